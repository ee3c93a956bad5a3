"""Value ranges and argument contracts of the attention kernels beyond the seeded N(0,1)
workloads, each against the oracle (online_attention.py:74-219 per row):

* large V scales: the PV weights and V operands are rounded to f16, so V scales big
  enough to overflow f16 (INT8 beyond ~3e4, E4M3FN beyond 448, E5M2 beyond ~5.7e4 in
  decode; any format beyond 65504 in chunk rows) must be carried by a power-of-two
  exponent instead; attention is linear in V, so V scales times 2^k give outputs 2^k
  as large, within the tolerance scaled the same way;
* extreme finite scores, after the reference's own test
  (tests/unit/test_inference_online_attention.py:79-98: q x 100, k x 100, against a
  float64 oracle), in decode rows (both split modes) and chunk rows;
* the checks on a caller's ``out`` and ``workspace``, and a ``max_query_len`` smaller
  than a row's query count (which would leave that row unwritten) raising the index
  flag."""

import numpy as np
import pytest
import torch

from aster_amd import KVQuantization, PagedKVCache
from aster_amd import workloads as wl
from tests.gpu_util import arena_numpy, assert_attention_close, oracle_decode

pytestmark = pytest.mark.gpu

FORMATS = ["int8", "fp8_e4m3fn", "fp8_e5m2"]


def _workload(q_lens, ctx, *, hq=32, hkv=8, dim=128, qdtype=torch.bfloat16, seed=11):
    ctx = np.asarray(ctx, np.int32)
    rng = np.random.default_rng(seed)
    tables, pool = wl._tables_from_lengths(ctx, rng, spare_blocks=3)
    q_lens = None if q_lens is None else np.asarray(q_lens, np.int32)
    return wl.DecodeWorkload("range", hq, hkv, dim, ctx, tables, pool, qdtype, seed, dim ** -0.5,
                             query_lens=q_lens)


def _build(w, device, fmt):
    cache = PagedKVCache(num_blocks=w.num_blocks, num_layers=1, num_kv_heads=w.num_kv_heads,
                         head_dim=w.head_dim, device=device, quantization=KVQuantization(fmt))
    wl.materialize(w, cache, device=device)
    tables, lens = wl.device_tables(w, device)
    return cache, tables, lens


def _attend(cache, w, q, tables, lens, **kw):
    if w.query_lens is not None:
        kw.update(query_start_loc=wl.device_query_start(w, q.device),
                  max_query_len=w.max_query_len)
    return cache.paged_attention(0, q, tables, lens, max_context_len=w.max_context_len,
                                 scale=w.scale, check=True, **kw)


DECODE_CTX = [1, 17, 255, 600, 33, 1000, 129, 2048]
MIXED_Q = [2, 31, 1, 32, 33, 1, 65, 129, 1, 7]
MIXED_CTX = [2, 71, 300, 48, 38, 1, 265, 462, 17, 1007]


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("qdtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("part", [0, 128])
@pytest.mark.parametrize("k", [9, 20])
def test_large_v_scales_in_decode_rows(device, fmt, qdtype, part, k):
    w = _workload(None, DECODE_CTX, qdtype=qdtype, seed=70 + k)
    cache, tables, lens = _build(w, device, fmt)
    cache.scales[:, 0, 1] *= 2.0 ** k
    q = wl.queries(w, device)
    out = _attend(cache, w, q, tables, lens, partition_tokens=part)
    assert torch.isfinite(out).all()
    assert_attention_close(out, oracle_decode(w, cache, q), atol=2e-3 * 2.0 ** k)


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("part", [0, 512])
@pytest.mark.parametrize("k", [9, 20])
def test_large_v_scales_in_chunk_rows(device, fmt, part, k):
    w = _workload(MIXED_Q, MIXED_CTX, seed=80 + k)
    cache, tables, lens = _build(w, device, fmt)
    cache.scales[:, 0, 1] *= 2.0 ** k
    q = wl.queries(w, device)
    out = _attend(cache, w, q, tables, lens, partition_tokens=part)
    assert torch.isfinite(out).all()
    assert_attention_close(out, oracle_decode(w, cache, q), atol=2e-3 * 2.0 ** k)


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("part", [0, 128])
@pytest.mark.parametrize("dim", [64, 128, 256])
def test_mixed_v_scale_ranges_within_rows(device, fmt, part, dim):
    """Every third block's V scales times 2^12, the others unchanged: pieces and query
    tiles meet blocks of both ranges (the weight factor or the block exponent changes
    mid-row), in decode and chunk rows of one step. Every head size: the decode blocks
    screen their scales after the QK MFMAs up to D = 128 and before them at D = 256."""
    w = _workload(MIXED_Q, MIXED_CTX, hq=16, hkv=4, dim=dim, seed=90 + dim)
    cache, tables, lens = _build(w, device, fmt)
    cache.scales[::3, 0, 1] *= 2.0 ** 12
    q = wl.queries(w, device)
    out = _attend(cache, w, q, tables, lens, partition_tokens=part)
    assert torch.isfinite(out).all()
    assert_attention_close(out, oracle_decode(w, cache, q), atol=2e-3 * 2.0 ** 12)


def _fp32_score_sensitivity(w, cache, query, exact):
    """Per output element, sum_t w_t |V_t - o| eps_t: how far the attention output of a
    query moves (to first order: d o / d s_t = w_t (V_t - o)) when each score s_t
    carries eps_t = 4 sqrt(D) 2^-24 sum_d |q_d k_td| scale, the rounding an fp32
    evaluation of the score (the reference's own included) may carry, with the exact
    weights and values (float64, dequantized codes, causal chunk positions). Nothing
    here depends on how the kernels compute: they are held to what any fp32 evaluation
    of the same codes may differ by."""
    kc, ks, vc, vs = arena_numpy(cache)
    q = query.double().cpu().numpy()
    dim, group = w.head_dim, w.num_q_heads // w.num_kv_heads
    qlens = w.q_lens
    extra = np.zeros_like(exact)
    cursor = 0
    for b, ctx in enumerate(w.context_lens.tolist()):
        n = int(qlens[b])
        if n == 0 or ctx == 0:
            cursor += n
            continue
        pages = w.block_tables[b][: (ctx + 15) // 16]
        keys = kc[pages].transpose(1, 0, 2, 3).reshape(w.num_kv_heads, -1, dim)[:, :ctx]
        kscl = ks[pages].transpose(1, 0, 2).reshape(w.num_kv_heads, -1)[:, :ctx]
        vals = vc[pages].transpose(1, 0, 2, 3).reshape(w.num_kv_heads, -1, dim)[:, :ctx]
        vscl = vs[pages].transpose(1, 0, 2).reshape(w.num_kv_heads, -1)[:, :ctx]
        k = keys.astype(np.float64) * kscl[..., None]
        v = vals.astype(np.float64) * vscl[..., None]
        for i in range(n):
            pos = ctx - n + i
            for h in range(w.num_q_heads):
                qh, kh, vh = q[cursor + i, h], k[h // group, : pos + 1], v[h // group, : pos + 1]
                s = kh @ qh * w.scale
                p = np.exp(s - s.max())
                p /= p.sum()
                eps = 4 * np.sqrt(dim) * 2.0 ** -24 * (np.abs(kh) @ np.abs(qh)) * w.scale
                extra[cursor + i, h] = (p * eps) @ np.abs(vh - exact[cursor + i, h])
        cursor += n
    return extra


def _assert_within_fp32_rounding(w, cache, q, out):
    """The tolerance around the exact (float64) result, widened only by the softmax's
    first-order response to fp32 rounding of the scores (zero where the attention is
    well posed)."""
    exact = oracle_decode(w, cache, q, fp64=True)
    extra = _fp32_score_sensitivity(w, cache, q, exact)
    err = np.abs(out.double().cpu().numpy() - exact)
    bound = 2e-3 + 1e-2 * np.abs(exact) + extra
    assert (err <= bound).all(), (float((err - bound).max()), int((err > bound).sum()))
    return extra


@pytest.mark.parametrize("qdtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("dim", [64, 128, 256])
@pytest.mark.parametrize("part", [0, 512])
def test_extreme_finite_scores(device, qdtype, dim, part):
    """q x 100 and k x 100 (test_inference_online_attention.py:79-98): scores of
    thousands, so every block past the first moves the running maximum far beyond the
    lazy-rescale slack; outputs stay finite and match the float64 oracle within the
    tolerance plus what fp32 rounding of the scores may move them
    (_fp32_score_sensitivity), in decode rows (both split modes) and chunk rows."""
    for q_lens, ctx in ((None, DECODE_CTX), (MIXED_Q, MIXED_CTX)):
        w = _workload(q_lens, ctx, hq=16, hkv=4, dim=dim, qdtype=qdtype, seed=dim + 5)
        cache, tables, lens = _build(w, device, "int8")
        cache.scales[:, 0, 0] *= 100.0
        q = (wl.queries(w, device).float() * 100.0).to(qdtype)
        out = _attend(cache, w, q, tables, lens, partition_tokens=part)
        assert torch.isfinite(out).all()
        extra = _assert_within_fp32_rounding(w, cache, q, out)
        assert (extra > 2e-3).any(-1).mean() < 0.05  # ill-posed (query, head) rows are rare


@pytest.mark.parametrize("part", [0, 128])
@pytest.mark.parametrize("dim", [64, 128])
def test_key_scale_outliers_past_the_group_tokens(device, part, dim):
    """One token of every block, at a slot r >= G (G = 4 here), carries a key scale
    x 400 while the other keys stay N(0,1): a test of large scores that looks only at
    the first G tokens of a block, or only at each column's own token, would miss it.
    Decode and chunk rows, held to the float64 oracle without any allowance for how
    the kernels quantize the query."""
    for q_lens, ctx in ((None, DECODE_CTX), (MIXED_Q, MIXED_CTX)):
        w = _workload(q_lens, ctx, hq=16, hkv=4, dim=dim, seed=dim + 17)
        cache, tables, lens = _build(w, device, "int8")
        cache.scales[:, 0, 0, :, 11] *= 400.0
        q = wl.queries(w, device)
        out = _attend(cache, w, q, tables, lens, partition_tokens=part)
        assert torch.isfinite(out).all()
        _assert_within_fp32_rounding(w, cache, q, out)


@pytest.mark.parametrize("dim", [64, 128, 256])
def test_scores_near_the_chunk_third_term_threshold(device, dim):
    """Keys x 3 and queries x 3: the chunk rows' steps sit around the key scale at
    which the prefill kernel adds its third query term (some take it, most not), and
    both kinds of step are held to the float64 oracle at the plain tolerance plus fp32
    rounding."""
    w = _workload(MIXED_Q, MIXED_CTX, hq=16, hkv=4, dim=dim, seed=dim + 29)
    cache, tables, lens = _build(w, device, "int8")
    cache.scales[:, 0, 0] *= 3.0
    q = (wl.queries(w, device).float() * 3.0).to(torch.bfloat16)
    out = _attend(cache, w, q, tables, lens)
    assert torch.isfinite(out).all()
    _assert_within_fp32_rounding(w, cache, q, out)


def test_out_and_workspace_are_checked(device):
    w = _workload(None, [40, 300, 17])
    cache, tables, lens = _build(w, device, "int8")
    q = wl.queries(w, device)
    kw = dict(max_context_len=w.max_context_len)
    for bad in (torch.empty(2, 32, 128, device=device, dtype=q.dtype),       # shape
                torch.empty_like(q, dtype=torch.float32),                     # dtype
                torch.empty(3, 32, 256, device=device, dtype=q.dtype)[..., ::2],  # strides
                torch.empty(q.shape, dtype=q.dtype)):                         # host
        with pytest.raises(ValueError, match="out must"):
            cache.paged_attention(0, q, tables, lens, out=bad, **kw)
    need = cache.workspace_bytes(3, 32, w.max_context_len)
    assert need > 0
    for bad in (torch.empty(need, dtype=torch.uint8),                           # host
                torch.empty(need // 4 + 1, dtype=torch.int32, device=device),  # dtype
                torch.empty(2 * need, dtype=torch.uint8, device=device)[::2]):  # strided
        with pytest.raises(ValueError, match="workspace must"):
            cache.paged_attention(0, q, tables, lens, workspace=bad, **kw)
    with pytest.raises(ValueError, match="bytes required"):
        cache.paged_attention(0, q, tables, lens, workspace=torch.empty(
            need - 256, dtype=torch.uint8, device=device), **kw)
    out = torch.empty_like(q)
    ws = torch.empty(need, dtype=torch.uint8, device=device)
    got = cache.paged_attention(0, q, tables, lens, out=out, workspace=ws, check=True, **kw)
    assert got.data_ptr() == out.data_ptr()
    assert_attention_close(out, oracle_decode(w, cache, q))


def test_max_query_len_below_a_rows_query_count_is_flagged(device):
    w = _workload([4, 1, 3], [20, 30, 40], seed=3)
    cache, tables, lens = _build(w, device, "int8")
    q = wl.queries(w, device)
    qsl = wl.device_query_start(w, device)
    for stale in (1, 3):  # 1: no chunk kernel at all; 3: row 0 (4 tokens) is too long
        with pytest.raises(ValueError, match="outside"):
            cache.paged_attention(0, q, tables, lens, max_context_len=40, query_start_loc=qsl,
                                  max_query_len=stale, check=True)
    out = cache.paged_attention(0, q, tables, lens, max_context_len=40, query_start_loc=qsl,
                                max_query_len=4, check=True)
    assert_attention_close(out, oracle_decode(w, cache, q))
