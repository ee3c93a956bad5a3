"""GPU parity of the mixed chunked-prefill + decode step (astr_paged_attention_varlen_i8)
against the oracle's row-by-row online softmax with multi-token rows
(online_attention.py:74-219 as called per row by paged_attention.py:168-215:
query i of an n-token chunk sits at position ctx - n + i), within the north_star
tolerance |a-b| <= 2e-3 + 1e-2|b|, plus cross-kernel and size-independent checks."""

import numpy as np
import pytest
import torch

from aster_amd import KernelWork, KVQuantization, PagedKVCache
from aster_amd import workloads as wl
from tests.gpu_util import assert_attention_close, mark_padding, oracle_decode

pytestmark = pytest.mark.gpu


def _mixed(q_lens, ctx, *, hq=32, hkv=8, dim=128, qdtype=torch.bfloat16, seed=11):
    q_lens = np.asarray(q_lens, np.int32)
    ctx = np.asarray(ctx, np.int32)
    rng = np.random.default_rng(seed)
    tables, pool = wl._tables_from_lengths(ctx, rng, spare_blocks=5)
    return wl.DecodeWorkload("mixed", hq, hkv, dim, ctx, tables, pool, qdtype, seed, dim ** -0.5,
                             query_lens=q_lens)


def _build(w, device, fmt="int8"):
    cache = PagedKVCache(num_blocks=w.num_blocks, num_layers=1, num_kv_heads=w.num_kv_heads,
                         head_dim=w.head_dim, device=device, quantization=KVQuantization(fmt))
    wl.materialize(w, cache, device=device)
    tables, lens = wl.device_tables(w, device)
    return cache, tables, lens, wl.device_query_start(w, device)


def _run(cache, w, q, tables, lens, qsl, **kw):
    return cache.paged_attention(0, q, tables, lens, max_context_len=w.max_context_len,
                                 scale=w.scale, query_start_loc=qsl,
                                 max_query_len=w.max_query_len, check=True, **kw)


# chunk lengths around the query-tile sizes (128/G tokens per workgroup) and
# priors that are not block multiples, mixed with decode rows and a 0-token row
Q_LENS = [2, 31, 1, 32, 33, 1, 65, 0, 129, 1, 7]
CTX = [2, 31 + 40, 300, 32 + 16, 33 + 5, 1, 65 + 200, 50, 129 + 333, 17, 7 + 1000]


@pytest.mark.parametrize("dim,hq,hkv", [(128, 32, 8), (128, 8, 8), (128, 32, 2), (64, 16, 2),
                                        (256, 8, 2), (128, 128, 8)])
@pytest.mark.parametrize("qdtype", [torch.bfloat16, torch.float16, torch.float32])
def test_mixed_rows_match_oracle(device, dim, hq, hkv, qdtype):
    w = _mixed(Q_LENS, CTX, hq=hq, hkv=hkv, dim=dim, qdtype=qdtype, seed=dim + hq)
    cache, tables, lens, qsl = _build(w, device)
    q = wl.queries(w, device)
    work = KernelWork()
    out = _run(cache, w, q, tables, lens, qsl, work=work)
    assert out.shape == q.shape and out.dtype == qdtype
    assert_attention_close(out, oracle_decode(w, cache, q))
    assert work.backend == "hip_int8_paged" and work.max_query_tile == 129


@pytest.mark.parametrize("window", [1, 5, 16, 40, 300])
@pytest.mark.parametrize("causal", [True, False])
def test_window_and_causality(device, window, causal):
    w = _mixed(Q_LENS, CTX, seed=5)
    cache, tables, lens, qsl = _build(w, device)
    q = wl.queries(w, device)
    out = _run(cache, w, q, tables, lens, qsl, window=window, causal=causal)
    assert_attention_close(out, oracle_decode(w, cache, q, window=window, causal=causal))


@pytest.mark.parametrize("dim,hq,hkv", [(128, 32, 8), (64, 16, 2), (256, 8, 2)])
@pytest.mark.parametrize("window", [None, 40])
def test_key_padding_in_chunks(device, dim, hq, hkv, window):
    """Padding keys, in the history and in the step's own chunk (the runner appends
    the chunk with its padding leaf before attention, paged_attention.py:190 and
    :228-229), are seen by no query of the prefill or decode rows."""
    w = _mixed(Q_LENS, CTX, hq=hq, hkv=hkv, dim=dim, seed=dim + 3)
    cache, tables, lens, qsl = _build(w, device)
    mark_padding(cache, w.block_tables, w.context_lens, 0.2, seed=dim, whole_blocks=2)
    q = wl.queries(w, device)
    out = _run(cache, w, q, tables, lens, qsl, window=window)
    assert_attention_close(out, oracle_decode(w, cache, q, window=window))


@pytest.mark.parametrize("fmt", ["fp8_e4m3fn", "fp8_e5m2"])
@pytest.mark.parametrize("dim,hq,hkv", [(128, 32, 8), (64, 16, 2), (256, 8, 2)])
@pytest.mark.parametrize("qdtype", [torch.bfloat16, torch.float16, torch.float32])
def test_fp8_kv_formats_in_mixed_steps(device, fmt, dim, hq, hkv, qdtype):
    """FP8 arenas on the prefill kernel's f16 QK path (chunk rows) and the decode kernels
    (decode rows) of one mixed step, causal and windowed."""
    w = _mixed(Q_LENS, CTX, hq=hq, hkv=hkv, dim=dim, qdtype=qdtype, seed=dim + 1)
    cache, tables, lens, qsl = _build(w, device, fmt)
    q = wl.queries(w, device)
    for window in (None, 40):
        out = _run(cache, w, q, tables, lens, qsl, window=window)
        assert_attention_close(out, oracle_decode(w, cache, q, window=window))


@pytest.mark.parametrize("fmt", ["int8", "fp8_e4m3fn", "fp8_e5m2"])
def test_small_values_keep_their_precision(device, fmt):
    """V scales times 2^-6 (exact) give outputs 2^-6 as large within the tolerance
    scaled the same way, on the chunk and decode rows of one step (E5M2's scales lie
    below f16's normal range unless lifted before the V operands are rounded)."""
    w = _mixed(Q_LENS, CTX, hq=32, hkv=8, dim=128, seed=62)
    cache, tables, lens, qsl = _build(w, device, fmt)
    cache.scales[:, 0, 1] *= 2.0 ** -6
    q = wl.queries(w, device)
    out = _run(cache, w, q, tables, lens, qsl)
    assert_attention_close(out, oracle_decode(w, cache, q), atol=2e-3 * 2.0 ** -6)


def test_tiny_query_heads(device):
    """Query heads scaled by 2^-100 (column maxima below the 2^-64 under which the int8
    query path lifts a column by 2^64 before quantizing it) beside heads at full scale
    in the same waves: the tiny heads' scores vanish (near-uniform attention over their
    visible keys) and the other heads are unaffected."""
    w = _mixed(Q_LENS, CTX, hq=32, hkv=8, dim=128, seed=63)
    cache, tables, lens, qsl = _build(w, device)
    q = wl.queries(w, device)
    q[:, 1::3] *= 2.0 ** -100
    out = _run(cache, w, q, tables, lens, qsl)
    assert torch.isfinite(out).all()
    assert_attention_close(out, oracle_decode(w, cache, q))


def test_step_without_query_tokens(device):
    """Rows with no query token this step (and a step where no row has one) write
    nothing and raise nothing."""
    w = _mixed([0, 0, 0], [40, 0, 300], hq=32, hkv=8, dim=128, seed=64)
    cache, tables, lens, qsl = _build(w, device)
    q = wl.queries(w, device)
    out = _run(cache, w, q, tables, lens, qsl)
    assert out.shape == (0, 32, 128)
    assert_attention_close(out, oracle_decode(w, cache, q))


@pytest.mark.parametrize("bad", [float("inf"), float("nan")])
@pytest.mark.parametrize("row_kind", ["decode", "chunk"])
@pytest.mark.parametrize("part,qdtype,fmt", [(0, torch.bfloat16, "int8"),
                                             (512, torch.bfloat16, "int8"),
                                             (0, torch.float32, "int8"),
                                             (0, torch.bfloat16, "fp8_e4m3fn")])
def test_non_finite_query_is_reported(device, bad, row_kind, part, qdtype, fmt):
    """A non-finite query element makes that head's scores non-finite, which the
    reference rejects (online_attention.py:193-196): the call raises ValueError, from a
    decode row (its interior and edge blocks) and from a chunk row alike."""
    w = _mixed(Q_LENS, CTX, hq=32, hkv=8, dim=128, qdtype=qdtype, seed=65)
    cache, tables, lens, qsl = _build(w, device, fmt)
    q = wl.queries(w, device)
    tok = 33 if row_kind == "decode" else 10  # row 2 (context 300) / a token of row 1's chunk
    q[tok, 5, 17] = bad
    with pytest.raises(ValueError, match="score overflow"):
        _run(cache, w, q, tables, lens, qsl, partition_tokens=part)


def test_non_causal_without_window(device):
    w = _mixed(Q_LENS, CTX, seed=6)
    cache, tables, lens, qsl = _build(w, device)
    q = wl.queries(w, device)
    out = _run(cache, w, q, tables, lens, qsl, causal=False)
    assert_attention_close(out, oracle_decode(w, cache, q, causal=False))


@pytest.mark.parametrize("part", [0, 512, 64])
def test_scaled_config3_matches_oracle(device, part):
    w = wl.config3(num_prefill=3, chunk=200, max_prior=600, num_decode=9)
    cache, tables, lens, qsl = _build(w, device)
    q = wl.queries(w, device)
    out = _run(cache, w, q, tables, lens, qsl, partition_tokens=part)
    assert_attention_close(out, oracle_decode(w, cache, q))


@pytest.mark.parametrize("rows", [256, 257])
def test_many_chunk_rows(device, rows):
    """Chunk rows are dispatched longest first up to 256 of them and in index order
    beyond: both sides of that boundary, with decode rows interleaved."""
    rng = np.random.default_rng(rows)
    q_lens = rng.integers(2, 24, rows + rows // 6)
    q_lens[rng.choice(q_lens.size, rows // 6, replace=False)] = 1  # exactly `rows` chunk rows
    ctx = q_lens + rng.integers(0, 160, q_lens.size)
    w = _mixed(q_lens, ctx, hq=4, hkv=2, dim=64, seed=rows)
    cache, tables, lens, qsl = _build(w, device)
    q = wl.queries(w, device)
    out = _run(cache, w, q, tables, lens, qsl)
    assert_attention_close(out, oracle_decode(w, cache, q))


def test_chunk_last_token_equals_decode_kernel(device):
    """The last query of a chunk sees exactly the keys a decode query at ctx-1 sees:
    the prefill kernel and the decode kernels agree on it."""
    w = _mixed([40, 97, 300], [40 + 64, 97 + 1000, 300 + 17], seed=9)
    cache, tables, lens, qsl = _build(w, device)
    q = wl.queries(w, device)
    out = _run(cache, w, q, tables, lens, qsl)
    last = torch.as_tensor(w.query_start_loc()[1:] - 1, device=device).long()
    dec = cache.paged_attention(0, q[last].contiguous(), tables, lens,
                                max_context_len=w.max_context_len, scale=w.scale, check=True)
    assert_attention_close(out[last], dec)


def test_full_config3_step(device):
    """The full config3 workload: quantize-append the step's 4216 tokens, then one
    mixed launch; oracle on two chunks and four decode rows, and every output row
    finite with |o| bounded by max|v| (a convex combination of dequantized values)."""
    w = wl.config3()
    cache = PagedKVCache(num_blocks=w.num_blocks, num_layers=1, num_kv_heads=w.num_kv_heads,
                         head_dim=w.head_dim, device=device)
    _, (k, v, slots) = wl.materialize(w, cache, device=device, hold_last=True)
    assert k.shape[0] == w.num_query_tokens == 8 * 512 + 120
    cache.append(0, k, v, slots, check=True)
    tables, lens = wl.device_tables(w, device)
    qsl = wl.device_query_start(w, device)
    q = wl.queries(w, device)
    out = _run(cache, w, q, tables, lens, qsl)
    assert torch.isfinite(out.float()).all()
    vmax = (cache.codes[:, 0, 1].float().abs().amax(-1) * cache.scales[:, 0, 1]).max()
    assert out.float().abs().max() <= vmax * 1.01
    rows = [0, 5, 8, 50, 100, 127]
    sub = wl.DecodeWorkload("sub", w.num_q_heads, w.num_kv_heads, w.head_dim,
                            w.context_lens[rows], w.block_tables[rows], w.num_blocks, w.q_dtype,
                            w.seed, w.scale, query_lens=w.q_lens[rows])
    qsl_h = w.query_start_loc()
    take = np.concatenate([np.arange(qsl_h[r], qsl_h[r + 1]) for r in rows])
    take_t = torch.as_tensor(take, device=device).long()
    assert_attention_close(out[take_t], oracle_decode(sub, cache, q[take_t]))


def test_invalid_offsets_and_short_context_are_flagged(device):
    w = _mixed([4, 1, 3], [20, 30, 40], seed=2)
    cache, tables, lens, qsl = _build(w, device)
    q = wl.queries(w, device)
    bad = qsl.clone()
    bad[1] = 9  # decreasing offsets: the affected rows are skipped, the step is flagged
    with pytest.raises(ValueError, match="outside"):
        _run(cache, w, q, tables, lens, bad)
    short = lens.clone()
    short[0] = 3  # a 4-token chunk cannot sit in a 3-token context
    with pytest.raises(ValueError, match="outside"):
        _run(cache, w, q, tables, short, qsl)
    out = _run(cache, w, q, tables, lens, qsl)  # the flag was cleared by the raise
    assert_attention_close(out, oracle_decode(w, cache, q))


@pytest.mark.parametrize("case", range(48))
def test_random_mixed_steps_match_oracle(device, case):
    """Seeded random mixed steps: head dim, GQA group, query dtype, decode/chunk/empty
    rows, causal or not, sliding window, split mode, code format and key padding drawn
    per case, each against the oracle at the north_star tolerance."""
    rng = np.random.default_rng(7000 + case)
    dim = int(rng.choice([64, 128, 256]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    g = int(rng.choice([1, 2, 4, 8, 16] if dim != 256 else [1, 2, 4, 8]))
    qdtype = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(3))]
    if qdtype == torch.float32:
        g = min(g, 8)  # fp32 decode rows run the exact VALU kernel (groups up to 8)
    nrows = int(rng.integers(1, 24))
    q_lens = np.where(rng.random(nrows) < 0.6, 1, rng.integers(2, 160, nrows)).astype(np.int32)
    q_lens[rng.random(nrows) < 0.05] = 0
    ctx = (q_lens + rng.integers(0, 900, nrows)).astype(np.int32)
    window = None if rng.random() < 0.6 else int(rng.integers(1, 400))
    causal = bool(rng.random() < 0.85)
    part = int(rng.choice([0, 0, 512, 64]))
    fmt = ["int8", "int8", "int8", "fp8_e4m3fn", "fp8_e5m2"][int(rng.integers(5))]
    w = _mixed(q_lens, ctx, hq=hkv * g, hkv=hkv, dim=dim, qdtype=qdtype, seed=9000 + case)
    cache, tables, lens, qsl = _build(w, device, fmt)
    if rng.random() < 0.3:
        mark_padding(cache, w.block_tables, w.context_lens, 0.15, seed=case)
    q = wl.queries(w, device)
    out = _run(cache, w, q, tables, lens, qsl, causal=causal, window=window,
               partition_tokens=part)
    assert_attention_close(out, oracle_decode(w, cache, q, causal=causal, window=window))
