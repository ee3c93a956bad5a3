"""The op-level API on the HIP kernels, against the oracle's restatement of
online_attention / online_attention_statistics / merge_softmax
(online_attention.py:42-63, 74-219): explicit ``AttentionBlock`` pages with gaps,
offsets, key and query padding, causal and non-causal rows, windows with and without
causality, GQA, the three code formats and three query dtypes."""

import numpy as np
import pytest
import torch

import aster_amd
from aster_amd import AttentionBlock, QuantizedKV, UnsupportedAttentionBackend
from oracle import reference_cpu as ref
from tests.gpu_util import assert_attention_close

pytestmark = pytest.mark.gpu

FP8_DTYPE = {"fp8_e4m3fn": torch.float8_e4m3fn, "fp8_e5m2": torch.float8_e5m2}


def _pages(rng, batch, hkv, dim, spans, fmt, qdtype, device, pad_fraction=0.0):
    """Blocks over the token spans [(offset, length), ...]: (device blocks, oracle blocks)."""
    dev_blocks, ref_blocks = [], []
    for offset, length in spans:
        sides = []
        for _ in range(2):
            x = rng.standard_normal((batch, hkv, length, dim)).astype(np.float32)
            q = ref.quantize_kv(x, fmt)
            codes = torch.from_numpy(np.ascontiguousarray(q.values)).to(device)
            if fmt != "int8":
                codes = codes.view(FP8_DTYPE[fmt])
            scales = torch.from_numpy(np.ascontiguousarray(q.scales)).to(device)
            sides.append((QuantizedKV(codes, scales, qdtype), q))
        padding = None
        if pad_fraction:
            padding = (rng.random((batch, length)) >= pad_fraction).astype(np.int32)
        dev_blocks.append(AttentionBlock(sides[0][0], sides[1][0], offset,
                                         None if padding is None else
                                         torch.from_numpy(padding).to(device)))
        ref_blocks.append(ref.AttentionBlock(sides[0][1], sides[1][1], offset, padding))
    return dev_blocks, ref_blocks


def _run(device, *, batch=2, hq=8, hkv=2, dim=128, queries=5, spans=((0, 20), (24, 33), (57, 7)),
         fmt="int8", qdtype=torch.bfloat16, causal=True, window=None, pad_fraction=0.0,
         query_pad=False, positions=None, seed=0):
    rng = np.random.default_rng(seed)
    dev_blocks, ref_blocks = _pages(rng, batch, hkv, dim, spans, fmt, qdtype, device, pad_fraction)
    q32 = rng.standard_normal((batch, hq, queries, dim)).astype(np.float32)
    query = torch.from_numpy(q32).to(device).to(qdtype)
    last = max(o + n for o, n in spans)
    if positions is None:
        positions = np.stack([np.sort(rng.choice(last + 3, queries, replace=False))
                              for _ in range(batch)])
    positions = np.asarray(positions, np.int64)
    qpad = (rng.random((batch, queries)) >= 0.3).astype(np.int32) if query_pad else None
    kw = dict(causal=causal, window=window, scale=dim ** -0.5)
    got = aster_amd.online_attention(
        query, dev_blocks, query_positions=torch.from_numpy(positions).to(device),
        query_padding=None if qpad is None else torch.from_numpy(qpad).to(device), **kw)
    want = ref.online_attention(query.double().cpu().numpy(), ref_blocks, query_positions=positions,
                                query_padding=qpad, **kw)
    assert got.shape == query.shape and got.dtype == qdtype and got.is_contiguous()
    assert_attention_close(got.float().cpu().numpy(), want)
    return got


@pytest.mark.parametrize("fmt", ["int8", "fp8_e4m3fn", "fp8_e5m2"])
@pytest.mark.parametrize("qdtype", [torch.bfloat16, torch.float16, torch.float32])
def test_formats_and_query_dtypes(device, fmt, qdtype):
    _run(device, fmt=fmt, qdtype=qdtype)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dim", [64, 128, 256])
def test_causality_and_head_dims(device, causal, dim):
    _run(device, causal=causal, dim=dim, seed=dim)


@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 2), (16, 1)])
def test_gqa_groups(device, hq, hkv):
    _run(device, hq=hq, hkv=hkv, seed=hq)


def test_window_key_and_query_padding(device):
    _run(device, window=12, pad_fraction=0.25, query_pad=True, queries=9, seed=3)


@pytest.mark.parametrize("window", [1, 5, 12, 40])
def test_noncausal_windows(device, window):
    """Windows without causality (online_attention.py:183-184): every key after
    ``p - window`` is visible, later keys included. Rows read their first visible
    block through a copy of their own; a window past the last key leaves no key."""
    positions = [[0, 3, 17, 30, 45, 64, 66, 90], [8, 16, 24, 31, 56, 63, 70, 200]]
    _run(device, causal=False, window=window, queries=8, positions=positions, seed=40 + window)


def test_noncausal_window_padding_and_formats(device):
    for k, fmt in enumerate(("int8", "fp8_e4m3fn", "fp8_e5m2")):
        _run(device, causal=False, window=9, pad_fraction=0.25, query_pad=True, queries=7,
             fmt=fmt, qdtype=(torch.bfloat16, torch.float16, torch.float32)[k], seed=50 + k)


def test_gaps_offsets_and_queries_before_any_key(device):
    # keys only at [40, 56) and [70, 100); queries at 0 and 10 see nothing (zero rows)
    got = _run(device, spans=((40, 16), (70, 30)), positions=[[0, 10, 45, 69, 99]] * 2, seed=4)
    assert torch.count_nonzero(got[:, :, :2]) == 0


def test_many_rows_take_the_partitioned_path(device):
    # 4 x 160 query tokens = 640 decode rows, beyond the stream-K kernel's 512
    _run(device, batch=4, queries=160, spans=((0, 90), (100, 80)), seed=5)


def test_work_counters_and_unsupported_cases(device):
    rng = np.random.default_rng(6)
    dev_blocks, _ = _pages(rng, 1, 2, 64, ((0, 16),), "int8", torch.bfloat16, device)
    q = torch.randn(1, 4, 2, 64, device=device, dtype=torch.bfloat16)
    pos = torch.tensor([[3, 15]], device=device)
    work = aster_amd.AttentionWork()
    aster_amd.online_attention(q, dev_blocks, query_positions=pos, work=work)
    assert work.query_tiles == 2 and work.key_tiles == 2 * 2 and work.max_key_tile == 16
    plain = AttentionBlock(torch.randn(1, 2, 16, 64, device=device, dtype=torch.bfloat16),
                           torch.randn(1, 2, 16, 64, device=device, dtype=torch.bfloat16), 0)
    with pytest.raises(UnsupportedAttentionBackend):  # unquantized pages
        aster_amd.online_attention(q, [plain], query_positions=pos)
    # a finite query whose scores exceed fp32 raises the reference's overflow error
    f32_blocks, _ = _pages(rng, 1, 2, 64, ((0, 16),), "int8", torch.float32, device)
    huge = torch.full((1, 4, 2, 64), 3e38, device=device)
    with pytest.raises(ValueError, match="overflow"):
        aster_amd.online_attention(huge, f32_blocks, query_positions=pos, scale=1.0)


def _state(rng, shape, width, device, kinds=()):
    m = rng.standard_normal(shape).astype(np.float32) * 4
    for index, value in kinds:
        m[index] = value
    l = rng.random(shape).astype(np.float32) + 0.5
    n = rng.standard_normal(shape + (width,)).astype(np.float32)
    dev = aster_amd.SoftmaxState(*(torch.from_numpy(a).to(device) for a in (m, l, n)))
    return dev, ref.SoftmaxState(m, l, n)


@pytest.mark.parametrize("width", [128, 6])
def test_merge_softmax(device, width):
    rng = np.random.default_rng(width)
    shape = (2, 3, 4, 5)
    specials_left = [((0, 0, 0, 0), -np.inf), ((0, 0, 0, 1), -np.inf), ((1, 2, 3, 4), np.nan)]
    specials_right = [((0, 0, 0, 0), -np.inf), ((0, 0, 0, 2), np.inf)]
    left, left_ref = _state(rng, shape, width, device, specials_left)
    right, right_ref = _state(rng, shape, width, device, specials_right)
    got = aster_amd.merge_softmax(left, right)
    want = ref.merge_softmax(left_ref, right_ref)
    for g, w in ((got.maximum, want.maximum), (got.mass, want.mass), (got.weighted, want.weighted)):
        np.testing.assert_allclose(g.cpu().numpy(), w, rtol=2e-6, atol=1e-6, equal_nan=True)
    # the merged state normalises to the attention output, as the reference's does
    np.testing.assert_allclose(got.output().cpu().numpy(), want.output(), rtol=2e-6, atol=1e-6,
                               equal_nan=True)
    with pytest.raises(ValueError, match="same queries"):
        bad, _ = _state(rng, (2, 3, 4, 6), width, device)
        aster_amd.merge_softmax(left, bad)


@pytest.mark.parametrize("causal,window", [(True, None), (True, 24), (False, None)])
def test_pages_at_large_offsets(device, causal, window):
    """Pages around position 1e5 (and a second group near 1e5 + 4000): the transient
    arena spans the keys, not their absolute offsets. Queries before every key, between
    the groups and past the last key, with and without a window."""
    spans = ((100000, 20), (100024, 33), (100057, 7), (104000, 40))
    positions = [[5, 100010, 100040, 100063, 102000, 104039, 104100, 200000],
                 [99999, 100000, 100030, 100064, 104000, 104020, 104063, 104070]]
    _run(device, spans=spans, queries=8, positions=positions, causal=causal, window=window,
         seed=31)


def _statistics(device, *, batch=2, hq=8, hkv=2, dim=128, queries=6,
                spans=((0, 20), (24, 33), (57, 7)), fmt="int8", qdtype=torch.float32,
                causal=True, window=None, pad_fraction=0.0, query_pad=False, positions=None,
                seed=0, split=None):
    """online_attention_statistics on the HIP kernels against the oracle's float64
    statistics: the exact maximum and the mass and numerator relative to it, -inf/0
    rows where nothing is visible. ``split`` also merges the statistics of the pages
    before and after it with merge_softmax and checks the output against the whole."""
    rng = np.random.default_rng(seed)
    dev_blocks, ref_blocks = _pages(rng, batch, hkv, dim, spans, fmt, qdtype, device, pad_fraction)
    query = torch.from_numpy(rng.standard_normal((batch, hq, queries, dim)).astype(np.float32))
    query = query.to(device).to(qdtype)
    last = max(o + n for o, n in spans)
    if positions is None:
        positions = np.stack([np.sort(rng.choice(last + 3, queries, replace=False))
                              for _ in range(batch)])
    positions = np.asarray(positions, np.int64)
    qpad = (rng.random((batch, queries)) >= 0.3).astype(np.int32) if query_pad else None
    kw = dict(causal=causal, window=window, scale=dim ** -0.5)
    dev_kw = dict(kw, query_positions=torch.from_numpy(positions).to(device),
                  query_padding=None if qpad is None else torch.from_numpy(qpad).to(device))
    ref_kw = dict(kw, query_positions=positions, query_padding=qpad)
    q64 = query.double().cpu().numpy()
    got = aster_amd.online_attention_statistics(query, dev_blocks, **dev_kw)
    want = ref.online_attention_statistics(q64, ref_blocks, **ref_kw)
    groups = hq // hkv
    assert got.maximum.shape == (batch, hkv, groups, queries) == want.maximum.shape
    assert got.weighted.shape == (batch, hkv, groups, queries, dim)
    assert all(t.dtype == torch.float32 for t in (got.maximum, got.mass, got.weighted))
    m, l, w = (t.cpu().numpy() for t in (got.maximum, got.mass, got.weighted))
    empty = ~np.isfinite(want.maximum)
    np.testing.assert_array_equal(~np.isfinite(m), empty)
    assert (m[empty] == -np.inf).all() and (l[empty] == 0).all() and (w[empty] == 0).all()
    # scores of N(0, 1) rows are O(1): fp32 scores against float64 ones
    np.testing.assert_allclose(m[~empty], want.maximum[~empty], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(l, want.mass, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(w, want.weighted, rtol=1e-4, atol=1e-4)
    # the state normalises to online_attention's rows
    out = aster_amd.online_attention(query, dev_blocks, **dev_kw)
    assert_attention_close(got.output(dtype=qdtype).float().cpu().numpy(), out.float().cpu().numpy())
    if split is not None:
        left = aster_amd.online_attention_statistics(query, dev_blocks[:split], **dev_kw)
        right = aster_amd.online_attention_statistics(query, dev_blocks[split:], **dev_kw)
        merged = aster_amd.merge_softmax(left, right).output().cpu().numpy()
        assert_attention_close(merged, want.output())
    return got


@pytest.mark.parametrize("fmt", ["int8", "fp8_e4m3fn", "fp8_e5m2"])
@pytest.mark.parametrize("qdtype", [torch.bfloat16, torch.float16, torch.float32])
def test_statistics_formats_and_query_dtypes(device, fmt, qdtype):
    _statistics(device, fmt=fmt, qdtype=qdtype, split=1)


@pytest.mark.parametrize("dim", [64, 128, 256])
@pytest.mark.parametrize("causal,window", [(True, None), (True, 10), (False, None), (False, 7)])
def test_statistics_masks_and_head_dims(device, dim, causal, window):
    _statistics(device, dim=dim, causal=causal, window=window, pad_fraction=0.2, query_pad=True,
                seed=dim + (window or 0), split=2)


@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 2), (16, 1)])
def test_statistics_gqa_and_empty_rows(device, hq, hkv):
    # keys only at [40, 56) and [70, 100): queries at 0 and 10 see nothing
    got = _statistics(device, hq=hq, hkv=hkv, spans=((40, 16), (70, 30)), queries=5,
                      positions=[[0, 10, 45, 69, 99]] * 2, seed=hq, split=1)
    assert (got.maximum[..., :2] == -torch.inf).all()


def test_statistics_long_rows_merge_partitions(device):
    # 1500 keys: three 512-token partitions per row, merged with the exact maximum
    _statistics(device, spans=((0, 700), (700, 800)), queries=4,
                positions=[[100, 600, 1200, 1499], [511, 512, 1023, 1600]], seed=70, split=1)


def test_statistics_extreme_scores(device):
    """Scores far beyond the decode kernels' lazy-rescale slack (2^8): the statistics
    keep the exact maximum, so the mass stays O(keys)."""
    rng = np.random.default_rng(80)
    dev_blocks, ref_blocks = _pages(rng, 1, 2, 64, ((0, 48),), "int8", torch.float32, device)
    query = torch.from_numpy(rng.standard_normal((1, 4, 3, 64)).astype(np.float32) * 60)
    query = query.to(device)
    positions = np.array([[10, 30, 47]])
    got = aster_amd.online_attention_statistics(
        query, dev_blocks, query_positions=torch.from_numpy(positions).to(device))
    want = ref.online_attention_statistics(query.double().cpu().numpy(), ref_blocks,
                                           query_positions=positions)
    np.testing.assert_allclose(got.maximum.cpu().numpy(), want.maximum, rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(got.mass.cpu().numpy(), want.mass, rtol=1e-3, atol=1e-4)
    np.testing.assert_allclose(got.weighted.cpu().numpy(), want.weighted, rtol=1e-3, atol=1e-3)
