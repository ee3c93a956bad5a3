"""GPU parity of the paged decode attention kernel against the oracle's page-by-page
online softmax (online_attention.py:74-219 via paged_attention.py:168-215), within
the north_star tolerance |a-b| <= 2e-3 + 1e-2|b|, plus size-independent
properties at the full BASELINE sizes."""

import math
import os

import numpy as np
import pytest
import torch

from aster_amd import KernelWork, KVQuantization, PagedKVCache, UnsupportedAttentionBackend
from aster_amd import workloads as wl
from tests.gpu_util import arena_numpy, assert_attention_close, mark_padding, oracle_decode

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _build(w, device, layers=1, fmt="int8"):
    cache = PagedKVCache(num_blocks=w.num_blocks, num_layers=layers, num_kv_heads=w.num_kv_heads,
                         head_dim=w.head_dim, device=device, quantization=KVQuantization(fmt))
    wl.materialize(w, cache, device=device)
    tables, lens = wl.device_tables(w, device)
    return cache, tables, lens


def test_config1_matches_golden_output(device):
    g = np.load(os.path.join(GOLDEN, "config1.npz"))
    cache = PagedKVCache(num_blocks=64, num_layers=1, num_kv_heads=4, head_dim=64, device=device)
    cache.append(0, torch.from_numpy(g["k"]).to(device), torch.from_numpy(g["v"]).to(device),
                 torch.from_numpy(g["slots"]).to(device), check=True)
    q = torch.from_numpy(g["q"]).to(device)
    tables = torch.from_numpy(g["block_tables"]).to(device)
    lens = torch.from_numpy(g["context_lens"]).to(device)
    work = KernelWork()
    for part in (0, 512, 64):
        out = cache.paged_attention(0, q, tables, lens, max_context_len=300, scale=64 ** -0.5,
                                    partition_tokens=part, work=work, check=True)
        assert out.dtype == torch.float32 and out.shape == (4, 4, 64)
        assert_attention_close(out, g["out"])
        # fp32 queries: far tighter than the north_star bound in practice
        assert_attention_close(out, g["out"], atol=2e-5, rtol=2e-5)
    assert work.backend == "hip_int8_paged" and work.fallback_reason is None


@pytest.mark.parametrize("builder,rows,max_len", [
    (wl.config2, 12, None),
    (wl.config4, 6, None),
    (wl.config5, 2, 3000),
])
@pytest.mark.parametrize("part", [0, 512, 64])
def test_scaled_configs_match_oracle(device, builder, rows, max_len, part):
    w = wl.scaled(builder(), num_seqs=rows, max_len=max_len)
    cache, tables, lens = _build(w, device)
    q = wl.queries(w, device)
    out = cache.paged_attention(0, q, tables, lens, max_context_len=w.max_context_len,
                                scale=w.scale, partition_tokens=part, check=True)
    assert out.dtype == w.q_dtype
    assert_attention_close(out, oracle_decode(w, cache, q))


@pytest.mark.parametrize("dim,hq,hkv", [(64, 8, 8), (128, 16, 8), (128, 32, 8), (128, 64, 8),
                                        (128, 128, 8), (256, 8, 2), (64, 16, 2)])
@pytest.mark.parametrize("qdtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("part", [0, 128])
def test_head_dims_groups_dtypes(device, dim, hq, hkv, qdtype, part):
    lens = np.array([1, 15, 16, 17, 255, 256, 257, 600, 0, 33], np.int32)
    rng = np.random.default_rng(dim + hq)
    tables, pool = wl._tables_from_lengths(lens, rng, spare_blocks=3)
    w = wl.DecodeWorkload("edge", hq, hkv, dim, lens, tables, pool, qdtype, 7, dim ** -0.5)
    cache, t, l = _build(w, device)
    q = wl.queries(w, device)
    out = cache.paged_attention(0, q, t, l, max_context_len=600, partition_tokens=part,
                                check=True)
    assert (out[8] == 0).all()
    assert_attention_close(out, oracle_decode(w, cache, q))


@pytest.mark.parametrize("window", [1, 7, 16, 100, 1000])
@pytest.mark.parametrize("part", [0, 128])
def test_sliding_window(device, window, part):
    w = wl.scaled(wl.config2(), num_seqs=6, max_len=700)
    cache, tables, lens = _build(w, device)
    q = wl.queries(w, device)
    out = cache.paged_attention(0, q, tables, lens, max_context_len=w.max_context_len,
                                window=window, partition_tokens=part, check=True)
    assert_attention_close(out, oracle_decode(w, cache, q, window=window))


@pytest.mark.parametrize("dim,hq,hkv", [(128, 32, 8), (64, 8, 2), (256, 8, 2)])
@pytest.mark.parametrize("qdtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("part", [0, 128])
def test_key_padding(device, dim, hq, hkv, qdtype, part):
    """Padding keys (the pages' padding leaf, online_attention.py:185-186) are never
    attended: a seeded 25 % of keys, two whole pages and one whole row (whose output
    is zero, online_attention.py:37), on every decode kernel (stream-K, fixed
    partitions, and the fp32 VALU kernel), with and without a sliding window."""
    lens = np.array([300, 17, 600, 1, 64, 250, 129, 40], np.int32)
    rng = np.random.default_rng(dim + hq)
    tables, pool = wl._tables_from_lengths(lens, rng, spare_blocks=3)
    w = wl.DecodeWorkload("pad", hq, hkv, dim, lens, tables, pool, qdtype, 5, dim ** -0.5)
    cache, t, l = _build(w, device)
    mark_padding(cache, tables, lens, 0.25, seed=dim, whole_rows=(5,), whole_blocks=2)
    q = wl.queries(w, device)
    for window in (None, 90):
        out = cache.paged_attention(0, q, t, l, max_context_len=600, partition_tokens=part,
                                    window=window, check=True)
        assert (out[5] == 0).all()
        assert_attention_close(out, oracle_decode(w, cache, q, window=window))


@pytest.mark.parametrize("fmt", ["fp8_e4m3fn", "fp8_e5m2"])
@pytest.mark.parametrize("dim,hq,hkv", [(128, 32, 8), (64, 8, 2), (256, 8, 2), (128, 64, 8)])
@pytest.mark.parametrize("qdtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("part", [0, 128])
def test_fp8_kv_formats(device, fmt, dim, hq, hkv, qdtype, part):
    """FP8 E4M3FN / E5M2 arenas (KVQuantization formats, kv_quantization.py:7-25):
    the codes enter the f16 MFMAs (or the fp32 VALU kernel) exactly, so the result
    matches the oracle's dequantize-then-attend within the same tolerance; with a
    window and key padding too."""
    lens = np.array([1, 15, 16, 17, 255, 256, 257, 600, 0, 33], np.int32)
    rng = np.random.default_rng(dim + hq)
    tables, pool = wl._tables_from_lengths(lens, rng, spare_blocks=3)
    w = wl.DecodeWorkload("fp8", hq, hkv, dim, lens, tables, pool, qdtype, 7, dim ** -0.5)
    cache, t, l = _build(w, device, fmt=fmt)
    q = wl.queries(w, device)
    out = cache.paged_attention(0, q, t, l, max_context_len=600, partition_tokens=part,
                                check=True)
    assert (out[8] == 0).all()
    assert_attention_close(out, oracle_decode(w, cache, q))
    mark_padding(cache, tables, lens, 0.2, seed=dim)
    out = cache.paged_attention(0, q, t, l, max_context_len=600, partition_tokens=part,
                                window=50, check=True)
    assert_attention_close(out, oracle_decode(w, cache, q, window=50))


@pytest.mark.parametrize("fmt", ["int8", "fp8_e4m3fn", "fp8_e5m2"])
@pytest.mark.parametrize("qdtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("part", [0, 128])
def test_small_values_keep_their_precision(device, fmt, qdtype, part):
    """Attention is linear in V: V scales times 2^-6 (an exact change of the arena)
    give outputs 2^-6 as large, within the tolerance scaled the same way. E5M2's
    scales (amax / 57344) lie below f16's normal range, so this needs the kernels to
    lift them before the PV weights are rounded to f16."""
    lens = np.array([1, 17, 255, 600, 33, 1000], np.int32)
    rng = np.random.default_rng(61)
    tables, pool = wl._tables_from_lengths(lens, rng, spare_blocks=3)
    w = wl.DecodeWorkload("small", 32, 8, 128, lens, tables, pool, qdtype, 9, 128 ** -0.5)
    cache, t, l = _build(w, device, fmt=fmt)
    cache.scales[:, 0, 1] *= 2.0 ** -6
    q = wl.queries(w, device)
    out = cache.paged_attention(0, q, t, l, max_context_len=1000, partition_tokens=part,
                                check=True)
    assert_attention_close(out, oracle_decode(w, cache, q), atol=2e-3 * 2.0 ** -6)


def test_empty_rows_are_zero_and_ctx_one_returns_value(device):
    lens = np.array([0, 1, 40, 0], np.int32)
    tables = np.array([[0, 0, 0], [1, 0, 0], [2, 3, 4], [0, 0, 0]], np.int32)
    w = wl.DecodeWorkload("empty", 8, 2, 128, lens, tables, 5, torch.bfloat16, 3, 128 ** -0.5)
    cache = PagedKVCache(num_blocks=5, num_layers=1, num_kv_heads=2, head_dim=128, device=device)
    wl.materialize(w, cache, device=device)
    t, l = wl.device_tables(w, device)
    q = wl.queries(w, device)
    out = cache.paged_attention(0, q, t, l, max_context_len=40, check=True)
    assert (out[0] == 0).all() and (out[3] == 0).all()
    # one visible key: the output is that dequantized value row (per kv head)
    kc, ks, vc, vs = arena_numpy(cache)
    vrow = vc[1, :, 0].astype(np.float32) * vs[1, :, 0, None]
    np.testing.assert_allclose(out[1].float().cpu().numpy(), np.repeat(vrow, 4, 0),
                               rtol=1e-2, atol=1e-6)


def test_full_config2_split_invariance_and_permutation(device):
    """The full config2 workload: split-K partition size does not change the result
    beyond tolerance, and relabelling physical blocks (permuting the arena and the
    block tables together) gives bit-identical output."""
    w = wl.config2()
    cache, tables, lens = _build(w, device)
    q = wl.queries(w, device)
    ref_out = cache.paged_attention(0, q, tables, lens, max_context_len=w.max_context_len,
                                    partition_tokens=4096, check=True)
    for part in (0, 512, 256, 64):
        out = cache.paged_attention(0, q, tables, lens, max_context_len=w.max_context_len,
                                    partition_tokens=part, check=True)
        assert_attention_close(out, ref_out.float().cpu().numpy())
    perm = torch.randperm(w.num_blocks, generator=torch.Generator().manual_seed(5))
    inverse = torch.argsort(perm).to(torch.int32)
    other = PagedKVCache(num_blocks=w.num_blocks, num_layers=1, num_kv_heads=8, head_dim=128,
                         device=device)
    other.codes.copy_(cache.codes[perm.to(device)])
    other.scales.copy_(cache.scales[perm.to(device)])
    tables2 = inverse.to(device)[tables.long()].to(torch.int32).contiguous()
    out2 = other.paged_attention(0, q, tables2, lens, max_context_len=w.max_context_len,
                                 check=True)
    out1 = cache.paged_attention(0, q, tables, lens, max_context_len=w.max_context_len,
                                 check=True)
    assert torch.equal(out1, out2)
    # a few full-length rows against the oracle
    sub = [int(i) for i in np.argsort(w.context_lens)[-2:]]
    ora = oracle_decode(w.block_tables[sub], cache, q[sub], context_lens=w.context_lens[sub],
                        scale=w.scale)
    assert_attention_close(out1[sub], ora)


def test_full_config5_long_context_rows_match_oracle(device):
    """32768-token rows with 10% x8 K outliers, 64 split-K partitions per row."""
    w = wl.config5()
    w = wl.DecodeWorkload(w.name, w.num_q_heads, w.num_kv_heads, w.head_dim, w.context_lens[:2],
                          w.block_tables[:2], w.num_blocks, w.q_dtype, w.seed, w.scale,
                          w.k_outlier_fraction)
    cache, tables, lens = _build(w, device)
    q = wl.queries(w, device)
    out = cache.paged_attention(0, q, tables, lens, max_context_len=32768, check=True)
    assert_attention_close(out, oracle_decode(w, cache, q))


def test_long_waves_stream_several_block_windows(device):
    """Stream-K waves streaming more than 64 blocks keep their block list in windows
    of 64 (the next window's ids load while the current one streams): 32 kv heads
    leave few ranges per head, so 48 ragged rows of 1000-5000 tokens give each wave
    well over 64 blocks, with row boundaries at many offsets inside later windows.
    Every row matches the fixed-partition kernel, four match the oracle, and an
    out-of-range block id deep inside a row is flagged, never read."""
    rng = np.random.default_rng(71)
    lens = rng.integers(1000, 5001, 48).astype(np.int32)
    tables, pool = wl._tables_from_lengths(lens, rng, spare_blocks=4)
    w = wl.DecodeWorkload("long_waves", 64, 32, 128, lens, tables, pool, torch.bfloat16, 72,
                          128 ** -0.5)
    cache, t, l = _build(w, device)
    q = wl.queries(w, device)
    mx = int(lens.max())
    sk = cache.paged_attention(0, q, t, l, max_context_len=mx, partition_tokens=0, check=True)
    part = cache.paged_attention(0, q, t, l, max_context_len=mx, partition_tokens=512,
                                 check=True)
    assert_attention_close(sk, part)
    rows = [0, 17, 30, 47]
    sub = wl.DecodeWorkload("long_waves_rows", 64, 32, 128, lens[rows], tables[rows], pool,
                            torch.bfloat16, 72, 128 ** -0.5)
    assert_attention_close(sk[rows], oracle_decode(sub, cache, q[rows]))
    bad = t.clone()
    longest = int(np.argmax(lens))
    bad[longest, int(lens[longest]) // 32] = w.num_blocks + 5
    with pytest.raises(ValueError, match="outside"):
        cache.paged_attention(0, q, bad, l, max_context_len=mx, partition_tokens=0, check=True)


def test_automatic_mode_beyond_stream_k_limits(device):
    """partition_tokens = 0 takes stream-K only for up to 512 sequences and 64 kv heads;
    beyond either limit it runs 512-token partitions: bit-identical to asking for them,
    and equal to the oracle (600 ragged rows, sampled; 80 kv heads; a 600-row mixed step)."""
    rng = np.random.default_rng(81)
    lens = rng.integers(1, 700, 600).astype(np.int32)
    tables, pool = wl._tables_from_lengths(lens, rng, spare_blocks=2)
    w = wl.DecodeWorkload("many_rows", 8, 2, 64, lens, tables, pool, torch.bfloat16, 82, 0.125)
    cache, t, l = _build(w, device)
    q = wl.queries(w, device)
    mx = int(lens.max())
    auto = cache.paged_attention(0, q, t, l, max_context_len=mx, partition_tokens=0, check=True)
    fixed = cache.paged_attention(0, q, t, l, max_context_len=mx, partition_tokens=512, check=True)
    assert torch.equal(auto, fixed)
    rows = [0, 1, 299, 598, 599]
    sub = wl.DecodeWorkload("many_rows_sample", 8, 2, 64, lens[rows], tables[rows], pool,
                            torch.bfloat16, 82, 0.125)
    assert_attention_close(auto[rows], oracle_decode(sub, cache, q[rows]))
    # the same rows as one mixed step: every fifth row brings a 3-token chunk
    qlens = np.where(np.arange(600) % 5 == 0, 3, 1).astype(np.int32)
    qlens = np.minimum(qlens, lens)
    mixed = wl.DecodeWorkload("many_rows_mixed", 8, 2, 64, lens, tables, pool, torch.bfloat16, 83,
                              0.125, query_lens=qlens)
    qm = wl.queries(mixed, device)
    qsl = wl.device_query_start(mixed, device)
    out = cache.paged_attention(0, qm, t, l, max_context_len=mx, query_start_loc=qsl,
                                max_query_len=int(qlens.max()), check=True)
    qsl_h = mixed.query_start_loc()
    take = np.concatenate([np.arange(qsl_h[r], qsl_h[r + 1]) for r in rows])
    subm = wl.DecodeWorkload("many_rows_mixed_sample", 8, 2, 64, lens[rows], tables[rows], pool,
                             torch.bfloat16, 83, 0.125, query_lens=qlens[rows])
    assert_attention_close(out[take], oracle_decode(subm, cache, qm[take]))
    # more kv heads than the stream-K counters cover
    lens80 = np.array([1, 40, 333, 17], np.int32)
    tables80, pool80 = wl._tables_from_lengths(lens80, rng, spare_blocks=2)
    w80 = wl.DecodeWorkload("heads80", 80, 80, 64, lens80, tables80, pool80, torch.bfloat16, 84,
                            0.125)
    cache80, t80, l80 = _build(w80, device)
    q80 = wl.queries(w80, device)
    out80 = cache80.paged_attention(0, q80, t80, l80, max_context_len=333, partition_tokens=0,
                                    check=True)
    assert_attention_close(out80, oracle_decode(w80, cache80, q80))


def test_duplicate_rows_and_prefix_sharing(device):
    """Rows aliasing the same blocks give identical outputs for identical queries."""
    w = wl.scaled(wl.config4(), num_seqs=4)
    cache, tables, lens = _build(w, device)
    q = wl.queries(w, device)
    t2 = tables.clone()
    t2[1] = t2[0]
    l2 = lens.clone()
    l2[1] = l2[0]
    q2 = q.clone()
    q2[1] = q2[0]
    # fixed partitions split both rows at the same token offsets: bit-identical
    out = cache.paged_attention(0, q2, t2, l2, max_context_len=w.max_context_len,
                                partition_tokens=512, check=True)
    assert torch.equal(out[0], out[1])
    # stream-K cuts the flattened block list into equal ranges, so the two copies are
    # split at different offsets: equal up to the merge's rounding
    sk = cache.paged_attention(0, q2, t2, l2, max_context_len=w.max_context_len,
                               partition_tokens=0, check=True)
    assert_attention_close(sk[1], sk[0])
    assert_attention_close(sk, out)


def test_errors(device):
    w = wl.scaled(wl.config2(), num_seqs=2, max_len=64)
    cache, tables, lens = _build(w, device)
    q = wl.queries(w, device)
    bad = tables.clone()
    bad[0, 0] = w.num_blocks + 7
    with pytest.raises(ValueError, match="outside"):
        cache.paged_attention(0, q, bad, lens, max_context_len=w.max_context_len, check=True)
    long_lens = lens.clone()
    long_lens[1] = tables.shape[1] * 16 + 5  # beyond the block table: clamped and flagged
    with pytest.raises(ValueError, match="outside"):
        cache.paged_attention(0, q, tables, long_lens, max_context_len=w.max_context_len,
                              check=True)
    with pytest.raises(ValueError):
        cache.paged_attention(0, q, tables, lens, max_context_len=10 ** 6)
    with pytest.raises(ValueError):
        cache.paged_attention(0, q, tables.long(), lens, max_context_len=64)
    with pytest.raises(UnsupportedAttentionBackend):
        cache.paged_attention(0, q.double(), tables, lens, max_context_len=64)
    with pytest.raises(ValueError, match="divide"):
        cache.paged_attention(0, torch.zeros(2, 12, 128, device=device, dtype=torch.bfloat16),
                              tables, lens, max_context_len=64)
    with pytest.raises(UnsupportedAttentionBackend):  # GQA group of 32 has no kernel
        cache.paged_attention(0, torch.zeros(2, 256, 128, device=device, dtype=torch.bfloat16),
                              tables, lens, max_context_len=64)
    assert math.isfinite(float(cache.paged_attention(0, q, tables, lens, max_context_len=64,
                                                     check=True).float().abs().max()))
