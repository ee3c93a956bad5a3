"""The planned decode path (a host schedule from astr_decode_plan, the planned kernel,
workgroup-local merges and the chunk merge) against the oracle's page-by-page online
softmax (online_attention.py:74-219 via paged_attention.py:168-215) at the north_star
tolerance, and against the unplanned stream-K call on the full BASELINE workloads;
plans that disagree with the device lengths or hold bad indices are flagged."""

import numpy as np
import pytest
import torch

from aster_amd import KVQuantization, PagedKVCache, UnsupportedAttentionBackend
from aster_amd import _native
from aster_amd import workloads as wl
from aster_amd.decode_plan import plan_decode
from tests.gpu_util import assert_attention_close, mark_padding, oracle_decode

pytestmark = pytest.mark.gpu

FORMAT_CODES = {"int8": _native.ASTR_KV_INT8, "fp8_e4m3fn": _native.ASTR_KV_FP8_E4M3FN,
                "fp8_e5m2": _native.ASTR_KV_FP8_E5M2}


def _build(w, device, fmt="int8"):
    cache = PagedKVCache(num_blocks=w.num_blocks, num_layers=1, num_kv_heads=w.num_kv_heads,
                         head_dim=w.head_dim, device=device, quantization=KVQuantization(fmt))
    wl.materialize(w, cache, device=device)
    tables, lens = wl.device_tables(w, device)
    return cache, tables, lens


def _planned(cache, w, q, tables, lens, *, window=None, fmt="int8", **plan_kw):
    plan = plan_decode(w.block_tables, w.context_lens, num_q_heads=w.num_q_heads,
                       num_kv_heads=w.num_kv_heads, head_dim=w.head_dim, q_dtype=w.q_dtype,
                       device=q.device, code_format=FORMAT_CODES[fmt], window=window, **plan_kw)
    out = cache.paged_attention(0, q, tables, lens, max_context_len=w.max_context_len,
                                scale=w.scale, window=window, decode_plan=plan, check=True)
    return out, plan


def _edge_workload(dim, hq, hkv, qdtype, seed=7):
    lens = np.array([1, 15, 16, 17, 255, 256, 257, 600, 0, 33, 2048, 90], np.int32)
    rng = np.random.default_rng(dim + hq + seed)
    tables, pool = wl._tables_from_lengths(lens, rng, spare_blocks=3)
    return wl.DecodeWorkload("edge", hq, hkv, dim, lens, tables, pool, qdtype, seed, dim ** -0.5)


@pytest.mark.parametrize("dim,hq,hkv", [(64, 8, 8), (128, 16, 8), (128, 32, 8), (128, 64, 8),
                                        (128, 128, 8), (256, 8, 2), (256, 32, 4), (64, 16, 2)])
@pytest.mark.parametrize("qdtype", [torch.bfloat16, torch.float16, torch.float32])
def test_head_dims_groups_dtypes(device, dim, hq, hkv, qdtype):
    w = _edge_workload(dim, hq, hkv, qdtype)
    cache, tables, lens = _build(w, device)
    q = wl.queries(w, device)
    out, _ = _planned(cache, w, q, tables, lens)
    assert (out[8] == 0).all()
    assert_attention_close(out, oracle_decode(w, cache, q))


@pytest.mark.parametrize("workgroups", [2, 3, 7, 40, 150])
@pytest.mark.parametrize("tail", [0, 3])
def test_rows_cut_across_workgroups(device, workgroups, tail):
    """Few workgroups: every long row is cut into chunks that several workgroups
    stream and the chunk kernel merges; many waves hold empty ranges."""
    w = _edge_workload(128, 32, 8, torch.bfloat16, seed=workgroups)
    cache, tables, lens = _build(w, device)
    q = wl.queries(w, device)
    out, plan = _planned(cache, w, q, tables, lens, num_workgroups=workgroups, tail_blocks=tail)
    nb = (w.context_lens + 15) // 16
    cost = 50 * nb + 135 * (nb > 0)
    share = cost.sum() * w.num_kv_heads / workgroups
    assert (plan.info.num_chunked > 0) == bool((cost > share).any())
    assert_attention_close(out, oracle_decode(w, cache, q))


@pytest.mark.parametrize("fmt", ["int8", "fp8_e4m3fn", "fp8_e5m2"])
@pytest.mark.parametrize("window", [None, 100])
def test_formats_windows_padding(device, fmt, window):
    w = _edge_workload(128, 16, 4, torch.bfloat16, seed=3)
    cache, tables, lens = _build(w, device, fmt)
    mark_padding(cache, w.block_tables, w.context_lens, 0.2, seed=5, whole_blocks=2)
    q = wl.queries(w, device)
    out, _ = _planned(cache, w, q, tables, lens, window=window, fmt=fmt, num_workgroups=9)
    assert_attention_close(out, oracle_decode(w, cache, q, window=window))


def test_large_v_scales_and_extreme_scores(device):
    from tests.test_gpu_hardening import _assert_within_fp32_rounding

    w = _edge_workload(128, 16, 4, torch.bfloat16, seed=11)
    cache, tables, lens = _build(w, device)
    cache.scales[::3, 0, 1] *= 2.0 ** 12
    q = wl.queries(w, device)
    out, _ = _planned(cache, w, q, tables, lens, num_workgroups=5)
    assert_attention_close(out, oracle_decode(w, cache, q), atol=2e-3 * 2.0 ** 12)
    cache, tables, lens = _build(w, device)
    cache.scales[:, 0, 0] *= 100.0
    q = (wl.queries(w, device).float() * 100.0).to(torch.bfloat16)
    out, _ = _planned(cache, w, q, tables, lens, num_workgroups=5)
    _assert_within_fp32_rounding(w, cache, q, out)


def _shared_workload(dim, hq, hkv, qdtype, seed=0, groups=(40, 7, 2), shared=(20, 9, 33),
                     own_max=300, empty_own=True):
    """Groups of sequences whose tables begin with their group's blocks (a forked
    prefix), then blocks of their own (some none); groups interleaved in the batch,
    and a few rows sharing nothing."""
    rng = np.random.default_rng(seed + dim + hq)
    rows, lens, nxt = [], [], 0
    for g, n in enumerate(groups):
        prefix = list(range(nxt, nxt + shared[g]))
        nxt += shared[g]
        for i in range(n):
            own = 0 if i % 9 == 4 and empty_own else int(rng.integers(1, own_max + 1))
            ctx = shared[g] * 16 + own
            nb = -(-ctx // 16)
            rows.append(prefix + list(range(nxt, nxt + nb - shared[g])))
            nxt += nb - shared[g]
            lens.append(ctx)
    for ctx in (5, 700, 0):
        nb = -(-ctx // 16)
        rows.append(list(range(nxt, nxt + nb)))
        nxt += nb
        lens.append(ctx)
    perm = rng.permutation(nxt + 3).astype(np.int32)
    tables = np.zeros((len(rows), max(len(r) for r in rows)), np.int32)
    for i, r in enumerate(rows):
        tables[i, :len(r)] = perm[r]
    order = rng.permutation(len(rows))
    return wl.DecodeWorkload("shared", hq, hkv, dim, np.asarray(lens, np.int32)[order],
                             tables[order], nxt + 3, qdtype, seed, dim ** -0.5)


@pytest.mark.parametrize("dim,hq,hkv", [(128, 32, 8), (128, 8, 8), (64, 32, 2), (256, 16, 4),
                                        (128, 128, 8)])
@pytest.mark.parametrize("qdtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("ranges", [0, 1, 3])
def test_shared_prefixes_in_tiles(device, dim, hq, hkv, qdtype, ranges):
    """Shared prefixes read in prefix tiles (the chunked-prefill kernel's column tiles,
    no mask, one partial per member row and key range) and merged with the rows' own
    blocks by the chunk kernel: the oracle's row-by-row result."""
    w = _shared_workload(dim, hq, hkv, qdtype)
    cache, tables, lens = _build(w, device)
    q = wl.queries(w, device)
    out, plan = _planned(cache, w, q, tables, lens, tile_ranges=ranges, num_workgroups=37)
    assert plan.info.num_tiles > 0 and plan.info.num_tile_members >= 40
    assert (out[torch.as_tensor(np.nonzero(w.context_lens == 0)[0], device=device)] == 0).all()
    assert_attention_close(out, oracle_decode(w, cache, q))


@pytest.mark.parametrize("fmt", ["int8", "fp8_e4m3fn", "fp8_e5m2"])
def test_shared_prefix_tiles_formats_and_padding(device, fmt):
    w = _shared_workload(128, 32, 8, torch.bfloat16, seed=3)
    cache, tables, lens = _build(w, device, fmt)
    mark_padding(cache, w.block_tables, w.context_lens, 0.2, seed=5, whole_blocks=2)
    cache.scales[::5, 0, 1] *= 2.0 ** 10  # V scales past the f16 weight range in some blocks
    q = wl.queries(w, device)
    out, plan = _planned(cache, w, q, tables, lens, fmt=fmt, tile_ranges=2)
    assert plan.info.num_tiles > 0
    assert_attention_close(out, oracle_decode(w, cache, q), atol=2e-3 * 2.0 ** 10)


def test_shared_prefix_tiles_extreme_scores(device):
    """q x100 and K scales x100: the tiles' scores take the third query term on every
    step, and every output stays within the fp32 rounding of the exact result."""
    from tests.test_gpu_hardening import _assert_within_fp32_rounding

    w = _shared_workload(128, 32, 8, torch.bfloat16, seed=9)
    cache, tables, lens = _build(w, device)
    cache.scales[:, 0, 0] *= 100.0
    q = (wl.queries(w, device).float() * 100.0).to(torch.bfloat16)
    out, plan = _planned(cache, w, q, tables, lens, tile_ranges=2)
    assert plan.info.num_tiles > 0
    _assert_within_fp32_rounding(w, cache, q, out)


def test_tile_plans_that_contradict_the_call_are_flagged(device):
    w = _shared_workload(128, 32, 8, torch.bfloat16, seed=5)
    cache, tables, lens = _build(w, device)
    q = wl.queries(w, device)
    plan = plan_decode(w.block_tables, w.context_lens, num_q_heads=32, num_kv_heads=8,
                       head_dim=128, q_dtype=torch.bfloat16, device=device, tile_ranges=2)
    assert plan.info.num_tiles > 0
    kw = dict(max_context_len=w.max_context_len, scale=w.scale, decode_plan=plan, check=True)
    info = plan.info
    member = int(plan.words[info.off_tile_members].item())
    # a member's device length shorter than its shared blocks
    other = lens.clone()
    other[member] = 3
    with pytest.raises(ValueError):
        cache.paged_attention(0, q, tables, other, **kw)
    # a tile naming a kv head past the arena's, a member past the batch, a slot span
    # beyond the chunk slots
    for offset, value in ((info.off_tiles + 2, 8), (info.off_tile_members, 10 ** 6),
                          (info.off_tile_members + 2, 10 ** 6)):
        words = plan.words.clone()
        plan.words[offset] = value
        with pytest.raises(ValueError):
            cache.paged_attention(0, q, tables, lens, **kw)
        plan.words.copy_(words)
    out = cache.paged_attention(0, q, tables, lens, **kw)
    assert_attention_close(out, oracle_decode(w, cache, q))


@pytest.mark.parametrize("builder", [wl.config2, wl.config4, wl.config5])
def test_full_configs_match_the_unplanned_call(device, builder):
    """BASELINE configs 2, 4 and 5 at full size: the planned call equals the stream-K
    call within the tolerance on every output, and the oracle on sampled rows."""
    w = builder()
    cache, tables, lens = _build(w, device)
    q = wl.queries(w, device)
    out, plan = _planned(cache, w, q, tables, lens)
    if builder is wl.config2:
        assert plan.info.num_chunked == 0
    if builder is wl.config5:
        assert plan.info.num_chunked > 0
    if builder is wl.config4:
        assert plan.info.num_tile_members == w.num_seqs  # the prefix in tiles
    ref = cache.paged_attention(0, q, tables, lens, max_context_len=w.max_context_len,
                                scale=w.scale, check=True)
    assert_attention_close(out, ref)
    rows = np.random.default_rng(0).choice(w.num_seqs, 3, replace=False)
    sub = wl.DecodeWorkload(w.name, w.num_q_heads, w.num_kv_heads, w.head_dim,
                            w.context_lens[rows], w.block_tables[rows], w.num_blocks, w.q_dtype,
                            w.seed, w.scale)
    assert_attention_close(out[torch.as_tensor(rows, device=device)],
                           oracle_decode(sub, cache, q[torch.as_tensor(rows, device=device)]))


def test_plans_that_contradict_the_call_are_flagged(device):
    w = _edge_workload(128, 32, 8, torch.bfloat16, seed=21)
    cache, tables, lens = _build(w, device)
    q = wl.queries(w, device)
    plan = plan_decode(w.block_tables, w.context_lens, num_q_heads=32, num_kv_heads=8,
                       head_dim=128, q_dtype=torch.bfloat16, device=device, num_workgroups=6)
    kw = dict(max_context_len=w.max_context_len, scale=w.scale, decode_plan=plan, check=True)
    # device lengths other than the plan's
    other = lens.clone()
    other[4] += 1
    with pytest.raises(ValueError):
        cache.paged_attention(0, q, tables, other, **kw)
    # a block id beyond the arena, an item naming a sequence past the batch, and wave
    # entries whose first block or piece are not the items' (or out of range)
    info = plan.info
    went = plan.words[info.off_waves:info.off_items].view(-1, 6)
    w0 = int(torch.nonzero(went[:, 2] > 0)[0, 0])  # a wave that prefetches
    e0 = info.off_waves + 6 * w0
    other_id = int((went[w0, 3] + 1) % w.num_blocks)
    for offset, value in ((info.off_ids + 3, w.num_blocks + 5), (info.off_items, 10 ** 6),
                          (e0 + 3, other_id), (e0 + 1, (int(went[w0, 1]) + 1) % 8),
                          (e0 + 0, 10 ** 6), (e0 + 2, 9)):
        words = plan.words.clone()
        plan.words[offset] = value
        with pytest.raises(ValueError):
            cache.paged_attention(0, q, tables, lens, **kw)
        plan.words.copy_(words)
    out = cache.paged_attention(0, q, tables, lens, **kw)  # the intact plan still serves
    assert_attention_close(out, oracle_decode(w, cache, q))
    with pytest.raises(ValueError, match="another batch"):
        cache.paged_attention(0, q[:5], tables[:5], lens[:5], max_context_len=w.max_context_len,
                              decode_plan=plan)


def test_fp32_queries_on_the_full_config2_and_config1(device):
    """fp32 queries take the planned MFMA path over int8 codes (three int8 query terms):
    config 1 against its golden output and config 2 against the exact fp32 kernel, at
    the north_star tolerance; fp32 queries over FP8 codes are refused."""
    import os

    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config1.npz"))
    cache = PagedKVCache(num_blocks=64, num_layers=1, num_kv_heads=4, head_dim=64, device=device)
    cache.append(0, torch.from_numpy(g["k"]).to(device), torch.from_numpy(g["v"]).to(device),
                 torch.from_numpy(g["slots"]).to(device), check=True)
    q = torch.from_numpy(g["q"]).to(device)
    plan = plan_decode(g["block_tables"], g["context_lens"], num_q_heads=4, num_kv_heads=4,
                       head_dim=64, q_dtype=torch.float32, device=device)
    out = cache.paged_attention(0, q, torch.from_numpy(g["block_tables"]).to(device),
                                torch.from_numpy(g["context_lens"]).to(device),
                                max_context_len=300, scale=64 ** -0.5, decode_plan=plan,
                                check=True)
    assert out.dtype == torch.float32
    assert_attention_close(out, g["out"])
    w = wl.config2()
    cache, tables, lens = _build(w, device)
    q = wl.queries(w, device).float()
    w32 = wl.DecodeWorkload(w.name, w.num_q_heads, w.num_kv_heads, w.head_dim, w.context_lens,
                            w.block_tables, w.num_blocks, torch.float32, w.seed, w.scale)
    out, _ = _planned(cache, w32, q, tables, lens)
    exact = cache.paged_attention(0, q, tables, lens, max_context_len=w.max_context_len,
                                  scale=w.scale, check=True)  # the exact fp32 VALU kernel
    assert_attention_close(out, exact)
    with pytest.raises(Exception):
        plan_decode(w.block_tables, w.context_lens, num_q_heads=32, num_kv_heads=8,
                    head_dim=128, q_dtype=torch.float32, device=device,
                    code_format=FORMAT_CODES["fp8_e4m3fn"])


# ---- the step's append inside the planned decode (astr_paged_attention_i8_planned_append)

def _held_batch(w, cache, device):
    """Fills `cache` with every token but each row's newest (position ctx - 1) and
    returns those as per-sequence rows in the query dtype, with their slots (a zero row
    and slot -1 where a row has no token)."""
    _, (k, v, slots) = wl.materialize(w, cache, device=device, hold_last=True)
    has = torch.from_numpy(w.context_lens > 0).to(device)
    shape = (w.num_seqs,) + tuple(k.shape[1:])
    key = torch.zeros(shape, dtype=w.q_dtype, device=device)
    value = torch.zeros(shape, dtype=w.q_dtype, device=device)
    slot = torch.full((w.num_seqs,), -1, dtype=torch.int64, device=device)
    key[has], value[has], slot[has] = k.to(w.q_dtype), v.to(w.q_dtype), slots
    return key, value, slot


def _append_pair(w, device, fmt="int8", window=None, padding=False, scale_v=False,
                 **plan_kw):
    """The same step twice: the reserved-slot append then the planned decode, and the
    planned decode that appends; returns both outputs and both arenas."""
    caches = []
    for _ in range(2):
        cache = PagedKVCache(num_blocks=w.num_blocks, num_layers=1,
                             num_kv_heads=w.num_kv_heads, head_dim=w.head_dim, device=device,
                             quantization=KVQuantization(fmt))
        held = _held_batch(w, cache, device)
        if padding:
            mark_padding(cache, w.block_tables, w.context_lens, 0.2, seed=5, whole_blocks=2)
        if scale_v:
            cache.scales[::5, 0, 1] *= 2.0 ** 10  # V scales past the f16 weight range
        caches.append(cache)
    tables, lens = wl.device_tables(w, device)
    q = wl.queries(w, device)
    plan = plan_decode(w.block_tables, w.context_lens, num_q_heads=w.num_q_heads,
                       num_kv_heads=w.num_kv_heads, head_dim=w.head_dim, q_dtype=w.q_dtype,
                       device=device, code_format=FORMAT_CODES[fmt], window=window, **plan_kw)
    key, value, slot = held
    kw = dict(max_context_len=w.max_context_len, scale=w.scale, window=window,
              decode_plan=plan, check=True)
    caches[0].append(0, key, value, slot, reserved=True, check=True)
    two = caches[0].paged_attention(0, q, tables, lens, **kw)
    one = caches[1].paged_attention(0, q, tables, lens, append=(key, value, slot), **kw)
    return two, one, caches, q, plan


def _assert_same_step(two, one, caches):
    assert torch.equal(two, one)
    assert torch.equal(caches[0].codes, caches[1].codes)
    assert torch.equal(caches[0].scales.view(torch.int32), caches[1].scales.view(torch.int32))


@pytest.mark.parametrize("dim,hq,hkv", [(128, 8, 8), (128, 32, 8), (128, 128, 8), (256, 8, 2),
                                        (256, 32, 4), (256, 16, 2)])
@pytest.mark.parametrize("qdtype", [torch.bfloat16, torch.float16])
def test_append_in_decode_equals_append_then_decode(device, dim, hq, hkv, qdtype):
    """Rows of 1..2048 tokens (and an empty one), newest tokens at every block offset:
    outputs and arena bit for bit as the append launch followed by the decode, and the
    oracle's result."""
    w = _edge_workload(dim, hq, hkv, qdtype, seed=11)
    two, one, caches, q, _ = _append_pair(w, device)
    _assert_same_step(two, one, caches)
    assert_attention_close(one, oracle_decode(w, caches[1], q))


@pytest.mark.parametrize("fmt", ["int8", "fp8_e4m3fn", "fp8_e5m2"])
@pytest.mark.parametrize("window", [None, 100])
def test_append_in_decode_formats_windows_padding(device, fmt, window):
    w = _edge_workload(128, 16, 4, torch.bfloat16, seed=13)
    two, one, caches, q, _ = _append_pair(w, device, fmt=fmt, window=window, padding=True,
                                          scale_v=True)
    _assert_same_step(two, one, caches)


@pytest.mark.parametrize("workgroups", [40, 150])
def test_append_in_decode_with_chunks_and_tiles(device, workgroups):
    """Rows cut across workgroups (the newest token in one chunk) and rows sharing
    prefixes (tiles end before any newest token's block)."""
    w = _edge_workload(128, 32, 8, torch.bfloat16, seed=workgroups)
    two, one, caches, _, plan = _append_pair(w, device, num_workgroups=workgroups)
    assert plan.info.num_chunked > 0
    _assert_same_step(two, one, caches)
    # every row's newest token in a block of its own, as the runner's copy-on-write
    # reservations keep it (a row with no block of its own would append into the pages
    # its group shares)
    w = _shared_workload(128, 32, 8, torch.bfloat16, seed=5, empty_own=False)
    two, one, caches, _, plan = _append_pair(w, device, num_workgroups=workgroups,
                                             tile_ranges=2)
    assert plan.info.num_tiles > 0
    _assert_same_step(two, one, caches)


def test_append_in_decode_full_configs(device):
    for w in (wl.config2(), wl.config4()):
        two, one, caches, _, _ = _append_pair(w, device)
        _assert_same_step(two, one, caches)


def test_append_in_decode_nonfinite_and_wrong_slots_are_flagged(device):
    w = _edge_workload(128, 32, 8, torch.bfloat16, seed=17)
    cache = PagedKVCache(num_blocks=w.num_blocks, num_layers=1, num_kv_heads=w.num_kv_heads,
                         head_dim=w.head_dim, device=device)
    key, value, slot = _held_batch(w, cache, device)
    tables, lens = wl.device_tables(w, device)
    q = wl.queries(w, device)
    plan = plan_decode(w.block_tables, w.context_lens, num_q_heads=w.num_q_heads,
                       num_kv_heads=w.num_kv_heads, head_dim=w.head_dim, q_dtype=w.q_dtype,
                       device=device)
    kw = dict(max_context_len=w.max_context_len, scale=w.scale, decode_plan=plan)
    # a non-finite value in one row: the input flag, and that token written nowhere
    bad = value.clone()
    bad[3, 2, 7] = float("nan")
    before = cache.codes.clone()
    cache.paged_attention(0, q, tables, lens, append=(key, bad, slot), **kw)
    with pytest.raises(ValueError, match="finite"):
        cache.raise_errors()
    s3 = int(slot[3])
    assert torch.equal(cache.codes[s3 // 16, 0, :, 2, s3 % 16], before[s3 // 16, 0, :, 2, s3 % 16])
    # a slot that is not the plan's position of the token: the index flag; the token goes
    # to the caller's slot (a spare block)
    used = {int(b) for r, n in enumerate(-(-w.context_lens // 16)) for b in w.block_tables[r, :n]}
    blk = min(set(range(w.num_blocks)) - used)
    wrong = slot.clone()
    wrong[5] = blk * 16 + 3
    cache.paged_attention(0, q, tables, lens, append=(key, value, wrong), **kw)
    with pytest.raises(ValueError, match="outside"):
        cache.raise_errors()
    probe = PagedKVCache(num_blocks=w.num_blocks, num_layers=1, num_kv_heads=w.num_kv_heads,
                         head_dim=w.head_dim, device=device)
    probe.append(0, key[5:6], value[5:6], wrong[5:6], check=True)
    assert torch.equal(cache.codes[blk, 0, :, :, 3], probe.codes[blk, 0, :, :, 3])
    with pytest.raises(ValueError, match="decode plan"):
        cache.paged_attention(0, q, tables, lens, max_context_len=w.max_context_len,
                              append=(key, value, slot))


def test_append_in_decode_head_dim_64_is_refused(device):
    """At head dim 64 the decode does not append (its token rows would cost the kernel
    its second workgroup per CU): refused, never run at half occupancy; the runner
    appends in a launch of its own there."""
    w = _edge_workload(64, 16, 2, torch.bfloat16, seed=19)
    cache = PagedKVCache(num_blocks=w.num_blocks, num_layers=1, num_kv_heads=w.num_kv_heads,
                         head_dim=w.head_dim, device=device)
    key, value, slot = _held_batch(w, cache, device)
    tables, lens = wl.device_tables(w, device)
    q = wl.queries(w, device)
    plan = plan_decode(w.block_tables, w.context_lens, num_q_heads=w.num_q_heads,
                       num_kv_heads=w.num_kv_heads, head_dim=w.head_dim, q_dtype=w.q_dtype,
                       device=device)
    assert not cache.decode_appends(torch.bfloat16)
    with pytest.raises(UnsupportedAttentionBackend):
        cache.paged_attention(0, q, tables, lens, max_context_len=w.max_context_len,
                              scale=w.scale, decode_plan=plan, append=(key, value, slot))
