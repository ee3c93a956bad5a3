"""Prefix packs on the GPU (astr_paged_attention_i8_shared): decode rows whose block
tables alias shared prefix blocks (the PrefixCache's shared page refs,
state.py:599-625) read them once per pack of 16 // G rows. Every output is held to
the oracle's row-by-row attention (online_attention.py:74-219 via
paged_attention.py:168-215) at the north_star tolerance, and to the kernels without
the plan; a plan that contradicts the call is flagged and its bad members fall back
to ordinary rows. Includes the config4 workload at full size (256 rows)."""

import numpy as np
import pytest
import torch

from aster_amd import KVQuantization, PagedKVCache, plan_prefix_packs
from aster_amd import workloads as wl
from tests.gpu_util import assert_attention_close, mark_padding, oracle_decode

pytestmark = pytest.mark.gpu


def _shared_workload(hq, hkv, dim, qdtype, seed):
    """20 rows: 9 alias one 12-block prefix (two of them end exactly at it, some
    end inside a partial block), 5 alias another 7-block prefix, 5 share nothing,
    one sees no key at all."""
    rng = np.random.default_rng(seed)
    lens = ([12 * 16, 12 * 16] + list(12 * 16 + rng.integers(1, 90, 7)) +
            list(7 * 16 + rng.integers(0, 200, 5)) + list(rng.integers(20, 300, 5)) + [0])
    lens = np.asarray(lens, np.int32)
    need = [-(-int(c) // 16) for c in lens]
    pool = 12 + 7 + sum(max(0, n - 12) for n in need[:9]) + sum(max(0, n - 7) for n in need[9:14])
    pool += sum(need[14:]) + 2
    perm = rng.permutation(pool).astype(np.int32)
    tables = np.zeros((len(lens), max(need) + 1), np.int32)
    cursor = 19
    for r, n in enumerate(need):
        lead = 12 if r < 9 else 7 if r < 14 else 0
        base = 0 if r < 9 else 12
        tables[r, :lead] = perm[base:base + lead]
        k = max(0, n - lead)
        tables[r, lead:lead + k] = perm[cursor:cursor + k]
        cursor += k
    return wl.DecodeWorkload("prefix_mix", hq, hkv, dim, lens, tables, pool, qdtype, seed,
                             dim ** -0.5)


def _build(w, device, fmt="int8"):
    cache = PagedKVCache(num_blocks=w.num_blocks, num_layers=1, num_kv_heads=w.num_kv_heads,
                         head_dim=w.head_dim, device=device, quantization=KVQuantization(fmt))
    wl.materialize(w, cache, device=device)
    tables, lens = wl.device_tables(w, device)
    return cache, tables, lens


def _plan(w, device, **kw):
    return plan_prefix_packs(w.block_tables, w.context_lens, w.num_q_heads, w.num_kv_heads,
                             device=device, **kw)


@pytest.mark.parametrize("fmt", ["int8", "fp8_e4m3fn", "fp8_e5m2"])
@pytest.mark.parametrize("qdtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dim", [64, 128, 256])
@pytest.mark.parametrize("hq", [4, 8, 16, 32])
def test_packs_match_oracle_and_the_unplanned_kernels(device, fmt, qdtype, dim, hq):
    w = _shared_workload(hq, 4, dim, qdtype, seed=hq * 7 + dim)
    plan = _plan(w, device)
    assert plan is not None and plan.num_packs >= 2
    cache, tables, lens = _build(w, device, fmt)
    q = wl.queries(w, device)
    kw = dict(max_context_len=w.max_context_len, scale=w.scale, check=True)
    out = cache.paged_attention(0, q, tables, lens, prefix_packs=plan, **kw)
    assert torch.isfinite(out).all()
    assert_attention_close(out, oracle_decode(w, cache, q))
    assert_attention_close(out, cache.paged_attention(0, q, tables, lens, **kw))
    assert (out[-1] == 0).all()  # the row without keys


@pytest.mark.parametrize("fmt", ["int8", "fp8_e4m3fn"])
def test_packs_with_padding_keys_and_large_v_scales(device, fmt):
    w = _shared_workload(32, 8, 128, torch.bfloat16, seed=5)
    plan = _plan(w, device)
    cache, tables, lens = _build(w, device, fmt)
    mark_padding(cache, w.block_tables, w.context_lens, 0.1, seed=3, whole_blocks=1)
    shared = torch.from_numpy(w.block_tables[0, :12].astype(np.int64)).to(device)
    cache.scales[shared[::2], 0, 1] *= 2.0 ** 13  # V of every other shared block
    q = wl.queries(w, device)
    out = cache.paged_attention(0, q, tables, lens, max_context_len=w.max_context_len,
                                scale=w.scale, prefix_packs=plan, check=True)
    assert torch.isfinite(out).all()
    assert_attention_close(out, oracle_decode(w, cache, q), atol=2e-3 * 2.0 ** 13)


@pytest.mark.parametrize("dim", [64, 128, 256])
def test_packs_with_extreme_finite_scores(device, dim):
    """q x 100 and the shared blocks' K x 100 (test_inference_online_attention.py:79-98):
    pack blocks, whose 16 query columns come from several rows; held to the float64
    oracle within the tolerance plus fp32 rounding of the scores, as in
    test_gpu_hardening."""
    from tests.test_gpu_hardening import _assert_within_fp32_rounding

    w = _shared_workload(16, 4, dim, torch.bfloat16, seed=40 + dim)
    plan = _plan(w, device)
    assert plan is not None and plan.num_packs >= 2
    cache, tables, lens = _build(w, device)
    shared = np.concatenate([w.block_tables[0, :12], w.block_tables[9, :7]]).astype(np.int64)
    cache.scales[torch.from_numpy(shared).to(device), 0, 0] *= 100.0
    q = (wl.queries(w, device).float() * 100.0).to(torch.bfloat16)
    out = cache.paged_attention(0, q, tables, lens, max_context_len=w.max_context_len,
                                scale=w.scale, prefix_packs=plan, check=True)
    assert torch.isfinite(out).all()
    _assert_within_fp32_rounding(w, cache, q, out)


def test_plans_that_contradict_the_call_are_flagged(device):
    """A member listed twice, a member that sees fewer keys than the shared blocks and
    a member index past the batch raise the index flag; those members are served as
    ordinary rows, so every output still matches the oracle."""
    w = _shared_workload(32, 8, 128, torch.bfloat16, seed=9)
    cache, tables, lens = _build(w, device)
    q = wl.queries(w, device)
    good = _plan(w, device)
    rec = good.records().copy()
    for bad in ("twice", "short", "range"):
        r = rec.copy()
        if bad == "twice":
            r[1, 1] = r[0, 1]
        elif bad == "short":
            r[0, 0] = 40  # more shared blocks than any member holds
        else:
            r[0, 2] = w.num_seqs + 3
        plan = good.__class__(torch.from_numpy(r.reshape(-1)).to(device), good.num_packs,
                              good.rows_per_pack, good.num_seqs, good.shared_blocks,
                              good.packed_rows, good.saved_block_reads)
        out = cache.paged_attention(0, q, tables, lens, max_context_len=w.max_context_len,
                                    scale=w.scale, prefix_packs=plan)
        with pytest.raises(ValueError, match="outside"):
            cache.raise_errors()
        assert_attention_close(out, oracle_decode(w, cache, q))


def test_python_arguments(device):
    w = _shared_workload(32, 8, 128, torch.bfloat16, seed=2)
    plan = _plan(w, device)
    cache, tables, lens = _build(w, device)
    q = wl.queries(w, device)
    kw = dict(max_context_len=w.max_context_len, prefix_packs=plan)
    for bad in (dict(partition_tokens=512), dict(window=64),
                dict(query_start_loc=wl.device_query_start(w, device))):
        with pytest.raises(ValueError, match="prefix packs"):
            cache.paged_attention(0, q, tables, lens, **kw, **bad)
    with pytest.raises(ValueError, match="planned for other"):
        cache.paged_attention(0, q[:-1], tables[:-1], lens[:-1], **kw)


def test_full_config4(device):
    """The config4 workload at full size: 256 rows aliasing one 128-block prefix. The plan
    packs all 256 rows; stream-K with packs agrees with fixed 512-token partitions over
    every row and with the oracle on sampled rows."""
    w = wl.config4()
    plan = _plan(w, device)
    assert plan.num_packs == 64 and plan.packed_rows == 256
    assert (plan.records()[:, 0] == 128).all()
    cache, tables, lens = _build(w, device)
    q = wl.queries(w, device)
    kw = dict(max_context_len=w.max_context_len, scale=w.scale, check=True)
    packed = cache.paged_attention(0, q, tables, lens, prefix_packs=plan, **kw)
    parts = cache.paged_attention(0, q, tables, lens, partition_tokens=512, **kw)
    assert_attention_close(packed, parts)
    rows = np.random.default_rng(0).choice(w.num_seqs, 12, replace=False)
    ref = oracle_decode(w.block_tables[rows], cache, q[rows], context_lens=w.context_lens[rows],
                        scale=w.scale)
    assert_attention_close(packed[rows], ref)
