"""Host-side semantics of the arena-backed PagedStatePool (state.py:166-493) on a CPU
stand-in arena: ownership, copy-on-write of a shared or leased tail page,
truncation, leases, transactional appends, capacity, block tables and storage
metrics. Modelled on the reference's test_hot_kv.py:45-75 and
test_inference_online_attention.py:106-135."""

import math

import numpy as np
import pytest
import torch

from aster_amd.paged_pool import CacheCapacityError, PagedStatePool, SlotReservation, StateError
from oracle import reference_cpu as ref
from tests.fake_arena import FakeArena

L, HKV, D, BS = 2, 2, 32, 16


def make_pool(blocks=12):
    return PagedStatePool(FakeArena(num_blocks=blocks, num_layers=L, num_kv_heads=HKV,
                                    head_dim=D, block_size=BS))


def layers(tokens, seed):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(1, HKV, tokens, D, generator=g), torch.randn(1, HKV, tokens, D, generator=g))
            for _ in range(L)]


def expected(state_layers):
    """Dequantized oracle values of the appended tokens (quantize_kv then
    dequantize, kv_quantization.py:66-94), per layer (k, v) [1, Hkv, T, D]."""
    out = []
    for k, v in state_layers:
        pair = []
        for x in (k, v):
            q = ref.quantize_kv_int8(x.numpy())
            pair.append(torch.from_numpy(q.dequantize()))
        out.append(tuple(pair))
    return out


def assert_state(pool, seq, want):
    got = pool.materialize(seq)
    for (gk, gv), (wk, wv) in zip(got, want):
        torch.testing.assert_close(gk, wk, atol=0, rtol=0)
        torch.testing.assert_close(gv, wv, atol=0, rtol=0)


def cat(a, b):
    return [(torch.cat([ka, kb], 2), torch.cat([va, vb], 2)) for (ka, va), (kb, vb) in zip(a, b)]


def test_append_materialize_and_slot_placement():
    pool = make_pool()
    seq = pool.create("tenant-policy")
    first, second = layers(21, 1), layers(13, 2)
    pool.append_delta(seq, first)
    assert seq.length == 21 and len(seq.pages) == 2
    pool.append_delta(seq, second)
    assert seq.length == 34 and len(seq.pages) == 3
    assert [r.index for r in seq.pages] == [0, 1, 2]  # lowest free index first
    assert_state(pool, seq, expected(cat(first, second)))
    # offset o lives in page pages[o // 16], slot o % 16 (state.py:339-344)
    arena = pool.cache
    codes = ref.quantize_kv_int8(second[1][0].numpy()).values  # layer 1, K
    for t in range(13):
        o = 21 + t
        b = seq.pages[o // BS].index
        np.testing.assert_array_equal(arena.codes[b, 1, 0, :, o % BS].numpy(), codes[0, :, t])
    assert pool.used_blocks == 3
    assert pool.storage_metrics() == {
        "format": "int8", "physical_pages": 3, "quantized_leaves": 3 * 2 * L,
        "allocated_tensor_bytes": 3 * (L * 2 * HKV * BS * D + L * 2 * HKV * BS * 4 + BS)}


def test_fork_then_append_copies_the_shared_tail_page():
    pool = make_pool()
    seq = pool.create("p")
    base = layers(21, 3)
    pool.append_delta(seq, base)
    fork = pool.fork(seq)
    tail = fork.pages[-1]
    extra = layers(2, 4)
    pool.append_delta(seq, extra)
    assert seq.pages[-1] != tail and fork.pages[-1] == tail
    assert pool.cache.copies == [([tail.index], [seq.pages[-1].index])]
    assert_state(pool, fork, expected(base))
    assert_state(pool, seq, expected(cat(base, extra)))
    # a full tail page is not copied: appending starts a fresh page
    pool.truncate(seq, 16)
    fork2 = pool.fork(seq)
    pool.append_delta(seq, layers(1, 5))
    assert len(pool.cache.copies) == 1 and seq.pages[0] == fork2.pages[0]


def test_leased_tail_is_copied_and_released_pages_outlive_their_lease():
    pool = make_pool()
    seq = pool.create("p")
    base = layers(5, 6)
    pool.append_delta(seq, base)
    with pool.read_pages(seq) as views:
        assert len(views) == 1 and views[0].offset == 0
        assert views[0].payload[0].values.shape == (1, HKV, 5, D)
        old = seq.pages[0]
        pool.append_delta(seq, layers(1, 7))  # leased partial tail -> private copy
        assert seq.pages[0] != old
        pool.release(seq)
        assert pool.used_blocks == 1  # the leased page stays until the lease ends
        k = views[0].payload[0].dequantize(dtype=torch.float32)
        torch.testing.assert_close(k, expected(base)[0][0], atol=0, rtol=0)
    assert pool.used_blocks == 0


def test_truncate_release_and_stale_references():
    pool = make_pool()
    seq = pool.create("p")
    base = layers(40, 8)
    pool.append_delta(seq, base)
    pool.truncate(seq, 17)
    assert seq.length == 17 and len(seq.pages) == 2 and pool.used_blocks == 2
    assert_state(pool, seq, [(k[..., :17, :], v[..., :17, :]) for k, v in expected(base)])
    with pytest.raises(ValueError):
        pool.truncate(seq, 18)
    stale = list(seq.pages)
    pool.release(seq)
    pool.release(seq)  # idempotent
    with pytest.raises(StateError):
        pool.append_delta(seq, layers(1, 9))
    other = pool.create("q")
    pool.append_delta(other, layers(1, 10))  # reuses page 0 with a new generation
    assert other.pages[0].index == stale[0].index and other.pages[0] != stale[0]
    with pytest.raises(StateError):
        pool._page(stale[0])
    with pytest.raises(StateError):
        make_pool().fork(other)  # foreign pool


def test_nonfinite_suffix_and_capacity_leave_state_unchanged():
    pool = make_pool(blocks=3)
    seq = pool.create("p")
    pool.append_delta(seq, layers(20, 11))
    before = (list(seq.pages), seq.length, pool.used_blocks)
    bad = layers(3, 12)
    bad[1][1][0, 0, 1, 0] = float("nan")
    with pytest.raises(ValueError, match="finite"):
        pool.append_delta(seq, bad)
    assert (list(seq.pages), seq.length, pool.used_blocks) == before
    with pytest.raises(CacheCapacityError):
        pool.append_delta(seq, layers(40, 13))
    assert (list(seq.pages), seq.length, pool.used_blocks) == before
    with pytest.raises(StateError):
        pool.append_delta(seq, layers(2, 14)[:1])  # layer count differs from the arena


def test_reservations_commit_abort_and_block_tables():
    pool = make_pool()
    a, b = pool.create("a"), pool.create("b")
    pool.append_delta(a, layers(30, 15))
    r = pool.reserve(a, 5)
    assert isinstance(r, SlotReservation) and r.start == 30 and r.length == 35
    assert r.slots == [r.pages[o // BS].index * BS + o % BS for o in range(30, 35)]
    assert a.length == 30  # nothing visible before commit
    with pool.block_tables([r, b]) as (tables, lens):
        assert tables.dtype == torch.int32 and tables.shape == (2, 3)
        assert tables[0].tolist() == [p.index for p in r.pages] and lens.tolist() == [35, 0]
        assert all(pool._pages[p.index].readers == 1 for p in r.pages)
    assert all(pool._pages[p.index].readers == 0 for p in r.pages)
    pool.commit(r)
    assert a.length == 35 and a.pages == r.pages
    with pytest.raises(StateError):
        pool.commit(r)
    used = pool.used_blocks
    r2 = pool.reserve(a, 20)
    assert pool.used_blocks == used + 1
    pool.abort(r2)
    assert pool.used_blocks == used and a.length == 35
    with pytest.raises(RuntimeError):
        with pool.transaction(a, 3):
            raise RuntimeError("step failed")
    assert a.length == 35 and pool.used_blocks == used


def test_capacity_matches_pages_needed_for_many_sequences():
    pool = make_pool(blocks=10)
    seqs = []
    for i in range(4):
        s = pool.create(f"s{i}")
        pool.append_delta(s, layers(33, 20 + i))  # 3 pages each
        seqs.append(s)
        if i == 2:
            break
    assert pool.used_blocks == 9
    last = pool.create("last")
    with pytest.raises(CacheCapacityError):
        pool.append_delta(last, layers(17, 30))
    pool.append_delta(last, layers(16, 31))
    assert pool.used_blocks == 10
    for s in seqs + [last]:
        pool.release(s)
    assert pool.used_blocks == 0 and pool.storage_metrics()["allocated_tensor_bytes"] == 0
    assert math.ceil(33 / BS) == 3


def test_padding_leaf_is_stored_exposed_and_copied_on_write():
    """The runner's suffix carries a padding leaf [1, 1, T, 1] (paged_attention.py:228):
    it lands in the slots' key bytes, comes back as the last of 2L+1 page leaves
    (paged_attention.py:171-182) and in materialize, follows a copied tail page, and a
    later suffix without a leaf marks its tokens real."""
    pool = make_pool()
    seq = pool.create("p")
    pad = torch.tensor([1, 0, 1, 1, 0, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 0, 1, 1], dtype=torch.bool)
    pool.append_delta(seq, layers(20, 1) + [(pad[None, None, :, None],)])
    assert pool.cache.has_padding
    with pool.read_pages(seq) as views:
        assert [len(v.payload) for v in views] == [2 * L + 1] * 2
        got = torch.cat([v.payload[-1][0, 0, :, 0] for v in views])
        assert views[1].payload[-1].shape == (1, 1, 4, 1) and views[1].payload[-1].dtype == torch.bool
    assert torch.equal(got, pad)
    state = pool.materialize(seq)
    assert len(state) == L + 1 and torch.equal(state[-1][0][0, 0, :, 0], pad)
    # a fork shares the tail page; appending to it copies the page with its padding bytes
    child = pool.fork(seq)
    pool.append_delta(child, layers(3, 2))  # no leaf: real tokens
    assert child.pages[-1].index != seq.pages[-1].index
    with pool.read_pages(child) as views:
        got_child = torch.cat([v.payload[-1][0, 0, :, 0] for v in views])
    assert torch.equal(got_child, torch.cat([pad, torch.ones(3, dtype=torch.bool)]))
    with pool.read_pages(seq) as views:
        assert torch.equal(torch.cat([v.payload[-1][0, 0, :, 0] for v in views]), pad)
    # the full-state append slices the leaf like every other leaf
    more = torch.tensor([0, 1, 1], dtype=torch.bool)
    whole = [(torch.cat([k, k2], 2), torch.cat([v, v2], 2))
             for (k, v), (k2, v2) in zip(pool.materialize(seq)[:L], layers(3, 3))]
    pool.append(seq, whole + [(torch.cat([pad, more])[None, None, :, None],)])
    assert torch.equal(pool.materialize(seq)[-1][0][0, 0, :, 0], torch.cat([pad, more]))
    with pytest.raises(StateError):
        pool.append_delta(seq, layers(2, 4) + [(torch.tensor([1, 2])[None, None, :, None],)])
    with pytest.raises(StateError):
        pool.append_delta(seq, layers(2, 4) + [(torch.ones(1, 1, 3, 1, dtype=torch.bool),)])
