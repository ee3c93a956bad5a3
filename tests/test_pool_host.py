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


def test_reference_constructor_and_lazy_arena():
    """PagedStatePool(*, block_size, max_blocks, codec, quantization) as ModelRunner
    builds it (runner.py:36-41, state.py:169-180): no layer shape is known until the
    first append, so the arena is allocated then (here it cannot be: the leaves live on
    the CPU, and the arena only on a HIP device)."""
    from aster_amd import KVQuantization, UnsupportedAttentionBackend
    from aster_amd.paged_pool import KVStateCodec

    q8 = KVQuantization("int8")
    with pytest.raises(ValueError, match="positive"):
        PagedStatePool(block_size=0, max_blocks=4, quantization=q8)
    with pytest.raises(ValueError, match="KVQuantization"):
        PagedStatePool(quantization="int8")
    with pytest.raises(UnsupportedAttentionBackend, match="quantized"):
        PagedStatePool()  # native (unquantized) storage is the reference backend's
    with pytest.raises(UnsupportedAttentionBackend, match="16-token"):
        PagedStatePool(block_size=4, quantization=q8)
    with pytest.raises(UnsupportedAttentionBackend, match="codec"):
        PagedStatePool(quantization=q8, codec=KVStateCodec(kind="mla_latent"))
    with pytest.raises(ValueError, match="codec tag"):
        KVStateCodec(kind="unknown")
    pool = PagedStatePool(block_size=16, max_blocks=4, codec=KVStateCodec(kind="gqa_kv"),
                          quantization=q8)
    assert pool.cache is None and pool.quantization is q8 and pool.codec.kind == "gqa_kv"
    seq = pool.create("tenant")
    child = pool.fork(seq)
    assert seq.kind == child.kind == "gqa_kv" and pool.materialize(seq) is None
    with pool.read_pages(seq) as views:
        assert views == ()
    assert pool.storage_metrics() == {"format": "int8", "allocated_tensor_bytes": 0,
                                      "quantized_leaves": 0, "physical_pages": 0}
    with pytest.raises(StateError, match="initialized"):
        pool.restore_pages((), identity="tenant", length=3)
    with pytest.raises(StateError, match="arena"):
        with pool.block_tables([seq]):
            pass
    with pytest.raises(UnsupportedAttentionBackend, match="HIP device"):
        pool.append_delta(seq, layers(3, 1))
    with pytest.raises(StateError, match="token/head"):
        pool.append_delta(seq, [(torch.zeros(1, 2, 3, 4, dtype=torch.int32),) * 2])
    pool.release(child)
    pool.release(seq)


def test_layout_lock_and_padding_leaf_detection():
    """The first append locks layers, heads, head dim and input dtype
    (state.py:285-300); a trailing one-element tuple is the padding leaf."""
    pool = make_pool()
    seq = pool.create("t")
    pool.append_delta(seq, layers(3, 1) + [(torch.ones(1, 1, 3, 1, dtype=torch.bool),)])
    with pytest.raises(StateError, match="layout"):
        pool.append_delta(seq, [(k.double(), v.double()) for k, v in layers(2, 2)])
    with pytest.raises(StateError, match="layout"):
        pool.append_delta(seq, [(k[:, :1], v[:, :1]) for k, v in layers(2, 3)])
    with pytest.raises(StateError, match="layout"):
        pool.append_delta(seq, layers(2, 4) + layers(2, 5))  # four layers
    assert seq.length == 3


def test_prefix_cache_internals_on_the_arena_pool():
    """The reference's PrefixCache reaches into the pool (state.py:547-640): it holds
    ``pool._lock``, calls ``pool._check``, reads ``pool._page(ref).valid``, adds and drops
    owners on ``pool._page(ref)``, builds ``PagedSequence(id(pool), pool.codec.kind, ...)``
    and returns pages with ``pool._collect(page)``. Those steps, as it takes them,
    keep the arena pool's free list exact."""
    from aster_amd.paged_pool import PagedSequence

    pool = make_pool(blocks=6)
    seq = pool.create("domain")
    pool.append_delta(seq, layers(40, 1))  # 2 full pages + 1 partial
    full = seq.pages[:2]
    # publish: full pages only, one owner more each
    with pool._lock:
        pool._check(seq)
        assert all(pool._page(ref).valid == BS for ref in full)
        for ref in full:
            pool._page(ref).owners += 1
    # lookup: a new sequence sharing the published pages
    with pool._lock:
        for ref in full:
            pool._page(ref).owners += 1
        hit = PagedSequence(id(pool), pool.codec.kind, "domain", list(full), 2 * BS)
    pool.append_delta(hit, layers(5, 2))  # extends onto a fresh page (tail was full)
    assert hit.pages[:2] == full and hit.length == 2 * BS + 5
    pool.release(seq)
    pool.release(hit)
    assert pool.used_blocks == 2  # still held by the cache entry
    # evict: drop the cache's owner and collect, as _evict_one_locked does
    with pool._lock:
        for ref in full:
            page = pool._page(ref)
            page.owners -= 1
            pool._collect(page)
            pool._collect(page)  # a second collect must not free the page twice
    assert pool.used_blocks == 0
    fresh = pool.create("domain")
    pool.append_delta(fresh, layers(6 * BS, 3))  # every page exactly once
    assert sorted(ref.index for ref in fresh.pages) == list(range(6))


def test_step_setup_failure_releases_leases_and_reservations(monkeypatch):
    """A failure after the step has reserved slots and leased its pages (an upload of
    the step's metadata, the padding write) undoes both."""
    from aster_amd import runner as runner_module

    pool = make_pool()
    seqs = [pool.create("t") for _ in range(2)]
    for i, s in enumerate(seqs):
        pool.append_delta(s, layers(20, 10 + i))
    used = pool.used_blocks
    calls = []

    def failing_upload(values, dtype, device):
        calls.append(dtype)
        if len(calls) == 2:
            raise RuntimeError("upload failed")
        return torch.tensor(values, dtype=dtype)

    monkeypatch.setattr(runner_module, "_device_ints", failing_upload)
    with pytest.raises(RuntimeError, match="upload failed"):
        runner_module.PagedAttentionStep(pool, seqs, [5, 30])
    assert pool.used_blocks == used
    assert all(pool._pages[ref.index].readers == 0 for s in seqs for ref in s.pages)
    monkeypatch.undo()

    def failing_padding(slots, valid=None):
        raise RuntimeError("padding write failed")

    monkeypatch.setattr(pool.cache, "write_key_valid", failing_padding)
    with pytest.raises(RuntimeError, match="padding write failed"):
        runner_module.PagedAttentionStep(pool, seqs, [5, 30])
    assert pool.used_blocks == used and [s.length for s in seqs] == [20, 20]
    assert all(pool._pages[ref.index].readers == 0 for s in seqs for ref in s.pages)
