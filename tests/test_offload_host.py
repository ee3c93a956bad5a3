"""Host-side rules of PagedStateArchive on a CPU stand-in pool (the transfers
themselves run on the GPU in test_gpu_pool.py): the async variants outlast their
caller's cancellation and then reclaim what the finished transfer produced
(test_paged_offload.py:100-141, async_work.py:20-37), errors pass through, and the
catalog keeps the byte budget, identities and counters (offload.py:140-228)."""

import asyncio
import threading

import pytest
import torch

from aster_amd.offload import PagedStateArchive, _Catalog, _PagedSnapshot
from aster_amd.paged_pool import CacheCapacityError, PagedStatePool, StateError
from tests.fake_arena import FakeArena


def make_archive(**kw):
    pool = PagedStatePool(FakeArena(num_blocks=8, num_layers=1, num_kv_heads=2, head_dim=16,
                                    block_size=16))
    return PagedStateArchive(pool, **kw)


def _snapshot(identity, length, nbytes):
    empty = torch.empty(0)
    return _PagedSnapshot(identity, length, empty, empty, empty, nbytes)


@pytest.mark.parametrize("operation", ["put", "restore"])
def test_cancelled_caller_waits_for_the_transfer_then_reclaims(operation, monkeypatch):
    archive = make_archive()
    entered, finish = threading.Event(), threading.Event()
    reclaimed = []

    def slow(*args, **kwargs):
        entered.set()
        assert finish.wait(5)
        return f"{operation}-result"

    monkeypatch.setattr(archive, operation, slow)
    if operation == "put":
        monkeypatch.setattr(archive, "release", lambda h, *, identity: reclaimed.append((h, identity)))
    else:
        monkeypatch.setattr(archive.pool, "release", lambda s: reclaimed.append(s))
    seq = archive.pool.create("tenant")

    async def run():
        task = asyncio.create_task(archive.put_async(seq) if operation == "put" else
                                   archive.restore_async("h", identity="tenant"))
        assert await asyncio.to_thread(entered.wait, 5)
        for _ in range(2):  # repeated cancellation does not abandon the transfer
            task.cancel()
            await asyncio.sleep(0)
            assert not task.done()
        finish.set()
        with pytest.raises(asyncio.CancelledError):
            await task

    try:
        asyncio.run(run())
    finally:
        finish.set()
    want = ("put-result", "tenant") if operation == "put" else "restore-result"
    assert reclaimed == [want]


def test_async_results_and_errors_pass_through(monkeypatch):
    archive = make_archive()
    seq = archive.pool.create("tenant")
    monkeypatch.setattr(archive, "put", lambda s: "handle")
    assert asyncio.run(archive.put_async(seq)) == "handle"

    def full(s):
        raise CacheCapacityError("Host KV archive is full")

    monkeypatch.setattr(archive, "put", full)
    with pytest.raises(CacheCapacityError):
        asyncio.run(archive.put_async(seq))


def test_cancellation_during_a_failing_transfer_reclaims_nothing(monkeypatch):
    archive = make_archive()
    entered, finish = threading.Event(), threading.Event()
    reclaimed = []

    def failing(*args, **kwargs):
        entered.set()
        assert finish.wait(5)
        raise StateError("Missing archived KV or identity mismatch")

    monkeypatch.setattr(archive, "restore", failing)
    monkeypatch.setattr(archive.pool, "release", reclaimed.append)

    async def run():
        task = asyncio.create_task(archive.restore_async("h", identity="x"))
        assert await asyncio.to_thread(entered.wait, 5)
        task.cancel()
        await asyncio.sleep(0)
        finish.set()
        with pytest.raises(asyncio.CancelledError):
            await task

    try:
        asyncio.run(run())
    finally:
        finish.set()
    assert reclaimed == []  # nothing was produced, nothing to give back


def test_catalog_budget_identity_and_counters():
    cat = _Catalog(100)
    cat.charge(60)
    with pytest.raises(CacheCapacityError):
        cat.charge(41)
    cat.charge(40)
    cat.refund(40)
    handle = cat.file(_snapshot("a", 7, 60))
    assert cat.lookup(handle, "a").length == 7
    for bad in ((handle, "b"), ("nope", "a")):
        with pytest.raises(StateError):
            cat.lookup(*bad)
        with pytest.raises(StateError):
            cat.discard(*bad)
    cat.note_restored(7)
    assert cat.report() == dict(host_bytes=60, snapshots=1, offloaded_tokens=7, restored_tokens=7)
    cat.discard(handle, "a")
    assert cat.report() == dict(host_bytes=0, snapshots=0, offloaded_tokens=7, restored_tokens=7)


def test_archive_arguments_and_metrics():
    archive = make_archive(max_bytes=1024)
    assert archive.stored_bytes == 0
    assert archive.metrics() == dict(host_bytes=0, snapshots=0, offloaded_tokens=0,
                                     restored_tokens=0, pinned_memory=False)
    for bad in (dict(max_bytes=0), dict(max_bytes=1.5), dict(pin_memory=1)):
        with pytest.raises(ValueError):
            make_archive(**bad)
    with pytest.raises(ValueError):
        PagedStateArchive(object())
    with pytest.raises(StateError):
        archive.release("nope", identity="a")
