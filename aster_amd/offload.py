"""Host swap of paged KV: ``PagedStateArchive`` over the arena-backed pool.

Keeps the behaviour callers of src/aster/inference/offload.py:120-230 rely on: a
bounded host store that holds the archived codes and scales exactly (no
requantization, no float history), restore into freshly reserved pages only under
the identity the snapshot was taken for, a byte budget, metrics, and async variants
that outlive the caller's cancellation and then give back what the finished
transfer produced (the rule of core/async_work.py:20-37).

The design is this library's own:

* ``_Catalog`` owns every piece of shared state (snapshots by handle, the byte
  budget, token counters) behind one lock, so the archive methods never touch the
  lock or the dict themselves;
* transfers are block copies, not per-leaf clones between two device
  synchronisations (offload.py:155-167): ``put`` gathers the sequence's blocks with
  one copy launch into a device staging buffer and DMAs it into (optionally pinned)
  host memory on a dedicated copy stream, under a read lease; ``restore`` DMAs the
  packed blocks back and scatters them into the reserved pages on the same stream
  (``PagedStatePool.restore_pages``). Only these transfers wait; the compute stream
  keeps running;
* the async variants run the blocking transfer on the event loop's executor and wait
  on it with ``asyncio.wait``, which never cancels what it waits for
  (``_outlast_cancellation``); a cancellation that arrives meanwhile is held until
  the worker returns, then the result is handed to a reclaim function and the
  cancellation raised.
"""

from __future__ import annotations

import asyncio
from dataclasses import dataclass
import functools
import math
import threading
import uuid

import torch

from .paged_pool import CacheCapacityError, PagedStatePool, StateError


@dataclass(frozen=True)
class _PagedSnapshot:
    identity: str
    length: int
    codes: torch.Tensor   # host int8 [P, L, 2, Hkv, bs, D]
    scales: torch.Tensor  # host fp32 [P, L, 2, Hkv, bs]
    valid: torch.Tensor   # host uint8 [P, bs]: the pages' padding leaves (0 = padding key)
    nbytes: int


class _Catalog:
    """Snapshots by handle, the host byte budget and the token counters. Every
    method holds the lock for its whole body, so transfers running in executor
    threads and the event loop can share one archive."""

    def __init__(self, budget):
        self.budget = budget
        self._guard = threading.RLock()
        self._snapshots = {}
        self.held_bytes = 0
        self.tokens_out = 0
        self.tokens_in = 0

    def charge(self, nbytes):
        """Hold ``nbytes`` of the budget for a transfer about to start."""
        with self._guard:
            if self.held_bytes + nbytes > self.budget:
                raise CacheCapacityError("Host KV archive is full")
            self.held_bytes += nbytes

    def refund(self, nbytes):
        with self._guard:
            self.held_bytes -= nbytes

    def file(self, snapshot):
        """Register a finished snapshot (its bytes are already charged)."""
        handle = uuid.uuid4().hex
        with self._guard:
            self._snapshots[handle] = snapshot
            self.tokens_out += snapshot.length
        return handle

    def lookup(self, handle, identity):
        with self._guard:
            snapshot = self._snapshots.get(handle)
        if snapshot is None or snapshot.identity != identity:
            raise StateError("Missing archived KV or identity mismatch")
        return snapshot

    def discard(self, handle, identity):
        with self._guard:
            snapshot = self.lookup(handle, identity)
            del self._snapshots[handle]
            self.held_bytes -= snapshot.nbytes

    def note_restored(self, tokens):
        with self._guard:
            self.tokens_in += tokens

    def report(self):
        with self._guard:
            return dict(host_bytes=self.held_bytes, snapshots=len(self._snapshots),
                        offloaded_tokens=self.tokens_out, restored_tokens=self.tokens_in)


async def _outlast_cancellation(call, reclaim):
    """Run ``call()`` on the event loop's default executor and return its result (or
    raise its error). A thread cannot be interrupted, and the transfer it runs owns
    pages and host memory, so a cancellation of the awaiting task does not end the
    wait: ``asyncio.wait`` leaves the job running, the loop goes back to waiting, and
    once the job has returned, a successful result goes to ``reclaim`` before the
    cancellation is raised (chained to the job's error, if it failed)."""
    job = asyncio.get_running_loop().run_in_executor(None, call)
    interrupted = False
    while not job.done():
        try:
            await asyncio.wait((job,))
        except asyncio.CancelledError:
            interrupted = True
    if not interrupted:
        return job.result()
    failure = job.exception()
    if failure is None:
        reclaim(job.result())
    raise asyncio.CancelledError from failure


class PagedStateArchive:
    """Bounded host storage preserving KV codes and scales exactly."""

    def __init__(self, pool, *, max_bytes=256 * 1024**2, pin_memory=False):
        if not isinstance(pool, PagedStatePool) or type(max_bytes) is not int or max_bytes < 1:
            raise ValueError("Archive requires the actual paged pool and a positive byte budget")
        if type(pin_memory) is not bool or (pin_memory and not torch.cuda.is_available()):
            raise ValueError("Pinned host archive requires a provisioned HIP allocator")
        self.pool, self.max_bytes, self.pin_memory = pool, max_bytes, pin_memory
        self._catalog = _Catalog(max_bytes)
        self._stream = None

    @property
    def stored_bytes(self):
        return self._catalog.held_bytes

    def _copy_stream(self):
        if self._stream is None:
            self._stream = torch.cuda.Stream(self.pool.cache.device)  # default priority
        return self._stream

    def _payload_bytes(self, length):
        """Bytes of the archived leaves: codes and scales of every committed token and
        its bool padding byte (what the reference sums over the narrowed page
        payloads, offload.py:146)."""
        c = self.pool.cache
        return length * (c.num_layers * 2 * c.num_kv_heads * (c.head_dim + 4) + 1)

    def _to_host(self, sequence):
        """Gather the sequence's blocks on the copy stream (after the work already
        queued on the compute stream) and DMA them into host tensors; returns once
        the host copies are complete."""
        device = self.pool.cache.device
        stream = self._copy_stream()
        stream.wait_stream(torch.cuda.current_stream(device))
        staged = self.pool.export_blocks(sequence, stream=stream)
        with torch.cuda.stream(stream):
            host = tuple(torch.empty(t.shape, dtype=t.dtype, pin_memory=self.pin_memory)
                         .copy_(t, non_blocking=self.pin_memory) for t in staged)
        finished = torch.cuda.Event()
        finished.record(stream)
        finished.synchronize()
        return host

    def put(self, sequence):
        """Copy the sequence's committed pages to host memory; returns the handle."""
        with self.pool.borrow(sequence):
            length = sequence.length
            if not length:
                raise StateError("Cannot offload an empty request state")
            nbytes = self._payload_bytes(length)
            self._catalog.charge(nbytes)
            try:
                codes, scales, valid = self._to_host(sequence)
            except BaseException:
                # a failed launch may leave copies queued that still read the pages
                torch.cuda.synchronize(self.pool.cache.device)
                self._catalog.refund(nbytes)
                raise
        return self._catalog.file(_PagedSnapshot(sequence.identity, length, codes, scales,
                                                 valid, nbytes))

    def restore(self, handle, *, identity):
        """Fresh pages holding the archived tokens, as a new sequence of ``identity``;
        the snapshot stays archived until ``release``."""
        snapshot = self._catalog.lookup(handle, identity)
        sequence = self.pool.restore_pages((snapshot.codes, snapshot.scales, snapshot.valid),
                                           identity=identity, length=snapshot.length,
                                           stream=self._copy_stream())
        self._catalog.note_restored(snapshot.length)
        return sequence

    def release(self, handle, *, identity):
        self._catalog.discard(handle, identity)

    def pages(self, handle, *, identity):
        """The archived pages as ``QuantizedKV`` leaves per page (host views), then the
        bool padding leaf, narrowed to the committed tokens, in the ``read_pages``
        payload order."""
        from .kv_quantization import QuantizedKV

        snapshot = self._catalog.lookup(handle, identity)
        bs = self.pool.block_size
        fmt = self.pool.quantization.dtype
        out = []
        for p in range(math.ceil(snapshot.length / bs)):
            count = min(bs, snapshot.length - p * bs)
            leaves = [QuantizedKV(snapshot.codes[p, layer, kv][None, :, :count].view(fmt),
                                  snapshot.scales[p, layer, kv][None, :, :count, None],
                                  torch.float32)
                      for layer in range(snapshot.codes.shape[1]) for kv in (0, 1)]
            leaves.append(snapshot.valid[p, :count].bool()[None, None, :, None])
            out.append(tuple(leaves))
        return tuple(out)

    async def put_async(self, sequence):
        """``put`` off the event loop; a cancelled caller's snapshot is released."""
        drop = functools.partial(self.release, identity=sequence.identity)
        return await _outlast_cancellation(functools.partial(self.put, sequence), drop)

    async def restore_async(self, handle, *, identity):
        """``restore`` off the event loop; a cancelled caller's pages are released."""
        return await _outlast_cancellation(
            functools.partial(self.restore, handle, identity=identity), self.pool.release)

    def metrics(self):
        return {**self._catalog.report(), "pinned_memory": self.pin_memory}
