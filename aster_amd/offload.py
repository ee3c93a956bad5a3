"""Host swap of paged KV: ``PagedStateArchive`` over the arena-backed pool.

Follows src/aster/inference/offload.py:120-230: bounded host storage that keeps
the archived codes and scales exactly (no requantization, no float history),
identity-checked restore into freshly reserved pages, byte budget and metrics,
and async variants that reclaim a result whose caller was cancelled
(core/async_work.py:20-37).

The transfers differ: instead of a per-leaf ``clone_kv`` between two device
synchronisations (offload.py:155-167), ``put`` gathers the sequence's blocks with
one copy launch into a device staging buffer and DMAs it into (optionally pinned)
host memory on a dedicated copy stream, under a read lease; ``restore`` DMAs the
packed blocks back and scatters them into the reserved pages on the same stream
(``PagedStatePool.restore_pages``). Only these transfers wait; the compute stream
keeps running.
"""

from __future__ import annotations

import asyncio
from dataclasses import dataclass
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


@dataclass(frozen=True)
class SettledWork:
    value: object = None
    cancelled: bool = False
    error: BaseException | None = None

    def unwrap(self):
        if self.error is not None:
            raise self.error
        return self.value


async def settle_thread(function, *args, **kwargs):
    """Run ``function`` in a worker thread and wait for it to settle even when the
    caller is cancelled, reporting the cancellation beside the result."""
    operation = asyncio.create_task(asyncio.to_thread(function, *args, **kwargs))
    cancelled = False
    while True:
        try:
            return SettledWork(await asyncio.shield(operation), cancelled)
        except asyncio.CancelledError:
            if operation.cancelled():
                raise
            cancelled = True
        except Exception as error:  # noqa: BLE001 - handed back to the caller
            return SettledWork(cancelled=cancelled, error=error)


class PagedStateArchive:
    """Bounded host storage preserving KV codes and scales exactly."""

    def __init__(self, pool, *, max_bytes=256 * 1024**2, pin_memory=False):
        if not isinstance(pool, PagedStatePool) or type(max_bytes) is not int or max_bytes < 1:
            raise ValueError("Archive requires the actual paged pool and a positive byte budget")
        if type(pin_memory) is not bool or (pin_memory and not torch.cuda.is_available()):
            raise ValueError("Pinned host archive requires a provisioned HIP allocator")
        self.pool, self.max_bytes, self.pin_memory = pool, max_bytes, pin_memory
        self._entries = {}
        self._lock = threading.RLock()
        self._stream = None
        self.stored_bytes = 0
        self.offloaded_tokens = self.restored_tokens = 0

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

    def put(self, sequence):
        pool = self.pool
        with pool.borrow(sequence):
            length = sequence.length
            if not length:
                raise StateError("Cannot offload an empty request state")
            size = self._payload_bytes(length)
            with self._lock:
                if self.stored_bytes + size > self.max_bytes:
                    raise CacheCapacityError("Host KV archive is full")
                self.stored_bytes += size
            try:
                stream = self._copy_stream()
                stream.wait_stream(torch.cuda.current_stream(pool.cache.device))
                blocks = pool.export_blocks(sequence, stream=stream)
                with torch.cuda.stream(stream):
                    host = []
                    for t in blocks:
                        h = torch.empty(t.shape, dtype=t.dtype, pin_memory=self.pin_memory)
                        h.copy_(t, non_blocking=self.pin_memory)
                        host.append(h)
                    host_codes, host_scales, host_valid = host
                done = torch.cuda.Event()
                done.record(stream)
                done.synchronize()
                handle = uuid.uuid4().hex
                with self._lock:
                    self._entries[handle] = _PagedSnapshot(sequence.identity, length, host_codes,
                                                           host_scales, host_valid, size)
                    self.offloaded_tokens += length
                return handle
            except BaseException:
                torch.cuda.synchronize(pool.cache.device)
                with self._lock:
                    self.stored_bytes -= size
                raise

    def restore(self, handle, *, identity):
        with self._lock:
            snapshot = self._entries.get(handle)
            if snapshot is None or snapshot.identity != identity:
                raise StateError("Missing archived KV or identity mismatch")
        state = self.pool.restore_pages((snapshot.codes, snapshot.scales, snapshot.valid),
                                        identity=identity,
                                        length=snapshot.length, stream=self._copy_stream())
        with self._lock:
            self.restored_tokens += snapshot.length
        return state

    def release(self, handle, *, identity):
        with self._lock:
            snapshot = self._entries.get(handle)
            if snapshot is None or snapshot.identity != identity:
                raise StateError("Missing archived KV or identity mismatch")
            self._entries.pop(handle)
            self.stored_bytes -= snapshot.nbytes

    def pages(self, handle, *, identity):
        """The archived pages as ``QuantizedKV`` leaves per page (host views), then the
        bool padding leaf, narrowed to the committed tokens, in the ``read_pages``
        payload order."""
        from .kv_quantization import QuantizedKV

        with self._lock:
            snapshot = self._entries.get(handle)
            if snapshot is None or snapshot.identity != identity:
                raise StateError("Missing archived KV or identity mismatch")
        bs = self.pool.block_size
        out = []
        for p in range(math.ceil(snapshot.length / bs)):
            count = min(bs, snapshot.length - p * bs)
            leaves = []
            for layer in range(snapshot.codes.shape[1]):
                for kv in (0, 1):
                    leaves.append(QuantizedKV(snapshot.codes[p, layer, kv][None, :, :count]
                                              .view(self.pool.quantization.dtype),
                                              snapshot.scales[p, layer, kv][None, :, :count, None],
                                              torch.float32))
            leaves.append(snapshot.valid[p, :count].bool()[None, None, :, None])
            out.append(tuple(leaves))
        return tuple(out)

    async def put_async(self, sequence):
        work = await settle_thread(self.put, sequence)
        if work.cancelled:
            if work.error is None:
                self.release(work.value, identity=sequence.identity)
            raise asyncio.CancelledError from work.error
        return work.unwrap()

    async def restore_async(self, handle, *, identity):
        work = await settle_thread(self.restore, handle, identity=identity)
        if work.cancelled:
            if work.error is None:
                self.pool.release(work.value)
            raise asyncio.CancelledError from work.error
        return work.unwrap()

    def metrics(self):
        with self._lock:
            return {
                "host_bytes": self.stored_bytes,
                "snapshots": len(self._entries),
                "offloaded_tokens": self.offloaded_tokens,
                "restored_tokens": self.restored_tokens,
                "pinned_memory": self.pin_memory,
            }
