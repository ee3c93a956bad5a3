"""The attention part of a paged forward step on the ``hip_int8_paged`` backend.

``PagedAttentionRunner.forward_batch`` (src/aster/inference/paged_attention.py:110-230)
takes read leases on every row's pages, and per layer runs one ``online_attention``
per row over the row's pages plus the chunk's own (quantized) K/V, appending the
chunk to the pool only after the step (:226-229). ``PagedAttentionStep`` replaces
that row loop:

  * on entry it reserves the step's slots in the pool for every row
    (transactionally: all rows or none) and builds one block table over the
    reserved pages, with ``query_start_loc`` packing ragged chunk lengths;
  * per layer, ``attend`` quantize-appends the chunk K/V of all rows into their
    slots in one launch and runs one ragged attention launch (decode rows on the
    decode kernels, chunk rows on the prefill kernel) over history + chunk,
    causal within the chunk, exactly the keys the reference's per-row call sees;
  * on exit it checks the device error flag and commits every reservation, or
    rolls all of them back if the step raised.

Row lengths need not match (the reference groups equal ``start``/``count`` per
call, :118-123). Chunk padding (``forward_batch(padding_masks=...)``, :137-143) is
written once per step into the reserved slots' key bytes: a padding token is
appended like any other but attended by no query, in this step or later, as the
reference's padding leaf does (:181, :190, :228).
"""

from __future__ import annotations

import torch

from .attention_backend import BACKEND, KernelWork
from .paged_pool import StateError


def pack_rows(x, counts):
    """Reference layout ``[B, H, Q, D]`` (rows padded to Q) -> packed ``[sum(counts), H, D]``."""
    if x.ndim != 4 or x.shape[0] != len(counts):
        raise ValueError("expected [batch, heads, tokens, head_dim] rows")
    rows = [x[b, :, :n].transpose(0, 1) for b, n in enumerate(counts)]
    return torch.cat(rows, 0).contiguous() if rows else x.new_empty((0, x.shape[1], x.shape[3]))


def unpack_rows(y, counts, width=None):
    """Packed ``[sum(counts), H, D]`` -> ``[B, H, width, D]`` (zero-padded rows)."""
    width = width or max(counts)
    out = y.new_zeros((len(counts), y.shape[1], width, y.shape[2]))
    cursor = 0
    for b, n in enumerate(counts):
        out[b, :, :n] = y[cursor : cursor + n].transpose(0, 1)
        cursor += n
    return out


def _padding_vector(padding, counts):
    """Chunk padding as a host bool vector packed like the step's tokens: one 0/1
    sequence per row (``len == counts[b]``) or a batch-by-token matrix whose row ``b``
    starts with the row's ``counts[b]`` tokens (paged_attention.py:137-143)."""
    rows = []
    if isinstance(padding, (list, tuple)):
        if len(padding) != len(counts):
            raise ValueError("Chunk padding must be a binary batch-by-token matrix")
        for row, n in zip(padding, counts):
            row = torch.as_tensor(row).cpu()
            if row.ndim != 1 or row.shape[0] != n:
                raise ValueError("Chunk padding must be a binary batch-by-token matrix")
            rows.append(row)
    else:
        matrix = torch.as_tensor(padding).cpu()
        if matrix.ndim != 2 or matrix.shape[0] != len(counts) or matrix.shape[1] < max(counts):
            raise ValueError("Chunk padding must be a binary batch-by-token matrix")
        rows = [matrix[b, :n] for b, n in enumerate(counts)]
    packed = torch.cat(rows)
    if not ((packed == 0) | (packed == 1)).all():
        raise ValueError("Chunk padding must be a binary batch-by-token matrix")
    return packed.bool()


class PagedAttentionStep:
    """One step of ``counts[b]`` new tokens for each sequence ``b`` of a batch."""

    def __init__(self, pool, sequences, counts, *, padding=None, work=None,
                 partition_tokens=0):
        if not sequences or len(sequences) != len(counts) or \
                len({id(s) for s in sequences}) != len(sequences):
            raise ValueError("Need a nonempty batch of distinct sequences and aligned chunks")
        if any(type(n) is not int or n < 1 for n in counts):
            raise ValueError("Every row needs at least one new token")
        if len({s.identity for s in sequences}) != 1:
            raise StateError("A projection batch cannot cross cache security domains")
        valid = None if padding is None else _padding_vector(padding, counts)
        self.pool, self.counts = pool, list(counts)
        self.work = work if work is not None else KernelWork()
        self.partition_tokens = partition_tokens
        self.reservations = []
        try:
            for sequence, n in zip(sequences, counts):
                self.reservations.append(pool.reserve(sequence, n))
        except BaseException:
            for r in self.reservations:
                pool.abort(r)
            raise
        cache = pool.cache
        device = cache.device
        self._tables = pool.block_tables(self.reservations)
        self.block_tables, self.context_lens = self._tables.__enter__()
        starts = [0]
        for n in counts:
            starts.append(starts[-1] + n)
        self.num_tokens = starts[-1]
        self.query_start_loc = torch.tensor(starts, dtype=torch.int32).to(device, non_blocking=True)
        self.positions = [r.start for r in self.reservations]
        self.max_query_len = max(counts)
        self.max_context_len = max(r.length for r in self.reservations)
        slots = [s for r in self.reservations for s in r.slots]
        self.slot_mapping = torch.tensor(slots, dtype=torch.int64).to(device, non_blocking=True)
        try:
            cache.write_key_valid(self.slot_mapping,
                                  None if valid is None else valid.to(device, non_blocking=True))
        except BaseException:
            self._tables.__exit__(None, None, None)
            for r in self.reservations:
                pool.abort(r)
            raise
        self._open = True

    def attend(self, layer, query, key, value, *, scale=None, window=None, out=None):
        """Append this layer's chunk K/V and attend. ``query`` ``[T, Hq, D]`` and
        ``key``/``value`` ``[T, Hkv, D]`` packed by row in batch order (``pack_rows``
        converts the reference's ``[B, H, Q, D]``). Returns ``[T, Hq, D]`` in the
        query dtype."""
        if not self._open:
            raise StateError("Step already committed or aborted")
        if query.shape[0] != self.num_tokens or key.shape[0] != self.num_tokens:
            raise ValueError("query/key rows must match the step's tokens")
        cache = self.pool.cache
        cache.append(layer, key, value, self.slot_mapping)
        ws_work = self.work
        return cache.paged_attention(
            layer, query, self.block_tables, self.context_lens,
            max_context_len=self.max_context_len, scale=scale, window=window,
            partition_tokens=self.partition_tokens, query_start_loc=self.query_start_loc,
            max_query_len=self.max_query_len, causal=True, out=out, work=ws_work)

    def commit(self):
        """Wait for the device, raise any flagged error (then nothing is committed),
        release the read leases and publish every row's tokens."""
        if not self._open:
            raise StateError("Step already committed or aborted")
        try:
            torch.cuda.synchronize(self.pool.cache.device)
            self.pool.cache.raise_errors()
        except BaseException:
            self.abort()
            raise
        self._close()
        for r in self.reservations:
            self.pool.commit(r)
        self.work.backend, self.work.fallback_reason = BACKEND, None

    def abort(self):
        if not self._open:
            return
        torch.cuda.synchronize(self.pool.cache.device)
        self._close()
        for r in self.reservations:
            self.pool.abort(r)

    def _close(self):
        self._open = False
        self._tables.__exit__(None, None, None)

    def __enter__(self):
        return self

    def __exit__(self, kind, error, trace):
        if kind is None:
            self.commit()
        else:
            self.abort()
        return False
