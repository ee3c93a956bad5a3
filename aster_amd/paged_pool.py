"""Arena-backed paged KV state pool.

Mirrors ``PagedStatePool`` (src/aster/inference/state.py:166-493): a sequence owns
a table of ``block_size``-token pages; ``fork`` shares pages (owners += 1),
``truncate``/``release`` drop them, ``borrow``/``read_pages`` take reader leases,
and appends are transactional: pages are reserved before anything is written,
a tail page that is shared or leased is copied before the writer extends it
(copy-on-write, state.py:306-337), and a failure leaves the page table unchanged.

What differs is where the pages live: not per-page tensors (state.py:319-327) but
blocks of one ``PagedKVCache`` arena, ``PageRef.index`` being the block index. An
append quantizes its tokens straight into their slots with the HIP kernel
(``slot = index * block_size + offset``, state.py:339-344); copy-on-write moves
whole blocks with ``astr_kv_copy_blocks``; attention reads pages through the block
tables of ``block_tables()``; ``restore_pages`` scatters archived blocks into
reserved pages (state.py:427-493). The runner-facing entry is ``reserve``: slots
for a step's tokens, written by per-layer appends and committed (or rolled back)
once the step is done.

Free pages are taken lowest index first, like the reference's scan (state.py:312-314),
from a heap instead of a scan over every page.

Construction follows the reference (state.py:169-180): ``PagedStatePool(*, block_size,
max_blocks, codec, quantization)`` knows no layer shape, and the arena is allocated
at the first append from its leaves (layers, kv heads, head dim, device), which also
locks the layout the way the reference's first append locks its leaf signature
(state.py:297-300). A pool can also wrap an existing ``PagedKVCache``.
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass, field
import heapq
import math
import threading

import torch

from .attention_backend import UnsupportedAttentionBackend
from .kv_quantization import KVQuantization, QuantizedKV, require_format


class StateError(RuntimeError):
    """Invalid use of pool state (state.py:28-29)."""


class CacheCapacityError(StateError):
    """Not enough free pages (state.py:32-33)."""


@dataclass(frozen=True)
class KVStateCodec:
    """The pool's state tag (the reference's ``KVStateCodec``, state.py:45-62, of which
    the arena pool needs only the kind): K/V leaves per layer with the token axis at
    dimension 2. Any object with a ``kind`` attribute (the reference's codec too) can be
    passed as ``codec``."""

    kind: str = "dense_kv"
    sequence_dim: int = 2

    def __post_init__(self):
        if self.kind not in {"dense_kv", "gqa_kv", "mla_latent_rope", "mla_latent", "indexed_mla"}:
            raise ValueError("An explicit supported KV codec tag is required")


@dataclass(frozen=True)
class PageRef:
    index: int
    generation: int


@dataclass
class _Page:
    index: int = 0
    generation: int = 0
    owners: int = 0
    readers: int = 0
    valid: int = 0
    free: bool = True  # on the free heap


@dataclass
class PagedSequence:
    """A request or prefix block table modified only by its owning pool."""

    owner: int
    kind: str
    identity: str
    pages: list = field(default_factory=list)
    length: int = 0
    released: bool = False


@dataclass(frozen=True)
class PageView:
    """A borrowed page: ``offset`` is the absolute position of its first token;
    ``payload`` holds zero-copy ``QuantizedKV`` views ``(k_0, v_0, k_1, v_1, ...)``
    of ``[1, Hkv, count, D]`` codes and ``[1, Hkv, count, 1]`` scales, then the
    padding leaf: a bool view ``[1, 1, count, 1]`` (True = real token), as the
    reference's ``2 * layers + 1`` leaves (paged_attention.py:171-182)."""

    offset: int
    payload: tuple


@dataclass
class SlotReservation:
    """Slots of ``count`` new tokens of ``sequence`` (positions ``start`` ..
    ``start + count - 1``) on the page table ``pages``, not committed yet."""

    sequence: PagedSequence
    start: int
    count: int
    pages: list
    slots: list
    allocated: list
    cow_source: PageRef | None
    done: bool = False

    @property
    def length(self):
        return self.start + self.count

    def slot_mapping(self, device):
        return torch.tensor(self.slots, dtype=torch.int64).to(device, non_blocking=True)


class PagedStatePool:
    evidence_kind = "hip_arena_storage"

    def __init__(self, cache=None, *, block_size=16, max_blocks=256, codec=None,
                 quantization=None, kind=None, device=None):
        if cache is not None:
            require_format(cache.quantization)
            if quantization is not None and quantization != cache.quantization:
                raise ValueError("quantization differs from the arena's format")
            block_size, max_blocks = cache.block_size, cache.num_blocks
            quantization = cache.quantization
        if type(block_size) is not int or type(max_blocks) is not int or block_size < 1 \
                or max_blocks < 1:
            raise ValueError("Cache capacities must be positive")
        if quantization is None:
            raise UnsupportedAttentionBackend(
                "hip_int8_paged pools store quantized codes: pass an explicit KVQuantization "
                "('int8', 'fp8_e4m3fn' or 'fp8_e5m2')")
        if not isinstance(quantization, KVQuantization):
            raise ValueError("An explicit immutable KVQuantization profile is required")
        require_format(quantization)
        if block_size != 16:
            raise UnsupportedAttentionBackend("hip_int8_paged kernels use 16-token blocks")
        if codec is None:
            codec = KVStateCodec(kind=kind or "gqa_kv")
        elif kind is not None and kind != codec.kind:
            raise ValueError("codec and kind disagree")
        if codec.kind not in {"dense_kv", "gqa_kv"} or getattr(codec, "sequence_dim", 2) != 2 \
                or getattr(codec, "sequence_dims", None):
            raise UnsupportedAttentionBackend(
                f"hip_int8_paged pools hold per-layer K/V leaves [1, Hkv, T, D]; codec kind "
                f"{codec.kind!r} is not served")
        self.codec, self.kind = codec, codec.kind
        self.cache = cache
        self.block_size, self.max_blocks = block_size, max_blocks
        self._quantization = quantization
        self._device = torch.device(device) if device is not None else None
        self._pages = [_Page(index=i) for i in range(self.max_blocks)]
        self._free = list(range(self.max_blocks))  # a sorted list is a valid heap
        self._lock = threading.RLock()
        # the arena's layout lock: (layers, kv heads, head dim, input dtype, padding leaf)
        self._signature = None

    @classmethod
    def with_arena(cls, *, num_layers, num_kv_heads, head_dim, block_size=16, max_blocks=256,
                   device="cuda", quantization=None):
        from .paged_kv import PagedKVCache

        return cls(PagedKVCache(num_blocks=max_blocks, num_layers=num_layers,
                                num_kv_heads=num_kv_heads, head_dim=head_dim,
                                block_size=block_size, device=device, quantization=quantization))

    @property
    def quantization(self):
        return self._quantization

    def bind_layout(self, *, num_layers, num_kv_heads, head_dim, device):
        """Allocate the arena for this layout, or check an allocated one against it."""
        with self._lock:
            device = torch.device(device)
            if device.type == "cuda" and device.index is None:
                device = torch.device("cuda", torch.cuda.current_device())
            if self.cache is None:
                if self._device is not None and self._device != device:
                    raise StateError("Cache layout changed within a model pool")
                from .paged_kv import PagedKVCache

                self.cache = PagedKVCache(num_blocks=self.max_blocks, num_layers=num_layers,
                                          num_kv_heads=num_kv_heads, head_dim=head_dim,
                                          block_size=self.block_size, device=device,
                                          quantization=self._quantization)
            c = self.cache
            if (c.num_layers, c.num_kv_heads, c.head_dim) != (num_layers, num_kv_heads, head_dim) \
                    or torch.device(c.device) != device:
                raise StateError("Cache layout changed within a model pool")
            return c

    def _lock_signature(self, signature):
        if self._signature is not None and signature != self._signature:
            raise StateError("Cache layout changed within a model pool")
        self._signature = signature

    # ---- page bookkeeping (state.py:190-206) --------------------------------
    def create(self, identity):
        if not identity:
            raise ValueError("Cache identity must bind an immutable policy")
        return PagedSequence(id(self), self.kind, identity)

    def _check(self, sequence):
        if sequence.owner != id(self) or sequence.kind != self.kind or sequence.released:
            raise StateError("Foreign, mistagged or released sequence")

    def _page(self, ref):
        page = self._pages[ref.index]
        if page.generation != ref.generation or (page.owners == 0 and page.readers == 0):
            raise StateError("Stale page reference")
        return page

    def _collect(self, page):
        """Return a page nobody owns or reads to the free heap (state.py:199-202;
        ``PrefixCache`` calls it with the page object after dropping an owner)."""
        if page.owners == 0 and page.readers == 0 and not page.free:
            page.valid = 0
            page.free = True
            heapq.heappush(self._free, page.index)

    def _allocate(self, count):
        """``count`` fresh pages (owners = 1) or CacheCapacityError, nothing taken."""
        if len(self._free) < count:
            raise CacheCapacityError("State page budget exhausted")
        refs = []
        for _ in range(count):
            index = heapq.heappop(self._free)
            page = self._pages[index]
            page.generation += 1
            page.owners, page.readers, page.valid, page.free = 1, 0, 0, False
            refs.append(PageRef(index, page.generation))
        return refs

    def _drop(self, refs):
        for ref in refs:
            page = self._page(ref)
            page.owners -= 1
            self._collect(page)

    @property
    def used_blocks(self):
        with self._lock:
            return self.max_blocks - len(self._free)

    def fork(self, sequence):
        with self._lock:
            self._check(sequence)
            for ref in sequence.pages:
                self._page(ref).owners += 1
            return PagedSequence(id(self), sequence.kind, sequence.identity, list(sequence.pages),
                                 sequence.length)

    def truncate(self, sequence, length):
        with self._lock:
            self._check(sequence)
            if not 0 <= length <= sequence.length:
                raise ValueError("Cannot extend state by truncation")
            count = math.ceil(length / self.block_size)
            self._drop(sequence.pages[count:])
            sequence.pages = sequence.pages[:count]
            sequence.length = length

    def release(self, sequence):
        with self._lock:
            if sequence.released:
                return
            self._check(sequence)
            self._drop(sequence.pages)
            sequence.released = True
            sequence.pages = []
            sequence.length = 0

    @contextmanager
    def borrow(self, sequence):
        """Reader leases on the sequence's pages for the duration (device work on
        them must have finished before the block exits, state.py:227-244)."""
        with self._lock:
            self._check(sequence)
            refs = tuple(sequence.pages)
            for ref in refs:
                self._page(ref).readers += 1
        try:
            yield sequence
        finally:
            self._unlease(refs)

    def _unlease(self, refs):
        with self._lock:
            for ref in refs:
                page = self._page(ref)
                page.readers -= 1
                self._collect(page)

    # ---- appends ---------------------------------------------------------------
    def reserve(self, sequence, count):
        """Reserve slots for ``count`` new tokens (state.py:301-337 up to the copies):
        fresh pages for the new tokens, and a private copy of a partially filled tail
        page that other sequences or readers hold (copied on the device now, before
        any token is written). Nothing is visible in the sequence until ``commit``."""
        if type(count) is not int or count < 0:
            raise ValueError("Token count must be a non-negative int")
        with self._lock:
            self._check(sequence)
            start = sequence.length
            old = list(sequence.pages)
            needed = math.ceil((start + count) / self.block_size)
            tail = start % self.block_size
            cow = bool(count and tail and old and (self._page(old[-1]).owners > 1
                                                   or self._page(old[-1]).readers > 0))
            allocated = self._allocate(needed - len(old) + int(cow))
            pages = list(old)
            cursor = 0
            try:
                if cow:
                    pages[-1] = allocated[0]
                    cursor = 1
                    self.cache.copy_blocks([old[-1].index], [allocated[0].index])
                    self._pages[allocated[0].index].valid = tail
                pages.extend(allocated[cursor:])
                slots = []
                for offset in range(start, start + count):
                    page, slot = divmod(offset, self.block_size)
                    slots.append(pages[page].index * self.block_size + slot)
            except BaseException:
                self._drop(allocated)
                raise
            return SlotReservation(sequence, start, count, pages, slots, allocated,
                                   old[-1] if cow else None)

    def commit(self, reservation):
        """Publish a reservation: the tokens count, the copied tail page replaces the
        shared one (whose owner count drops), fresh pages join the table."""
        with self._lock:
            if reservation.done:
                raise StateError("Reservation already committed or aborted")
            sequence = reservation.sequence
            self._check(sequence)
            if sequence.length != reservation.start:
                raise StateError("Sequence changed while a reservation was open")
            for offset in range(reservation.start, reservation.length):
                page, slot = divmod(offset, self.block_size)
                entry = self._page(reservation.pages[page])
                entry.valid = max(entry.valid, slot + 1)
            if reservation.cow_source is not None:
                self._drop([reservation.cow_source])
            sequence.pages, sequence.length = list(reservation.pages), reservation.length
            reservation.done = True

    def abort(self, reservation):
        """Drop a reservation: fresh pages (and the private tail copy) are freed."""
        with self._lock:
            if reservation.done:
                return
            self._drop(reservation.allocated)
            reservation.done = True

    @contextmanager
    def transaction(self, sequence, count):
        reservation = self.reserve(sequence, count)
        try:
            yield reservation
        except BaseException:
            self.abort(reservation)
            raise
        self.commit(reservation)

    def append_delta(self, sequence, layers, *, check=True):
        """Commit new-token K/V of every layer (state.py:261-267): ``layers`` is one
        ``(key, value)`` per arena layer, ``[1, Hkv, T, D]`` (the reference's state
        leaves) or ``[T, Hkv, D]`` floating device tensors, optionally followed by the
        padding leaf ``(padding,)``: ``[1, 1, T, 1]`` (or ``[T]``) bool/0-1, True = real
        token, as the runner appends it (paged_attention.py:228-229). Quantized on the
        device into reserved slots; non-finite input raises ValueError and commits
        nothing (kv_quantization.py:77-81)."""
        rows, padding = self._token_rows(layers)
        count = rows[0][0].shape[0]
        with self.transaction(sequence, count) as reservation:
            if count:
                slots = reservation.slot_mapping(self.cache.device)
                for layer, (key, value) in enumerate(rows):
                    self.cache.append(layer, key, value, slots)
                self.cache.write_key_valid(slots, padding)
                if check:
                    self.cache.raise_errors()
        return reservation

    def append(self, sequence, layers, *, check=True):
        """Append the suffix of a full state (state.py:254-258): tokens from the
        sequence's committed length on."""
        rows, padding = self._token_rows(layers)
        total = rows[0][0].shape[0]
        if total < sequence.length:
            raise StateError("Append cannot shrink state")
        start = sequence.length
        suffix = [(k[start:], v[start:]) for k, v in rows]
        if padding is not None:
            suffix.append((padding[start:],))
        return self.append_delta(sequence, suffix, check=check)

    def _token_rows(self, layers):
        """``(rows, padding)``: one ``[T, Hkv, D]`` ``(key, value)`` per layer and the
        padding leaf as a bool device vector ``[T]`` (None when absent; a trailing
        one-element tuple is the padding leaf, as the runner appends it,
        paged_attention.py:228). The first append allocates the arena from these
        leaves; every append must match its layout, input dtype and device
        (state.py:285-300)."""
        layers = tuple(layers)
        if not layers:
            raise StateError("KV state must be a nonempty tuple tree of tensors")
        padding = None
        last = layers[-1]
        if not (isinstance(last, (tuple, list)) and len(last) == 2):
            padding = last[0] if isinstance(last, (tuple, list)) and len(last) == 1 else last
            layers = layers[:-1]
        rows = []
        for item in layers:
            if not (isinstance(item, (tuple, list)) and len(item) == 2):
                raise StateError("Cache layout changed within a model pool")
            pair = []
            for t in item:
                if not isinstance(t, torch.Tensor) or not t.is_floating_point():
                    raise StateError(
                        "Quantized KV requires token/head vectors, not an arbitrary state tensor")
                if t.ndim == 4:
                    if t.shape[0] != 1:
                        raise StateError("Page storage accepts single-sequence states only")
                    t = t[0].transpose(0, 1)  # [1, Hkv, T, D] -> [T, Hkv, D] view
                if t.ndim != 3:
                    raise StateError("Invalid KV tensor layout")
                pair.append(t)
            if pair[0].shape != pair[1].shape:
                raise StateError("Every cache leaf must describe the same token span")
            rows.append(tuple(pair))
        if not rows:
            raise StateError("KV state must be a nonempty tuple tree of tensors")
        first = rows[0][0]
        if any(t.shape[1:] != first.shape[1:] or t.dtype != first.dtype
               or t.device != first.device for pair in rows for t in pair):
            raise StateError("Cache layout changed within a model pool")
        if len({k.shape[0] for k, _ in rows}) != 1:
            raise StateError("Every cache leaf must describe the same token span")
        with self._lock:
            cache = self.bind_layout(num_layers=len(rows), num_kv_heads=first.shape[1],
                                     head_dim=first.shape[2], device=first.device)
            self._lock_signature((len(rows), first.shape[1], first.shape[2], first.dtype))
        if padding is not None:
            padding = torch.as_tensor(padding, device=cache.device)
            if padding.ndim == 4:
                if padding.shape[0] != 1 or padding.shape[1] != 1 or padding.shape[3] != 1:
                    raise StateError("Padding leaf must be [1, 1, tokens, 1]")
                padding = padding[0, 0, :, 0]
            if padding.ndim != 1 or not ((padding == 0) | (padding == 1)).all():
                raise StateError("Padding leaf must be a binary token vector")
            if padding.shape[0] != first.shape[0]:
                raise StateError("Every cache leaf must describe the same token span")
            padding = padding.bool()
        return rows, padding

    # ---- reads --------------------------------------------------------------
    @contextmanager
    def read_pages(self, sequence):
        """Zero-copy page views narrowed to committed tokens, under reader leases
        (state.py:358-390)."""
        with self._lock:
            self._check(sequence)
            refs, length = tuple(sequence.pages), sequence.length
            if len(refs) != math.ceil(length / self.block_size):
                raise StateError("Block table length differs from committed tokens")
            views = []
            for index, ref in enumerate(refs):
                page = self._page(ref)
                count = min(self.block_size, length - index * self.block_size)
                if page.valid < count:
                    raise StateError("Cannot expose an uninitialized page")
                payload = []
                for layer in range(self.cache.num_layers):
                    for leaf in self.cache.page(ref.index, layer):
                        payload.append(leaf.narrow(2, 0, count))
                payload.append(self.cache.padding_leaf(ref.index)[:, :, :count])
                views.append(PageView(index * self.block_size, tuple(payload)))
            for ref in refs:
                self._page(ref).readers += 1
        try:
            yield tuple(views)
        finally:
            self._unlease(refs)

    @contextmanager
    def block_tables(self, items, *, width=None):
        """Block tables and context lengths of a step's rows for the attention
        kernels, under reader leases: ``items`` are sequences (committed length) or
        reservations (length including the reserved tokens). Yields int32 device
        tensors ``block_tables [B, width]`` and ``context_lens [B]``."""
        with self._lock:
            tables, lengths, refs = [], [], []
            for item in items:
                if isinstance(item, SlotReservation):
                    if item.done:
                        raise StateError("Reservation already committed or aborted")
                    self._check(item.sequence)
                    pages, length = item.pages, item.length
                else:
                    self._check(item)
                    pages, length = item.pages, item.length
                for ref in pages:
                    self._page(ref)
                tables.append([ref.index for ref in pages])
                lengths.append(length)
                refs.extend(pages)
            width = width or max([len(t) for t in tables] + [1])
            if any(len(t) > width for t in tables):
                raise ValueError("block table width too small")
            if self.cache is None:
                raise StateError("The pool's arena is not allocated before its first append")
            for ref in refs:
                self._page(ref).readers += 1
        try:
            host = torch.zeros((len(tables), width), dtype=torch.int32)
            for row, t in enumerate(tables):
                host[row, : len(t)] = torch.tensor(t, dtype=torch.int32)
            device = self.cache.device
            yield (host.to(device, non_blocking=True),
                   torch.tensor(lengths, dtype=torch.int32).to(device, non_blocking=True))
        finally:
            self._unlease(refs)

    def materialize(self, sequence):
        """Dequantized history ``((k, v), ..., (padding,))``: per layer ``[1, Hkv, T, D]``
        fp32, then the padding leaf ``[1, 1, T, 1]`` bool, the structure the runner
        appends (state.py:392-409); None for an empty sequence."""
        with self._lock:
            self._check(sequence)
            if not sequence.length:
                return None
            for index, ref in enumerate(sequence.pages):
                count = min(self.block_size, sequence.length - index * self.block_size)
                if self._page(ref).valid < count:
                    raise StateError("Uninitialized cache page")
            blocks = torch.tensor([ref.index for ref in sequence.pages], dtype=torch.long,
                                  device=self.cache.device)
            layers = []
            for layer in range(self.cache.num_layers):
                pair = []
                for kv in (0, 1):
                    codes = self.cache.codes[blocks, layer, kv]    # [P, Hkv, bs, D]
                    scales = self.cache.scales[blocks, layer, kv]  # [P, Hkv, bs]
                    x = self.cache.code_view(codes).float() * scales[..., None]
                    x = x.permute(1, 0, 2, 3).reshape(x.shape[1], -1, x.shape[-1])
                    pair.append(x[None, :, : sequence.length])
                layers.append(tuple(pair))
            padding = self.cache.key_valid[blocks].reshape(-1)[: sequence.length]
            layers.append((padding.bool()[None, None, :, None],))
            return tuple(layers)

    def storage_metrics(self):
        """Persistent page storage including scales (state.py:411-425): every page
        in use holds 2 * num_layers quantized leaves and the bool padding leaf."""
        with self._lock:
            used = self.used_blocks
            c = self.cache
            per_page = (c.block_code_bytes + c.block_scale_bytes + c.block_size) if c else 0
            return {
                "format": self.quantization.format,
                "allocated_tensor_bytes": used * per_page,
                "quantized_leaves": used * 2 * c.num_layers if c else 0,
                "physical_pages": used,
            }

    # ---- host swap ------------------------------------------------------------
    def export_blocks(self, sequence, *, stream=None):
        """Device copies ``(codes, scales, valid)`` of the sequence's pages packed in
        page order (the gather half of host swap), enqueued on ``stream``; the caller
        holds a read lease until the copy has finished."""
        with self._lock:
            self._check(sequence)
            blocks = [ref.index for ref in sequence.pages]
        return self.cache.gather_blocks(blocks, stream=stream)

    def restore_pages(self, payloads, *, identity, length, stream=None):
        """Reserve every destination page, move the archived codes and scales in
        without requantization, publish after the copy completes (state.py:427-493).

        ``payloads``: one tuple per page of ``2 * num_layers`` ``QuantizedKV`` leaves
        ``(k_0, v_0, ...)`` of ``[1, Hkv, count, D]`` codes (in the format's dtype) and
        ``[1, Hkv, count, 1]`` fp32 scales, optionally followed by the padding leaf
        ``[1, 1, count, 1]`` (what ``read_pages`` exposes and ``PagedStateArchive``
        keeps), or ``(codes, scales[, valid])`` already packed in the
        ``export_blocks`` layout on the host."""
        sequence = self.create(identity)
        if type(length) is not int or length < 1:
            raise StateError("Archived page count and token length differ")
        if self.cache is None:  # no arena yet: its layout is unknown (state.py:453-454)
            raise StateError("Restore requires this initialized model pool")
        count = math.ceil(length / self.block_size)
        packed = self._pack(payloads, length) if not _is_packed(payloads) else payloads
        codes, scales = packed[0], packed[1]
        valid = packed[2] if len(packed) == 3 else None
        if valid is not None:
            if tuple(valid.shape) != (codes.shape[0], self.block_size):
                raise StateError("Archived padding layout differs from model pool")
            if bool(valid.reshape(-1)[:length].bool().all()):
                valid = None  # every committed key real: the arena needs no padding bytes
        if codes.shape[0] != count:
            raise StateError("Archived page count and token length differ")
        with self._lock:
            refs = self._allocate(count)
        stream = stream or torch.cuda.current_stream(self.cache.device)
        try:
            # pages just freed may still be read by work queued before their release
            stream.wait_stream(torch.cuda.current_stream(self.cache.device))
            with torch.cuda.stream(stream):
                dcodes = codes.to(self.cache.device, non_blocking=True)
                dscales = scales.to(self.cache.device, non_blocking=True)
                dvalid = (valid.to(torch.uint8).to(self.cache.device, non_blocking=True)
                          if valid is not None else None)
            self.cache.scatter_blocks([ref.index for ref in refs], dcodes, dscales, dvalid,
                                      stream=stream)
            done = torch.cuda.Event()
            done.record(stream)
            done.synchronize()
            torch.cuda.current_stream(self.cache.device).wait_event(done)
        except BaseException:
            torch.cuda.synchronize(self.cache.device)
            with self._lock:
                self._drop(refs)
            raise
        with self._lock:
            for i, ref in enumerate(refs):
                self._page(ref).valid = min(self.block_size, length - i * self.block_size)
            sequence.pages, sequence.length = refs, length
        return sequence

    def _pack(self, payloads, length):
        """Page leaves -> host tensors in the export_blocks layout (validated like
        state.py:436-451)."""
        c = self.cache
        count = math.ceil(length / self.block_size)
        if len(payloads) != count:
            raise StateError("Archived page count and token length differ")
        codes = torch.zeros((count,) + tuple(c.codes.shape[1:]), dtype=torch.int8)
        scales = torch.ones((count,) + tuple(c.scales.shape[1:]), dtype=torch.float32)
        valid = torch.ones((count, self.block_size), dtype=torch.uint8)
        for p, leaves in enumerate(payloads):
            tokens = min(self.block_size, length - p * self.block_size)
            if len(leaves) == 2 * c.num_layers + 1:
                pad = leaves[-1]
                if isinstance(pad, QuantizedKV) or tuple(pad.shape) != (1, 1, tokens, 1) or \
                        not ((pad == 0) | (pad == 1)).all():
                    raise StateError("Archived padding leaf differs")
                valid[p, :tokens] = pad[0, 0, :, 0].to(torch.uint8).cpu()
                leaves = leaves[:-1]
            if len(leaves) != 2 * c.num_layers:
                raise StateError("Archived leaf plan differs")
            for i, leaf in enumerate(leaves):
                if not isinstance(leaf, QuantizedKV):
                    raise StateError("Archived low-bit format differs")
                if leaf.values.dtype != self.quantization.dtype:
                    raise StateError("Archived quantization format changed")
                want = (1, c.num_kv_heads, tokens, c.head_dim)
                if tuple(leaf.values.shape) != want or tuple(leaf.scales.shape) != want[:3] + (1,):
                    raise StateError("Archived KV layout differs from model pool")
                layer, kv = divmod(i, 2)
                codes[p, layer, kv, :, :tokens] = leaf.values[0].cpu().view(torch.int8)
                scales[p, layer, kv, :, :tokens] = leaf.scales[0, ..., 0].cpu()
        return codes, scales, valid


def _is_packed(payloads):
    return (isinstance(payloads, tuple) and len(payloads) in (2, 3)
            and all(isinstance(t, torch.Tensor) for t in payloads))
