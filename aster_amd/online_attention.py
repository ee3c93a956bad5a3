"""Op-level attention over explicit KV pages on the HIP path: the reference's
``online_attention``, ``online_attention_statistics`` and ``merge_softmax``
(src/aster/optimization/online_attention.py) for callers that hold ``AttentionBlock``
pages rather than a paged arena.

Both attention calls check their arguments as the reference does (same exceptions and
messages, online_attention.py:89-147), then lay the blocks' quantized codes and
scales into a transient single-layer arena. Each block's token ``t`` goes to
absolute position ``offset + t``; positions no block covers, and key padding, become
padding keys. Each query token then attends as one decode row of the library's
paged kernels, its context ending at its own position (causal) or at the last key.
That gives the causal mask (``k <= p``) and the window (``k > p - window``) of
online_attention.py:175-188. ``online_attention`` returns the rows' outputs;
``online_attention_statistics`` the rows' unnormalised states from the exact fp32
decode kernels (``astr_paged_attention_i8_statistics``). ``merge_softmax`` runs a
HIP kernel over fp32 states (``astr_merge_softmax_f32``).

Not served (``UnsupportedAttentionBackend``, never a silent downgrade):
  * plain tensor K/V, since the path attends to quantized pages;
  * blocks of different code formats, and value widths unlike the key width;
  * fp64 queries or states.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _native
from .attention_backend import UnsupportedAttentionBackend
from .kv_quantization import KVQuantization, QuantizedKV
from .paged_kv import PagedKVCache

BLOCK = 16
_FORMAT_OF_DTYPE = {torch.int8: "int8", torch.float8_e4m3fn: "fp8_e4m3fn",
                    torch.float8_e5m2: "fp8_e5m2"}


@dataclass(frozen=True)
class AttentionBlock:
    """One KV page: ``key``/``value`` ``[B, Hkv, T, D]``, the absolute position of its
    first token and optional key padding ``[B, T]`` (online_attention.py:10-15)."""

    key: object
    value: object
    offset: int
    padding: torch.Tensor | None = None


@dataclass(frozen=True)
class SoftmaxState:
    """``maximum`` and ``mass`` ``[B, Hkv, G, Q]``, ``weighted`` ``[B, Hkv, G, Q, Dv]``
    (online_attention.py:29-39)."""

    maximum: torch.Tensor
    mass: torch.Tensor
    weighted: torch.Tensor

    def output(self, *, dtype=None):
        value = self.weighted / self.mass.clamp_min(torch.finfo(self.mass.dtype).tiny)[..., None]
        batch, heads, groups, query, width = value.shape
        return value.reshape(batch, heads * groups, query, width).to(dtype or value.dtype)


@torch.no_grad()
def merge_softmax(left, right):
    """Merge the statistics of two disjoint KV partitions (online_attention.py:42-63)
    with ``astr_merge_softmax_f32``; fp32 device states."""
    if (
        left.maximum.shape != right.maximum.shape
        or left.weighted.shape != right.weighted.shape
        or left.maximum.dtype != right.maximum.dtype
        or left.maximum.device != right.maximum.device
    ):
        raise ValueError(
            "Attention partitions must describe the same queries and accumulator layout")
    tensors = (left.maximum, left.mass, left.weighted, right.maximum, right.mass, right.weighted)
    if any(t.device.type != "cuda" for t in tensors):
        raise UnsupportedAttentionBackend("hip_int8_paged merges device states")
    if any(t.device != left.maximum.device for t in tensors):
        raise ValueError(
            "Attention partitions must describe the same queries and accumulator layout")
    if any(t.dtype != torch.float32 for t in tensors):
        raise UnsupportedAttentionBackend("hip_int8_paged merges fp32 softmax states")
    if (left.mass.shape != left.maximum.shape or right.mass.shape != right.maximum.shape
            or left.weighted.shape[:-1] != left.maximum.shape):
        raise ValueError(
            "Attention partitions must describe the same queries and accumulator layout")
    ma, la, na, mb, lb, nb = (t.contiguous() for t in tensors)
    mo, lo, no = torch.empty_like(ma), torch.empty_like(la), torch.empty_like(na)
    rows, width = ma.numel(), na.shape[-1]
    stream = torch.cuda.current_stream(ma.device).cuda_stream
    rc = _native.lib().astr_merge_softmax_f32(
        ma.data_ptr(), la.data_ptr(), na.data_ptr(), mb.data_ptr(), lb.data_ptr(), nb.data_ptr(),
        mo.data_ptr(), lo.data_ptr(), no.data_ptr(), rows, width, stream)
    _native.check(rc, "merge_softmax")
    return SoftmaxState(mo, lo, no)


def _binary_mask(value, shape, device, name):
    if value is None:
        return None
    if value.shape != shape or value.device != device or not ((value == 0) | (value == 1)).all():
        raise ValueError(name + " must be a colocated aligned binary mask")
    return value.bool()


def _finite(value):
    if isinstance(value, QuantizedKV):
        return bool(torch.isfinite(value.values.float()).all() and torch.isfinite(value.scales).all()
                    and (value.scales > 0).all())
    return bool(torch.isfinite(value).all())


def _length(value):
    return value.shape[-2]


def _check(query, blocks, query_positions, causal, window, query_padding, scale,
           query_block_size, key_block_size):
    """The reference's argument checks (online_attention.py:89-147), in its order."""
    if (
        query.ndim != 4
        or min(query.shape) < 1
        or not query.is_floating_point()
        or type(query_block_size) is not int
        or type(key_block_size) is not int
        or min(query_block_size, key_block_size) < 1
        or not blocks
    ):
        raise ValueError("Need nonempty query/pages and positive integer tile sizes")
    if not torch.isfinite(query).all():
        raise ValueError("Query must be finite")
    if type(causal) is not bool or (window is not None and (type(window) is not int or window < 1)):
        raise ValueError("Invalid causal/window semantics")
    batch, query_heads, queries, key_width = query.shape
    if (
        query_positions.shape != (batch, queries)
        or query_positions.device != query.device
        or query_positions.dtype not in {torch.int32, torch.int64}
        or (query_positions < 0).any()
    ):
        raise ValueError("Query positions must explicitly align the absolute token axis")
    query_padding = _binary_mask(query_padding, (batch, queries), query.device, "query padding")
    if (not isinstance(blocks[0], AttentionBlock) or blocks[0].key.ndim != 4
            or blocks[0].value.ndim != 4):
        raise ValueError("Expected explicit rank-four KV blocks")
    heads, value_width = blocks[0].key.shape[1], blocks[0].value.shape[-1]
    if heads < 1 or query_heads % heads:
        raise ValueError("Query heads must divide into KV groups")
    intervals = []
    for block in blocks:
        if (
            not isinstance(block, AttentionBlock)
            or block.key.ndim != 4
            or block.value.ndim != 4
            or tuple(block.key.shape[:2]) != (batch, heads)
            or block.key.shape[-1] != key_width
            or tuple(block.key.shape[:3]) != tuple(block.value.shape[:3])
            or block.value.shape[-1] != value_width
            or block.key.shape[-2] < 1
            or type(block.offset) is not int
            or block.offset < 0
            or block.key.device != query.device
            or block.value.device != query.device
            or block.key.dtype != query.dtype
            or block.value.dtype != query.dtype
        ):
            raise ValueError("KV page layout/dtype/device differs from query")
        _binary_mask(block.padding, (batch, block.key.shape[-2]), query.device, "key padding")
        if not _finite(block.key) or not _finite(block.value):
            raise ValueError("KV blocks must contain finite values")
        intervals.append((block.offset, block.offset + block.key.shape[-2]))
    intervals.sort()
    if any(left[1] > right[0] for left, right in zip(intervals, intervals[1:])):
        raise ValueError("Overlapping KV blocks would count the same key twice")
    scale = key_width**-0.5 if scale is None else scale
    if not math.isfinite(scale) or scale <= 0:
        raise ValueError("Attention scale must be finite and positive")
    return query_padding, scale, heads, value_width


class _Rows:
    """The transient arena of one call and its decode rows (one per query token)."""

    def __init__(self, cache, queries, tables, ctx, span, window):
        self.cache, self.queries, self.tables, self.ctx = cache, queries, tables, ctx
        self.span, self.window = span, window


def _rows(query, blocks, positions, causal, window, query_padding, heads, width, fmt):
    """Lay the blocks' codes and scales into a transient single-layer arena and give
    every query token a decode row whose visible keys are the reference's
    (online_attention.py:175-188).

    Row ``b`` owns arena blocks ``[b * nb, (b + 1) * nb)`` holding positions from
    ``base`` (the first page's offset rounded down to a block) on: causal and window
    masks are translation invariant, so memory and streamed blocks follow the span of
    keys, not their absolute offsets. Positions between pages are padding keys.

    * causal: the row's context ends at its own position (``k <= p``), capped at the
      last key unless a window counts back from the position (the kernels' window
      keeps the ``window`` keys that end the context, ``k > p - window``);
    * not causal: the context ends at the last key; with a window the first visible
      key ``p - window + 1`` falls inside a block that the row reads through a copy of
      its own, whose padding bytes hide the keys before it, and the row's table goes on
      with the shared blocks after it.

    A padded query, or one whose window or causal bound leaves no key, sees nothing
    (context 0) and comes out as the empty state."""
    batch, queries = positions.shape
    device = positions.device
    base = min(b.offset for b in blocks) // BLOCK * BLOCK
    end = max(b.offset + _length(b.key) for b in blocks)  # one past the last key
    first = None  # not causal, windowed: the first visible key of each row, from base
    if causal:
        ctx = positions + 1 - base
        if window is None:
            ctx = torch.clamp(ctx, max=end - base)
        else:
            ctx = torch.where(positions + 1 - window >= end, torch.zeros_like(ctx), ctx)
        ctx = torch.clamp(ctx, min=0)
        kernel_window = window
    else:
        ctx = torch.full_like(positions, end - base)
        if window is not None:
            first = torch.clamp(positions - window + 1 - base, min=0)
            ctx = torch.where(first >= end - base, torch.zeros_like(ctx), ctx)
        kernel_window = None
    if query_padding is not None:
        ctx = torch.where(query_padding, ctx, torch.zeros_like(ctx))
    span = max(int(ctx.max()), 1)
    if span >= 2**31:
        raise UnsupportedAttentionBackend("hip_int8_paged contexts are int32")
    nb = -(-span // BLOCK)
    own = batch * queries if first is not None else 0  # per-row first-block copies
    cache = PagedKVCache(num_blocks=batch * nb + own, num_layers=1, num_kv_heads=heads,
                         head_dim=width, device=device, quantization=KVQuantization(fmt))
    cache._enable_padding()
    cache.key_valid.zero_()
    rows = torch.arange(batch, device=device)[:, None]
    for block in blocks:
        pos = block.offset - base + torch.arange(_length(block.key), device=device)
        keep = pos < nb * BLOCK                                     # keys no row can see
        pos = pos[keep]
        blk = rows * nb + pos[None, :] // BLOCK                     # [B, T]
        slot = (pos % BLOCK).expand(batch, -1)                      # [B, T]
        for side, kv in ((0, block.key), (1, block.value)):
            codes = kv.values.view(torch.int8)[:, :, keep].permute(0, 2, 1, 3)  # [B, T, Hkv, D]
            cache.codes[blk, 0, side, :, slot, :] = codes
            cache.scales[blk, 0, side, :, slot] = kv.scales[:, :, keep, 0].permute(0, 2, 1).float()
        real = (torch.ones_like(blk, dtype=torch.uint8) if block.padding is None
                else block.padding[:, keep].to(torch.uint8))
        cache.key_valid[blk, slot] = real

    ctx = ctx.reshape(-1)
    seq_rows = torch.arange(batch * queries, device=device) // queries       # [B * Q]
    cols = torch.arange(nb, device=device)[None, :]
    if first is None:
        tables = (seq_rows[:, None] * nb + cols).to(torch.int32)
    else:
        lead = torch.clamp(first.reshape(-1), max=nb * BLOCK - 1) // BLOCK   # [B * Q]
        src = seq_rows * nb + lead
        dst = batch * nb + torch.arange(batch * queries, device=device)
        cache.codes[dst] = cache.codes[src]
        cache.scales[dst] = cache.scales[src]
        hide = torch.arange(BLOCK, device=device)[None, :] < (first.reshape(-1) - lead * BLOCK)[:, None]
        cache.key_valid[dst] = torch.where(hide, torch.zeros_like(cache.key_valid[src]),
                                           cache.key_valid[src])
        shared = seq_rows[:, None] * nb + torch.clamp(lead[:, None] + cols, max=nb - 1)
        tables = torch.where(cols == 0, dst[:, None], shared).to(torch.int32)
        ctx = torch.where(ctx > 0, ctx - lead * BLOCK, ctx)
    q_rows = query.permute(0, 2, 1, 3).reshape(batch * queries, query.shape[1], width)
    return _Rows(cache, q_rows, tables.contiguous(), ctx.to(torch.int32).contiguous(), nb * BLOCK,
                 kernel_window)


def _prepare(query, blocks, query_positions, causal, window, query_padding, scale,
             query_block_size, key_block_size):
    """The reference's checks, then the HIP path's own gates (never a silent downgrade)."""
    blocks = tuple(blocks)
    query_padding, scale, heads, value_width = _check(
        query, blocks, query_positions, causal, window, query_padding, scale,
        query_block_size, key_block_size)
    if query.device.type != "cuda":
        raise UnsupportedAttentionBackend("hip_int8_paged attends to device pages")
    if query.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise UnsupportedAttentionBackend("hip_int8_paged takes fp32/fp16/bf16 queries")
    if not all(isinstance(b.key, QuantizedKV) and isinstance(b.value, QuantizedKV) for b in blocks):
        raise UnsupportedAttentionBackend("hip_int8_paged attends to quantized KV pages")
    formats = {_FORMAT_OF_DTYPE.get(v.values.dtype) for b in blocks for v in (b.key, b.value)}
    if len(formats) != 1 or None in formats:
        raise UnsupportedAttentionBackend("hip_int8_paged needs one KV code format per call")
    if value_width != query.shape[-1]:
        raise UnsupportedAttentionBackend("hip_int8_paged needs equal key and value widths")
    rows = _rows(query, blocks, query_positions.to(torch.int64), causal, window, query_padding,
                 heads, query.shape[-1], formats.pop())
    return rows, scale, heads


def _record(work, rows, heads, query_heads):
    if work is None:
        return
    visible = int(((rows.ctx.to(torch.int64) + BLOCK - 1) // BLOCK).sum())
    work.query_tiles += rows.ctx.numel()
    work.key_tiles += visible * heads
    work.max_query_tile = max(work.max_query_tile, 1)
    work.max_key_tile = max(work.max_key_tile, BLOCK)
    work.max_score_elements = max(work.max_score_elements, query_heads * BLOCK)


@torch.no_grad()
def online_attention_statistics(query, blocks, *, query_positions, causal=True, window=None,
                                query_padding=None, scale=None, query_block_size=32,
                                key_block_size=64, work=None):
    """``online_attention_statistics`` (online_attention.py:74-214) on the HIP kernels:
    the same arguments as :func:`online_attention`; returns the fp32
    :class:`SoftmaxState` with ``maximum`` and ``mass`` ``[B, Hkv, G, Q]`` and
    ``weighted`` ``[B, Hkv, G, Q, D]``. ``maximum`` is the largest visible score,
    ``mass`` the sum of ``exp(score - maximum)`` and ``weighted`` the numerator; a row
    that sees no key keeps the initial state ``(-inf, 0, 0)``. The query enters the
    kernels in fp32 (the reference's accumulator dtype, :158-159), on the exact fp32
    fixed-partition decode kernels."""
    rows, scale, heads = _prepare(query, blocks, query_positions, causal, window, query_padding,
                                  scale, query_block_size, key_block_size)
    batch, query_heads, queries, width = query.shape
    maximum, mass, weighted = rows.cache.paged_attention_statistics(
        0, rows.queries.float().contiguous(), rows.tables, rows.ctx,
        max_context_len=rows.span, scale=scale, window=rows.window, check=True)
    _record(work, rows, heads, query_heads)
    groups = query_heads // heads
    shape = (batch, queries, heads, groups)
    return SoftmaxState(maximum.reshape(shape).permute(0, 2, 3, 1).contiguous(),
                        mass.reshape(shape).permute(0, 2, 3, 1).contiguous(),
                        weighted.reshape(*shape, width).permute(0, 2, 3, 1, 4).contiguous())


@torch.no_grad()
def online_attention(query, blocks, *, query_positions, causal=True, window=None,
                     query_padding=None, scale=None, query_block_size=32, key_block_size=64,
                     work=None):
    """``online_attention`` (online_attention.py:217-219) on the HIP kernels:
    ``query`` ``[B, Hq, Q, D]`` (fp32/fp16/bf16, device), ``blocks`` of
    ``QuantizedKV`` pages, ``query_positions`` ``[B, Q]``; returns ``[B, Hq, Q, D]``
    in the query dtype. The tile sizes are checked as the reference checks them; the
    kernels' own tiles (16-token blocks, one decode row per query token) are what
    ``work`` records."""
    rows, scale, heads = _prepare(query, blocks, query_positions, causal, window, query_padding,
                                  scale, query_block_size, key_block_size)
    batch, query_heads, queries, width = query.shape
    out = rows.cache.paged_attention(0, rows.queries.contiguous(), rows.tables, rows.ctx,
                                     max_context_len=rows.span, scale=scale, window=rows.window,
                                     check=True)
    _record(work, rows, heads, query_heads)
    return out.reshape(batch, queries, query_heads, width).permute(0, 2, 1, 3).contiguous()
