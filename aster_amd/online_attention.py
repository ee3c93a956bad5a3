"""Op-level attention over explicit KV pages on the HIP path: the reference's
``online_attention`` and ``merge_softmax`` (src/aster/optimization/online_attention.py)
for callers that hold ``AttentionBlock`` pages rather than a paged arena.

``online_attention`` checks its arguments as the reference does (same exceptions and
messages, online_attention.py:89-147), then lays the blocks' quantized codes and
scales into a transient single-layer arena. Each block's token ``t`` goes to
absolute position ``offset + t``; positions no block covers, and key padding, become
padding keys. Each query token then attends as one decode row of the library's
paged kernels, its context ending at its own position. That gives the causal mask
(``k <= p``) and the window (``k > p - window``) of online_attention.py:175-188.
``merge_softmax`` runs a HIP kernel over fp32 states (``astr_merge_softmax_f32``).

Not served (``UnsupportedAttentionBackend``, never a silent downgrade):
  * plain tensor K/V, since the path attends to quantized pages;
  * blocks of different code formats, and value widths unlike the key width;
  * windows without causality;
  * fp64 queries or states;
  * ``online_attention_statistics``, because the kernels return normalised rows,
    not the unnormalised (maximum, mass, numerator) state.
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
    batch, query_heads, queries, width = query.shape
    if value_width != width:
        raise UnsupportedAttentionBackend("hip_int8_paged needs equal key and value widths")
    if window is not None and not causal:
        raise UnsupportedAttentionBackend("hip_int8_paged windows are causal")
    device = query.device
    positions = query_positions.to(torch.int64)

    # transient arena: row b owns blocks [b * nb, (b + 1) * nb) holding positions from
    # `base` (the first page's offset rounded down to a block) on: causal and window
    # masks are translation invariant, so memory and streamed blocks follow the span of
    # keys, not their absolute offsets. Positions between pages are padding keys.
    base = min(b.offset for b in blocks) // BLOCK * BLOCK
    end = max(b.offset + _length(b.key) for b in blocks)  # one past the last key
    # one decode row per query token, its context ending at its position (causal), or
    # at the last key; keys past the last page are never visible, so a causal row's
    # context stops there unless a window counts back from its own position (then a
    # row whose window starts past the last key sees nothing); a padded query, or one
    # before every key, sees nothing and comes out zero
    if causal:
        ctx = positions + 1 - base
        if window is None:
            ctx = torch.clamp(ctx, max=end - base)
        else:
            ctx = torch.where(positions + 1 - window >= end, torch.zeros_like(ctx), ctx)
        ctx = torch.clamp(ctx, min=0)
    else:
        ctx = torch.full_like(positions, end - base)
    if query_padding is not None:
        ctx = torch.where(query_padding, ctx, torch.zeros_like(ctx))
    span = max(int(ctx.max()), 1)
    if span >= 2**31:
        raise UnsupportedAttentionBackend("hip_int8_paged contexts are int32")
    nb = -(-span // BLOCK)
    cache = PagedKVCache(num_blocks=batch * nb, num_layers=1, num_kv_heads=heads,
                         head_dim=width, device=device,
                         quantization=KVQuantization(formats.pop()))
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

    ctx = ctx.reshape(-1).to(torch.int32).contiguous()
    tables = (rows * nb + torch.arange(nb, device=device)[None, :]).to(torch.int32)
    tables = tables.repeat_interleave(queries, dim=0).contiguous()  # [B * Q, nb]
    q_rows = query.permute(0, 2, 1, 3).reshape(batch * queries, query_heads, width).contiguous()
    out = cache.paged_attention(0, q_rows, tables, ctx, max_context_len=nb * BLOCK, scale=scale,
                                window=window if causal else None, check=True)
    if work is not None:
        visible = int(((ctx.to(torch.int64) + BLOCK - 1) // BLOCK).sum())
        work.query_tiles += batch * queries
        work.key_tiles += visible * heads
        work.max_query_tile = max(work.max_query_tile, 1)
        work.max_key_tile = max(work.max_key_tile, BLOCK)
        work.max_score_elements = max(work.max_score_elements, query_heads * BLOCK)
    return out.reshape(batch, queries, query_heads, width).permute(0, 2, 1, 3).contiguous()
