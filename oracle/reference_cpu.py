"""numpy restatement of the reference's low-bit (INT8, FP8 E4M3FN, FP8 E5M2)
paged-decode arithmetic.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): the product never imports
this module. Every function cites the reference file:line it restates, relative
to the sutiankang/aster source tree (``src/aster/...``).

Parity status of each function (how it is pinned, in ``tests/test_oracle.py``):
  quantize_kv_int8          pinned: reference known-answer test (seed-76 tensor,
                            test_hot_kv.py:22-42), exact ties, zero row,
                            FLT_MIN clamp, true-division vs reciprocal cases,
                            error bound and |code|max == 127 invariants.
  dequantize                pinned: closed form fp32(code)*scale (atol 0).
  fp8_values / fp8_round    pinned: every one of the 256 codes against torch's
                            float8_e4m3fn / float8_e5m2 -> float32 conversion, and
                            the rounding against torch's float32 -> float8
                            conversion on random, tie, subnormal and extreme values.
  quantize_kv_fp8           pinned: against the reference's own torch expression
                            (amax / finfo.max, clamp, .to(float8)) on the CPU.
  merge_softmax / output    pinned: partition merge == whole, -inf partitions.
  online_attention_statistics
                            pinned: fp64 brute-force dense softmax (dense.py),
                            page order invariance, fully-masked rows == 0,
                            single-key and equal-score closed forms.
  paged_attention           pinned through online_attention_statistics plus
                            block-table permutation invariance.
"""

from __future__ import annotations

from dataclasses import dataclass
import math

import numpy as np

FLT_TINY = np.float32(np.finfo(np.float32).tiny)
DBL_TINY = np.float64(np.finfo(np.float64).tiny)
INT8_MAXIMUM = 127.0  # kv_quantization.py:23-25 (KVQuantization("int8").maximum)
# KVQuantization(...).maximum of the FP8 formats: torch.finfo(dtype).max (:23-25)
FP8_MAXIMUM = {"fp8_e4m3fn": 448.0, "fp8_e5m2": 57344.0}


# ----------------------------------------------------------------------------
# quantization (src/aster/optimization/kv_quantization.py)
# ----------------------------------------------------------------------------


@dataclass(frozen=True)
class QuantizedKV:
    """codes [..., T, D] and scales [..., T, 1] (kv_quantization.py:28-68): int8 values,
    or uint8 FP8 bit patterns of format ``fmt``."""

    values: np.ndarray
    scales: np.ndarray
    fmt: str = "int8"

    @property
    def shape(self):
        return self.values.shape

    def narrow(self, start, count):
        """Token-axis slice (kv_quantization.py:57-64)."""
        return QuantizedKV(
            self.values[..., start : start + count, :], self.scales[..., start : start + count, :],
            self.fmt,
        )

    def code_values(self):
        """The codes as exact floats (int8 values, or decoded FP8)."""
        if self.fmt == "int8":
            return self.values.astype(np.float64)
        return fp8_values(self.fmt)[self.values.astype(np.uint8)]

    def dequantize(self, dtype=None):
        """``values.to(scales.dtype) * scales`` then cast (kv_quantization.py:66-68)."""
        out = self.code_values().astype(self.scales.dtype) * self.scales
        return out if dtype is None else out.astype(dtype)


def quantize_kv_int8(x):
    """Per-(token, head) symmetric INT8 codes + scales (kv_quantization.py:71-94).

    ``x`` is a float16/float32/float64 array ``[..., T, D]`` (bf16 data is passed
    as the float32 array holding the same values, which is what ``.to(float32)``
    at :82-83 produces). Accumulation is float64 only for float64 input (:82).
    Steps: amax over the last dim (:84); scale = 1 where amax == 0 else
    max(amax / 127, tiny) with true division (:86-90); codes =
    round_half_even(clamp(x / scale, -127, 127)) (:91-93).
    """
    x = np.asarray(x)
    if x.ndim < 3 or x.shape[-1] < 1:
        raise ValueError("Quantized KV needs explicit layout [...,tokens,width] and format")
    if x.dtype not in (np.float16, np.float32, np.float64) or not np.isfinite(x).all():
        raise ValueError("Quantized KV requires finite floating input")
    acc = np.float64 if x.dtype == np.float64 else np.float32
    tiny = DBL_TINY if acc == np.float64 else FLT_TINY
    source = x.astype(acc)
    maximum = np.abs(source).max(axis=-1, keepdims=True)
    divided = np.divide(maximum, acc(INT8_MAXIMUM), dtype=acc)
    scales = np.where(maximum == 0, acc(1.0), np.maximum(divided, tiny)).astype(acc)
    normalized = np.clip(np.divide(source, scales, dtype=acc), -INT8_MAXIMUM, INT8_MAXIMUM)
    codes = np.rint(normalized).astype(np.int8)
    return QuantizedKV(codes, scales)


def fp8_values(fmt):
    """The 256 FP8 codes' values (float64; NaN/Inf codes as NaN/Inf), from the OCP
    format definition: E4M3FN bias 7, 3 mantissa bits, no Inf, 0x7F/0xFF NaN; E5M2
    bias 15, 2 mantissa bits, IEEE-style Inf/NaN (torch.float8_e4m3fn / float8_e5m2,
    the dtypes of KVQuantization.dtype, kv_quantization.py:16-21)."""
    e_bits, m_bits, bias = (4, 3, 7) if fmt == "fp8_e4m3fn" else (5, 2, 15)
    out = np.empty(256, np.float64)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        e = (code >> m_bits) & ((1 << e_bits) - 1)
        m = code & ((1 << m_bits) - 1)
        if fmt == "fp8_e4m3fn" and (code & 0x7F) == 0x7F:
            out[code] = np.nan
        elif fmt == "fp8_e5m2" and e == 31:
            out[code] = sign * np.inf if m == 0 else np.nan
        elif e == 0:
            out[code] = sign * m * 2.0 ** (1 - bias - m_bits)
        else:
            out[code] = sign * (1 + m / (1 << m_bits)) * 2.0 ** (e - bias)
    return out


def fp8_round(c, fmt):
    """float32 ``c`` (finite, |c| <= the format's maximum) -> FP8 codes (uint8),
    round to the nearest representable value, ties to the even code, sign kept (-0
    for negative values that round to zero): the float32 -> float8 conversion of
    ``.to(dtype)`` at kv_quantization.py:94. Restated as a nearest-value search over
    the format's finite non-negative values (exact in float64)."""
    c = np.asarray(c, np.float32)
    values = fp8_values(fmt)
    finite = np.isfinite(values[:128])
    grid = values[:128][finite]          # non-negative values, increasing with the code
    codes = np.arange(128)[finite]
    a = np.abs(c.astype(np.float64))
    hi = np.clip(np.searchsorted(grid, a), 0, len(grid) - 1)
    lo = np.clip(hi - 1, 0, len(grid) - 1)
    dlo, dhi = a - grid[lo], grid[hi] - a
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (codes[hi] % 2 == 0) & (hi != lo))
    pick = np.where(a <= grid[0], 0, np.where(pick_hi, hi, lo))
    code = codes[pick].astype(np.uint8)
    return code | np.where(np.signbit(c), np.uint8(0x80), np.uint8(0))


def quantize_kv_fp8(x, fmt):
    """Per-(token, head) FP8 codes + scales (kv_quantization.py:71-94 with an FP8
    profile): scale = 1 where amax == 0 else max(amax / M, tiny) (M =
    finfo(dtype).max, :86-90), codes = float8(clamp(x / scale, -M, M)) (:91-94; no
    rounding step before the cast, :92-93 apply to int8 only)."""
    x = np.asarray(x)
    if x.ndim < 3 or x.shape[-1] < 1:
        raise ValueError("Quantized KV needs explicit layout [...,tokens,width] and format")
    if x.dtype not in (np.float16, np.float32) or not np.isfinite(x).all():
        raise ValueError("Quantized KV requires finite floating input")
    maximum_code = np.float32(FP8_MAXIMUM[fmt])
    source = x.astype(np.float32)
    maximum = np.abs(source).max(axis=-1, keepdims=True)
    divided = np.divide(maximum, maximum_code, dtype=np.float32)
    scales = np.where(maximum == 0, np.float32(1.0), np.maximum(divided, FLT_TINY)).astype(np.float32)
    normalized = np.clip(np.divide(source, scales, dtype=np.float32), -maximum_code, maximum_code)
    return QuantizedKV(fp8_round(normalized, fmt), scales, fmt)


def quantize_kv(x, fmt="int8"):
    """``quantize_kv`` for any of the three formats."""
    return quantize_kv_int8(x) if fmt == "int8" else quantize_kv_fp8(x, fmt)


# ----------------------------------------------------------------------------
# online softmax (src/aster/optimization/online_attention.py)
# ----------------------------------------------------------------------------


@dataclass(frozen=True)
class AttentionBlock:
    """One KV page: key/value ``[B, Hkv, T, D]`` float arrays or QuantizedKV,
    absolute token offset and optional key padding ``[B, T]`` (online_attention.py:10-15)."""

    key: object
    value: object
    offset: int
    padding: np.ndarray | None = None


@dataclass(frozen=True)
class SoftmaxState:
    """(maximum, mass, weighted) over ``[B, Hkv, G, Q]`` (online_attention.py:29-39)."""

    maximum: np.ndarray
    mass: np.ndarray
    weighted: np.ndarray

    def output(self):
        """``weighted / max(mass, tiny)`` reshaped to ``[B, Hq, Q, Dv]`` (:35-39)."""
        tiny = DBL_TINY if self.mass.dtype == np.float64 else FLT_TINY
        value = self.weighted / np.maximum(self.mass, tiny)[..., None]
        b, h, g, q, w = value.shape
        return value.reshape(b, h * g, q, w)


def _exp_where_finite(m, safe):
    out = np.zeros_like(m)
    finite = np.isfinite(m)
    out[finite] = np.exp(m[finite] - safe[finite])
    return out


def merge_softmax(left, right):
    """LSE merge of disjoint partitions; non-finite maxima weigh 0 (online_attention.py:42-63)."""
    if left.maximum.shape != right.maximum.shape or left.weighted.shape != right.weighted.shape:
        raise ValueError("Attention partitions must describe the same queries and accumulator layout")
    maximum = np.maximum(left.maximum, right.maximum)
    safe = np.where(np.isfinite(maximum), maximum, 0).astype(maximum.dtype)
    a = _exp_where_finite(left.maximum, safe)
    b = _exp_where_finite(right.maximum, safe)
    return SoftmaxState(
        maximum,
        left.mass * a + right.mass * b,
        left.weighted * a[..., None] + right.weighted * b[..., None],
    )


def _tile(value, start, count, dtype):
    """kv_tile (kv_quantization.py:130-132): dequantize a token slice."""
    if isinstance(value, QuantizedKV):
        return value.narrow(start, count).dequantize(dtype)
    return value[..., start : start + count, :].astype(dtype)


def _length(value):
    return value.values.shape[-2] if isinstance(value, QuantizedKV) else value.shape[-2]


def online_attention_statistics(
    query,
    blocks,
    *,
    query_positions,
    causal=True,
    window=None,
    query_padding=None,
    scale=None,
    query_block_size=32,
    key_block_size=64,
):
    """Blockwise online softmax over a list of pages (online_attention.py:74-214).

    ``query`` ``[B, Hq, Q, D]``; GQA maps query head ``h`` to kv head ``h // G``
    through the ``[B, Hkv, G, Q, D]`` reshape (:157-161). Visibility per tile
    (:175-188): causal ``kpos <= qpos``, window ``kpos > qpos - window``, key and
    query padding. Fully-invisible tiles are skipped (:189-190); non-finite
    scores raise (:193-196); each tile's (max, sum, P@V) is merged into the
    running state with ``merge_softmax`` (:197-206).
    """
    blocks = tuple(blocks)
    query = np.asarray(query)
    if query.ndim != 4 or min(query.shape) < 1 or not blocks:
        raise ValueError("Need nonempty query/pages and positive integer tile sizes")
    if not np.isfinite(query).all():
        raise ValueError("Query must be finite")
    acc = np.float64 if query.dtype == np.float64 else np.float32
    batch, query_heads, queries, width = query.shape
    heads = blocks[0].key.shape[1]
    value_width = blocks[0].value.shape[-1]
    if heads < 1 or query_heads % heads:
        raise ValueError("Query heads must divide into KV groups")
    intervals = sorted((b.offset, b.offset + _length(b.key)) for b in blocks)
    if any(l[1] > r[0] for l, r in zip(intervals, intervals[1:])):
        raise ValueError("Overlapping KV blocks would count the same key twice")
    scale = width**-0.5 if scale is None else scale
    if not math.isfinite(scale) or scale <= 0:
        raise ValueError("Attention scale must be finite and positive")
    scale = acc(scale)
    groups = query_heads // heads
    positions_all = np.asarray(query_positions)
    maxima, masses, numerators = [], [], []
    for begin in range(0, queries, query_block_size):
        end = min(queries, begin + query_block_size)
        q = query[:, :, begin:end, :].astype(acc).reshape(batch, heads, groups, end - begin, width)
        positions = positions_all[:, begin:end]
        shape = (batch, heads, groups, end - begin)
        state = SoftmaxState(
            np.full(shape, -np.inf, dtype=acc),
            np.zeros(shape, dtype=acc),
            np.zeros(shape + (value_width,), dtype=acc),
        )
        for block in blocks:
            length = _length(block.key)
            for start in range(0, length, key_block_size):
                stop = min(length, start + key_block_size)
                keys = _tile(block.key, start, stop - start, acc)
                values = _tile(block.value, start, stop - start, acc)
                key_positions = np.arange(block.offset + start, block.offset + stop)
                visible = np.ones((batch, end - begin, stop - start), dtype=bool)
                if causal:
                    visible &= key_positions[None, None, :] <= positions[:, :, None]
                if window is not None:
                    visible &= key_positions[None, None, :] > positions[:, :, None] - window
                if block.padding is not None:
                    visible &= np.asarray(block.padding, dtype=bool)[:, None, start:stop]
                if query_padding is not None:
                    visible &= np.asarray(query_padding, dtype=bool)[:, begin:end, None]
                if not visible.any():
                    continue
                scores = np.einsum("bhgqd,bhkd->bhgqk", q, keys) * scale
                if not np.isfinite(scores).all():
                    raise ValueError(
                        "Attention score overflow; cannot repair an infinite dot product with softmax"
                    )
                scores = np.where(visible[:, None, None], scores, -np.inf).astype(acc)
                maximum = scores.max(-1)
                safe = np.where(np.isfinite(maximum), maximum, 0).astype(acc)
                probability = np.exp(scores - safe[..., None])
                local = SoftmaxState(
                    maximum,
                    probability.sum(-1),
                    np.einsum("bhgqk,bhkd->bhgqd", probability, values),
                )
                state = merge_softmax(state, local)
        maxima.append(state.maximum)
        masses.append(state.mass)
        numerators.append(state.weighted)
    return SoftmaxState(
        np.concatenate(maxima, -1), np.concatenate(masses, -1), np.concatenate(numerators, -2)
    )


def online_attention(query, blocks, **kwargs):
    """``online_attention_statistics(...).output()`` (online_attention.py:217-219),
    returned in the accumulator dtype (the cast to the query dtype is left to the
    caller so parity can be checked before the final rounding)."""
    return online_attention_statistics(query, blocks, **kwargs).output()


# ----------------------------------------------------------------------------
# paged runner assembly (src/aster/inference/paged_attention.py, state.py)
# ----------------------------------------------------------------------------


def page_blocks(k_codes, k_scales, v_codes, v_scales, block_table, length, block_size,
                padding=None, fmt="int8"):
    """One AttentionBlock per page, narrowed to its valid tokens, at absolute
    offset ``index * block_size`` (state.py:358-390 read_pages;
    paged_attention.py:170-183). Arena layout: codes ``[blocks, Hkv, bs, D]``,
    scales ``[blocks, Hkv, bs]``; ``padding`` optional ``[blocks, bs]`` bool."""
    blocks = []
    for index in range(math.ceil(length / block_size)):
        page = int(block_table[index])
        count = min(block_size, length - index * block_size)
        key = QuantizedKV(k_codes[page][None, :, :count], k_scales[page][None, :, :count, None], fmt)
        value = QuantizedKV(v_codes[page][None, :, :count], v_scales[page][None, :, :count, None],
                            fmt)
        pad = None if padding is None else padding[page][None, :count]
        blocks.append(AttentionBlock(key, value, index * block_size, pad))
    return blocks


def paged_attention(query, k_codes, k_scales, v_codes, v_scales, block_tables, context_lens,
                    *, block_size, scale, query_lens=None, causal=True, window=None,
                    query_block_size=32, key_block_size=64, padding=None, fmt="int8"):
    """Ragged paged attention over a committed arena, row by row, as
    ``PagedAttentionRunner.forward_batch`` does (paged_attention.py:168-215).

    ``query`` ``[total_q, Hq, D]`` packed by ``query_lens`` (default: one query
    token per sequence). Row ``b``'s ``n_b`` queries sit at absolute positions
    ``context_lens[b] - n_b .. context_lens[b] - 1`` (the chunk has already been
    appended, so ``context_lens`` counts it). Returns ``[total_q, Hq, Dv]`` in the
    accumulator dtype.
    """
    query = np.asarray(query)
    n = len(context_lens)
    query_lens = [1] * n if query_lens is None else [int(x) for x in query_lens]
    outputs = []
    cursor = 0
    for b in range(n):
        ctx, qn = int(context_lens[b]), query_lens[b]
        q = query[cursor : cursor + qn].transpose(1, 0, 2)[None]
        cursor += qn
        if qn == 0:  # a sequence with no query token this step produces no rows
            continue
        if ctx == 0:  # no visible key: the fully-masked row is zero (online_attention.py:37)
            width = v_codes.shape[-1]
            acc = np.float64 if query.dtype == np.float64 else np.float32
            outputs.append(np.zeros((qn, query.shape[1], width), dtype=acc))
            continue
        blocks = page_blocks(k_codes, k_scales, v_codes, v_scales, block_tables[b], ctx,
                             block_size, padding, fmt)
        positions = np.arange(ctx - qn, ctx)[None]
        out = online_attention(q, blocks, query_positions=positions, causal=causal, window=window,
                               scale=scale, query_block_size=query_block_size,
                               key_block_size=key_block_size)
        outputs.append(out[0].transpose(1, 0, 2))
    if not outputs:  # no sequence has a query token this step
        acc = np.float64 if query.dtype == np.float64 else np.float32
        return np.zeros((0, query.shape[1], v_codes.shape[-1]), dtype=acc)
    return np.concatenate(outputs, 0)


def quantize_append(k, v, slot_mapping, k_codes, k_scales, v_codes, v_scales, block_size,
                    fmt="int8"):
    """Quantize new tokens and copy raw codes/scales into ``slot // bs, slot % bs``
    (state.py:292 quantize, :339-344 per-token copy_kv). ``k``/``v`` ``[T, Hkv, D]``;
    slots < 0 are skipped. Mutates the arena arrays in place."""
    qk = quantize_kv(np.asarray(k).transpose(1, 0, 2)[None], fmt)
    qv = quantize_kv(np.asarray(v).transpose(1, 0, 2)[None], fmt)
    for t, slot in enumerate(np.asarray(slot_mapping).tolist()):
        if slot < 0:
            continue
        page, offset = divmod(int(slot), block_size)
        k_codes[page, :, offset] = qk.values[0, :, t]
        k_scales[page, :, offset] = qk.scales[0, :, t, 0]
        v_codes[page, :, offset] = qv.values[0, :, t]
        v_scales[page, :, offset] = qv.scales[0, :, t, 0]
    return qk, qv
