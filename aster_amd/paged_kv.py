"""Device arena of the paged low-bit KV cache and the two hot-path calls on it.

Arena layout (one allocation per model, block-major so a physical page of all
layers is contiguous for copy-on-write and host swap):

    codes     int8  [num_blocks, num_layers, 2 (K, V), num_kv_heads, block_size, head_dim]
                    (one byte per code: int8 values, or FP8 E4M3FN / E5M2 bit patterns)
    scales    fp32  [num_blocks, num_layers, 2 (K, V), num_kv_heads, block_size]
    key_valid uint8 [num_blocks, block_size]   (0: the slot holds a padding key)

Block ``b`` is the reference's ``PageRef.index`` (src/aster/inference/state.py:131-134):
the reference keeps per page and layer a ``QuantizedKV`` of codes ``[1, Hkv, bs, D]``
and scales ``[1, Hkv, bs, 1]`` (state.py:319-327, kv_quantization.py:97-110);
here those are ``codes[b, layer, 0|1]`` / ``scales[b, layer, 0|1]`` of one arena,
and the page's padding leaf ``[1, 1, bs, 1]`` (state.py:319-327; the runner appends it
with every chunk, paged_attention.py:228) is ``key_valid[b]``, shared by all layers.
The kernels see ``key_valid`` only once a padding key has been written
(``write_key_valid``): until then every key is real and they skip the mask.

``append`` replaces quantize_kv + the per-token copy_kv loop of
``PagedStatePool._append_leaves`` (state.py:292, 339-344): token ``t`` goes to
slot ``slot_mapping[t] = page * block_size + offset``. ``paged_attention``
replaces the per-row ``online_attention`` calls of
``PagedAttentionRunner.forward_batch`` (src/aster/inference/paged_attention.py:168-215)
with one launch over all rows.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _native
from .attention_backend import BACKEND, KernelWork, UnsupportedAttentionBackend
from .kv_quantization import KVQuantization, QuantizedKV, _DTYPE_CODES, require_format

DEFAULT_PARTITION_TOKENS = 0  # automatic: stream-K for bf16/fp16, else 512-token partitions


class PagedKVCache:
    """Caller-owned device arena for ``num_layers`` layers of paged K/V in one of the
    reference's formats (``KVQuantization``: int8, fp8_e4m3fn, fp8_e5m2)."""

    def __init__(self, *, num_blocks, num_layers, num_kv_heads, head_dim, block_size=16,
                 device="cuda", quantization=None):
        quantization = KVQuantization("int8") if quantization is None else quantization
        self.code_format = require_format(quantization)
        if min(num_blocks, num_layers, num_kv_heads, head_dim, block_size) < 1:
            raise ValueError("Cache capacities must be positive")
        if block_size != 16:
            raise UnsupportedAttentionBackend("hip_int8_paged kernels use 16-token blocks")
        device = torch.device(device)
        if device.type != "cuda":
            raise UnsupportedAttentionBackend("hip_int8_paged arenas live in HIP device memory")
        self.quantization = quantization
        self.num_blocks, self.num_layers = num_blocks, num_layers
        self.num_kv_heads, self.head_dim, self.block_size = num_kv_heads, head_dim, block_size
        self.device = device
        self.codes = torch.zeros((num_blocks, num_layers, 2, num_kv_heads, block_size, head_dim),
                                 dtype=torch.int8, device=device)
        self.scales = torch.ones((num_blocks, num_layers, 2, num_kv_heads, block_size),
                                 dtype=torch.float32, device=device)
        self.key_valid = torch.ones((num_blocks, block_size), dtype=torch.uint8, device=device)
        self.has_padding = False  # some slot may hold a padding key (descriptors carry key_valid)
        self.err_flag = torch.zeros(1, dtype=torch.int32, device=device)
        self._workspace = None
        self._descs = [self._make_desc(layer) for layer in range(num_layers)]

    # ---- descriptors --------------------------------------------------------
    def _make_desc(self, layer):
        c, s = self.codes, self.scales
        return _native.PagedKVDesc(
            k_codes=c[0, layer, 0].data_ptr(), v_codes=c[0, layer, 1].data_ptr(),
            k_scales=s[0, layer, 0].data_ptr(), v_scales=s[0, layer, 1].data_ptr(),
            code_block_stride=c.stride(0), code_head_stride=c.stride(3),
            scale_block_stride=s.stride(0), scale_head_stride=s.stride(3),
            num_blocks=self.num_blocks, block_size=self.block_size,
            num_kv_heads=self.num_kv_heads, head_dim=self.head_dim,
            key_valid=self.key_valid.data_ptr() if self.has_padding else None,
            code_format=self.code_format)

    def _enable_padding(self):
        if not self.has_padding:
            self.has_padding = True
            self._descs = [self._make_desc(layer) for layer in range(self.num_layers)]

    def layer_desc(self, layer):
        return self._descs[layer]

    @property
    def nbytes(self):
        return self.codes.numel() + self.scales.numel() * 4 + self.key_valid.numel()

    def page(self, block, layer):
        """Zero-copy ``QuantizedKV`` views ``[1, Hkv, bs, D]`` of one page
        (the reference's ``PageView.payload[2*layer : 2*layer+2]``, state.py:158-163)."""
        k = QuantizedKV(self.code_view(self.codes[block, layer, 0][None]),
                        self.scales[block, layer, 0][None, ..., None], torch.float32)
        v = QuantizedKV(self.code_view(self.codes[block, layer, 1][None]),
                        self.scales[block, layer, 1][None, ..., None], torch.float32)
        return k, v

    def code_view(self, raw):
        """Raw code bytes (int8 storage) viewed in the format's dtype (int8,
        float8_e4m3fn or float8_e5m2), zero-copy; ``.float()`` of it is the code value."""
        return raw.view(self.quantization.dtype)

    def padding_leaf(self, block):
        """Zero-copy bool view ``[1, 1, bs, 1]`` of one page's padding leaf (True =
        real token; the reference's ``PageView.payload[-1]``, state.py:158-163)."""
        return self.key_valid[block].view(torch.bool)[None, None, :, None]

    # ---- error flag ---------------------------------------------------------
    def pending_errors(self):
        """Read (synchronising) and clear the sticky device error flag."""
        flags = int(self.err_flag.item())
        if flags:
            self.err_flag.zero_()
        return flags

    def raise_errors(self):
        """Raise the reference's ValueError for any flagged device error."""
        flags = self.pending_errors()
        if flags & _native.FLAG_NONFINITE_INPUT:
            raise ValueError("Quantized KV requires finite floating input")
        if flags & _native.FLAG_NONFINITE_SCORE:
            raise ValueError(
                "Attention score overflow; cannot repair an infinite dot product with softmax")
        if flags & _native.FLAG_BAD_INDEX:
            raise ValueError("Slot, block table or context length outside the KV arena")

    # ---- hot path -----------------------------------------------------------
    def append(self, layer, key, value, slot_mapping, *, check=False, reserved=False):
        """Quantize ``key``/``value`` ``[T, Hkv, D]`` (fp32/fp16/bf16, device) into
        the slots ``slot_mapping`` (int64 ``[T]``; negative = skip). With
        ``check=True`` synchronise and raise ``ValueError`` on non-finite input, as
        quantize_kv does (kv_quantization.py:77-81); otherwise the error stays in
        the sticky flag (and blocks further appends) until ``raise_errors``.

        A non-finite input leaves every slot as it was; with ``reserved=True`` (slots
        the caller rolls back when the call is flagged, as the runner's step does) the
        append takes one launch instead of two, and only the non-finite rows are
        guaranteed to stay unwritten."""
        _check_rows(key, "key", self.num_kv_heads, self.head_dim, self.device)
        _check_rows(value, "value", self.num_kv_heads, self.head_dim, self.device)
        if key.shape != value.shape or key.dtype != value.dtype:
            raise ValueError("key and value must share shape and dtype")
        if (slot_mapping.dtype != torch.int64 or slot_mapping.shape != (key.shape[0],)
                or slot_mapping.device != self.device or not slot_mapping.is_contiguous()):
            raise ValueError("slot_mapping must be a contiguous int64 device vector [T]")
        stream = torch.cuda.current_stream(self.device).cuda_stream
        lib = _native.lib()
        fn = lib.astr_kv_quantize_append_i8_reserved if reserved else lib.astr_kv_quantize_append_i8
        _native.check(
            fn(
                self._descs[layer], key.data_ptr(), value.data_ptr(), _DTYPE_CODES[key.dtype],
                key.shape[0], key.stride(0), key.stride(1), value.stride(0), value.stride(1),
                slot_mapping.data_ptr(), self.err_flag.data_ptr(), stream),
            "quantize_append")
        if check:
            self.raise_errors()

    def write_key_valid(self, slot_mapping, valid=None):
        """Key-padding bytes of new tokens: ``valid`` (bool/uint8 device ``[T]``,
        True = real token) into slots ``slot_mapping`` (int64 ``[T]``, negative =
        skip); None marks every token real. Written once per step for all layers
        (the padding leaf of state.py:292, 339-344). Without any padding so far and
        ``valid`` None this is a no-op: every slot is still real."""
        if (slot_mapping.dtype != torch.int64 or slot_mapping.ndim != 1
                or slot_mapping.device != self.device or not slot_mapping.is_contiguous()):
            raise ValueError("slot_mapping must be a contiguous int64 device vector [T]")
        if valid is None and not self.has_padding:
            return
        if valid is not None:
            valid = torch.as_tensor(valid, device=self.device)
            if valid.shape != slot_mapping.shape or valid.dtype not in (torch.bool, torch.uint8):
                raise ValueError("key padding must be a bool/uint8 vector aligned with slot_mapping")
            valid = valid.to(torch.uint8).contiguous()
            self._enable_padding()
        stream = torch.cuda.current_stream(self.device).cuda_stream
        _native.check(
            _native.lib().astr_kv_write_key_valid(
                self._descs[0], slot_mapping.data_ptr(),
                valid.data_ptr() if valid is not None else None, slot_mapping.shape[0],
                self.err_flag.data_ptr(), stream),
            "write_key_valid")

    # ---- whole-block moves (copy-on-write, host swap) ------------------------
    @property
    def block_code_bytes(self):
        """Bytes of one block's codes, all layers (one contiguous arena stretch)."""
        return self.codes[0].numel()

    @property
    def block_scale_bytes(self):
        return self.scales[0].numel() * self.scales.element_size()

    def _copy(self, src, src_stride, src_index, src_blocks, dst, dst_stride, dst_index,
              dst_blocks, block_bytes, count, stream):
        _native.check(
            _native.lib().astr_kv_copy_blocks(
                src, src_stride, src_index, src_blocks, dst, dst_stride, dst_index, dst_blocks,
                block_bytes, count, self.err_flag.data_ptr(), stream),
            "copy_blocks")

    def _index(self, blocks):
        return torch.as_tensor(list(blocks), dtype=torch.int32).to(self.device, non_blocking=True)

    def copy_blocks(self, src_blocks, dst_blocks, *, stream=None):
        """Copy whole blocks (codes and scales of every layer) ``src[i] -> dst[i]``
        inside the arena, bit-exact (copy-on-write of a shared tail page,
        state.py:330-337). One launch per array for any number of blocks."""
        if len(src_blocks) != len(dst_blocks):
            raise ValueError("src_blocks and dst_blocks differ in length")
        if not len(src_blocks):
            return
        stream = stream or torch.cuda.current_stream(self.device)
        with torch.cuda.stream(stream):
            src, dst = self._index(src_blocks), self._index(dst_blocks)
        cb, sb, vb = self.block_code_bytes, self.block_scale_bytes, self.block_size
        for base, nbytes in ((self.codes.data_ptr(), cb), (self.scales.data_ptr(), sb),
                             (self.key_valid.data_ptr(), vb)):
            self._copy(base, nbytes, src.data_ptr(), self.num_blocks, base, nbytes, dst.data_ptr(),
                       self.num_blocks, nbytes, len(src_blocks), stream.cuda_stream)
        src.record_stream(stream), dst.record_stream(stream)

    def gather_blocks(self, blocks, *, stream=None):
        """Blocks ``blocks`` packed into new device tensors ``codes [P, L, 2, Hkv, bs, D]``,
        ``scales [P, L, 2, Hkv, bs]`` and ``valid [P, bs]`` (the gather half of host
        swap), enqueued on ``stream``."""
        stream = stream or torch.cuda.current_stream(self.device)
        count = len(blocks)
        with torch.cuda.stream(stream):
            codes = torch.empty((count,) + tuple(self.codes.shape[1:]), dtype=self.codes.dtype,
                                device=self.device)
            scales = torch.empty((count,) + tuple(self.scales.shape[1:]), dtype=self.scales.dtype,
                                 device=self.device)
            valid = torch.empty((count, self.block_size), dtype=torch.uint8, device=self.device)
            if count:
                index = self._index(blocks)
                for src, dst, nbytes in ((self.codes, codes, self.block_code_bytes),
                                         (self.scales, scales, self.block_scale_bytes),
                                         (self.key_valid, valid, self.block_size)):
                    self._copy(src.data_ptr(), nbytes, index.data_ptr(), self.num_blocks,
                               dst.data_ptr(), nbytes, None, count, nbytes, count,
                               stream.cuda_stream)
        return codes, scales, valid

    def scatter_blocks(self, blocks, codes, scales, valid=None, *, stream=None):
        """Write packed device blocks (``gather_blocks`` layout) into arena blocks
        ``blocks`` (the scatter half of host swap), enqueued on ``stream``. ``valid``
        None marks every restored key real; a given ``valid`` makes the arena carry
        padding bytes from now on."""
        count = len(blocks)
        if valid is not None and (valid.shape != (count, self.block_size)
                                  or valid.dtype != torch.uint8 or valid.device != self.device
                                  or not valid.is_contiguous()):
            raise ValueError("packed padding bytes do not match the arena layout")
        if codes.shape != (count,) + tuple(self.codes.shape[1:]) or codes.dtype != self.codes.dtype \
                or scales.shape != (count,) + tuple(self.scales.shape[1:]) \
                or scales.dtype != self.scales.dtype or not codes.is_contiguous() \
                or not scales.is_contiguous() or codes.device != self.device \
                or scales.device != self.device:
            raise ValueError("packed blocks do not match the arena layout")
        if not count:
            return
        stream = stream or torch.cuda.current_stream(self.device)
        with torch.cuda.stream(stream):
            index = self._index(blocks)
        if valid is None:
            with torch.cuda.stream(stream):
                valid = torch.ones((count, self.block_size), dtype=torch.uint8, device=self.device)
        else:
            self._enable_padding()
        for src, dst, nbytes in ((codes, self.codes, self.block_code_bytes),
                                 (scales, self.scales, self.block_scale_bytes),
                                 (valid, self.key_valid, self.block_size)):
            self._copy(src.data_ptr(), nbytes, None, count, dst.data_ptr(), nbytes, index.data_ptr(),
                       self.num_blocks, nbytes, count, stream.cuda_stream)
        index.record_stream(stream)

    def workspace_bytes(self, num_seqs, num_q_heads, max_context_len,
                        partition_tokens=DEFAULT_PARTITION_TOKENS, prefix_packs=None):
        if prefix_packs is not None:
            return int(_native.lib().astr_paged_attention_i8_shared_workspace_bytes(
                num_seqs, num_q_heads, self.num_kv_heads, self.head_dim, max_context_len,
                prefix_packs.num_packs, prefix_packs.rows_per_pack))
        return int(_native.lib().astr_paged_attention_i8_workspace_bytes(
            num_seqs, num_q_heads, self.num_kv_heads, self.head_dim, max_context_len,
            partition_tokens))

    def workspace(self, num_seqs, num_q_heads, max_context_len,
                  partition_tokens=DEFAULT_PARTITION_TOKENS, prefix_packs=None):
        """Split-K scratch owned by this cache, grown on demand (None when unneeded)."""
        return self._scratch(self.workspace_bytes(num_seqs, num_q_heads, max_context_len,
                                                  partition_tokens, prefix_packs))

    def _scratch(self, need):
        if not need:
            return None
        if self._workspace is None or self._workspace.numel() < need:
            self._workspace = torch.empty(need, dtype=torch.uint8, device=self.device)
        return self._workspace

    def paged_attention(self, layer, query, block_tables, context_lens, *, max_context_len,
                        scale=None, window=None, partition_tokens=DEFAULT_PARTITION_TOKENS,
                        query_start_loc=None, max_query_len=None, causal=True,
                        out=None, workspace=None, work=None, check=False, prefix_packs=None,
                        decode_plan=None, append=None):
        """Paged attention of this layer's arena for every row of a step.

        Decode (``query_start_loc=None``): one query token per sequence, ``query``
        ``[S, Hq, D]``; the token sits at position ``ctx - 1``.

        Mixed step (chunked prefill + decode): ``query`` ``[T, Hq, D]`` packed by
        sequence, ``query_start_loc`` int32 ``[S + 1]`` device offsets (sequence
        ``s`` owns rows ``[qsl[s], qsl[s+1])``), ``max_query_len`` the host-side
        bound of the per-sequence query count (computed with a device sync when
        omitted). Query ``i`` of a sequence with ``n`` queries sits at position
        ``ctx - n + i`` (the chunk is already appended, paged_attention.py:185-192)
        and sees keys ``<= position`` when ``causal`` (online_attention.py:181-182).

        ``block_tables`` int32 ``[S, max_blocks]``; ``context_lens`` int32 ``[S]``
        (committed length including the step's tokens); ``max_context_len`` host
        upper bound of ``context_lens``. ``scale`` defaults to ``head_dim ** -0.5``
        (nn/attention.py:130); ``window`` keeps keys ``k > position - window``
        (online_attention.py:183-184). Returns the query's shape in the query
        dtype (online_attention.py:219).

        ``prefix_packs`` (decode, automatic split, no window): a
        ``prefix_plan.plan_prefix_packs`` plan of the same block tables; rows of a
        pack read their shared prefix blocks once for the whole pack. Same outputs
        as without it.

        ``decode_plan`` (decode, bf16/fp16 queries): a ``decode_plan.plan_decode``
        schedule of the same block tables and lengths (and window); the planned kernel
        streams the blocks the plan names and does not read ``block_tables``. Same
        outputs as without it.

        ``append`` (with ``decode_plan``, bf16/fp16): ``(key, value, slot_mapping)`` of the
        step's newest tokens, key/value ``[S, Hkv, D]`` in the query dtype and int64 slots
        ``[S]`` the caller reserved. The decode quantizes and writes each token into the
        arena and attends to it in the same launch: the outputs and the arena equal
        ``append(..., reserved=True)`` followed by the call without it."""
        if query.ndim != 3 or query.shape[-1] != self.head_dim or query.device != self.device:
            raise ValueError("query must be [tokens, num_q_heads, head_dim] on the cache device")
        if query.dtype not in _DTYPE_CODES:
            raise UnsupportedAttentionBackend(f"query dtype {query.dtype} is not fp32/fp16/bf16")
        if query.stride(-1) != 1:
            raise ValueError("query rows must be contiguous")
        num_tokens, num_q_heads = query.shape[0], query.shape[1]
        if num_q_heads % self.num_kv_heads:
            raise ValueError("Query heads must divide into KV groups")
        _check_index(block_tables, "block_tables", 2, self.device)
        _check_index(context_lens, "context_lens", 1, self.device)
        num_seqs = block_tables.shape[0]
        if context_lens.shape[0] != num_seqs:
            raise ValueError("block_tables/context_lens must have one row per sequence")
        if query_start_loc is None:
            if num_tokens != num_seqs:
                raise ValueError("decode attention takes one query row per sequence")
        else:
            _check_index(query_start_loc, "query_start_loc", 1, self.device)
            if query_start_loc.shape[0] != num_seqs + 1:
                raise ValueError("query_start_loc must have num_seqs + 1 entries")
            if max_query_len is None:
                lens = query_start_loc[1:] - query_start_loc[:-1]
                max_query_len = int(lens.max().item()) if num_seqs else 0
            if type(max_query_len) is not int or max_query_len < 0:
                raise ValueError("max_query_len must be a non-negative int")
        if max_context_len > block_tables.shape[1] * self.block_size:
            raise ValueError("max_context_len exceeds the block table capacity")
        scale = self.head_dim ** -0.5 if scale is None else float(scale)
        if not math.isfinite(scale) or scale <= 0:
            raise ValueError("Attention scale must be finite and positive")
        if window is not None and (type(window) is not int or window < 1):
            raise ValueError("Invalid causal/window semantics")
        if prefix_packs is not None:
            if query_start_loc is not None or partition_tokens != 0 or window is not None:
                raise ValueError("prefix packs serve decode batches under the automatic split "
                                 "without a window")
            if prefix_packs.num_seqs != num_seqs or prefix_packs.table.device != self.device:
                raise ValueError("prefix packs were planned for other block tables")
        if decode_plan is not None:
            if query_start_loc is not None or partition_tokens != 0 or prefix_packs is not None:
                raise ValueError("a decode plan serves decode batches under the automatic "
                                 "split, without prefix packs")
            if (decode_plan.num_seqs != num_seqs or decode_plan.num_q_heads != num_q_heads
                    or decode_plan.head_dim != self.head_dim or decode_plan.window != window
                    or decode_plan.info.num_kv_heads != self.num_kv_heads
                    or decode_plan.words.device != self.device):
                raise ValueError("the decode plan was built for another batch")
        if append is not None:
            if decode_plan is None:
                raise ValueError("an appending decode runs on a decode plan")
            key, value, slots = append
            _check_rows(key, "key", self.num_kv_heads, self.head_dim, self.device)
            _check_rows(value, "value", self.num_kv_heads, self.head_dim, self.device)
            if (key.dtype != query.dtype or value.dtype != query.dtype
                    or query.dtype not in (torch.bfloat16, torch.float16)
                    or key.shape[0] != num_tokens or value.shape[0] != num_tokens):
                raise ValueError("an appending decode takes bf16/fp16 key/value rows "
                                 "[S, Hkv, D] in the query dtype")
            if not self.decode_appends(query.dtype):
                raise UnsupportedAttentionBackend(
                    "hip_int8_paged decodes append at head dims 128 and 256")
            if (slots.dtype != torch.int64 or slots.shape != (num_tokens,)
                    or slots.device != self.device or not slots.is_contiguous()):
                raise ValueError("slot_mapping must be a contiguous int64 device vector [S]")
        if out is None:
            out = torch.empty_like(query)
        elif (not isinstance(out, torch.Tensor) or out.shape != query.shape
              or out.dtype != query.dtype or out.device != self.device or out.stride(-1) != 1):
            raise ValueError("out must match the query's shape, dtype and device, with "
                             "contiguous rows")
        need = (decode_plan.workspace_bytes() if decode_plan is not None else
                self.workspace_bytes(num_seqs, num_q_heads, max_context_len, partition_tokens,
                                     prefix_packs))
        if need and workspace is None:
            workspace = self._scratch(need)
        elif need:
            if (not isinstance(workspace, torch.Tensor) or workspace.dtype != torch.uint8
                    or workspace.device != self.device or not workspace.is_contiguous()):
                raise ValueError("workspace must be a contiguous uint8 tensor on the cache device")
            if workspace.numel() < need:
                raise ValueError(f"workspace of {need} bytes required")
        stream = torch.cuda.current_stream(self.device).cuda_stream
        ws = workspace.data_ptr() if need else None
        lib = _native.lib()
        if append is not None:
            key, value, slots = append
            rc = lib.astr_paged_attention_i8_planned_append(
                self._descs[layer], query.data_ptr(), _DTYPE_CODES[query.dtype], query.stride(0),
                query.stride(1), out.data_ptr(), out.stride(0), out.stride(1), key.data_ptr(),
                value.data_ptr(), key.stride(0), key.stride(1), value.stride(0), value.stride(1),
                slots.data_ptr(), context_lens.data_ptr(), num_q_heads, scale,
                decode_plan.words.data_ptr(), ctypes.byref(decode_plan.info), ws, need,
                self.err_flag.data_ptr(), stream)
        elif decode_plan is not None:
            rc = lib.astr_paged_attention_i8_planned(
                self._descs[layer], query.data_ptr(), _DTYPE_CODES[query.dtype], query.stride(0),
                query.stride(1), out.data_ptr(), out.stride(0), out.stride(1),
                context_lens.data_ptr(), num_q_heads, scale, decode_plan.words.data_ptr(),
                ctypes.byref(decode_plan.info), ws, need, self.err_flag.data_ptr(), stream)
        elif prefix_packs is not None:
            rc = lib.astr_paged_attention_i8_shared(
                self._descs[layer], query.data_ptr(), _DTYPE_CODES[query.dtype], query.stride(0),
                query.stride(1), out.data_ptr(), out.stride(0), out.stride(1),
                block_tables.data_ptr(), block_tables.stride(0), context_lens.data_ptr(),
                num_seqs, num_q_heads, max_context_len, scale, 0, prefix_packs.table.data_ptr(),
                prefix_packs.num_packs, prefix_packs.rows_per_pack, ws, need,
                self.err_flag.data_ptr(), stream)
        elif query_start_loc is None:
            rc = lib.astr_paged_attention_i8(
                self._descs[layer], query.data_ptr(), _DTYPE_CODES[query.dtype], query.stride(0),
                query.stride(1), out.data_ptr(), out.stride(0), out.stride(1),
                block_tables.data_ptr(), block_tables.stride(0), context_lens.data_ptr(),
                num_seqs, num_q_heads, max_context_len, scale, window or 0, partition_tokens,
                ws, need, self.err_flag.data_ptr(), stream)
        else:
            rc = lib.astr_paged_attention_varlen_i8(
                self._descs[layer], query.data_ptr(), _DTYPE_CODES[query.dtype], query.stride(0),
                query.stride(1), out.data_ptr(), out.stride(0), out.stride(1),
                query_start_loc.data_ptr(), num_tokens, max_query_len, 1 if causal else 0,
                block_tables.data_ptr(), block_tables.stride(0), context_lens.data_ptr(),
                num_seqs, num_q_heads, max_context_len, scale, window or 0, partition_tokens,
                ws, need, self.err_flag.data_ptr(), stream)
        _native.check(rc, "paged_attention")
        if work is not None:
            prefill = query_start_loc is not None and max_query_len > 1
            work.backend, work.fallback_reason = BACKEND, None
            work.page_launches += (2 if need else 1) + (1 if prefill else 0)
            work.query_tiles += 1
            work.max_query_tile = max(work.max_query_tile, max_query_len if prefill else 1)
            work.max_key_tile = max(work.max_key_tile, self.block_size)
            work.compiler_version = lib.astr_version().decode()
        if check:
            self.raise_errors()
        return out

    def decode_appends(self, dtype):
        """Whether a planned decode of this arena appends the step's ``dtype`` rows itself
        (``paged_attention(append=...)``): bf16/fp16 at head dims 128 and 256 (at 64 the
        token rows would cost the kernel its second workgroup per CU)."""
        return dtype in (torch.bfloat16, torch.float16) and self.head_dim in (128, 256)

    def paged_attention_statistics(self, layer, query, block_tables, context_lens, *,
                                   max_context_len, scale=None, window=None,
                                   partition_tokens=DEFAULT_PARTITION_TOKENS, check=False):
        """Decode rows' softmax states instead of their outputs
        (``online_attention_statistics``, online_attention.py:74-214): ``query`` fp32
        ``[S, Hq, D]``, other arguments as :meth:`paged_attention`. Returns
        ``(maximum, mass, weighted)``: ``[S, Hq]``, ``[S, Hq]`` and ``[S, Hq, D]`` fp32,
        the largest visible score, ``sum(exp(score - maximum))`` and the numerator
        ``sum(exp(score - maximum) * value)``; a row with no visible key gets
        ``(-inf, 0, 0)``."""
        if (query.ndim != 3 or query.shape[-1] != self.head_dim or query.device != self.device
                or query.dtype != torch.float32 or query.stride(-1) != 1):
            raise ValueError("query must be fp32 [tokens, num_q_heads, head_dim] on the cache "
                             "device with contiguous rows")
        num_seqs, num_q_heads = query.shape[0], query.shape[1]
        if num_q_heads % self.num_kv_heads:
            raise ValueError("Query heads must divide into KV groups")
        _check_index(block_tables, "block_tables", 2, self.device)
        _check_index(context_lens, "context_lens", 1, self.device)
        if block_tables.shape[0] != num_seqs or context_lens.shape[0] != num_seqs:
            raise ValueError("block_tables/context_lens must have one row per query row")
        if max_context_len > block_tables.shape[1] * self.block_size:
            raise ValueError("max_context_len exceeds the block table capacity")
        scale = self.head_dim ** -0.5 if scale is None else float(scale)
        if not math.isfinite(scale) or scale <= 0:
            raise ValueError("Attention scale must be finite and positive")
        if window is not None and (type(window) is not int or window < 1):
            raise ValueError("Invalid causal/window semantics")
        weighted = torch.empty_like(query)
        stats = torch.empty((num_seqs, num_q_heads, 2), dtype=torch.float32, device=self.device)
        need = self.workspace_bytes(num_seqs, num_q_heads, max_context_len, partition_tokens)
        ws = self._scratch(need).data_ptr() if need else None
        stream = torch.cuda.current_stream(self.device).cuda_stream
        rc = _native.lib().astr_paged_attention_i8_statistics(
            self._descs[layer], query.data_ptr(), query.stride(0), query.stride(1),
            weighted.data_ptr(), weighted.stride(0), weighted.stride(1), stats.data_ptr(),
            block_tables.data_ptr(), block_tables.stride(0), context_lens.data_ptr(), num_seqs,
            num_q_heads, max_context_len, scale, window or 0, partition_tokens, ws, need,
            self.err_flag.data_ptr(), stream)
        _native.check(rc, "paged_attention_statistics")
        if check:
            self.raise_errors()
        return stats[..., 0], stats[..., 1], weighted


def _check_rows(tensor, name, heads, width, device):
    if (not isinstance(tensor, torch.Tensor) or tensor.ndim != 3 or tensor.shape[1] != heads
            or tensor.shape[2] != width or tensor.device != device or tensor.stride(-1) != 1):
        raise ValueError(f"{name} must be a [T, num_kv_heads, head_dim] device tensor with "
                         "contiguous rows")
    if tensor.dtype not in _DTYPE_CODES:
        raise ValueError("Quantized KV requires finite floating input")


def _check_index(tensor, name, ndim, device):
    if (not isinstance(tensor, torch.Tensor) or tensor.dtype != torch.int32 or tensor.ndim != ndim
            or tensor.device != device or tensor.stride(-1) != 1):
        raise ValueError(f"{name} must be an int32 device tensor of rank {ndim} with "
                         "contiguous rows")
