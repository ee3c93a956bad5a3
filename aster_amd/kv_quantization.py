"""KV format profiles (INT8, FP8 E4M3FN, FP8 E5M2) and the device quantizer
(reference names and semantics).

Follows src/aster/optimization/kv_quantization.py: ``KVQuantization`` (:7-25),
``QuantizedKV`` (:28-68) and ``quantize_kv`` (:71-94). Quantization itself runs
in the gfx950 kernel behind ``astr_kv_quantize_append_i8`` (the arena descriptor
carries the code format); this module only validates, lays out the call and raises
the reference's exceptions.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _native
from .attention_backend import UnsupportedAttentionBackend

_DTYPE_CODES = {torch.float32: _native.ASTR_F32, torch.float16: _native.ASTR_F16,
                torch.bfloat16: _native.ASTR_BF16}
FORMAT_CODES = {"int8": _native.ASTR_KV_INT8, "fp8_e4m3fn": _native.ASTR_KV_FP8_E4M3FN,
                "fp8_e5m2": _native.ASTR_KV_FP8_E5M2}


@dataclass(frozen=True)
class KVQuantization:
    """Explicit KV storage format (kv_quantization.py:7-25): ``int8``, ``fp8_e4m3fn``
    or ``fp8_e5m2``, all three implemented by the HIP kernels (one byte per code)."""

    format: str = "int8"

    def __post_init__(self):
        if self.format not in {"int8", "fp8_e4m3fn", "fp8_e5m2"}:
            raise ValueError("KV format must be explicit INT8 / FP8 E4M3FN / FP8 E5M2")

    @property
    def dtype(self):
        return {
            "int8": torch.int8,
            "fp8_e4m3fn": torch.float8_e4m3fn,
            "fp8_e5m2": torch.float8_e5m2,
        }[self.format]

    @property
    def maximum(self):
        return 127.0 if self.format == "int8" else torch.finfo(self.dtype).max


@dataclass(frozen=True)
class QuantizedKV:
    """Codes ``[..., T, D]`` and fp32 scales ``[..., T, 1]`` (kv_quantization.py:28-68)."""

    values: torch.Tensor
    scales: torch.Tensor
    source_dtype: torch.dtype

    @property
    def shape(self):
        return self.values.shape

    @property
    def ndim(self):
        return self.values.ndim

    @property
    def dtype(self):
        return self.source_dtype

    @property
    def device(self):
        return self.values.device

    @property
    def nbytes(self):
        return (self.values.numel() * self.values.element_size()
                + self.scales.numel() * self.scales.element_size())

    def narrow(self, dim, start, count):
        if dim != self.ndim - 2:
            raise ValueError("Quantized KV token axis must immediately precede feature width")
        return QuantizedKV(self.values.narrow(dim, start, count),
                           self.scales.narrow(dim, start, count), self.source_dtype)

    def dequantize(self, *, dtype=None):
        """``fp32(code) * scale`` cast to ``dtype`` (kv_quantization.py:66-68); a plain
        tensor expression used for inspection/materialisation, not by the kernels."""
        return (self.values.to(self.scales.dtype) * self.scales).to(dtype or self.source_dtype)


def require_format(config):
    """The code format of an explicit profile (an ``astr_kv_format`` value)."""
    if not isinstance(config, KVQuantization):
        raise ValueError("An explicit immutable KVQuantization profile is required")
    return FORMAT_CODES[config.format]


@torch.no_grad()
def quantize_kv(value, config):
    """Device ``quantize_kv`` (kv_quantization.py:71-94), bit-exact with the reference.

    Same contract: ``None`` config or non-floating input passes through; rank < 3
    or empty width, non fp16/bf16/fp32 dtype or non-finite values raise
    ``ValueError``. Runs on the HIP device (a CPU tensor raises
    ``UnsupportedAttentionBackend``); the codes come back in the profile's dtype
    (``int8``, ``float8_e4m3fn`` or ``float8_e5m2``). Synchronises to report
    non-finite input as the reference does.
    """
    if config is None or not value.is_floating_point():
        return value
    if not isinstance(config, KVQuantization) or value.ndim < 3 or value.shape[-1] < 1:
        raise ValueError("Quantized KV needs explicit layout [...,tokens,width] and format")
    if value.dtype not in {torch.float16, torch.bfloat16, torch.float32, torch.float64}:
        raise ValueError("Quantized KV requires finite floating input")
    code_format = require_format(config)
    if value.dtype == torch.float64:
        raise UnsupportedAttentionBackend("hip_int8_paged stores fp32 scales; fp64 KV is not supported")
    if value.device.type != "cuda":
        raise UnsupportedAttentionBackend("hip_int8_paged quantizes HIP device tensors only")
    source = value.detach().contiguous()
    tokens, width = source.shape[-2], source.shape[-1]
    rows = source.numel() // max(tokens * width, 1)
    codes = torch.empty(source.shape, dtype=torch.int8, device=source.device)
    scales = torch.empty(source.shape[:-1] + (1,), dtype=torch.float32, device=source.device)
    if source.numel() == 0:
        return QuantizedKV(codes, scales, value.dtype)
    flag = torch.zeros(1, dtype=torch.int32, device=source.device)
    slots = torch.arange(tokens, dtype=torch.int64, device=source.device)
    desc = _native.PagedKVDesc(
        k_codes=codes.data_ptr(), v_codes=codes.data_ptr(), k_scales=scales.data_ptr(),
        v_scales=scales.data_ptr(), code_block_stride=rows * tokens * width,
        code_head_stride=tokens * width, scale_block_stride=rows * tokens,
        scale_head_stride=tokens, num_blocks=1, block_size=tokens, num_kv_heads=rows,
        head_dim=width, code_format=code_format)
    stream = torch.cuda.current_stream(source.device).cuda_stream
    _native.check(
        _native.lib().astr_kv_quantize_append_i8(
            desc, source.data_ptr(), None, _DTYPE_CODES[source.dtype], tokens,
            width, tokens * width, 0, 0, slots.data_ptr(), flag.data_ptr(), stream),
        "quantize_kv")
    if int(flag.item()) & _native.FLAG_NONFINITE_INPUT:
        raise ValueError("Quantized KV requires finite floating input")
    return QuantizedKV(codes.view(config.dtype), scales, value.dtype)
