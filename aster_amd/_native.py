"""ctypes binding of ``libaster_kv.so`` (the C ABI declared in ``include/aster_kv.h``).

The library is built in-tree by ``__graft_entry__.build()`` (or ``python -m
aster_amd.build``) into ``aster_amd/_lib/``. There is deliberately no fallback:
if the library is missing, :func:`lib` raises so the HIP path can never be
silently replaced by something else.
"""

from __future__ import annotations

import ctypes
import os
import threading

LIB_NAME = "libaster_kv.so"
LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib")
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)

ASTR_KV_INT8, ASTR_KV_FP8_E4M3FN, ASTR_KV_FP8_E5M2 = 0, 1, 2  # astr_kv_format
ASTR_EINVAL = -1
ASTR_EUNSUPPORTED = -2

FLAG_NONFINITE_INPUT = 1
FLAG_NONFINITE_SCORE = 2
FLAG_BAD_INDEX = 4

ASTR_F32, ASTR_F16, ASTR_BF16 = 0, 1, 2

# Every symbol include/aster_kv.h declares (checked by tests/test_capi.py).
EXPORTED_SYMBOLS = (
    "astr_kv_quantize_append_i8",
    "astr_kv_quantize_append_i8_reserved",
    "astr_kv_write_key_valid",
    "astr_paged_attention_i8",
    "astr_paged_attention_varlen_i8",
    "astr_paged_attention_i8_noalloc",
    "astr_paged_attention_i8_statistics",
    "astr_paged_attention_i8_shared",
    "astr_paged_attention_i8_workspace_bytes",
    "astr_paged_attention_i8_shared_workspace_bytes",
    "astr_kv_copy_blocks",
    "astr_merge_softmax_f32",
    "astr_decode_plan_workgroups",
    "astr_decode_plan_words_bound",
    "astr_decode_plan",
    "astr_paged_attention_i8_planned_workspace_bytes",
    "astr_paged_attention_i8_planned",
    "astr_paged_attention_i8_planned_append",
    "astr_last_error",
    "astr_version",
)


class PagedKVDesc(ctypes.Structure):
    """Mirror of ``astr_paged_kv``."""

    _fields_ = [
        ("k_codes", ctypes.c_void_p),
        ("v_codes", ctypes.c_void_p),
        ("k_scales", ctypes.c_void_p),
        ("v_scales", ctypes.c_void_p),
        ("code_block_stride", ctypes.c_int64),
        ("code_head_stride", ctypes.c_int64),
        ("scale_block_stride", ctypes.c_int64),
        ("scale_head_stride", ctypes.c_int64),
        ("num_blocks", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("key_valid", ctypes.c_void_p),
        ("code_format", ctypes.c_int32),
    ]


_lock = threading.Lock()
_lib = None


class NativeLibraryMissing(ImportError):
    """The HIP library is not built; build it with ``python -m aster_amd.build``."""


def lib():
    """Load ``libaster_kv.so`` once and declare its signatures."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise NativeLibraryMissing(
                f"{LIB_PATH} is missing: build the gfx950 HIP library first "
                "(python -m aster_amd.build); there is no CPU fallback"
            )
        handle = ctypes.CDLL(LIB_PATH)
        c_i32, c_i64, c_vp, c_sz = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t
        desc_p = ctypes.POINTER(PagedKVDesc)
        handle.astr_kv_quantize_append_i8.argtypes = [
            desc_p, c_vp, c_vp, c_i32, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp,
        ]
        handle.astr_kv_quantize_append_i8.restype = ctypes.c_int
        handle.astr_kv_quantize_append_i8_reserved.argtypes = [
            desc_p, c_vp, c_vp, c_i32, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp,
        ]
        handle.astr_kv_quantize_append_i8_reserved.restype = ctypes.c_int
        handle.astr_kv_write_key_valid.argtypes = [desc_p, c_vp, c_vp, c_i64, c_vp, c_vp]
        handle.astr_kv_write_key_valid.restype = ctypes.c_int
        handle.astr_paged_attention_i8.argtypes = [
            desc_p, c_vp, c_i32, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp, c_i32, c_vp, c_i32,
            c_i32, c_i32, ctypes.c_float, c_i32, c_i32, c_vp, c_sz, c_vp, c_vp,
        ]
        handle.astr_paged_attention_i8.restype = ctypes.c_int
        handle.astr_paged_attention_i8_noalloc.argtypes = [
            desc_p, c_vp, c_i32, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp, c_i32, c_vp, c_i32,
            c_i32, c_i32, ctypes.c_float, c_i32, c_i32, c_vp, c_vp,
        ]
        handle.astr_paged_attention_i8_noalloc.restype = ctypes.c_int
        handle.astr_paged_attention_i8_statistics.argtypes = [
            desc_p, c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp, c_vp, c_i32, c_vp, c_i32,
            c_i32, c_i32, ctypes.c_float, c_i32, c_i32, c_vp, c_sz, c_vp, c_vp,
        ]
        handle.astr_paged_attention_i8_statistics.restype = ctypes.c_int
        handle.astr_paged_attention_i8_shared.argtypes = [
            desc_p, c_vp, c_i32, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp, c_i32, c_vp, c_i32,
            c_i32, c_i32, ctypes.c_float, c_i32, c_vp, c_i32, c_i32, c_vp, c_sz, c_vp, c_vp,
        ]
        handle.astr_paged_attention_i8_shared.restype = ctypes.c_int
        handle.astr_paged_attention_varlen_i8.argtypes = [
            desc_p, c_vp, c_i32, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp, c_i32, c_i32, c_i32,
            c_vp, c_i32, c_vp, c_i32, c_i32, c_i32, ctypes.c_float, c_i32, c_i32, c_vp, c_sz,
            c_vp, c_vp,
        ]
        handle.astr_paged_attention_varlen_i8.restype = ctypes.c_int
        handle.astr_kv_copy_blocks.argtypes = [
            c_vp, c_i64, c_vp, c_i32, c_vp, c_i64, c_vp, c_i32, c_i64, c_i32, c_vp, c_vp,
        ]
        handle.astr_kv_copy_blocks.restype = ctypes.c_int
        handle.astr_merge_softmax_f32.argtypes = [c_vp] * 9 + [c_i64, c_i32, c_vp]
        handle.astr_merge_softmax_f32.restype = ctypes.c_int
        handle.astr_paged_attention_i8_workspace_bytes.argtypes = [c_i32] * 6
        handle.astr_paged_attention_i8_workspace_bytes.restype = c_sz
        handle.astr_paged_attention_i8_shared_workspace_bytes.argtypes = [c_i32] * 7
        handle.astr_paged_attention_i8_shared_workspace_bytes.restype = c_sz
        i32p = ctypes.POINTER(c_i32)
        handle.astr_decode_plan_workgroups.argtypes = [c_i32] * 5 + [i32p, i32p]
        handle.astr_decode_plan_workgroups.restype = ctypes.c_int
        handle.astr_decode_plan_words_bound.argtypes = [c_i32, c_i32, c_i64, c_i32, c_i32, c_i32]
        handle.astr_decode_plan_words_bound.restype = c_i64
        handle.astr_decode_plan.argtypes = [i32p, c_i32, i32p, c_i32, c_i32, c_i32, c_i32, c_i32,
                                            c_i32, c_i32, c_i32, i32p, c_i64, c_vp]
        handle.astr_decode_plan.restype = ctypes.c_int
        handle.astr_paged_attention_i8_planned_workspace_bytes.argtypes = [c_vp, c_i32, c_i32]
        handle.astr_paged_attention_i8_planned_workspace_bytes.restype = c_sz
        handle.astr_paged_attention_i8_planned.argtypes = [
            desc_p, c_vp, c_i32, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp, c_i32, ctypes.c_float,
            c_vp, c_vp, c_vp, c_sz, c_vp, c_vp,
        ]
        handle.astr_paged_attention_i8_planned.restype = ctypes.c_int
        handle.astr_paged_attention_i8_planned_append.argtypes = [
            desc_p, c_vp, c_i32, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp, c_vp, c_i64, c_i64,
            c_i64, c_i64, c_vp, c_vp, c_i32, ctypes.c_float, c_vp, c_vp, c_vp, c_sz, c_vp, c_vp,
        ]
        handle.astr_paged_attention_i8_planned_append.restype = ctypes.c_int
        handle.astr_last_error.argtypes = []
        handle.astr_last_error.restype = ctypes.c_char_p
        handle.astr_version.argtypes = []
        handle.astr_version.restype = ctypes.c_char_p
        _lib = handle
        return _lib


def last_error() -> str:
    return lib().astr_last_error().decode("utf-8", "replace")


def check(code: int, what: str) -> None:
    """Map a C-ABI return code to the reference's exception types."""
    if code == 0:
        return
    message = f"{what}: {last_error()}"
    if code == ASTR_EUNSUPPORTED:
        from .attention_backend import UnsupportedAttentionBackend

        raise UnsupportedAttentionBackend(message)
    if code == ASTR_EINVAL:
        raise ValueError(message)
    raise RuntimeError(f"{message} (hipError {code})")
