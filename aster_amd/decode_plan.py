"""Host-built schedules of decode batches (``astr_decode_plan``) for the planned decode
kernel.

The runner holds every row's page list and length on the host
(``PagedStatePool.read_pages``, src/aster/inference/state.py:358-390, is what the
reference's row loop reads per step), so the split of a decode batch over the GPU is
settled there once per step and serves every layer of the step: the plan carries the
rows' physical block ids, each workgroup's rows and each wave's range of blocks. The
kernel then starts streaming after one round trip for its block ids, and merges the
pieces of a row inside the workgroup that holds them. A plan is valid only for the
tables and lengths it was built from (the kernel checks the lengths against the device
copy and every index against the arena and the batch).
"""

from __future__ import annotations

import ctypes
import threading

import numpy as np
import torch

from . import _native


class DecodePlanInfo(ctypes.Structure):
    """Mirror of ``astr_decode_plan_info``."""

    _fields_ = [(name, ctypes.c_int32) for name in (
        "num_workgroups", "waves_per_workgroup", "num_items", "num_blocks", "num_ids",
        "num_chunks", "num_chunked", "num_seqs", "num_kv_heads", "window", "tail_blocks",
        "item_stride", "num_tiles", "tile_rows", "tile_ranges", "num_tile_members")] + \
        [(name, ctypes.c_int64) for name in (
            "off_workgroups", "off_waves", "off_items", "off_ids", "off_chunked", "off_tiles",
            "off_tile_members", "plan_words")]


# Blocks at the end of each wave's range that it loads two at a time (the waves that
# finish first leave memory bandwidth to the ones still streaming).
DEFAULT_TAIL_BLOCKS = 0
# Shared prefixes read in prefix tiles: the fewest shared blocks that make a tile.
DEFAULT_MIN_SHARED_BLOCKS = 8


def tile_columns(head_dim):
    """Query columns of a prefix tile (the chunked-prefill kernel's per workgroup)."""
    return 64 if head_dim == 256 else 128

_lock = threading.Lock()
_workgroups = {}


def plan_workgroups(head_dim, num_q_heads, num_kv_heads, q_dtype_code, code_format, device):
    """(resident workgroups, waves per workgroup) of the planned kernel on ``device``."""
    key = (torch.device(device).index, head_dim, num_q_heads, num_kv_heads, q_dtype_code,
           code_format)
    with _lock:
        if key not in _workgroups:
            wg, nw = ctypes.c_int32(0), ctypes.c_int32(0)
            with torch.cuda.device(device):
                rc = _native.lib().astr_decode_plan_workgroups(
                    head_dim, num_q_heads, num_kv_heads, q_dtype_code, code_format,
                    ctypes.byref(wg), ctypes.byref(nw))
            _native.check(rc, "decode plan workgroups")
            _workgroups[key] = (wg.value, nw.value)
        return _workgroups[key]


class DecodePlan:
    """A decode batch's schedule: ``info`` (host record) and ``words`` (the int32 plan on
    the device), with the shapes it was built for."""

    def __init__(self, info, words, host, num_q_heads, head_dim, window):
        self.info, self.words, self._host = info, words, host
        self.num_q_heads, self.head_dim, self.window = num_q_heads, head_dim, window

    @property
    def num_seqs(self):
        return self.info.num_seqs

    def workspace_bytes(self):
        return int(_native.lib().astr_paged_attention_i8_planned_workspace_bytes(
            ctypes.byref(self.info), self.num_q_heads, self.head_dim))


def plan_decode(block_tables, context_lens, *, num_q_heads, num_kv_heads, head_dim, q_dtype,
                device, code_format=_native.ASTR_KV_INT8, window=None,
                tail_blocks=DEFAULT_TAIL_BLOCKS, num_workgroups=None, shared_prefixes=True,
                tile_rows=None, tile_ranges=0, min_shared_blocks=DEFAULT_MIN_SHARED_BLOCKS):
    """Plan the decode rows of one step from host ``block_tables`` (int ``[S, width]``)
    and ``context_lens`` (``[S]``, the lengths the device copy will hold) for the
    planned kernel on ``device``; the plan's words are uploaded asynchronously on the
    current stream. ``num_workgroups`` overrides the device's resident workgroups
    (tests). With ``shared_prefixes``, sequences whose tables begin with the same
    ``min_shared_blocks`` blocks or more read them in prefix tiles of ``tile_rows``
    sequences (default: as many as a tile's query columns hold) over ``tile_ranges``
    key ranges (0: chosen by the planner)."""
    tables = np.ascontiguousarray(np.asarray(block_tables), dtype=np.int32)
    lens = np.ascontiguousarray(np.asarray(context_lens), dtype=np.int32)
    if tables.ndim != 2 or lens.ndim != 1 or tables.shape[0] != lens.shape[0]:
        raise ValueError("block_tables [S, width] and context_lens [S] are required")
    if window is not None and (type(window) is not int or window < 1):
        raise ValueError("Invalid causal/window semantics")
    from .paged_kv import _DTYPE_CODES

    if q_dtype not in _DTYPE_CODES:
        raise ValueError(f"query dtype {q_dtype} is not fp32/fp16/bf16")
    wg, nw = plan_workgroups(head_dim, num_q_heads, num_kv_heads, _DTYPE_CODES[q_dtype],
                             code_format, device)
    if num_workgroups is not None:
        wg = int(num_workgroups)
    rows = 0
    if shared_prefixes:
        rows = tile_rows if tile_rows is not None else tile_columns(head_dim) // (
            num_q_heads // num_kv_heads)
        if type(rows) is not int or rows < 0:
            raise ValueError("tile_rows must be a non-negative int")
        rows = rows if rows >= 2 else 0
    lib = _native.lib()
    win = window or 0
    ctx = lens.astype(np.int64)
    first = np.where((win > 0) & (ctx > win), ctx - win, 0) // 16
    visible = int(np.maximum(-(-ctx // 16) - first, 0).sum())
    bound = lib.astr_decode_plan_words_bound(lens.shape[0], num_kv_heads, visible, wg, nw, rows)
    host = torch.empty(max(int(bound), 1), dtype=torch.int32, pin_memory=True)
    info = DecodePlanInfo()
    i32p = ctypes.POINTER(ctypes.c_int32)
    rc = lib.astr_decode_plan(tables.ctypes.data_as(i32p), tables.shape[1],
                              lens.ctypes.data_as(i32p), lens.shape[0], num_kv_heads, win, wg,
                              nw, rows, tile_ranges, min_shared_blocks,
                              ctypes.cast(host.data_ptr(), i32p), host.numel(),
                              ctypes.byref(info))
    _native.check(rc, "decode plan")
    info.tail_blocks = tail_blocks
    words = host[: max(info.plan_words, 1)].to(device, non_blocking=True)
    return DecodePlan(info, words, host, num_q_heads, head_dim, window)
