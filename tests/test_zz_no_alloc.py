"""The allocation-free decode entry point (astr_paged_attention_i8_noalloc: split-K
partials in the library's fixed device array) against astr_paged_attention_i8 with a
caller workspace, through the C ABI: the same kernels, so the same outputs bit for bit,
on two calls in a row (the second smaller, so it meets the first call's leftovers in
the array), in both split modes; and a launch whose partials exceed the array is
refused before anything runs."""

import ctypes

import numpy as np
import pytest
import torch

from aster_amd import PagedKVCache, _native
from aster_amd import workloads as wl
from tests.gpu_util import assert_attention_close, oracle_decode

pytestmark = pytest.mark.gpu


def _call(lib, cache, w, q, out, tables, lens, part, *, workspace=None):
    stream = torch.cuda.current_stream(cache.device).cuda_stream
    args = (cache.layer_desc(0), q.data_ptr(), _native.ASTR_BF16, q.stride(0), q.stride(1),
            out.data_ptr(), out.stride(0), out.stride(1), tables.data_ptr(), tables.stride(0),
            lens.data_ptr(), w.num_seqs, w.num_q_heads, w.max_context_len,
            ctypes.c_float(w.scale), 0, part)
    if workspace is None:
        return lib.astr_paged_attention_i8_noalloc(*args, cache.err_flag.data_ptr(), stream)
    return lib.astr_paged_attention_i8(*args, workspace.data_ptr(), workspace.numel(),
                                       cache.err_flag.data_ptr(), stream)


@pytest.mark.parametrize("part", [0, 512])
def test_noalloc_matches_workspace_entry_point(device, part):
    lib = _native.lib()
    big = wl.scaled(wl.config2(), num_seqs=48)
    small = wl.scaled(wl.config2(), num_seqs=5, max_len=900, seed=77)
    for w in (big, small):  # the second call reuses the array the first one filled
        cache = PagedKVCache(num_blocks=w.num_blocks, num_layers=1,
                             num_kv_heads=w.num_kv_heads, head_dim=w.head_dim, device=device)
        wl.materialize(w, cache, device=device)
        tables, lens = wl.device_tables(w, device)
        q = wl.queries(w, device)
        ws = cache.workspace(w.num_seqs, w.num_q_heads, w.max_context_len, part)
        ref = torch.empty_like(q)
        got = torch.full_like(q, float("nan"))
        _native.check(_call(lib, cache, w, q, ref, tables, lens, part, workspace=ws), "ws")
        _native.check(_call(lib, cache, w, q, got, tables, lens, part), "noalloc")
        torch.cuda.synchronize(device)
        cache.raise_errors()
        assert torch.equal(got, ref)
        assert_attention_close(got, oracle_decode(w, cache, q))


def test_noalloc_refuses_partials_beyond_its_array(device):
    lib = _native.lib()
    lens = np.full(512, 4096, np.int32)
    tables = np.zeros((512, 256), np.int32)
    w = wl.DecodeWorkload("big", 64, 8, 128, lens, tables, 4, torch.bfloat16, 1, 128 ** -0.5)
    cache = PagedKVCache(num_blocks=4, num_layers=1, num_kv_heads=8, head_dim=128, device=device)
    q = torch.zeros(512, 64, 128, device=device, dtype=torch.bfloat16)
    out = torch.empty_like(q)
    t, l = wl.device_tables(w, device)
    # 64-token partitions: 512 x 64 heads x 64 partitions x 130 floats, far over 32 MiB
    rc = _call(lib, cache, w, q, out, t, l, 64)
    assert rc == _native.ASTR_EINVAL
    assert "allocation-free" in _native.last_error()
