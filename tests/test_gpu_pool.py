"""GPU checks of the arena-backed pool and host swap: device appends and copy-on-write
are bit-exact against the oracle quantizer, astr_kv_copy_blocks moves blocks
bit-exactly (and flags bad indices), attention over pool block tables matches the
oracle, and PagedStateArchive round trips codes and scales at atol=0 with the
reference's budget/identity/transaction rules (test_paged_offload.py:31-79)."""

import asyncio

import numpy as np
import pytest
import torch

from aster_amd import KVQuantization, PagedKVCache
from aster_amd import _native
from aster_amd.offload import PagedStateArchive
from aster_amd.paged_pool import CacheCapacityError, PagedStatePool, StateError
from oracle import reference_cpu as ref
from tests.gpu_util import assert_attention_close, oracle_decode

pytestmark = pytest.mark.gpu
L, HKV, D = 2, 4, 64


def make_pool(device, blocks=16, fmt="int8"):
    return PagedStatePool(PagedKVCache(num_blocks=blocks, num_layers=L, num_kv_heads=HKV,
                                       head_dim=D, device=device,
                                       quantization=KVQuantization(fmt)))


def layers(tokens, seed, device, dtype=torch.bfloat16):
    g = torch.Generator(device=device).manual_seed(seed)
    return [tuple(torch.randn(1, HKV, tokens, D, generator=g, device=device).to(dtype)
                  for _ in range(2)) for _ in range(L)]


def oracle_state(state_layers, fmt="int8"):
    return [tuple(torch.from_numpy(ref.quantize_kv(x.float().cpu().numpy(), fmt).dequantize())
                  for x in pair) for pair in state_layers]


def assert_state(pool, seq, want):
    for (gk, gv), (wk, wv) in zip(pool.materialize(seq), want):
        torch.testing.assert_close(gk.cpu(), wk, atol=0, rtol=0)
        torch.testing.assert_close(gv.cpu(), wv, atol=0, rtol=0)


def cat(a, b):
    return [(torch.cat([ka, kb], 2), torch.cat([va, vb], 2)) for (ka, va), (kb, vb) in zip(a, b)]


def test_device_append_fork_cow_truncate_bit_exact(device):
    pool = make_pool(device)
    seq = pool.create("tenant-policy")
    base = layers(21, 1, device)
    pool.append_delta(seq, base)
    assert_state(pool, seq, oracle_state(base))
    fork = pool.fork(seq)
    tail = fork.pages[-1]
    extra = layers(3, 2, device)
    pool.append_delta(seq, extra)
    assert seq.pages[-1] != tail == fork.pages[-1]
    assert_state(pool, fork, oracle_state(base))          # the shared page is untouched
    assert_state(pool, seq, oracle_state(cat(base, extra)))  # the copy carries the prefix
    pool.truncate(seq, 18)
    assert_state(pool, seq, [(k[..., :18, :], v[..., :18, :]) for k, v in oracle_state(base)])
    pool.release(seq), pool.release(fork)
    assert pool.used_blocks == 0 and pool.storage_metrics()["allocated_tensor_bytes"] == 0


def test_copy_blocks_gather_scatter_and_bad_index(device):
    cache = PagedKVCache(num_blocks=9, num_layers=L, num_kv_heads=HKV, head_dim=D, device=device)
    g = torch.Generator(device=device).manual_seed(3)
    cache.codes.copy_(torch.randint(-127, 128, cache.codes.shape, generator=g, device=device,
                                    dtype=torch.int8))
    cache.scales.copy_(torch.rand(cache.scales.shape, generator=g, device=device))
    cache.key_valid.copy_(torch.randint(0, 2, cache.key_valid.shape, generator=g, device=device,
                                        dtype=torch.uint8))
    before_c, before_s, before_v = cache.codes.clone(), cache.scales.clone(), cache.key_valid.clone()
    codes, scales, valid = cache.gather_blocks([7, 2, 5])
    assert torch.equal(codes, before_c[[7, 2, 5]]) and torch.equal(scales, before_s[[7, 2, 5]])
    assert torch.equal(valid, before_v[[7, 2, 5]])
    cache.scatter_blocks([0, 8, 1], codes, scales, valid)
    assert cache.has_padding
    assert torch.equal(cache.codes[[0, 8, 1]], before_c[[7, 2, 5]])
    assert torch.equal(cache.scales[[0, 8, 1]], before_s[[7, 2, 5]])
    assert torch.equal(cache.key_valid[[0, 8, 1]], before_v[[7, 2, 5]])
    cache.copy_blocks([3], [4])
    assert torch.equal(cache.codes[4], before_c[3]) and torch.equal(cache.scales[4], before_s[3])
    assert torch.equal(cache.key_valid[4], before_v[3])
    untouched = [2, 3, 5, 6, 7]
    assert torch.equal(cache.codes[untouched], before_c[untouched])
    # an index outside the arena is flagged and that block is skipped
    snap = cache.codes.clone()
    cache.copy_blocks([3, 2], [9, 6])
    assert cache.pending_errors() & _native.FLAG_BAD_INDEX
    assert torch.equal(cache.codes[6], before_c[2]) and torch.equal(cache.codes[:6], snap[:6])
    # unaligned byte path (odd sizes): a raw copy through the C ABI
    src = torch.arange(3 * 37, dtype=torch.uint8, device=device)
    dst = torch.zeros(4 * 41, dtype=torch.uint8, device=device)
    idx = torch.tensor([2, 0, 1], dtype=torch.int32, device=device)
    flag = torch.zeros(1, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream().cuda_stream
    _native.check(_native.lib().astr_kv_copy_blocks(
        src.data_ptr() + 1, 37, None, 3, dst.data_ptr() + 3, 41, idx.data_ptr(), 4, 35, 3,
        flag.data_ptr(), stream), "copy")
    torch.cuda.synchronize()
    want = np.zeros(4 * 41, np.uint8)
    s = np.arange(3 * 37, dtype=np.uint8)
    for i, d in enumerate([2, 0, 1]):
        want[3 + d * 41: 3 + d * 41 + 35] = s[1 + i * 37: 1 + i * 37 + 35]
    np.testing.assert_array_equal(dst.cpu().numpy(), want)
    assert int(flag.item()) == 0


def test_attention_over_pool_block_tables_matches_oracle(device):
    pool = make_pool(device, blocks=40)
    seqs = []
    for i, n in enumerate([1, 17, 60, 130]):
        s = pool.create(f"s{i}")
        pool.append_delta(s, layers(n, 10 + i, device))
        seqs.append(s)
    fork = pool.fork(seqs[2])
    pool.append_delta(fork, layers(5, 20, device))  # private tail copy for the fork
    rows = seqs + [fork]
    g = torch.Generator(device=device).manual_seed(5)
    q = torch.randn(len(rows), 2 * HKV, D, generator=g, device=device).to(torch.bfloat16)
    for layer in range(L):
        with pool.block_tables(rows) as (tables, lens):
            out = pool.cache.paged_attention(layer, q, tables, lens, max_context_len=135,
                                             check=True)
            torch.cuda.synchronize()
            want = oracle_decode(tables.cpu().numpy(), pool.cache, q, layer=layer,
                                 context_lens=lens.cpu().numpy(), scale=D ** -0.5)
        assert_attention_close(out, want)


@pytest.mark.parametrize("pin", [False, True])
@pytest.mark.parametrize("padded", [False, True])
def test_archive_roundtrip_is_bit_exact(device, pin, padded):
    pool = make_pool(device)
    seq = pool.create("tenant-policy")
    suffix = layers(37, 30, device)
    pad = torch.arange(37) % 5 != 3
    if padded:
        suffix = suffix + [(pad[None, None, :, None],)]
    pool.append_delta(seq, suffix)

    def codes(sequence):
        with pool.read_pages(sequence) as pages:
            return [[(x.values.clone(), x.scales.clone()) for x in page.payload[:-1]]
                    + [page.payload[-1].clone()] for page in pages]

    before = codes(seq)
    archive = PagedStateArchive(pool, pin_memory=pin)
    handle = archive.put(seq)
    pool.release(seq)
    assert pool.used_blocks == 0 and archive.stored_bytes == 37 * (L * 2 * HKV * (D + 4) + 1)
    pages = archive.pages(handle, identity="tenant-policy")
    assert len(pages) == 3 and pages[-1][0].values.shape == (1, HKV, 5, D)
    assert len(pages[0]) == 2 * L + 1 and pages[-1][-1].shape == (1, 1, 5, 1)
    restored = archive.restore(handle, identity="tenant-policy")
    assert restored.length == 37
    after = codes(restored)
    for page_a, page_b in zip(before, after):
        for (ca, sa), (cb, sb) in zip(page_a[:-1], page_b[:-1]):
            assert torch.equal(ca, cb) and torch.equal(sa, sb)
        assert torch.equal(page_a[-1], page_b[-1])
    got_pad = torch.cat([p[-1][0, 0, :, 0].cpu() for p in after])
    assert torch.equal(got_pad, pad if padded else torch.ones(37, dtype=torch.bool))
    archive.release(handle, identity="tenant-policy")
    pool.release(restored)
    assert archive.metrics() == dict(host_bytes=0, snapshots=0, offloaded_tokens=37,
                                     restored_tokens=37, pinned_memory=pin)
    assert pool.used_blocks == 0


def test_archive_budget_identity_and_failed_restore_are_transactional(device, monkeypatch):
    pool = make_pool(device, blocks=3)
    seq = pool.create("tenant-policy")
    pool.append_delta(seq, layers(33, 40, device))  # 3 pages
    archive = PagedStateArchive(pool)
    handle = archive.put(seq)
    with pytest.raises(StateError):
        archive.restore(handle, identity="other-tenant")
    with pytest.raises(StateError):
        archive.release(handle, identity="other-tenant")
    with pytest.raises(CacheCapacityError):
        archive.restore(handle, identity="tenant-policy")  # the pool is full
    assert pool.used_blocks == 3 and archive.metrics()["snapshots"] == 1
    full = PagedStateArchive(pool, max_bytes=archive.stored_bytes - 1)
    with pytest.raises(CacheCapacityError):
        full.put(seq)
    assert full.stored_bytes == 0
    pool.release(seq)

    def broken(*args, **kwargs):
        raise RuntimeError("injected transfer failure")

    monkeypatch.setattr(pool.cache, "scatter_blocks", broken)
    with pytest.raises(RuntimeError, match="injected"):
        archive.restore(handle, identity="tenant-policy")
    assert pool.used_blocks == 0 and archive.metrics()["snapshots"] == 1
    monkeypatch.undo()
    recovered = archive.restore(handle, identity="tenant-policy")
    archive.release(handle, identity="tenant-policy")
    pool.release(recovered)
    assert pool.used_blocks == 0


def test_async_put_and_restore(device):
    pool = make_pool(device)
    seq = pool.create("p")
    pool.append_delta(seq, layers(20, 50, device))
    archive = PagedStateArchive(pool, pin_memory=True)

    async def run():
        handle = await archive.put_async(seq)
        pool.release(seq)
        return await archive.restore_async(handle, identity="p"), handle

    restored, handle = asyncio.run(run())
    assert restored.length == 20 and pool.used_blocks == 2
    archive.release(handle, identity="p")
    pool.release(restored)


@pytest.mark.parametrize("fmt", ["fp8_e4m3fn", "fp8_e5m2"])
def test_fp8_pool_append_fork_archive_and_attention(device, fmt):
    """An FP8 arena behind the pool: appends dequantize to the oracle's FP8 values, page
    views carry the profile's float8 dtype, copy-on-write and the host archive move the
    bytes unchanged, and attention over the pool's block tables matches the oracle."""
    pool = make_pool(device, blocks=24, fmt=fmt)
    seq = pool.create("tenant")
    base = layers(21, 50, device)
    pool.append_delta(seq, base)
    assert_state(pool, seq, oracle_state(base, fmt))
    fork = pool.fork(seq)
    extra = layers(6, 51, device)
    pool.append_delta(fork, extra)  # copy of the shared partial tail page
    assert_state(pool, seq, oracle_state(base, fmt))
    assert_state(pool, fork, oracle_state([(torch.cat([a, c], 2), torch.cat([b, d], 2))
                                           for (a, b), (c, d) in zip(base, extra)], fmt))
    with pool.read_pages(fork) as views:
        assert views[0].payload[0].values.dtype == KVQuantization(fmt).dtype
        before = [[(x.values.view(torch.uint8).clone(), x.scales.clone()) for x in v.payload[:-1]]
                  for v in views]
    archive = PagedStateArchive(pool)
    handle = archive.put(fork)
    pool.release(fork)
    restored = archive.restore(handle, identity="tenant")
    with pool.read_pages(restored) as views:
        after = [[(x.values.view(torch.uint8).clone(), x.scales.clone()) for x in v.payload[:-1]]
                 for v in views]
    for pa, pb in zip(before, after):
        for (ca, sa), (cb, sb) in zip(pa, pb):
            assert torch.equal(ca, cb) and torch.equal(sa, sb)
    g = torch.Generator(device=device).manual_seed(52)
    q = torch.randn(2, 2 * HKV, D, generator=g, device=device).to(torch.bfloat16)
    for layer in range(L):
        with pool.block_tables([seq, restored]) as (tables, lens):
            out = pool.cache.paged_attention(layer, q, tables, lens, max_context_len=27, check=True)
            torch.cuda.synchronize()
            want = oracle_decode(tables.cpu().numpy(), pool.cache, q, layer=layer,
                                 context_lens=lens.cpu().numpy(), scale=D ** -0.5)
        assert_attention_close(out, want)
