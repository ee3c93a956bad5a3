"""GPU parity of the quantize-and-append kernel: bit-exact codes, scales and slot
placement against the oracle (kv_quantization.py:71-94, state.py:339-344)."""

import os

import numpy as np
import pytest
import torch

from aster_amd import KVQuantization, PagedKVCache, UnsupportedAttentionBackend, quantize_kv
from aster_amd import workloads as wl
from oracle import reference_cpu as ref
from tests.gpu_util import arena_numpy

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


FORMATS = ["int8", "fp8_e4m3fn", "fp8_e5m2"]


def _cache(device, blocks, heads, dim, layers=1, fmt="int8"):
    return PagedKVCache(num_blocks=blocks, num_layers=layers, num_kv_heads=heads, head_dim=dim,
                        device=device, quantization=KVQuantization(fmt))


def test_config1_append_matches_golden_arena(device):
    g = np.load(os.path.join(GOLDEN, "config1.npz"))
    cache = _cache(device, 64, 4, 64)
    k = torch.from_numpy(g["k"]).to(device)
    v = torch.from_numpy(g["v"]).to(device)
    slots = torch.from_numpy(g["slots"]).to(device)
    cache.append(0, k, v, slots, check=True)
    kc, ks, vc, vs = arena_numpy(cache)
    used = np.unique(g["slots"] // 16)
    np.testing.assert_array_equal(kc[used], g["k_codes"][used])
    np.testing.assert_array_equal(vc[used], g["v_codes"][used])
    assert (ks[used].view(np.uint32) == g["k_scales"][used].view(np.uint32)).all()
    assert (vs[used].view(np.uint32) == g["v_scales"][used].view(np.uint32)).all()
    # untouched blocks keep their initial contents
    untouched = np.setdiff1d(np.arange(64), used)
    assert (kc[untouched] == 0).all() and (ks[untouched] == 1).all()


def test_quantize_kv_api_seed76_known_answer(device):
    g = np.load(os.path.join(GOLDEN, "quantize_seed76.npz"))
    packed = quantize_kv(torch.from_numpy(g["x"]).to(device), KVQuantization("int8"))
    assert packed.values.dtype == torch.int8 and packed.scales.shape == (2, 3, 9, 1)
    np.testing.assert_array_equal(packed.values.cpu().numpy(), g["codes"])
    np.testing.assert_array_equal(packed.scales.cpu().numpy(), g["scales"])
    torch.testing.assert_close(packed.dequantize().cpu(),
                               torch.from_numpy(g["codes"].astype(np.float32) * g["scales"]),
                               atol=0, rtol=0)


def _edge_rows(dim, rng, fmt="int8"):
    """Rows that stress every branch: zero row, FLT_MIN clamp (denormal and tiny
    normal amax), exact half-way ties, +-127 clamp, x8 outliers, mixed magnitudes;
    for FP8 also rows whose scale is a power of two (amax = max * 2^e), so that
    midpoints between neighbouring FP8 values are exact ties and subnormal codes
    appear."""
    tiny = np.finfo(np.float32).tiny
    rows = [np.zeros(dim, np.float32)]
    if fmt != "int8":
        values = ref.fp8_values(fmt)[:128]
        finite = values[np.isfinite(values)]
        mids = ((finite[1:] + finite[:-1]) / 2).astype(np.float32)
        for e in (-20, 0, 5):
            for start in range(0, mids.size, dim - 1):
                r = np.zeros(dim, np.float32)
                r[0] = ref.FP8_MAXIMUM[fmt]
                chunk = mids[start : start + dim - 1]
                r[1 : 1 + chunk.size] = chunk * np.where(np.arange(chunk.size) % 2, -1, 1)
                rows.append((r * np.float32(2.0**e)).astype(np.float32))
    r = np.zeros(dim, np.float32)
    r[:3] = [1e-40, -7e-41, 3e-45]
    rows.append(r)
    r = np.zeros(dim, np.float32)
    r[:3] = [1e-37, -2e-38, 5e-39]
    rows.append(r)
    r = np.zeros(dim, np.float32)
    r[:2] = [127 * tiny, -tiny]
    rows.append(r)
    ties = np.array([127, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -125.5, 3.5], np.float32)
    for e in (-10, 0, 7):
        r = np.zeros(dim, np.float32)
        n = min(dim, ties.size)
        r[:n] = ties[:n] * np.float32(2.0**e)
        rows.append(r)
    rows.append(rng.standard_normal(dim).astype(np.float32) * 8)
    # mixed magnitudes that stay finite in fp16 (max 65504)
    rows.append((rng.standard_normal(dim) * 10.0 ** rng.uniform(-6, 4, dim)).astype(np.float32))
    rows.append(np.full(dim, -3.25, np.float32))
    for _ in range(20):
        rows.append(rng.standard_normal(dim).astype(np.float32))
    return np.stack(rows)


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("dim", [64, 128, 32, 200])
def test_append_edge_rows_bit_exact(device, dtype, dim, fmt):
    rng = np.random.default_rng(dim)
    rows = _edge_rows(dim, rng, fmt)
    if dtype == torch.float16:  # FP8 E5M2 ties reach 57344 * 2^5: keep fp16-finite rows
        rows = rows[np.abs(rows).max(1) < 60000]
    heads = 2
    tokens = rows.shape[0] // heads
    src = rows[: tokens * heads].reshape(tokens, heads, dim)
    k = torch.from_numpy(src).to(dtype)
    v = torch.from_numpy(src[::-1].copy()).to(dtype)
    # the oracle sees exactly the values the kernel reads (after the dtype cast)
    kf, vf = k.float().numpy(), v.float().numpy()
    if dtype == torch.float16:
        kf, vf = k.numpy(), v.numpy()
    blocks = (tokens + 15) // 16 + 3
    slots = np.random.default_rng(1).permutation(blocks * 16)[:tokens].astype(np.int64)
    cache = _cache(device, blocks, heads, dim, fmt=fmt)
    cache.append(0, k.to(device), v.to(device), torch.from_numpy(slots).to(device), check=True)
    shape = (blocks, heads, 16, dim)
    want = [np.zeros(shape, np.int8), np.ones(shape[:3], np.float32),
            np.zeros(shape, np.int8), np.ones(shape[:3], np.float32)]
    ref.quantize_append(kf, vf, slots, want[0], want[1], want[2], want[3], 16, fmt)
    got = arena_numpy(cache)
    for name, a, b in zip(("k_codes", "k_scales", "v_codes", "v_scales"), got, want):
        if a.dtype == np.float32:
            assert (a.view(np.uint32) == b.view(np.uint32)).all(), name
        else:
            np.testing.assert_array_equal(a, b, err_msg=name)


def test_config2_step_append_bit_exact(device):
    """The config2 workload's step: 64 new bf16 tokens (one per sequence) appended via
    slot_mapping into a shuffled pool, with strided (non-contiguous) K/V rows."""
    w = wl.config2()
    cache = _cache(device, w.num_blocks, w.num_kv_heads, w.head_dim)
    gen = torch.Generator(device=device)
    gen.manual_seed(22)
    qkv = torch.randn((64, 3, 8, 128), generator=gen, device=device).to(torch.bfloat16)
    k, v = qkv[:, 1], qkv[:, 2]  # strided views of a fused projection
    slots = np.array([wl.token_slots(w, r)[-1] for r in range(64)], np.int64)
    cache.append(0, k, v, torch.from_numpy(slots).to(device), check=True)
    shape = (w.num_blocks, 8, 16, 128)
    want = [np.zeros(shape, np.int8), np.ones(shape[:3], np.float32),
            np.zeros(shape, np.int8), np.ones(shape[:3], np.float32)]
    ref.quantize_append(k.float().cpu().numpy(), v.float().cpu().numpy(), slots, *want, 16)
    for a, b in zip(arena_numpy(cache), want):
        np.testing.assert_array_equal(a, b)


def test_nonfinite_input_mutates_no_slot(device):
    cache = _cache(device, 4, 2, 64)
    k = torch.randn(5, 2, 64, device=device)
    v = torch.randn(5, 2, 64, device=device)
    v[3, 1, 17] = float("inf")
    before = cache.codes.clone(), cache.scales.clone()
    with pytest.raises(ValueError, match="finite"):
        cache.append(0, k, v, torch.arange(5, device=device), check=True)
    assert torch.equal(cache.codes, before[0]) and torch.equal(cache.scales, before[1])
    # the flag was acknowledged: a clean append now lands
    cache.append(0, k, torch.randn_like(v), torch.arange(5, device=device), check=True)
    assert not torch.equal(cache.codes, before[0])
    with pytest.raises(ValueError):
        quantize_kv(torch.tensor([[[float("nan"), 1.0]]], device=device), KVQuantization())


def test_negative_slots_skip_and_bad_slots_flag(device):
    cache = _cache(device, 2, 1, 64)
    k = torch.randn(3, 1, 64, device=device)
    cache.append(0, k, k, torch.tensor([-1, 5, -1], device=device), check=True)
    codes = cache.codes[:, 0, 0, 0].cpu()
    assert (codes[0, 5] != 0).any() and (codes[0, [0, 1, 2, 3, 4, 6]] == 0).all()
    assert (codes[1] == 0).all()
    with pytest.raises(ValueError, match="outside"):
        cache.append(0, k, k, torch.tensor([0, 1, 32], device=device), check=True)


def test_quantize_kv_passthrough_and_unsupported(device):
    ints = torch.ones(1, 1, 2, 4, dtype=torch.int32, device=device)
    assert quantize_kv(ints, KVQuantization()) is ints
    x = torch.randn(1, 1, 2, 4, device=device)
    assert quantize_kv(x, None) is x
    with pytest.raises(UnsupportedAttentionBackend):
        quantize_kv(x.cpu(), KVQuantization())
    with pytest.raises(ValueError):
        quantize_kv(torch.randn(4, 4, device=device), KVQuantization())


@pytest.mark.parametrize("fmt", ["fp8_e4m3fn", "fp8_e5m2"])
def test_quantize_kv_api_fp8_matches_oracle(device, fmt):
    """quantize_kv with an FP8 profile returns codes in the profile's float8 dtype,
    bit-exact with the oracle (itself pinned to torch's float32 -> float8 cast)."""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((2, 3, 9, 64)) * np.exp(rng.uniform(-8, 8, (2, 3, 9, 1))))
    x = x.astype(np.float32)
    packed = quantize_kv(torch.from_numpy(x).to(device), KVQuantization(fmt))
    want = ref.quantize_kv_fp8(x, fmt)
    assert packed.values.dtype == KVQuantization(fmt).dtype
    np.testing.assert_array_equal(packed.values.cpu().view(torch.uint8).numpy(), want.values)
    np.testing.assert_array_equal(packed.scales.cpu().numpy(), want.scales)
    np.testing.assert_array_equal(packed.dequantize().cpu().numpy(), want.dequantize())


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("dim", [64, 128, 96])
def test_reserved_append_matches_guarded_append(device, fmt, dtype, dim):
    """The one-launch append for reserved slots writes the same codes and scales as
    the two-launch append, bit for bit (vector and strided row loads)."""
    rng = np.random.default_rng(dim)
    x = np.concatenate([_edge_rows(dim, rng, fmt), rng.standard_normal((40, dim)) * 3])
    x = x[: (len(x) // 4) * 4].astype(np.float32).reshape(-1, 2, 2, dim)  # [T, K|V, Hkv, D]
    # edge rows beyond the input dtype's range become zeros, not infinities
    k, v = (torch.from_numpy(np.ascontiguousarray(x[:, i])).to(device).to(dtype)
            .nan_to_num(0.0, 0.0, 0.0) for i in (0, 1))
    slots = torch.from_numpy(rng.permutation(64)[: k.shape[0]].astype(np.int64)).to(device)
    slots[1] = -1  # a padding token keeps its slot
    guarded, reserved = _cache(device, 4, 2, dim, fmt=fmt), _cache(device, 4, 2, dim, fmt=fmt)
    guarded.append(0, k, v, slots, check=True)
    reserved.append(0, k, v, slots, check=True, reserved=True)
    assert torch.equal(guarded.codes, reserved.codes)
    assert torch.equal(guarded.scales.view(torch.int32), reserved.scales.view(torch.int32))


def test_reserved_append_leaves_nonfinite_rows_unwritten(device):
    cache = _cache(device, 4, 2, 64)
    k = torch.randn(5, 2, 64, device=device)
    v = torch.randn(5, 2, 64, device=device)
    v[3, 1, 17] = float("nan")
    k[0, 0, 3] = float("-inf")
    before = cache.codes.clone(), cache.scales.clone()
    with pytest.raises(ValueError, match="finite"):
        cache.append(0, k, v, torch.arange(5, device=device), check=True, reserved=True)
    # the non-finite rows' slots: V of token 3 head 1, K of token 0 head 0 (block 0)
    assert torch.equal(cache.codes[0, 0, 1, 1, 3], before[0][0, 0, 1, 1, 3])
    assert torch.equal(cache.codes[0, 0, 0, 0, 0], before[0][0, 0, 0, 0, 0])
    assert cache.scales[0, 0, 1, 1, 3] == before[1][0, 0, 1, 1, 3]
    # the flag was acknowledged: a clean append now lands everywhere
    cache.append(0, k.nan_to_num(0.0, 0.0, 0.0), v.nan_to_num(0.0), torch.arange(5, device=device),
                 check=True, reserved=True)
    assert (cache.codes[0, 0, :, :, :5] != 0).any(-1).all()
