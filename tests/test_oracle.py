"""Pin the numpy oracle (oracle/reference_cpu.py) before it is trusted as the checker.

Each check is chosen so that a plausible restatement mistake fails it: the
reference's own known-answer test, exact half-way ties (half-away-from-zero
rounding), reciprocal-multiply instead of true division, a wrong maximum
constant, missing zero-row / FLT_MIN branches, a dropped online-softmax rescale,
a wrong GQA head mapping, a transposed operand, broken partition merging.
"""

from fractions import Fraction
import os

import numpy as np
import pytest

from oracle import dense
from oracle import reference_cpu as ref

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
F32 = np.float32


def f32_exact_div(a, b):
    """Correctly rounded float32 quotient computed from exact rationals."""
    q = Fraction(float(a)) / Fraction(float(b))
    d = float(q)  # nearest double
    f = F32(d)
    # guard against double rounding: the double must not sit on a float32 midpoint
    lo, hi = np.nextafter(f, F32(-np.inf)), np.nextafter(f, F32(np.inf))
    for n in (lo, hi):
        assert Fraction(float(f)) + Fraction(float(n)) != 2 * Fraction(d)
    return f


# ---------------------------------------------------------------------------------------
# quantize_kv (kv_quantization.py:71-94)
# ---------------------------------------------------------------------------------------


def test_quantize_reference_known_answer_seed76():
    """tests/unit/test_hot_kv.py:22-42: same input, the test's independent scalar
    oracle, atol=0, dequant exact, error bound <= 0.5001 * scale."""
    g = np.load(os.path.join(GOLDEN, "quantize_seed76.npz"))
    x = g["x"]
    assert x.shape == (2, 3, 9, 32) and x[0, 0, 0].max() == 0 and x[0, 0, 0].min() == 0
    q = ref.quantize_kv_int8(x)
    assert q.values.dtype == np.int8 and q.scales.dtype == np.float32
    np.testing.assert_array_equal(q.scales, g["scales"])
    np.testing.assert_array_equal(q.values, g["codes"])
    deq = q.dequantize()
    np.testing.assert_array_equal(deq, g["codes"].astype(F32) * g["scales"])
    assert (np.abs(x - deq) <= q.scales * 0.5001).all()
    assert q.scales[0, 0, 0, 0] == 1.0  # zero row -> scale 1


def test_quantize_seed76_fixture_matches_torch_generator():
    torch = pytest.importorskip("torch")
    torch.manual_seed(76)
    x = torch.randn(2, 3, 9, 32)
    x[0, 0, 0] = 0
    g = np.load(os.path.join(GOLDEN, "quantize_seed76.npz"))
    np.testing.assert_array_equal(x.numpy(), g["x"])


@pytest.mark.parametrize("exponent", [-20, -3, 0, 5, 40])
def test_quantize_exact_ties_round_half_to_even(exponent):
    """amax = 127 * 2^e gives scale = 2^e exactly, so x/scale hits n + 0.5 exactly."""
    unit = F32(2.0**exponent)
    row = np.array([127, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -125.5, 3.5], F32) * unit
    q = ref.quantize_kv_int8(row.reshape(1, 1, -1))
    assert q.scales.item() == unit
    # half-to-even; half-away-from-zero would give 1, 2, 3, -1, -2, -3, 127, -126, 4
    np.testing.assert_array_equal(q.values.ravel(), [127, 0, 2, 2, 0, -2, -2, 126, -126, 4])


def test_quantize_zero_row_and_flt_min_clamp():
    tiny = np.finfo(F32).tiny
    rows = np.zeros((1, 4, 8), F32)
    rows[0, 1, :3] = [1e-40, -5e-41, 0]          # denormal amax -> scale clamped to FLT_MIN
    rows[0, 2, :3] = [1e-37, -3e-38, 2e-39]      # amax/127 < FLT_MIN as well
    rows[0, 3, :2] = [127 * tiny, tiny]           # amax/127 == FLT_MIN exactly, no clamp needed
    q = ref.quantize_kv_int8(rows)
    s = q.scales.ravel()
    assert s[0] == 1.0 and (q.values[0, 0] == 0).all()
    assert s[1] == tiny and s[2] == tiny and s[3] == tiny
    # codes from exact rationals: x / FLT_MIN
    for h in (1, 2):
        for d in range(3):
            want = np.rint(np.clip(f32_exact_div(rows[0, h, d], tiny), -127, 127))
            assert q.values[0, h, d] == want
    np.testing.assert_array_equal(q.values[0, 3, :2], [127, 1])


def test_quantize_uses_true_division_not_reciprocal():
    """Rows where x*(1/scale) and x/scale round to different codes: the oracle must
    follow IEEE true division (torch CPU `source / scales`, kv_quantization.py:91)."""
    rng = np.random.default_rng(7)
    found = 0
    for _ in range(4000):
        amax = F32(rng.uniform(0.5, 4.0))
        scale = F32(amax / F32(127))
        n = rng.integers(-126, 126)
        # x near (n + 0.5) * scale, scanned over neighbouring float32 values
        x0 = F32((n + 0.5) * float(scale))
        for x in (x0, np.nextafter(x0, F32(np.inf)), np.nextafter(x0, F32(-np.inf))):
            true_q = f32_exact_div(x, scale)
            recip_q = F32(x * F32(F32(1) / scale))
            if np.rint(true_q) == np.rint(recip_q):
                continue
            row = np.array([amax, x], F32).reshape(1, 1, 2)
            q = ref.quantize_kv_int8(row)
            assert q.scales.item() == f32_exact_div(amax, 127.0)
            assert q.values[0, 0, 1] == np.rint(true_q)
            found += 1
    assert found >= 3, "test did not exercise a reciprocal/true-division disagreement"


def test_quantize_scale_and_extreme_codes():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((3, 5, 40, 16)).astype(F32) * rng.uniform(1e-3, 1e3, (3, 5, 40, 1)).astype(F32)
    q = ref.quantize_kv_int8(x)
    amax = np.abs(x).max(-1)
    for idx in np.ndindex(amax.shape):
        assert q.scales[idx][0] == f32_exact_div(amax[idx], 127.0)
    # the absmax element maps to +-127 and nothing exceeds it (wrong maximum constant fails)
    assert (np.abs(q.values.astype(int)).max(-1) == 127).all()
    assert (np.abs(x - q.dequantize()) <= q.scales * 0.5001).all()


def test_quantize_input_validation():
    with pytest.raises(ValueError):
        ref.quantize_kv_int8(np.zeros((4, 8), F32))
    bad = np.zeros((1, 1, 2, 4), F32)
    bad[0, 0, 1, 2] = np.nan
    with pytest.raises(ValueError):
        ref.quantize_kv_int8(bad)
    with pytest.raises(ValueError):
        ref.quantize_kv_int8(np.zeros((1, 1, 2, 4), np.int32))


def test_quantize_float16_source_matches_float32_of_same_values():
    rng = np.random.default_rng(3)
    x16 = rng.standard_normal((2, 3, 7, 32)).astype(np.float16)
    a = ref.quantize_kv_int8(x16)
    b = ref.quantize_kv_int8(x16.astype(F32))
    np.testing.assert_array_equal(a.values, b.values)
    np.testing.assert_array_equal(a.scales, b.scales)


# ---------------------------------------------------------------------------------------
# online attention (online_attention.py:42-219) against the fp64 dense brute force
# ---------------------------------------------------------------------------------------


def _page_scan_inputs():
    """Geometry of tests/unit/test_inference_online_attention.py:34-59."""
    rng = np.random.default_rng(123)
    q = rng.standard_normal((2, 6, 13, 8))
    key = rng.standard_normal((2, 2, 31, 8))
    value = rng.standard_normal((2, 2, 31, 5))
    positions = np.broadcast_to(np.arange(18, 31), (2, 13)).copy()
    padding = np.ones((2, 31), bool)
    padding[0, 2::3] = False
    padding[1] = False
    query_padding = np.ones((2, 13), bool)
    query_padding[0, -1] = False
    bounds = [0, 3, 10, 14, 21, 31]
    blocks = [ref.AttentionBlock(key[..., a:b, :], value[..., a:b, :], a, padding[:, a:b])
              for a, b in zip(bounds, bounds[1:])]
    return q, key, value, positions, padding, query_padding, blocks


@pytest.mark.parametrize("window", [None, 1, 5, 17])
@pytest.mark.parametrize("causal", [True, False])
def test_online_attention_fp64_matches_dense(window, causal):
    q, key, value, positions, padding, qpad, blocks = _page_scan_inputs()
    kw = dict(query_positions=positions, causal=causal, window=window, query_padding=qpad,
              query_block_size=4, key_block_size=5)
    got = ref.online_attention(q, blocks, **kw)
    want = dense.dense_attention(q, key, value, positions, causal=causal, window=window,
                                 key_padding=padding, query_padding=qpad)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    # partition merge == whole; page order irrelevant; fully masked rows are zero
    left = ref.online_attention_statistics(q, blocks[:2], **kw)
    right = ref.online_attention_statistics(q, blocks[2:], **kw)
    np.testing.assert_allclose(ref.merge_softmax(left, right).output(), want, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(ref.online_attention(q, blocks[::-1], **kw), want, rtol=1e-12,
                               atol=1e-12)
    assert np.count_nonzero(got[1]) == 0 and np.count_nonzero(got[0, :, -1]) == 0


def test_merge_with_empty_partition_keeps_state():
    q, key, value, positions, padding, qpad, blocks = _page_scan_inputs()
    kw = dict(query_positions=positions, query_block_size=4, key_block_size=5)
    whole = ref.online_attention_statistics(q, blocks, **kw)
    empty = ref.SoftmaxState(np.full_like(whole.maximum, -np.inf), np.zeros_like(whole.mass),
                             np.zeros_like(whole.weighted))
    merged = ref.merge_softmax(empty, whole)
    np.testing.assert_array_equal(merged.output(), whole.output())


def test_quantized_tile_attention_matches_dense_dequantized():
    """tests/unit/test_hot_kv.py:78-109 geometry in fp32: 4q/2kv heads, 23 keys in
    pages of 4, window 12, qb=2, kb=3, Dv=24."""
    rng = np.random.default_rng(13)
    q = rng.standard_normal((1, 4, 5, 32)).astype(F32)
    k = rng.standard_normal((1, 2, 23, 32)).astype(F32)
    v = rng.standard_normal((1, 2, 23, 24)).astype(F32)
    pk, pv = ref.quantize_kv_int8(k), ref.quantize_kv_int8(v)
    pos = np.arange(18, 23)[None]
    want = dense.dense_attention(q, pk.dequantize(), pv.dequantize(), pos, window=12)
    blocks = [ref.AttentionBlock(pk.narrow(i, min(4, 23 - i)), pv.narrow(i, min(4, 23 - i)), i)
              for i in range(0, 23, 4)]
    got = ref.online_attention(q, blocks, query_positions=pos, window=12, query_block_size=2,
                               key_block_size=3)
    assert got.dtype == np.float32
    np.testing.assert_allclose(got, want, atol=5e-7, rtol=3e-5)


def test_closed_forms_single_key_equal_scores_and_zero_query():
    rng = np.random.default_rng(5)
    v = rng.standard_normal((1, 1, 6, 4))
    k = rng.standard_normal((1, 1, 6, 4))
    # one visible key: output is exactly that value row
    out = ref.online_attention(rng.standard_normal((1, 2, 1, 4)),
                               [ref.AttentionBlock(k, v, 0)],
                               query_positions=np.array([[0]]))
    np.testing.assert_allclose(out[0, :, 0], np.repeat(v[0, :, 0], 2, 0), rtol=0, atol=1e-15)
    # zero query: uniform weights -> plain mean of the visible values
    out = ref.online_attention(np.zeros((1, 1, 1, 4)),
                               [ref.AttentionBlock(k[..., :3, :], v[..., :3, :], 0),
                                ref.AttentionBlock(k[..., 3:, :], v[..., 3:, :], 3)],
                               query_positions=np.array([[5]]), key_block_size=2)
    np.testing.assert_allclose(out[0, 0, 0], v[0, 0].mean(0), rtol=1e-14, atol=1e-14)
    # identical keys: same as the mean even with a nonzero query
    kk = np.repeat(k[..., :1, :], 6, axis=2)
    out = ref.online_attention(rng.standard_normal((1, 1, 1, 4)), [ref.AttentionBlock(kk, v, 0)],
                               query_positions=np.array([[5]]), key_block_size=4)
    np.testing.assert_allclose(out[0, 0, 0], v[0, 0].mean(0), rtol=1e-13, atol=1e-13)


def test_gqa_head_mapping_is_h_div_g():
    """Query head h must read kv head h // G (online_attention.py:157-161); a modulo
    mapping would pair heads differently and fail."""
    rng = np.random.default_rng(9)
    q = rng.standard_normal((1, 4, 1, 8))
    k = rng.standard_normal((1, 2, 5, 8))
    v = rng.standard_normal((1, 2, 5, 8))
    got = ref.online_attention(q, [ref.AttentionBlock(k, v, 0)], query_positions=np.array([[4]]))
    for h in range(4):
        one = ref.online_attention(q[:, h : h + 1], [ref.AttentionBlock(k[:, h // 2 : h // 2 + 1],
                                                                        v[:, h // 2 : h // 2 + 1], 0)],
                                   query_positions=np.array([[4]]))
        np.testing.assert_allclose(got[:, h], one[:, 0], rtol=1e-14, atol=1e-14)


def test_overlap_and_nonfinite_rejected():
    k = np.ones((1, 1, 3, 2))
    blocks = [ref.AttentionBlock(k, k, 0), ref.AttentionBlock(k, k, 2)]
    with pytest.raises(ValueError, match="Overlapping"):
        ref.online_attention(np.ones((1, 1, 1, 2)), blocks, query_positions=np.array([[4]]))
    huge = np.full((1, 1, 2, 2), 1e308)
    with pytest.raises(ValueError, match="overflow"):
        ref.online_attention(huge[:, :, :1], [ref.AttentionBlock(huge, huge, 0)],
                             query_positions=np.array([[1]]))


# ---------------------------------------------------------------------------------------
# paged assembly (paged_attention.py:168-215) and the config-1 golden fixture
# ---------------------------------------------------------------------------------------


def _config1():
    return np.load(os.path.join(GOLDEN, "config1.npz"))


def test_config1_fixture_regenerates_bit_for_bit():
    import sys

    sys.path.insert(0, GOLDEN)
    import make_golden

    g = _config1()
    w, q, k, v, slots = make_golden.config1_inputs()
    for name, arr in (("q", q), ("k", k), ("v", v), ("slots", slots),
                      ("block_tables", w.block_tables), ("context_lens", w.context_lens)):
        np.testing.assert_array_equal(arr, g[name], err_msg=name)
    k_codes, k_scales, v_codes, v_scales, out = make_golden.config1_expected(w, q, k, v, slots)
    np.testing.assert_array_equal(k_codes, g["k_codes"])
    np.testing.assert_array_equal(v_scales, g["v_scales"])
    np.testing.assert_allclose(out, g["out"], rtol=1e-6, atol=1e-7)


def test_config1_paged_oracle_matches_dense_fp64():
    g = _config1()
    out = g["out"]
    cursor = 0
    for row, ctx in enumerate(g["context_lens"].tolist()):
        pages = g["block_tables"][row][np.arange(ctx) // 16]
        offs = np.arange(ctx) % 16
        kd = (g["k_codes"][pages, :, offs].astype(np.float64)
              * g["k_scales"][pages, :, offs][..., None].astype(np.float64))
        vd = (g["v_codes"][pages, :, offs].astype(np.float64)
              * g["v_scales"][pages, :, offs][..., None].astype(np.float64))
        want = dense.dense_attention(g["q"][row][None, :, None, :], kd.transpose(1, 0, 2)[None],
                                     vd.transpose(1, 0, 2)[None], np.array([[ctx - 1]]),
                                     scale=64 ** -0.5)
        np.testing.assert_allclose(out[row], want[0, :, 0], rtol=2e-5, atol=2e-6)
        # codes are the quantized sources written to the right slots
        src = g["k"][cursor : cursor + ctx]
        qk = ref.quantize_kv_int8(src.transpose(1, 0, 2)[None])
        np.testing.assert_array_equal(g["k_codes"][pages, :, offs], qk.values[0].transpose(1, 0, 2))
        cursor += ctx


def test_paged_oracle_invariant_to_physical_block_permutation():
    g = _config1()
    perm = np.random.default_rng(0).permutation(64)
    inverse = np.argsort(perm)
    args = [g[n][perm] for n in ("k_codes", "k_scales", "v_codes", "v_scales")]
    tables = inverse[g["block_tables"]].astype(np.int32)
    out = ref.paged_attention(g["q"], *args, tables, g["context_lens"], block_size=16,
                              scale=64 ** -0.5)
    np.testing.assert_array_equal(out, ref.paged_attention(
        g["q"], g["k_codes"], g["k_scales"], g["v_codes"], g["v_scales"], g["block_tables"],
        g["context_lens"], block_size=16, scale=64 ** -0.5))


def test_paged_oracle_step_without_query_tokens():
    """Rows that carry no query token this step produce no output rows; a step where
    no row does returns an empty [0, Hq, Dv] array."""
    g = _config1()
    n = len(g["context_lens"])
    out = ref.paged_attention(g["q"][:0], g["k_codes"], g["k_scales"], g["v_codes"],
                              g["v_scales"], g["block_tables"], g["context_lens"], block_size=16,
                              scale=64 ** -0.5, query_lens=[0] * n)
    assert out.shape == (0, g["q"].shape[1], g["v_codes"].shape[-1])
    one = [0] * n
    one[2] = 1
    out = ref.paged_attention(g["q"][2:3], g["k_codes"], g["k_scales"], g["v_codes"],
                              g["v_scales"], g["block_tables"], g["context_lens"], block_size=16,
                              scale=64 ** -0.5, query_lens=one)
    whole = ref.paged_attention(g["q"], g["k_codes"], g["k_scales"], g["v_codes"], g["v_scales"],
                                g["block_tables"], g["context_lens"], block_size=16,
                                scale=64 ** -0.5)
    np.testing.assert_array_equal(out, whole[2:3])


def test_runner_order_equivalence_chunk_block_vs_appended_page():
    """The reference attends old pages plus the quantized chunk as a separate block and
    appends afterwards (paged_attention.py:185-229); appending first and attending
    over pages gives the same keys, so results agree to fp32 rounding."""
    g = _config1()
    row, ctx = 2, int(g["context_lens"][2])
    pages = ref.page_blocks(g["k_codes"], g["k_scales"], g["v_codes"], g["v_scales"],
                            g["block_tables"][row], ctx, 16)
    q = g["q"][row][None, :, None, :]
    pos = np.array([[ctx - 1]])
    appended = ref.online_attention(q, pages, query_positions=pos, scale=64 ** -0.5)
    old = ref.page_blocks(g["k_codes"], g["k_scales"], g["v_codes"], g["v_scales"],
                          g["block_tables"][row], ctx - 1, 16)
    last = pages[-1].key.narrow(pages[-1].key.shape[-2] - 1, 1)
    lastv = pages[-1].value.narrow(pages[-1].value.shape[-2] - 1, 1)
    chunk = ref.AttentionBlock(last, lastv, ctx - 1)
    separate = ref.online_attention(q, old + [chunk], query_positions=pos, scale=64 ** -0.5)
    np.testing.assert_allclose(appended, separate, rtol=1e-5, atol=1e-6)


# ---- FP8 formats (KVQuantization("fp8_e4m3fn"/"fp8_e5m2"), kv_quantization.py:7-25, 71-94)
import torch  # noqa: E402  (CPU conversions: the library routine FP8 reduces to)

FP8 = {"fp8_e4m3fn": torch.float8_e4m3fn, "fp8_e5m2": torch.float8_e5m2}


@pytest.mark.parametrize("fmt", sorted(FP8))
def test_fp8_code_values_match_torch_for_all_256_codes(fmt):
    got = ref.fp8_values(fmt)
    want = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(FP8[fmt]).double().numpy()
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    keep = ~np.isnan(want)
    np.testing.assert_array_equal(got[keep], want[keep])
    assert ref.FP8_MAXIMUM[fmt] == torch.finfo(FP8[fmt]).max


@pytest.mark.parametrize("fmt", sorted(FP8))
def test_fp8_rounding_matches_torch_conversion(fmt):
    """Random magnitudes over the whole range, exact midpoints between neighbouring
    codes (ties to even), subnormal steps, +-0, the maximum and the values just below
    it: codes equal torch's float32 -> float8 bits."""
    rng = np.random.default_rng(9)
    top = ref.FP8_MAXIMUM[fmt]
    values = ref.fp8_values(fmt)[:128]
    finite = values[np.isfinite(values)]
    mids = (finite[1:] + finite[:-1]) / 2  # exact in float32 for these short mantissas
    probe = np.concatenate([
        rng.uniform(-top, top, 20000),
        np.exp(rng.uniform(np.log(1e-12), np.log(top), 20000)) * rng.choice([-1, 1], 20000),
        mids, -mids, finite, -finite,
        np.nextafter(mids.astype(np.float32), np.float32(0)),
        np.nextafter(mids.astype(np.float32), np.float32(np.inf)),
        [0.0, -0.0, top, -top, np.nextafter(np.float32(top), np.float32(0))],
    ]).astype(np.float32)
    probe = np.clip(probe, -top, top).astype(np.float32)
    want = torch.from_numpy(probe).to(FP8[fmt]).view(torch.uint8).numpy()
    np.testing.assert_array_equal(ref.fp8_round(probe, fmt), want)
    # a plausible mistake: ties away from zero instead of to even
    assert (ref.fp8_round(mids.astype(np.float32), fmt) % 2 == 0).all()


@pytest.mark.parametrize("fmt", sorted(FP8))
def test_quantize_kv_fp8_matches_reference_torch_expression(fmt):
    """The reference's quantize_kv body (amax / finfo.max, FLT_MIN clamp, clamp,
    .to(float8)) evaluated by torch on the CPU, on rows of very different ranges,
    a zero row and fp16 input: identical codes and scales."""
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((2, 3, 17, 64)) * np.exp(rng.uniform(-12, 12, (2, 3, 17, 1))))
    x = x.astype(np.float32)
    x[1, 2, 5] = 0.0
    for arr in (x, (x / np.abs(x).max() * 30000).astype(np.float16)):
        got = ref.quantize_kv_fp8(arr, fmt)
        source = torch.from_numpy(arr).float()
        maximum = source.abs().amax(-1, keepdim=True)
        top = torch.finfo(FP8[fmt]).max
        scales = torch.where(maximum == 0, torch.ones_like(maximum),
                             (maximum / top).clamp_min(torch.finfo(torch.float32).tiny))
        codes = (source / scales).clamp(-top, top).to(FP8[fmt])
        np.testing.assert_array_equal(got.scales, scales.numpy())
        np.testing.assert_array_equal(got.values, codes.view(torch.uint8).numpy())
        np.testing.assert_array_equal(got.dequantize(), (codes.float() * scales).numpy())
