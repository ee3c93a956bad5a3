// Shared device helpers for the gfx950 INT8 paged-KV kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <cfloat>
#include <stdint.h>

#include "aster_kv.h"

namespace astr {

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

// Record a message for astr_last_error() and return `code`.
int fail(int code, const char* fmt, ...);
int hip_fail(hipError_t err, const char* what);

// A roctx range over one C-ABI call on the host (argument checks and launches), named
// after the entry point: `rocprofv3 --marker-trace` shows each call beside the
// kernels it enqueued. Without a profiler attached the push and pop are no-ops.
struct CallRange {
  explicit CallRange(const char* name);
  ~CallRange();
  CallRange(const CallRange&) = delete;
  CallRange& operator=(const CallRange&) = delete;
};

// ---- element conversion -----------------------------------------------------

struct bf16_t {
  uint16_t bits;
};

template <typename T>
__device__ __forceinline__ float to_float(T v);
template <>
__device__ __forceinline__ float to_float<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_float<_Float16>(_Float16 v) { return (float)v; }
template <>
__device__ __forceinline__ float to_float<bf16_t>(bf16_t v) {
  return __builtin_bit_cast(float, (uint32_t)v.bits << 16);
}

template <typename T>
__device__ __forceinline__ T from_float(float v);
template <>
__device__ __forceinline__ float from_float<float>(float v) { return v; }
template <>
__device__ __forceinline__ _Float16 from_float<_Float16>(float v) { return (_Float16)v; }
template <>
__device__ __forceinline__ bf16_t from_float<bf16_t>(float v) {
  // round-to-nearest-even fp32 -> bf16, NaN stays NaN (v_cvt_pk_bf16_f32)
  return bf16_t{__builtin_bit_cast(uint16_t, (__bf16)v)};
}

// Two values rounded to nearest even and packed in one word, a in the low half
// (one v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32).
typedef float f32x2_t __attribute__((ext_vector_type(2)));
template <typename T>
__device__ __forceinline__ uint32_t pack2(float a, float b);
template <>
__device__ __forceinline__ uint32_t pack2<bf16_t>(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}
template <>
__device__ __forceinline__ uint32_t pack2<_Float16>(float a, float b) {
  typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, f16x2_t));
}

// ---- cross-lane reductions ----------------------------------------------------
// DPP control words (GCN/CDNA encoding).
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7-i inside each 8-lane half row
constexpr int kDppMirror = 0x140;      // lane i <-> 15-i inside each 16-lane row
constexpr int kDppRor8 = 0x128;        // lane i <- (i+8)%16 inside each row

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of N consecutive lanes (N in 1,2,4,8,16); every lane
// of the group receives the group total.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (N >= 2) x += dpp<kDppXor1>(x);
  if constexpr (N >= 4) x += dpp<kDppXor2>(x);
  if constexpr (N >= 8) x += dpp<kDppHalfMirror>(x);
  if constexpr (N >= 16) x += dpp<kDppMirror>(x);
  return x;
}

__device__ __forceinline__ float shfl_xor(float x, int mask) { return __shfl_xor(x, mask, kWave); }

// Reduce over lanes whose index differs only in bits >= log2(STRIDE): every
// lane receives the total over its residue class (lane % STRIDE).
template <int STRIDE>
__device__ __forceinline__ float strided_sum(float x) {
  if constexpr (STRIDE <= 8) x += dpp<kDppRor8>(x);
  if constexpr (STRIDE <= 16) x += shfl_xor(x, 16);
  x += shfl_xor(x, 32);
  if constexpr (STRIDE <= 4) x += shfl_xor(x, 4);
  return x;
}

template <int STRIDE>
__device__ __forceinline__ float strided_max(float x) {
  if constexpr (STRIDE <= 8) x = fmaxf(x, dpp<kDppRor8>(x));
  if constexpr (STRIDE <= 16) x = fmaxf(x, shfl_xor(x, 16));
  x = fmaxf(x, shfl_xor(x, 32));
  if constexpr (STRIDE <= 4) x = fmaxf(x, shfl_xor(x, 4));
  return x;
}

__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp<kDppXor1>(x));
  x = fmaxf(x, dpp<kDppXor2>(x));
  x = fmaxf(x, dpp<kDppHalfMirror>(x));
  x = fmaxf(x, dpp<kDppMirror>(x));
  x = fmaxf(x, shfl_xor(x, 16));
  x = fmaxf(x, shfl_xor(x, 32));
  return x;
}

// Sum over the 64 lanes (every lane gets it): after the xor-1/xor-2 butterflies a
// lane holds its quad's sum, and each mirror step adds the mirrored (disjoint)
// group of the same size.
__device__ __forceinline__ float wave_sum(float x) {
  x += dpp<kDppXor1>(x);
  x += dpp<kDppXor2>(x);
  x += dpp<kDppHalfMirror>(x);
  x += dpp<kDppMirror>(x);
  x += shfl_xor(x, 16);
  x += shfl_xor(x, 32);
  return x;
}

// Code formats (astr_kv_format) as template arguments.
constexpr int kInt8 = ASTR_KV_INT8;
constexpr int kE4M3 = ASTR_KV_FP8_E4M3FN;
constexpr int kE5M2 = ASTR_KV_FP8_E5M2;

// Largest code magnitude of a format (KVQuantization.maximum, kv_quantization.py:23-25).
template <int KF>
__device__ __forceinline__ constexpr float format_max() {
  return KF == kInt8 ? 127.f : KF == kE4M3 ? 448.f : 57344.f;
}

// Finite c with |c| <= format_max -> FP8 bits, round to nearest even. With M mantissa
// bits and exponent bias B: below the smallest normal 2^(1-B) the value counts
// subnormal steps of 2^(1-B-M), rint(|c| * 2^(B-1+M)) in 0..2^M (scaling by a power of
// two is exact; 2^M is the smallest normal's code); above it the fp32 mantissa is
// rounded to M bits at bit 23-M (half to even, a carry steps the exponent) and the
// exponent rebiased from 127 to B. The sign is kept (-0 for a negative underflow).
template <int KF>
__device__ __forceinline__ uint8_t fp8_round(float c) {
  constexpr int M = KF == kE4M3 ? 3 : 2;
  constexpr int B = KF == kE4M3 ? 7 : 15;
  const uint32_t bits = __builtin_bit_cast(uint32_t, c);
  const uint32_t sign = (bits >> 24) & 0x80u;
  const uint32_t mag = bits & 0x7fffffffu;
  uint32_t code;
  if (mag < ((uint32_t)(128 - B) << 23)) {
    code = (uint32_t)__builtin_rintf(__builtin_bit_cast(float, mag) * (float)(1 << (B - 1 + M)));
  } else {
    const uint32_t r = mag + ((1u << (22 - M)) - 1u) + ((mag >> (23 - M)) & 1u);
    code = (r >> (23 - M)) - ((uint32_t)(127 - B) << M);
  }
  return (uint8_t)(code | sign);
}
// The row's scale from its largest magnitude (kv_quantization.py:86-90): true
// division, then the FLT_MIN clamp; an all-zero row gets scale 1.
template <int KF>
__device__ __forceinline__ float quant_scale(float amax) {
  return amax == 0.f ? 1.f : fmaxf(amax / format_max<KF>(), FLT_MIN);
}

// One code (kv_quantization.py:91-94): divide by the scale, clamp to the format's
// range, round half to even (int8) or to the nearest-even FP8 value; as a byte.
template <int KF>
__device__ __forceinline__ int8_t quant_code(float x, float scale) {
  constexpr float kMax = format_max<KF>();
  const float n = fminf(fmaxf(x / scale, -kMax), kMax);
  if constexpr (KF == kInt8) return (int8_t)__builtin_rintf(n);
  else return (int8_t)fp8_round<KF>(n);
}

// The f16 conversions below give a code's value times 2^-8 for E4M3FN (its bits
// land one exponent step of 8 apart from f16's) and the value itself otherwise;
// code_scale undoes that (exactly: a power of two) where the scales are applied.
template <int KF>
__device__ __forceinline__ constexpr float code_scale() {
  return KF == kE4M3 ? 256.f : 1.f;
}

// PV weights and V operands are rounded to f16 after the V scale is applied, so the
// scale enters times v_weight_scale: for E4M3FN that undoes its codes' 2^-8; E5M2's
// scales (amax / 57344) lie below f16's normal range for |V| up to ~3.5, and 2^8
// lifts them into it. Where the E5M2 codes enter at their own value (the decode
// kernels) the softmax normaliser carries the same 2^8 (norm_scale), which cancels
// in acc / l; the prefill kernel takes E5M2 codes times 2^-8 instead (exact in f16).
template <int KF>
__device__ __forceinline__ constexpr float v_weight_scale() {
  return KF == kInt8 ? 1.f : 256.f;
}
template <int KF>
__device__ __forceinline__ constexpr float norm_scale() {
  return KF == kE5M2 ? 256.f : 1.f;
}

// FP8 codes placed in the high byte of each f16 half (low bytes zero) -> the f16
// pair: E5M2 is the top byte of the f16 with the same value; E4M3FN keeps its
// sign and shifts |code| right by one bit into f16's exponent/mantissa fields,
// which is its value times 2^-8 (subnormals included).
template <int KF>
__device__ __forceinline__ uint32_t fp8_hi_bytes_to_f16(uint32_t h) {
  if constexpr (KF == kE5M2) return h;
  else return ((h >> 1) & 0x3f803f80u) | (h & 0x80008000u);
}

// Code byte `b` of a packed dword, as float (exact; times 2^-8 for E4M3FN).
template <int KF>
__device__ __forceinline__ float code_to_f(uint32_t w, int b) {
  if constexpr (KF == kInt8) {
    return (float)(int8_t)(w >> (8 * b));
  } else {
    const uint32_t h = fp8_hi_bytes_to_f16<KF>(((w >> (8 * b)) & 0xffu) << 8);
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  }
}

// int8 byte `b` of a packed dword, as float (exact).
__device__ __forceinline__ float i8_to_f(uint32_t w, int b) { return code_to_f<kInt8>(w, b); }

}  // namespace astr
