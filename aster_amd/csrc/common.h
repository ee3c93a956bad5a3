// Shared device helpers for the gfx950 INT8 paged-KV kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "aster_kv.h"

namespace astr {

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

// Record a message for astr_last_error() and return `code`.
int fail(int code, const char* fmt, ...);
int hip_fail(hipError_t err, const char* what);

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
  // round-to-nearest-even fp32 -> bf16 (NaN kept quiet)
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return bf16_t{(uint16_t)((u >> 16) | 0x40u)};
  u += 0x7fffu + ((u >> 16) & 1u);
  return bf16_t{(uint16_t)(u >> 16)};
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

// int8 byte `b` of a packed dword, as float (exact).
__device__ __forceinline__ float i8_to_f(uint32_t w, int b) {
  return (float)(int8_t)(w >> (8 * b));
}

}  // namespace astr
