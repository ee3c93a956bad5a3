// Fused quantize-and-append of new K/V token rows into the paged arena (INT8, FP8
// E4M3FN or FP8 E5M2 codes).
//
// Arithmetic follows quantize_kv (src/aster/optimization/kv_quantization.py:82-94)
// bit for bit: fp32 source, amax over the row, scale = amax==0 ? 1 :
// max(amax/M, FLT_MIN) with an IEEE-correct division (M = 127, 448 or 57344),
// c = clamp(x/scale, -M, M) again with IEEE division (never x*(1/scale)); int8
// codes are rint(c) (half to even, v_rndne), FP8 codes c rounded to nearest even
// in the format (the float32 -> float8 conversion of .to(dtype), :94). The library
// is built with -fhip-fp32-correctly-rounded-divide-sqrt and without denormal
// flushing.
//
// Two launches per call: a finiteness scan that sets ASTR_FLAG_NONFINITE_INPUT,
// then the quantize/scatter kernel that does nothing when that bit is set, so a
// bad suffix mutates no slot (kv_quantization.py:77-81, state.py:292 runs the
// check before any copy). For slots the caller has reserved and rolls back when
// the flag is raised (the runner's step), one launch: the quantize/scatter kernel
// checks its own row and leaves a non-finite row unwritten.
#include <cfloat>

#include "common.h"

namespace astr {
namespace {

constexpr int kRowsPerBlock = 4;  // one wave per (token, head, K|V) row

constexpr int kMaxPerLane = 8;    // head_dim <= 512

struct AppendArgs {
  const void* key;
  const void* value;
  int64_t key_token_stride, key_head_stride, value_token_stride, value_head_stride;
  int64_t num_tokens;
  const int64_t* slot_mapping;
  astr_paged_kv cache;
  int32_t* err_flag;
};

// Row (token t, head h, K or V) handled by this wave; false past the last row.
struct RowRef {
  int t, h;
  bool is_v;
};

__device__ __forceinline__ bool row_of(const AppendArgs& a, RowRef& rr) {
  const int heads = a.cache.num_kv_heads;
  const int rows = (int)a.num_tokens * heads;  // host checks rows * 2 < 2^31
  const int row = blockIdx.x * kRowsPerBlock + (int)(threadIdx.x >> 6);
  if (row >= (a.value ? 2 : 1) * rows) return false;
  rr.is_v = row >= rows;
  const int r = rr.is_v ? row - rows : row;
  rr.t = r / heads;
  rr.h = r - rr.t * heads;
  return true;
}

template <typename T>
__device__ __forceinline__ const T* row_src(const AppendArgs& a, const RowRef& rr) {
  return static_cast<const T*>(rr.is_v ? a.value : a.key) +
         rr.t * (rr.is_v ? a.value_token_stride : a.key_token_stride) +
         rr.h * (rr.is_v ? a.value_head_stride : a.key_head_stride);
}

// Load the row into registers: VEC consecutive elements per lane when
// head_dim == 64*VEC (one vector load), otherwise a strided fallback whose
// loads are clamped in bounds so they all issue before the first use.
template <typename T, int VEC>
__device__ __forceinline__ void load_row(const T* src, int D, int lane, float (&x)[kMaxPerLane]) {
  if constexpr (VEC > 0) {
    struct alignas(sizeof(T) * VEC) Pack {
      T e[VEC];
    };
    const Pack w = *reinterpret_cast<const Pack*>(src + lane * VEC);
#pragma unroll
    for (int i = 0; i < VEC; ++i) x[i] = to_float<T>(w.e[i]);
  } else {
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
      const int d = lane + i * kWave;
      const float v = to_float<T>(src[d < D ? d : D - 1]);
      x[i] = d < D ? v : 0.f;
    }
  }
}

template <typename T, int VEC>
__global__ __launch_bounds__(256) void finite_scan_kernel(AppendArgs a) {
  RowRef rr;
  if (!row_of(a, rr)) return;
  const int lane = threadIdx.x & 63;
  float x[kMaxPerLane];
  load_row<T, VEC>(row_src<T>(a, rr), a.cache.head_dim, lane, x);
  bool bad = false;
#pragma unroll
  for (int i = 0; i < (VEC > 0 ? VEC : kMaxPerLane); ++i) bad |= !__builtin_isfinite(x[i]);
  if (__ballot(bad) != 0 && lane == 0) atomicOr(a.err_flag, ASTR_FLAG_NONFINITE_INPUT);
}

template <typename T, int VEC, int KF, bool kOwnCheck>
__global__ __launch_bounds__(256) void quantize_append_kernel(AppendArgs a) {
  // All-or-nothing: the finite scan of this call (or an unacknowledged earlier
  // one) flagged the input, so leave every slot untouched. The flag, slot and
  // row loads are independent and issue together. kOwnCheck (reserved slots, no
  // scan launch): the row's own check keeps a non-finite row out of its slot.
  RowRef rr;
  if (!row_of(a, rr)) return;
  const int lane = threadIdx.x & 63;
  const int flag = __atomic_load_n(a.err_flag, __ATOMIC_RELAXED);
  const int64_t slot = a.slot_mapping[rr.t];
  const int D = a.cache.head_dim;
  float x[kMaxPerLane];
  load_row<T, VEC>(row_src<T>(a, rr), D, lane, x);
  constexpr int N = VEC > 0 ? VEC : kMaxPerLane;
  if constexpr (kOwnCheck) {
    bool bad = false;
#pragma unroll
    for (int i = 0; i < N; ++i) bad |= !__builtin_isfinite(x[i]);
    if (__ballot(bad) != 0) {
      if (lane == 0) atomicOr(a.err_flag, ASTR_FLAG_NONFINITE_INPUT);
      return;
    }
  }
  if (flag & ASTR_FLAG_NONFINITE_INPUT) return;
  if (slot < 0) return;  // padding token: no slot
  const int64_t block = slot / a.cache.block_size, offset = slot - block * a.cache.block_size;
  if (block >= a.cache.num_blocks) {
    if (lane == 0) atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
    return;
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < N; ++i) amax = fmaxf(amax, fabsf(x[i]));
  amax = wave_max(amax);
  const float scale = quant_scale<KF>(amax);
  int8_t* codes = (rr.is_v ? a.cache.v_codes : a.cache.k_codes) +
                  block * a.cache.code_block_stride + rr.h * a.cache.code_head_stride + offset * D;
  int8_t q[N];
#pragma unroll
  for (int i = 0; i < N; ++i) q[i] = quant_code<KF>(x[i], scale);
  if constexpr (VEC > 0) {
    struct alignas(VEC) Pack {
      int8_t e[VEC];
    };
    Pack w;
#pragma unroll
    for (int i = 0; i < VEC; ++i) w.e[i] = q[i];
    *reinterpret_cast<Pack*>(codes + lane * VEC) = w;
  } else {
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
      const int d = lane + i * kWave;
      if (d < D) codes[d] = q[i];
    }
  }
  if (lane == 0) {
    float* scales = (rr.is_v ? a.cache.v_scales : a.cache.k_scales) +
                    block * a.cache.scale_block_stride + rr.h * a.cache.scale_head_stride + offset;
    *scales = scale;
  }
}

template <typename T, int VEC, bool kOwnCheck>
void launch_quantize(const AppendArgs& a, uint32_t blocks, hipStream_t stream) {
  switch (a.cache.code_format) {
    case kInt8:
      hipLaunchKernelGGL((quantize_append_kernel<T, VEC, kInt8, kOwnCheck>), dim3(blocks),
                         dim3(256), 0, stream, a);
      break;
    case kE4M3:
      hipLaunchKernelGGL((quantize_append_kernel<T, VEC, kE4M3, kOwnCheck>), dim3(blocks),
                         dim3(256), 0, stream, a);
      break;
    default:
      hipLaunchKernelGGL((quantize_append_kernel<T, VEC, kE5M2, kOwnCheck>), dim3(blocks),
                         dim3(256), 0, stream, a);
      break;
  }
}

// reserved: the caller rolls the slots back on a flagged call, so no scan launch
template <typename T, int VEC>
int launch_append(const AppendArgs& a, bool reserved, hipStream_t stream) {
  const int64_t rows = (a.value ? 2 : 1) * a.num_tokens * a.cache.num_kv_heads;
  const uint32_t blocks = (uint32_t)((rows + kRowsPerBlock - 1) / kRowsPerBlock);
  if (reserved) {
    launch_quantize<T, VEC, true>(a, blocks, stream);
  } else {
    hipLaunchKernelGGL((finite_scan_kernel<T, VEC>), dim3(blocks), dim3(256), 0, stream, a);
    launch_quantize<T, VEC, false>(a, blocks, stream);
  }
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "quantize_append launch");
}

template <typename T>
int launch_append_dim(const AppendArgs& a, bool reserved, hipStream_t stream) {
  const int D = a.cache.head_dim;
  // The vector path needs every row start aligned to a whole vector.
  const int64_t vec = D >= 64 ? D / 64 : 1;
  auto aligned = [&](const void* p, int64_t tok, int64_t head) {
    return p == nullptr || (reinterpret_cast<uintptr_t>(p) % (sizeof(T) * vec) == 0 &&
                            tok % vec == 0 && head % vec == 0);
  };
  const bool codes_ok = a.cache.code_block_stride % vec == 0 && a.cache.code_head_stride % vec == 0 &&
                        reinterpret_cast<uintptr_t>(a.cache.k_codes) % vec == 0 &&
                        (a.value == nullptr || reinterpret_cast<uintptr_t>(a.cache.v_codes) % vec == 0);
  if (aligned(a.key, a.key_token_stride, a.key_head_stride) &&
      aligned(a.value, a.value_token_stride, a.value_head_stride) && codes_ok) {
    switch (D) {
      case 64: return launch_append<T, 1>(a, reserved, stream);
      case 128: return launch_append<T, 2>(a, reserved, stream);
      case 256: return launch_append<T, 4>(a, reserved, stream);
      case 512: return launch_append<T, 8>(a, reserved, stream);
      default: break;
    }
  }
  return launch_append<T, 0>(a, reserved, stream);
}

// One thread per token: the slot's key-padding byte (state.py:339-344 copies the
// padding leaf into the page like every other leaf).
__global__ __launch_bounds__(256) void write_key_valid_kernel(uint8_t* key_valid, int64_t slots,
                                                              const int64_t* slot_mapping,
                                                              const uint8_t* token_valid,
                                                              int64_t num_tokens, int32_t* err_flag) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= num_tokens) return;
  const int64_t slot = slot_mapping[i];
  if (slot < 0) return;
  if (slot >= slots) {
    atomicOr(err_flag, ASTR_FLAG_BAD_INDEX);
    return;
  }
  key_valid[slot] = token_valid == nullptr || token_valid[i] != 0 ? 1 : 0;
}

}  // namespace
}  // namespace astr

extern "C" int astr_kv_write_key_valid(const astr_paged_kv* cache, const int64_t* slot_mapping,
                                       const uint8_t* token_valid, int64_t num_tokens,
                                       int32_t* err_flag, void* stream) {
  astr::CallRange range("astr_kv_write_key_valid");
  using namespace astr;
  if (cache == nullptr || err_flag == nullptr)
    return fail(ASTR_EINVAL, "cache descriptor and err_flag are required");
  if (cache->key_valid == nullptr) return fail(ASTR_EINVAL, "cache key_valid pointer is required");
  if (num_tokens < 0) return fail(ASTR_EINVAL, "num_tokens must be >= 0");
  if (num_tokens == 0) return 0;
  if (slot_mapping == nullptr) return fail(ASTR_EINVAL, "slot_mapping is required");
  if (cache->num_blocks < 1 || cache->block_size < 1)
    return fail(ASTR_EINVAL, "cache sizes must be positive");
  const int64_t blocks = (num_tokens + 255) / 256;
  if (blocks > INT32_MAX) return fail(ASTR_EINVAL, "too many tokens for one launch");
  hipLaunchKernelGGL(write_key_valid_kernel, dim3((uint32_t)blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), cache->key_valid,
                     (int64_t)cache->num_blocks * cache->block_size, slot_mapping, token_valid,
                     num_tokens, err_flag);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "write_key_valid launch");
}

namespace {

int quantize_append(const astr_paged_kv* cache, const void* key, const void* value,
                    int32_t in_dtype, int64_t num_tokens, int64_t key_token_stride,
                    int64_t key_head_stride, int64_t value_token_stride,
                    int64_t value_head_stride, const int64_t* slot_mapping, int32_t* err_flag,
                    void* stream, bool reserved) {
  using namespace astr;
  if (cache == nullptr || err_flag == nullptr)
    return fail(ASTR_EINVAL, "cache descriptor and err_flag are required");
  if (num_tokens < 0) return fail(ASTR_EINVAL, "num_tokens must be >= 0");
  if (num_tokens == 0) return 0;
  if (key == nullptr || slot_mapping == nullptr)
    return fail(ASTR_EINVAL, "key and slot_mapping are required");
  if (cache->k_codes == nullptr || cache->k_scales == nullptr ||
      (value != nullptr && (cache->v_codes == nullptr || cache->v_scales == nullptr)))
    return fail(ASTR_EINVAL, "cache code/scale pointers are required");
  if (cache->head_dim < 1 || cache->head_dim > kWave * kMaxPerLane)
    return fail(ASTR_EUNSUPPORTED, "head_dim %d outside 1..%d", cache->head_dim,
                kWave * kMaxPerLane);
  if (cache->num_kv_heads < 1 || cache->block_size < 1 || cache->num_blocks < 1)
    return fail(ASTR_EINVAL, "cache sizes must be positive");
  if (cache->code_format != ASTR_KV_INT8 && cache->code_format != ASTR_KV_FP8_E4M3FN &&
      cache->code_format != ASTR_KV_FP8_E5M2)
    return fail(ASTR_EUNSUPPORTED, "code format %d is not int8 / fp8 e4m3fn / fp8 e5m2",
                cache->code_format);
  if ((value ? 2 : 1) * num_tokens * (int64_t)cache->num_kv_heads >= INT32_MAX)
    return fail(ASTR_EINVAL, "too many rows for one append launch");
  AppendArgs a{key, value, key_token_stride, key_head_stride, value_token_stride,
               value_head_stride, num_tokens, slot_mapping, *cache, err_flag};
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (in_dtype) {
    case ASTR_F32: return launch_append_dim<float>(a, reserved, s);
    case ASTR_F16: return launch_append_dim<_Float16>(a, reserved, s);
    case ASTR_BF16: return launch_append_dim<bf16_t>(a, reserved, s);
    default: return fail(ASTR_EUNSUPPORTED, "input dtype %d is not f32/f16/bf16", in_dtype);
  }
}

}  // namespace

extern "C" int astr_kv_quantize_append_i8(const astr_paged_kv* cache, const void* key,
                                          const void* value, int32_t in_dtype, int64_t num_tokens,
                                          int64_t key_token_stride, int64_t key_head_stride,
                                          int64_t value_token_stride, int64_t value_head_stride,
                                          const int64_t* slot_mapping, int32_t* err_flag,
                                          void* stream) {
  astr::CallRange range("astr_kv_quantize_append_i8");
  return quantize_append(cache, key, value, in_dtype, num_tokens, key_token_stride,
                         key_head_stride, value_token_stride, value_head_stride, slot_mapping,
                         err_flag, stream, false);
}

extern "C" int astr_kv_quantize_append_i8_reserved(
    const astr_paged_kv* cache, const void* key, const void* value, int32_t in_dtype,
    int64_t num_tokens, int64_t key_token_stride, int64_t key_head_stride,
    int64_t value_token_stride, int64_t value_head_stride, const int64_t* slot_mapping,
    int32_t* err_flag, void* stream) {
  astr::CallRange range("astr_kv_quantize_append_i8_reserved");
  return quantize_append(cache, key, value, in_dtype, num_tokens, key_token_stride,
                         key_head_stride, value_token_stride, value_head_stride, slot_mapping,
                         err_flag, stream, true);
}
