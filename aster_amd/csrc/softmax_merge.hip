// merge_softmax on the device: combines two softmax states (maximum, mass, weighted
// numerator) of disjoint key partitions of the same queries, the rule of
// merge_softmax (online_attention.py:42-63):
//   M = max(m_a, m_b) (NaN propagates, as torch.maximum), s = M where finite else 0,
//   w_x = exp(m_x - s) where m_x is finite else 0,
//   mass = l_a w_a + l_b w_b,  weighted = n_a w_a + n_b w_b.
// fp32 states, contiguous: [rows] maxima and masses, [rows, width] numerators.
// HBM-bound: 3 (rows + rows * width) floats read, (2 rows + rows * width) written.
#include "common.h"

namespace astr {
namespace {

__device__ __forceinline__ float merged_max(float a, float b) {
  return (a != a || b != b) ? __builtin_nanf("") : fmaxf(a, b);
}

__device__ __forceinline__ float weight_of(float m, float safe) {
  return __builtin_isfinite(m) ? expf(m - safe) : 0.f;
}

// One thread per 4 numerator elements of one row (width % 4 == 0) or per element;
// lane 0 of each row also writes the row's maximum and mass.
template <int V>
__global__ __launch_bounds__(256) void merge_softmax_kernel(
    const float* __restrict__ ma, const float* __restrict__ la, const float* __restrict__ na,
    const float* __restrict__ mb, const float* __restrict__ lb, const float* __restrict__ nb,
    float* __restrict__ mo, float* __restrict__ lo, float* __restrict__ no, int64_t rows,
    int width) {
  const int per_row = width / V;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * per_row) return;
  const int64_t row = i / per_row;
  const int col = (int)(i % per_row) * V;
  const float xa = ma[row], xb = mb[row];
  const float m = merged_max(xa, xb);
  const float safe = __builtin_isfinite(m) ? m : 0.f;
  const float wa = weight_of(xa, safe), wb = weight_of(xb, safe);
  if (col == 0) {
    mo[row] = m;
    lo[row] = la[row] * wa + lb[row] * wb;
  }
  const int64_t at = row * width + col;
  if constexpr (V == 4) {
    const float4 a = *reinterpret_cast<const float4*>(na + at);
    const float4 b = *reinterpret_cast<const float4*>(nb + at);
    *reinterpret_cast<float4*>(no + at) =
        float4{a.x * wa + b.x * wb, a.y * wa + b.y * wb, a.z * wa + b.z * wb, a.w * wa + b.w * wb};
  } else {
    no[at] = na[at] * wa + nb[at] * wb;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// [p, p + bytes) and [q, q + bytes_q) share a byte.
bool overlap(const void* p, size_t bytes, const void* q, size_t bytes_q) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p), b = reinterpret_cast<uintptr_t>(q);
  return a < b + bytes_q && b < a + bytes;
}

}  // namespace
}  // namespace astr

extern "C" int astr_merge_softmax_f32(const float* left_max, const float* left_mass,
                                      const float* left_weighted, const float* right_max,
                                      const float* right_mass, const float* right_weighted,
                                      float* out_max, float* out_mass, float* out_weighted,
                                      int64_t rows, int32_t width, void* stream) {
  astr::CallRange range("astr_merge_softmax_f32");
  using astr::fail;
  if (rows < 0 || width < 1) return fail(ASTR_EINVAL, "rows must be >= 0 and width >= 1");
  if (rows == 0) return 0;
  if (!left_max || !left_mass || !left_weighted || !right_max || !right_mass ||
      !right_weighted || !out_max || !out_mass || !out_weighted)
    return fail(ASTR_EINVAL, "every state pointer is required");
  // Every thread of a row reads the row's two maxima while one of them writes the
  // merged maximum: an output over an input would let later threads of the row weigh
  // by the merged maximum. Outputs therefore may not overlap any input or each other.
  const size_t rb = (size_t)rows * sizeof(float), wb = rb * (size_t)width;
  const void* in[6] = {left_max, left_mass, left_weighted, right_max, right_mass, right_weighted};
  const size_t in_bytes[6] = {rb, rb, wb, rb, rb, wb};
  const void* outs[3] = {out_max, out_mass, out_weighted};
  const size_t out_bytes[3] = {rb, rb, wb};
  for (int o = 0; o < 3; ++o) {
    for (int i = 0; i < 6; ++i)
      if (astr::overlap(outs[o], out_bytes[o], in[i], in_bytes[i]))
        return fail(ASTR_EINVAL, "merge_softmax outputs must not overlap its inputs");
    for (int p = 0; p < o; ++p)
      if (astr::overlap(outs[o], out_bytes[o], outs[p], out_bytes[p]))
        return fail(ASTR_EINVAL, "merge_softmax outputs must not overlap each other");
  }
  const bool vec = width % 4 == 0 && astr::aligned16(left_weighted) &&
                   astr::aligned16(right_weighted) && astr::aligned16(out_weighted);
  const int v = vec ? 4 : 1;
  const int64_t threads = rows * (width / v);
  const int64_t blocks = (threads + 255) / 256;
  if (blocks > INT32_MAX) return fail(ASTR_EUNSUPPORTED, "merge_softmax state too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (vec)
    hipLaunchKernelGGL(astr::merge_softmax_kernel<4>, dim3((uint32_t)blocks), dim3(256), 0, s,
                       left_max, left_mass, left_weighted, right_max, right_mass, right_weighted,
                       out_max, out_mass, out_weighted, rows, width);
  else
    hipLaunchKernelGGL(astr::merge_softmax_kernel<1>, dim3((uint32_t)blocks), dim3(256), 0, s,
                       left_max, left_mass, left_weighted, right_max, right_mass, right_weighted,
                       out_max, out_mass, out_weighted, rows, width);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : astr::hip_fail(err, "merge_softmax launch");
}
