// Raw block copies inside and out of the paged arena (gfx950): copy-on-write of
// a shared tail page, and the gather/scatter halves of host swap. The reference
// moves pages with per-token narrow().copy_() (copy_kv, kv_quantization.py:113-127)
// from state.py:330-337 (COW) and state.py:427-493 / offload.py:140-190 (restore,
// archive). Here one launch moves any number of whole blocks, bit-exact: block i
// goes from src + src_index[i] * src_stride to dst + dst_index[i] * dst_stride.
#include "common.h"

namespace astr {
namespace {

constexpr int kThreads = 256;
constexpr int kTileBytes = kThreads * 16 * 4;  // bytes one workgroup moves per tile (4 x 16 B per thread)

struct CopyArgs {
  const char* src;
  char* dst;
  int64_t src_stride, dst_stride, block_bytes;
  const int32_t* src_index;
  const int32_t* dst_index;
  int32_t src_blocks, dst_blocks, num_blocks;
  int32_t tiles_per_block;
  int32_t* err_flag;
};

// grid.x = num_blocks * tiles_per_block; each workgroup moves one tile of one block.
template <bool kVec16>
__global__ __launch_bounds__(kThreads) void copy_blocks_kernel(CopyArgs a) {
  const int64_t item = blockIdx.x / a.tiles_per_block;
  const int64_t tile = blockIdx.x % a.tiles_per_block;
  if (item >= a.num_blocks) return;
  const int64_t s = a.src_index ? a.src_index[item] : item;
  const int64_t d = a.dst_index ? a.dst_index[item] : item;
  if (s < 0 || s >= a.src_blocks || d < 0 || d >= a.dst_blocks) {
    if (tile == 0 && threadIdx.x == 0) atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
    return;
  }
  const char* src = a.src + s * a.src_stride;
  char* dst = a.dst + d * a.dst_stride;
  const int64_t begin = tile * kTileBytes;
  const int64_t end = begin + kTileBytes < a.block_bytes ? begin + kTileBytes : a.block_bytes;
  if constexpr (kVec16) {
    // all four 16-byte loads of a thread issue before its stores
    uint4 v[4];
    int64_t off[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      off[k] = begin + ((int64_t)k * kThreads + threadIdx.x) * 16;
      if (off[k] < end) v[k] = *reinterpret_cast<const uint4*>(src + off[k]);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (off[k] < end) *reinterpret_cast<uint4*>(dst + off[k]) = v[k];
  } else {
    for (int64_t o = begin + threadIdx.x; o < end; o += kThreads) dst[o] = src[o];
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace astr

extern "C" int astr_kv_copy_blocks(const void* src, int64_t src_stride, const int32_t* src_index,
                                   int32_t src_blocks, void* dst, int64_t dst_stride,
                                   const int32_t* dst_index, int32_t dst_blocks,
                                   int64_t block_bytes, int32_t num_blocks, int32_t* err_flag,
                                   void* stream) {
  astr::CallRange range("astr_kv_copy_blocks");
  using namespace astr;
  if (num_blocks < 0 || block_bytes < 0 || src_blocks < 0 || dst_blocks < 0)
    return fail(ASTR_EINVAL, "counts and sizes must be >= 0");
  if (num_blocks == 0 || block_bytes == 0) return 0;
  if (src == nullptr || dst == nullptr || err_flag == nullptr)
    return fail(ASTR_EINVAL, "src, dst and err_flag are required");
  if (block_bytes > src_stride || block_bytes > dst_stride)
    return fail(ASTR_EINVAL, "block_bytes %lld exceeds a block stride", (long long)block_bytes);
  if (src_index == nullptr && num_blocks > src_blocks)
    return fail(ASTR_EINVAL, "num_blocks exceeds src_blocks");
  if (dst_index == nullptr && num_blocks > dst_blocks)
    return fail(ASTR_EINVAL, "num_blocks exceeds dst_blocks");
  const int64_t tiles = (block_bytes + kTileBytes - 1) / kTileBytes;
  const int64_t grid = tiles * num_blocks;
  if (grid > INT32_MAX) return fail(ASTR_EUNSUPPORTED, "copy too large for one launch");
  CopyArgs a{static_cast<const char*>(src), static_cast<char*>(dst), src_stride, dst_stride,
             block_bytes, src_index, dst_index, src_blocks, dst_blocks, num_blocks,
             (int32_t)tiles, err_flag};
  const bool vec = aligned16(src) && aligned16(dst) && src_stride % 16 == 0 &&
                   dst_stride % 16 == 0 && block_bytes % 16 == 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (vec)
    hipLaunchKernelGGL(copy_blocks_kernel<true>, dim3((uint32_t)grid), dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL(copy_blocks_kernel<false>, dim3((uint32_t)grid), dim3(kThreads), 0, s, a);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "kv_copy_blocks launch");
}
