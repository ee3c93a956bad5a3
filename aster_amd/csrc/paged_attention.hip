// Ragged paged decode attention over the INT8 KV arena (gfx950).
//
// One workgroup (4 waves) per (sequence, kv head, split-K partition). Every
// wave owns whole 16-token blocks of the partition and serves ALL G query heads
// of the GQA group from the same registers, so each K/V byte is read from HBM
// once per (sequence, kv head). Inside a wave, a 16-token block of one kv head
// (16*D int8 codes, contiguous) is read with 16-byte-per-lane coalesced loads;
// lane l holds the 16 codes [16*(l % LPT), +16) of token rows l / LPT (+ TPL*j),
// dequantization is folded into the score (q . (c*s) == s * (q . c)) and into
// the probability (p * s_v), so codes are converted int8 -> fp32 in registers
// and never materialised as a tile.
//
// Online softmax in base 2 with a lazily-raised reference maximum: a block only
// rescales the running (l, acc) when one of its scores exceeds the reference by
// more than kRescaleSlack (a wave-uniform branch, taken on the first block and
// rarely after), so the common path has no cross-lane max at all. The final
// state (m, l, acc) is the reference's SoftmaxState (online_attention.py:29-39)
// up to the exp -> exp2 change of base, which cancels in acc / l.
//
// Partitions of more than one per (sequence, kv head) write (m, l, acc)
// partials that merge_kernel combines with the merge_softmax rule
// (online_attention.py:42-63): non-finite maxima weigh 0, output =
// acc / max(l, FLT_MIN) (:35-39).
#include <cfloat>
#include <cmath>

#include "common.h"

namespace astr {
namespace {

constexpr int kBlockTokens = 16;
constexpr int kWaves = 4;
constexpr float kRescaleSlack = 8.0f;  // p = exp2(s - m) <= 2^8 between rescales

struct DecodeArgs {
  const void* q;
  int64_t q_tok, q_head;
  void* out;
  int64_t o_tok, o_head;
  astr_paged_kv cache;
  const int32_t* block_tables;
  int32_t bt_stride;
  const int32_t* context_lens;
  int32_t num_seqs, num_q_heads;
  float qk_scale_log2;  // softmax scale * log2(e)
  int32_t window;
  int32_t part_blocks;  // blocks per split-K partition
  int32_t max_parts;
  float* ws_ml;  // [num_seqs][num_q_heads][max_parts][2]  (m, l)
  float* ws_o;   // [num_seqs][num_q_heads][max_parts][D]  unnormalised acc
  int32_t* err_flag;
};

// Visible key range [kv_begin, ctx) of a decode row and its partition count.
struct RowPlan {
  int ctx, kv_begin, first_blk, last_blk, num_parts;
};

__device__ __forceinline__ RowPlan plan_row(const DecodeArgs& a, int seq, bool report) {
  RowPlan r;
  int ctx = a.context_lens[seq];
  const int cap = a.bt_stride * kBlockTokens;
  if (ctx < 0 || ctx > cap) {
    if (report) atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
    ctx = ctx < 0 ? 0 : cap;
  }
  r.ctx = ctx;
  r.kv_begin = (a.window > 0 && ctx > a.window) ? ctx - a.window : 0;
  r.first_blk = r.kv_begin / kBlockTokens;
  r.last_blk = (ctx + kBlockTokens - 1) / kBlockTokens;
  int parts = (r.last_blk - r.first_blk + a.part_blocks - 1) / a.part_blocks;
  parts = parts < 1 ? 1 : parts;
  if (parts > a.max_parts) {
    if (report) atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
    parts = a.max_parts;
  }
  r.num_parts = parts;
  return r;
}

template <int NL>
struct Tile {
  uint4 k[NL];
  uint4 v[NL];
  float ks[NL];
  float vs[NL];
};

template <typename QT, int D, int G>
__global__ __launch_bounds__(256) void decode_kernel(DecodeArgs a) {
  constexpr int LPT = D / 16;               // lanes per token row
  constexpr int TPL = kWave / LPT;          // token rows per load instruction
  constexpr int NL = kBlockTokens / TPL;    // load instructions per block
  constexpr int kLoadBytes = kWave * 16;    // bytes per load instruction
  static_assert(NL >= 1 && NL * TPL == kBlockTokens, "unsupported head_dim");

  const int part = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const RowPlan row = plan_row(a, seq, part == 0 && kvh == 0 && threadIdx.x == 0);
  if (part >= row.num_parts) return;
  const int pb0 = row.first_blk + part * a.part_blocks;
  const int pb1 = min(row.last_blk, pb0 + a.part_blocks);

  const int lrow = lane / LPT;
  const int d0 = (lane % LPT) * 16;

  // Query slice [d0, d0+16) of the G heads kvh*G .. kvh*G+G-1, in fp32.
  float qf[G][16];
  {
    const QT* qp = static_cast<const QT*>(a.q) + seq * a.q_tok + (int64_t)kvh * G * a.q_head + d0;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      constexpr int kVec = 16 / sizeof(QT);
      const uint4* src = reinterpret_cast<const uint4*>(qp + g * a.q_head);
#pragma unroll
      for (int c = 0; c < 16 / kVec; ++c) {
        uint4 w = src[c];
        const QT* e = reinterpret_cast<const QT*>(&w);
#pragma unroll
        for (int i = 0; i < kVec; ++i) qf[g][c * kVec + i] = to_float<QT>(e[i]);
      }
    }
  }

  float m[G], l[G], acc[G][16];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[g][i] = 0.f;
  }

  const int32_t* bt = a.block_tables + (int64_t)seq * a.bt_stride;
  const int8_t* kbase = a.cache.k_codes + (int64_t)kvh * a.cache.code_head_stride;
  const int8_t* vbase = a.cache.v_codes + (int64_t)kvh * a.cache.code_head_stride;
  const float* ksbase = a.cache.k_scales + (int64_t)kvh * a.cache.scale_head_stride;
  const float* vsbase = a.cache.v_scales + (int64_t)kvh * a.cache.scale_head_stride;

  auto load_tile = [&](int blk, Tile<NL>& t) -> bool {
    const int phys = bt[blk];
    if ((unsigned)phys >= (unsigned)a.cache.num_blocks) return false;
    const int8_t* kp = kbase + (int64_t)phys * a.cache.code_block_stride + lane * 16;
    const int8_t* vp = vbase + (int64_t)phys * a.cache.code_block_stride + lane * 16;
    const float* ksp = ksbase + (int64_t)phys * a.cache.scale_block_stride + lrow;
    const float* vsp = vsbase + (int64_t)phys * a.cache.scale_block_stride + lrow;
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      t.k[j] = *reinterpret_cast<const uint4*>(kp + j * kLoadBytes);
      t.v[j] = *reinterpret_cast<const uint4*>(vp + j * kLoadBytes);
      t.ks[j] = ksp[j * TPL];
      t.vs[j] = vsp[j * TPL];
    }
    return true;
  };

  int blk = pb0 + wave;
  Tile<NL> cur;
  bool cur_ok = blk < pb1 ? load_tile(blk, cur) : false;
  bool bad_index = false, bad_score = false;
  for (; blk < pb1; blk += kWaves) {
    Tile<NL> nxt;
    const int nblk = blk + kWaves;
    const bool nxt_ok = nblk < pb1 ? load_tile(nblk, nxt) : false;
    if (!cur_ok) {
      bad_index = true;
    } else {
      // ---- scores s[j][g] = (q_g . k_t) * scale_k(t) * softmax_scale * log2e
      float s[NL][G];
#pragma unroll
      for (int j = 0; j < NL; ++j) {
        const uint32_t w[4] = {cur.k[j].x, cur.k[j].y, cur.k[j].z, cur.k[j].w};
        float kf[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) kf[i] = i8_to_f(w[i / 4], i % 4);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float dot = 0.f;
#pragma unroll
          for (int i = 0; i < 16; ++i) dot = fmaf(qf[g][i], kf[i], dot);
          s[j][g] = group_sum<LPT>(dot);
        }
      }
      bool need = false, nonfinite = false;
#pragma unroll
      for (int j = 0; j < NL; ++j) {
        const int tok = blk * kBlockTokens + j * TPL + lrow;
        const bool valid = tok >= row.kv_begin && tok < row.ctx;
        const float f = cur.ks[j] * a.qk_scale_log2;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float v = s[j][g] * f;
          nonfinite |= valid && !__builtin_isfinite(v);
          s[j][g] = valid ? v : -INFINITY;
          need |= s[j][g] > m[g] + kRescaleSlack;
        }
      }
      if (__ballot(nonfinite) != 0) bad_score = true;
      if (__ballot(need) != 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float tmax = s[0][g];
#pragma unroll
          for (int j = 1; j < NL; ++j) tmax = fmaxf(tmax, s[j][g]);
          tmax = strided_max<LPT>(tmax);
          const float mn = fmaxf(m[g], tmax);
          const float alpha = m[g] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[g] - mn);
          l[g] *= alpha;
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[g][i] *= alpha;
          m[g] = mn;
        }
      }
      // ---- P . V with the value scale folded into p
#pragma unroll
      for (int j = 0; j < NL; ++j) {
        const uint32_t w[4] = {cur.v[j].x, cur.v[j].y, cur.v[j].z, cur.v[j].w};
        float vf[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) vf[i] = i8_to_f(w[i / 4], i % 4);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float p = __builtin_amdgcn_exp2f(s[j][g] - m[g]);
          l[g] += p;
          const float pv = p * cur.vs[j];
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[g][i] = fmaf(pv, vf[i], acc[g][i]);
        }
      }
    }
    cur = nxt;
    cur_ok = nxt_ok;
  }
  if (bad_index && lane == 0) atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
  if (bad_score && lane == 0) atomicOr(a.err_flag, ASTR_FLAG_NONFINITE_SCORE);

  // ---- reduce the wave's token rows (lanes of one d-chunk hold other tokens)
#pragma unroll
  for (int g = 0; g < G; ++g) {
    l[g] = strided_sum<LPT>(l[g]);
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[g][i] = strided_sum<LPT>(acc[g][i]);
  }

  // ---- merge the 4 waves through LDS
  __shared__ float s_m[kWaves][G], s_l[kWaves][G];
  __shared__ float s_o[kWaves][G][D];
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      s_m[wave][g] = m[g];
      s_l[wave][g] = l[g];
    }
  }
  if (lrow == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 16; ++i) s_o[wave][g][d0 + i] = acc[g][i];
  }
  __syncthreads();

  const bool split = row.num_parts > 1;
  for (int idx = threadIdx.x; idx < G * D; idx += blockDim.x) {
    const int g = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w][g]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float mw = s_m[w][g];
      const float f = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
      L = fmaf(s_l[w][g], f, L);
      O = fmaf(s_o[w][g][d], f, O);
    }
    const int h = kvh * G + g;
    if (!split) {
      QT* op = static_cast<QT*>(a.out) + seq * a.o_tok + (int64_t)h * a.o_head;
      op[d] = from_float<QT>(O / fmaxf(L, FLT_MIN));
    } else {
      const int64_t base = ((int64_t)seq * a.num_q_heads + h) * a.max_parts + part;
      a.ws_o[base * D + d] = O;
      if (d == 0) {
        a.ws_ml[base * 2] = M;
        a.ws_ml[base * 2 + 1] = L;
      }
    }
  }
}

// Split-K combine: merge_softmax over the partitions of each (sequence, q head).
template <typename QT, int D>
__global__ __launch_bounds__(256) void merge_kernel(DecodeArgs a) {
  const int h = blockIdx.x, seq = blockIdx.y;
  const RowPlan row = plan_row(a, seq, false);
  if (row.num_parts <= 1) return;
  const int64_t base = ((int64_t)seq * a.num_q_heads + h) * a.max_parts;
  float M = -INFINITY;
  for (int p = 0; p < row.num_parts; ++p) M = fmaxf(M, a.ws_ml[(base + p) * 2]);
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float L = 0.f, O = 0.f;
    for (int p = 0; p < row.num_parts; ++p) {
      const float mp = a.ws_ml[(base + p) * 2];
      const float f = mp == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mp - M);
      L = fmaf(a.ws_ml[(base + p) * 2 + 1], f, L);
      O = fmaf(a.ws_o[(base + p) * D + d], f, O);
    }
    QT* op = static_cast<QT*>(a.out) + seq * a.o_tok + (int64_t)h * a.o_head;
    op[d] = from_float<QT>(O / fmaxf(L, FLT_MIN));
  }
}

template <typename QT, int D, int G>
int launch_decode(const DecodeArgs& a, hipStream_t stream) {
  const dim3 grid((uint32_t)a.max_parts, (uint32_t)a.cache.num_kv_heads, (uint32_t)a.num_seqs);
  hipLaunchKernelGGL((decode_kernel<QT, D, G>), grid, dim3(kWaves * kWave), 0, stream, a);
  if (a.max_parts > 1) {
    hipLaunchKernelGGL((merge_kernel<QT, D>), dim3((uint32_t)a.num_q_heads, (uint32_t)a.num_seqs),
                       dim3(D < 256 ? D : 256), 0, stream, a);
  }
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "paged_attention launch");
}

template <typename QT, int D>
int dispatch_group(const DecodeArgs& a, int G, hipStream_t s) {
  switch (G) {
    case 1: return launch_decode<QT, D, 1>(a, s);
    case 2: return launch_decode<QT, D, 2>(a, s);
    case 4: return launch_decode<QT, D, 4>(a, s);
    case 8: return launch_decode<QT, D, 8>(a, s);
    default: return fail(ASTR_EUNSUPPORTED, "GQA group size %d not in {1,2,4,8}", G);
  }
}

template <typename QT>
int dispatch_dim(const DecodeArgs& a, int G, hipStream_t s) {
  switch (a.cache.head_dim) {
    case 64: return dispatch_group<QT, 64>(a, G, s);
    case 128: return dispatch_group<QT, 128>(a, G, s);
    case 256: return dispatch_group<QT, 256>(a, G, s);
    default: return fail(ASTR_EUNSUPPORTED, "head_dim %d not in {64,128,256}", a.cache.head_dim);
  }
}

constexpr int kDefaultPartitionTokens = 512;

int resolve_partition(int32_t partition_tokens) {
  return partition_tokens == 0 ? kDefaultPartitionTokens : partition_tokens;
}

int64_t max_parts_for(int32_t max_context_len, int32_t partition_tokens) {
  const int64_t blocks = ((int64_t)max_context_len + kBlockTokens - 1) / kBlockTokens;
  const int64_t pb = partition_tokens / kBlockTokens;
  const int64_t parts = (blocks + pb - 1) / pb;
  return parts < 1 ? 1 : parts;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace astr

extern "C" size_t astr_paged_attention_i8_workspace_bytes(int32_t num_seqs, int32_t num_q_heads,
                                                          int32_t head_dim,
                                                          int32_t max_context_len,
                                                          int32_t partition_tokens) {
  using namespace astr;
  if (num_seqs < 0 || num_q_heads < 0 || head_dim < 0 || max_context_len < 0) return 0;
  const int pt = resolve_partition(partition_tokens);
  if (pt <= 0 || pt % (kBlockTokens * kWaves) != 0) return 0;
  const int64_t parts = max_parts_for(max_context_len, pt);
  if (parts <= 1) return 0;
  return (size_t)num_seqs * num_q_heads * parts * (head_dim + 2) * sizeof(float);
}

extern "C" int astr_paged_attention_i8(const astr_paged_kv* cache, const void* query,
                                       int32_t q_dtype, int64_t q_token_stride,
                                       int64_t q_head_stride, void* out, int64_t out_token_stride,
                                       int64_t out_head_stride, const int32_t* block_tables,
                                       int32_t block_table_stride, const int32_t* context_lens,
                                       int32_t num_seqs, int32_t num_q_heads,
                                       int32_t max_context_len, float scale, int32_t window,
                                       int32_t partition_tokens, void* workspace,
                                       size_t workspace_bytes, int32_t* err_flag, void* stream) {
  using namespace astr;
  if (cache == nullptr || err_flag == nullptr)
    return fail(ASTR_EINVAL, "cache descriptor and err_flag are required");
  if (num_seqs < 0 || num_q_heads < 1 || max_context_len < 0 || block_table_stride < 0)
    return fail(ASTR_EINVAL, "num_seqs/max_context_len/block_table_stride must be >= 0 and "
                             "num_q_heads >= 1");
  if (num_seqs == 0) return 0;
  if (query == nullptr || out == nullptr || block_tables == nullptr || context_lens == nullptr)
    return fail(ASTR_EINVAL, "query, out, block_tables and context_lens are required");
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(ASTR_EINVAL, "attention scale must be finite and positive");
  if (window < 0) return fail(ASTR_EINVAL, "window must be >= 0 (0 = no window)");
  if (cache->block_size != kBlockTokens)
    return fail(ASTR_EUNSUPPORTED, "block_size %d != 16", cache->block_size);
  if (cache->num_kv_heads < 1 || num_q_heads % cache->num_kv_heads != 0)
    return fail(ASTR_EINVAL, "num_q_heads %d must be a multiple of num_kv_heads %d", num_q_heads,
                cache->num_kv_heads);
  if (cache->num_blocks < 1) return fail(ASTR_EINVAL, "cache has no blocks");
  const int pt = resolve_partition(partition_tokens);
  if (pt <= 0 || pt % (kBlockTokens * kWaves) != 0)
    return fail(ASTR_EINVAL, "partition_tokens %d must be a positive multiple of %d", pt,
                kBlockTokens * kWaves);
  if ((int64_t)max_context_len > (int64_t)block_table_stride * kBlockTokens)
    return fail(ASTR_EINVAL, "max_context_len %d exceeds block table capacity %lld",
                max_context_len, (long long)block_table_stride * kBlockTokens);
  const int esize = q_dtype == ASTR_F32 ? 4 : 2;
  if (q_dtype != ASTR_F32 && q_dtype != ASTR_F16 && q_dtype != ASTR_BF16)
    return fail(ASTR_EUNSUPPORTED, "query dtype %d is not f32/f16/bf16", q_dtype);
  if (!aligned16(query) || !aligned16(out) || (q_token_stride * esize) % 16 ||
      (q_head_stride * esize) % 16 || (out_token_stride * esize) % 16 ||
      (out_head_stride * esize) % 16)
    return fail(ASTR_EINVAL, "query/out rows must be 16-byte aligned");
  if (!aligned16(cache->k_codes) || !aligned16(cache->v_codes) ||
      cache->code_block_stride % 16 || cache->code_head_stride % 16)
    return fail(ASTR_EINVAL, "cache code blocks must be 16-byte aligned");
  const int64_t parts = max_parts_for(max_context_len, pt);
  if (parts > 65535) return fail(ASTR_EUNSUPPORTED, "too many split-K partitions (%lld)",
                                 (long long)parts);
  const size_t need = astr_paged_attention_i8_workspace_bytes(
      num_seqs, num_q_heads, cache->head_dim, max_context_len, partition_tokens);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(ASTR_EINVAL, "workspace of %zu bytes required, %zu given", need, workspace_bytes);

  DecodeArgs a{};
  a.q = query;
  a.q_tok = q_token_stride;
  a.q_head = q_head_stride;
  a.out = out;
  a.o_tok = out_token_stride;
  a.o_head = out_head_stride;
  a.cache = *cache;
  a.block_tables = block_tables;
  a.bt_stride = block_table_stride;
  a.context_lens = context_lens;
  a.num_seqs = num_seqs;
  a.num_q_heads = num_q_heads;
  a.qk_scale_log2 = scale * kLog2e;
  a.window = window;
  a.part_blocks = pt / kBlockTokens;
  a.max_parts = (int32_t)parts;
  a.ws_o = static_cast<float*>(workspace);
  a.ws_ml = need > 0 ? a.ws_o + (size_t)num_seqs * num_q_heads * parts * cache->head_dim : nullptr;
  a.err_flag = err_flag;
  const int G = num_q_heads / cache->num_kv_heads;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (q_dtype) {
    case ASTR_F32: return dispatch_dim<float>(a, G, s);
    case ASTR_F16: return dispatch_dim<_Float16>(a, G, s);
    default: return dispatch_dim<bf16_t>(a, G, s);
  }
}
