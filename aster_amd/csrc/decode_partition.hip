// Paged decode attention with fixed-size split-K partitions (gfx950).
//
// Work decomposition: one workgroup (4 waves) per (sequence, kv head,
// partition of part_blocks 16-token blocks). Every wave owns blocks w, w+4, ...
// of the partition and serves all G query heads of the GQA group, so each K/V
// byte is read from HBM once per (sequence, kv head); the 4 waves' states merge
// through LDS at the end. This path serves any batch size and is the one used
// for fp32 queries; the stream-K path (decode_streamk.hip) balances bf16/fp16
// batches of up to 512 sequences better.
//
// bf16/fp16 queries -> decode_mfma_kernel (blocks staged into LDS by direct
// global->LDS loads, MFMA step of attention_common.h). fp32 queries ->
// decode_valu_kernel: the same schedule in exact fp32 VALU arithmetic (int8 ->
// fp32 in registers, 16-wide dot products per lane reduced with DPP), used where
// f16 operands would lose query precision.
//
// Both fold dequantization into the score (q.(c*s) = s*(q.c)) and into the
// probability (p*s_v), and run the online softmax in base 2 with a lazily raised
// reference maximum: a block rescales the running (l, acc) only when one of its
// scores exceeds the reference by more than kRescaleSlack. The final state is
// the reference's SoftmaxState (online_attention.py:29-39) up to the exp -> exp2
// change of base, which cancels in acc / l.
//
// Partitions of one (sequence, kv head) write (m, l, acc) partials and
// merge_kernel, launched next on the same stream, combines them with the
// merge_softmax rule (online_attention.py:42-63): non-finite maxima weigh 0,
// output = acc / max(l, FLT_MIN) (:35-39). (An in-kernel last-finisher merge
// needs agent-scope fences, which on gfx950 write back and invalidate the whole
// L2 of the XCD per workgroup; the kernel boundary is far cheaper.)
#include "attention_common.h"

namespace astr {
namespace attn {
namespace {

#ifndef ASTR_KF
#define ASTR_KF 0
#endif
constexpr int KF = ASTR_KF;  // this translation unit's code format

constexpr int kStages = 2;  // LDS stages per wave in the MFMA kernel

struct RowPlan : RowSpan {
  int num_parts;
};

__device__ __forceinline__ RowPlan plan_row(const AttnArgs& a, int seq, bool report) {
  RowPlan r;
  static_cast<RowSpan&>(r) = row_span(a, clamp_ctx(a, a.context_lens[seq], report));
  int parts = (r.last_blk - r.first_blk + a.part_blocks - 1) / a.part_blocks;
  parts = parts < 1 ? 1 : parts;
  if (parts > a.max_parts) {
    if (report) atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
    parts = a.max_parts;
  }
  r.num_parts = parts;
  return r;
}

// Per-workgroup shared state: the 4 waves' (m, l, acc).
template <int G, int D>
struct Shared {
  float m[kWaves][G];
  float l[kWaves][G];
  float o[kWaves][G][D];
};

// Combine the 4 waves of the workgroup (already in `sh`, heads head0 .. head0+G-1)
// and write either the normalised output (single partition) or this partition's
// partial.
template <typename QT, int G, int D>
__device__ void finish_partition(const AttnArgs& a, Shared<G, D>& sh, const RowPlan& row,
                                 int seq, int tok, int head0, int part) {
  const bool split = row.num_parts > 1;
  for (int idx = threadIdx.x; idx < G * D; idx += blockDim.x) {
    const int g = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sh.m[w][g]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float mw = sh.m[w][g];
      const float f = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
      L = fmaf(sh.l[w][g], f, L);
      O = fmaf(sh.o[w][g][d], f, O);
    }
    const int h = head0 + g;
    if (!split) {
      QT* op = static_cast<QT*>(a.out) + (int64_t)tok * a.o_tok + (int64_t)h * a.o_head;
      if (a.stats != nullptr) {  // the row's state itself
        op[d] = from_float<QT>(O);
        if (d == 0) store_row_stats(a.stats, (int64_t)tok * a.num_q_heads + h, M, L);
      } else {
        op[d] = from_float<QT>(O / fmaxf(L, FLT_MIN));
      }
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

// Physical block ids of this wave's blocks (first + 4*i), one per lane.
__device__ __forceinline__ int wave_block_ids(const AttnArgs& a, int seq, int first, int nbw,
                                              int lane) {
  const int32_t* bt = a.block_tables + (int64_t)seq * a.bt_stride;
  return lane < nbw ? bt[first + kWaves * lane] : 0;
}

template <int D, int G>
constexpr int stage0_bytes() {
  constexpr int staging = kWaves * Stage<D>::kBytes;
  constexpr int merge = (int)sizeof(Shared<G, D>);
  return staging > merge ? staging : merge;
}

// ================================ MFMA kernel (bf16 / fp16 queries)

template <typename QT, int D, int G, int NS>
__global__ __launch_bounds__(256) void decode_mfma_kernel(AttnArgs a) {
  static_assert(D == 64 || D == 128 || D == 256, "head_dim");
  static_assert(G >= 1 && G <= 16, "GQA group");
  static_assert(NS == 2 || NS == 3, "stages");
  using S = Stage<D>;
  constexpr int NPV = D / 16;
  constexpr int VB = D / 16;

  // One __shared__ object per stage (the ring is unrolled over them).
  __shared__ __attribute__((aligned(16))) char lds0[stage0_bytes<D, G>()];
  __shared__ __attribute__((aligned(16))) char lds1[kWaves * S::kBytes];
  __shared__ __attribute__((aligned(16))) char lds2[NS == 3 ? kWaves * S::kBytes : 16];
  const int part = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int r = lane & 15, qg = lane >> 4;
  const bool gvalid = r < G;
  const int tok = decode_token(a, seq);
  if (tok < 0) return;  // not a decode row

  // ---- prologue: the query and (for window == 0) this wave's block ids do not
  // depend on the context length, so their loads issue together with it.
  QueryRaw<D> qraw;
  load_query<QT, D, G>(a, tok, kvh, r, qg, qraw);
  const int32_t* bt = a.block_tables + (int64_t)seq * a.bt_stride;
  const int per_wave = (a.part_blocks + kWaves - 1) / kWaves;
  const int spec = part * a.part_blocks + wave + kWaves * lane;  // block index if kv_begin == 0
  int ids = (a.window == 0 && lane < per_wave && spec < a.bt_stride) ? bt[spec] : 0;
  const RowPlan row = plan_row(a, seq, part == 0 && kvh == 0 && threadIdx.x == 0);
  if (part >= row.num_parts) return;
  const int pb0 = row.first_blk + part * a.part_blocks;
  const int pb1 = min(row.last_blk, pb0 + a.part_blocks);
  const int first = pb0 + wave;
  const int nbw = first < pb1 ? (pb1 - first + kWaves - 1) / kWaves : 0;
  if (a.window != 0) ids = wave_block_ids(a, seq, first, nbw, lane);
  // One bad block id poisons the partition: flag it and stage nothing, so the
  // stage/wait bookkeeping below never sees a skipped load.
  const bool bad_index = __ballot(lane < nbw && (unsigned)ids >= (unsigned)a.cache.num_blocks) != 0;
  const int nblk = bad_index ? 0 : nbw;

  char* const st0 = lds0 + wave * S::kBytes;
  char* const st1 = lds1 + wave * S::kBytes;
  char* const st2 = lds2 + (NS == 3 ? wave * S::kBytes : 0);
  if (0 < nblk) stage_block<D>(a, __builtin_amdgcn_readlane(ids, 0), kvh, lane, st0);
  if (1 < nblk) stage_block<D>(a, __builtin_amdgcn_readlane(ids, 1), kvh, lane, st1);
  if (NS == 3 && 2 < nblk) stage_block<D>(a, __builtin_amdgcn_readlane(ids, 2), kvh, lane, st2);

  QkOperand<D, KF> qop;
  const float cf = qk_operand<QT, D, KF>(qraw, gvalid, a.qk_scale_log2, qop);
  float4_t acc[NPV + 1];  // [NPV]: weight sums (INT8)
#pragma unroll
  for (int n = 0; n <= NPV; ++n) acc[n] = float4_t{0.f, 0.f, 0.f, 0.f};
  // invalid head columns never contribute; a finite start makes a block whose keys are
  // all masked (padding) give exp2(-inf) = 0, not exp2(-inf + inf)
  float m = gvalid ? -FLT_MAX : 0.f;
  float l = 0.f;
  VRange vr = vrange_start<KF>();
  bool bad_score = false;

  auto step = [&](int i, char* st) __attribute__((always_inline)) {
    // wait until block i has landed: later stages (up to NS-1) may stay in flight
    const int later = min(NS - 1, nblk - 1 - i);
    if (later >= 2) wait_vmcnt<2 * S::kLoads>();
    else if (later == 1) wait_vmcnt<S::kLoads>();
    else wait_vmcnt<0>();
    mfma_block<QT, D, KF>(st, qop, cf, (first + kWaves * i) * kBlockTokens, row.kv_begin, row.ctx,
                          gvalid, r, qg, acc, m, l, vr, bad_score, a.cache.key_valid != nullptr);
    // refill this stage with block i + NS (its LDS reads above fed the MFMAs)
    if (i + NS < nblk) stage_block<D>(a, __builtin_amdgcn_readlane(ids, i + NS), kvh, lane, st);
  };
  for (int i = 0; i < nblk; i += NS) {
    step(i, st0);
    if (i + 1 >= nblk) break;
    step(i + 1, st1);
    if constexpr (NS == 3) {
      if (i + 2 >= nblk) break;
      step(i + 2, st2);
    }
  }
  if (bad_index && lane == 0) atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
  if (bad_score && lane == 0) atomicOr(a.err_flag, ASTR_FLAG_NONFINITE_SCORE);

  // ---- per-wave state to LDS (aliases the stages: wait for every wave first)
  end_piece<D, KF>(acc, r);
  l += shfl_xor(l, 16);
  l += shfl_xor(l, 32);
  l *= norm_scale<KF>();  // the factor the PV weights carry
  __syncthreads();
  Shared<G, D>& sh = *reinterpret_cast<Shared<G, D>*>(lds0);
  if (gvalid) {
    if (qg == 0) {
      sh.m[wave][r] = m;
      sh.l[wave][r] = l;
    }
#pragma unroll
    for (int n = 0; n < NPV; ++n)
#pragma unroll
      for (int j = 0; j < 4; ++j) sh.o[wave][r][VB * (4 * qg + j) + n] = acc[n][j];
  }
  __syncthreads();
  finish_partition<QT, G, D>(a, sh, row, seq, tok, kvh * G, part);
}

// ================================ exact fp32 VALU kernel (fp32 queries)

template <int NL>
struct ValuTile {
  uint4 k[NL];
  uint4 v[NL];
  float ks[NL];
  float vs[NL];
  uint8_t kv[NL];  // key padding bytes (1 without a mask)
};

// Heads of a GQA group one VALU workgroup serves: a lane keeps 16 query values and
// 16 accumulators per head in registers, so large groups at D >= 128 are served
// in passes of 4 heads (each pass re-reads the group's K/V) instead of spilling, as
// are groups of 16 at any D. (FP8 codes convert with a few more live registers: passes
// of 4 heads from D = 64 up.)
constexpr int valu_heads(int D, int group) {
  return (((D >= 128 || KF != kInt8) && group > 4) || group > 8) ? 4 : group;
}

// GROUP: the GQA group size; G: the heads of it this workgroup serves
// (blockIdx.y = kv head * GROUP/G + pass).
template <typename QT, int D, int GROUP, int G>
__global__ __launch_bounds__(256) void decode_valu_kernel(AttnArgs a) {
  static_assert(GROUP % G == 0, "passes must tile the group");
  constexpr int LPT = D / 16;             // lanes per token row
  constexpr int TPL = kWave / LPT;        // token rows per load instruction
  constexpr int NL = kBlockTokens / TPL;  // load instructions per block
  constexpr int kLoadBytes = kWave * 16;
  static_assert(NL >= 1 && NL * TPL == kBlockTokens, "unsupported head_dim");

  __shared__ Shared<G, D> sh;
  const int part = blockIdx.x, seq = blockIdx.z;
  const int kvh = blockIdx.y / (GROUP / G);
  const int head0 = kvh * GROUP + (blockIdx.y % (GROUP / G)) * G;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int tok = decode_token(a, seq);
  if (tok < 0) return;  // not a decode row
  const RowPlan row = plan_row(a, seq, part == 0 && kvh == 0 && threadIdx.x == 0);
  if (part >= row.num_parts) return;
  const int pb0 = row.first_blk + part * a.part_blocks;
  const int pb1 = min(row.last_blk, pb0 + a.part_blocks);
  const int first = pb0 + wave;
  const int nbw = first < pb1 ? (pb1 - first + kWaves - 1) / kWaves : 0;
  const int lrow = lane / LPT;
  const int d0 = (lane % LPT) * 16;

  float qf[G][16];
  {
    const QT* qp = static_cast<const QT*>(a.q) + (int64_t)tok * a.q_tok + (int64_t)head0 * a.q_head + d0;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      constexpr int kVec = 16 / sizeof(QT);
      const uint4* src = reinterpret_cast<const uint4*>(qp + g * a.q_head);
#pragma unroll
      for (int c = 0; c < 16 / kVec; ++c) {
        const uint4 w = src[c];
        const QT* e = reinterpret_cast<const QT*>(&w);
#pragma unroll
        for (int i = 0; i < kVec; ++i) qf[g][c * kVec + i] = to_float<QT>(e[i]);
      }
    }
  }
  float m[G], l[G], acc[G][16];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -FLT_MAX;  // finite: an all-masked block gives exp2(-inf) = 0
    l[g] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[g][i] = 0.f;
  }
  const int8_t* kbase = a.cache.k_codes + (int64_t)kvh * a.cache.code_head_stride + lane * 16;
  const int8_t* vbase = a.cache.v_codes + (int64_t)kvh * a.cache.code_head_stride + lane * 16;
  const float* ksbase = a.cache.k_scales + (int64_t)kvh * a.cache.scale_head_stride + lrow;
  const float* vsbase = a.cache.v_scales + (int64_t)kvh * a.cache.scale_head_stride + lrow;
  const bool masks = a.cache.key_valid != nullptr;  // key padding bytes of the token rows
  const uint8_t* kvbase = masks ? a.cache.key_valid + lrow : nullptr;
  // statistics mode raises the reference on every larger score, so that it ends as the
  // row's exact maximum
  const float slack = a.stats != nullptr ? 0.f : kRescaleSlack;
  auto load = [&](int phys, ValuTile<NL>& t) __attribute__((always_inline)) {
    const int8_t* kp = kbase + (int64_t)phys * a.cache.code_block_stride;
    const int8_t* vp = vbase + (int64_t)phys * a.cache.code_block_stride;
    const float* ksp = ksbase + (int64_t)phys * a.cache.scale_block_stride;
    const float* vsp = vsbase + (int64_t)phys * a.cache.scale_block_stride;
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      t.k[j] = *reinterpret_cast<const uint4*>(kp + j * kLoadBytes);
      t.v[j] = *reinterpret_cast<const uint4*>(vp + j * kLoadBytes);
      t.ks[j] = ksp[j * TPL] * code_scale<KF>();  // 2^8 for E4M3FN (its codes convert to 2^-8 x)
      t.vs[j] = vsp[j * TPL] * code_scale<KF>();
      t.kv[j] = masks ? kvbase[(int64_t)phys * kBlockTokens + j * TPL] : (uint8_t)1;
    }
  };

  const int ids = wave_block_ids(a, seq, first, nbw, lane);
  bool bad_index = false, bad_score = false;
  auto fetch = [&](int i, ValuTile<NL>& t) __attribute__((always_inline)) -> bool {
    const int phys = __builtin_amdgcn_readlane(ids, i);
    const bool ok = (unsigned)phys < (unsigned)a.cache.num_blocks;
    if (ok) load(phys, t);
    return ok;
  };
  auto process = [&](int i, const ValuTile<NL>& cur) __attribute__((always_inline)) {
    const int blk = first + kWaves * i;
    float s[NL][G];
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const uint32_t w[4] = {cur.k[j].x, cur.k[j].y, cur.k[j].z, cur.k[j].w};
      float kf[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) kf[e] = code_to_f<KF>(w[e / 4], e % 4);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float dot = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) dot = fmaf(qf[g][e], kf[e], dot);
        s[j][g] = group_sum<LPT>(dot);
      }
    }
    bool need = false, nonfinite = false;
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const int tok = blk * kBlockTokens + j * TPL + lrow;
      const bool valid = tok >= row.kv_begin && tok < row.ctx && cur.kv[j] != 0;
      const float f = cur.ks[j] * a.qk_scale_log2;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float v = s[j][g] * f;
        nonfinite |= valid && !__builtin_isfinite(v);
        s[j][g] = valid ? v : -INFINITY;
        need |= s[j][g] > m[g] + slack;
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
        for (int e = 0; e < 16; ++e) acc[g][e] *= alpha;
        m[g] = mn;
      }
    }
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const uint32_t w[4] = {cur.v[j].x, cur.v[j].y, cur.v[j].z, cur.v[j].w};
      float vf[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) vf[e] = code_to_f<KF>(w[e / 4], e % 4);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float p = __builtin_amdgcn_exp2f(s[j][g] - m[g]);
        l[g] += p;
        const float pv = p * cur.vs[j];
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[g][e] = fmaf(pv, vf[e], acc[g][e]);
      }
    }
  };
  ValuTile<NL> t0, t1;
  bool ok0 = nbw > 0 ? fetch(0, t0) : false, ok1 = false;
  for (int i = 0; i < nbw; i += 2) {
    if (i + 1 < nbw) ok1 = fetch(i + 1, t1);
    if (ok0) process(i, t0); else bad_index = true;
    if (i + 1 >= nbw) break;
    if (i + 2 < nbw) ok0 = fetch(i + 2, t0);
    if (ok1) process(i + 1, t1); else bad_index = true;
  }
  if (bad_index && lane == 0) atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
  if (bad_score && lane == 0) atomicOr(a.err_flag, ASTR_FLAG_NONFINITE_SCORE);

#pragma unroll
  for (int g = 0; g < G; ++g) {
    l[g] = strided_sum<LPT>(l[g]);
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[g][e] = strided_sum<LPT>(acc[g][e]);
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      sh.m[wave][g] = m[g];
      sh.l[wave][g] = l[g];
    }
  }
  if (lrow == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 16; ++e) sh.o[wave][g][d0 + e] = acc[g][e];
  }
  __syncthreads();
  finish_partition<QT, G, D>(a, sh, row, seq, tok, head0, part);
}


// ================================ split-K merge

// One wave per (sequence, q head) with more than one partition: lanes load the
// partitions' (m, l) in parallel, take the wave max, and every lane then sums
// its d-slice over the partitions with the merge_softmax weights exp2(m_p - M).
template <typename QT, int D>
__global__ __launch_bounds__(256) void merge_kernel(AttnArgs a) {
  constexpr int kPerLane = (D + kWave - 1) / kWave;
  const int lane = threadIdx.x % kWave;
  const int unit = blockIdx.x * kWaves + threadIdx.x / kWave;  // seq * Hq + h
  if (unit >= a.num_seqs * a.num_q_heads) return;
  const int seq = unit / a.num_q_heads, h = unit % a.num_q_heads;
  const int tok = decode_token(a, seq);
  if (tok < 0) return;
  const RowPlan row = plan_row(a, seq, false);
  if (row.num_parts <= 1) return;
  const int64_t base = (int64_t)unit * a.max_parts;
  float M = -INFINITY;
  for (int p = lane; p < row.num_parts; p += kWave) M = fmaxf(M, a.ws_ml[(base + p) * 2]);
  M = wave_max(M);
  float L = 0.f, O[kPerLane];
#pragma unroll
  for (int e = 0; e < kPerLane; ++e) O[e] = 0.f;
  for (int p0 = 0; p0 < row.num_parts; p0 += kWave) {
    const int p = p0 + lane;
    float w = 0.f, lw = 0.f;
    if (p < row.num_parts) {
      const float mp = a.ws_ml[(base + p) * 2];
      w = mp == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mp - M);
      lw = a.ws_ml[(base + p) * 2 + 1] * w;
    }
    // L = sum over partitions (every lane gets the total)
    lw += shfl_xor(lw, 1);
    lw += shfl_xor(lw, 2);
    lw += shfl_xor(lw, 4);
    lw += shfl_xor(lw, 8);
    lw += shfl_xor(lw, 16);
    lw += shfl_xor(lw, 32);
    L += lw;
    const int np = min(kWave, row.num_parts - p0);
    // 8 partitions per round: all their loads issue before the first use
    for (int q0 = 0; q0 < np; q0 += 8) {
      float v[8][kPerLane], wq[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int q = min(q0 + u, np - 1);
        wq[u] = q0 + u < np ? __shfl(w, q, kWave) : 0.f;
        const float* op = a.ws_o + (base + p0 + q) * D;
#pragma unroll
        for (int e = 0; e < kPerLane; ++e) {
          const int d = lane + e * kWave;
          v[u][e] = d < D ? op[d] : 0.f;
        }
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int e = 0; e < kPerLane; ++e) O[e] = fmaf(v[u][e], wq[u], O[e]);
    }
  }
  QT* out = static_cast<QT*>(a.out) + (int64_t)tok * a.o_tok + (int64_t)h * a.o_head;
  // statistics mode: the merged state itself
  const float inv_l = a.stats != nullptr ? 1.f : 1.f / fmaxf(L, FLT_MIN);
  if (a.stats != nullptr && lane == 0)
    store_row_stats(a.stats, (int64_t)tok * a.num_q_heads + h, M, L);
#pragma unroll
  for (int e = 0; e < kPerLane; ++e) {
    const int d = lane + e * kWave;
    if (d < D) out[d] = from_float<QT>(O[e] * inv_l);
  }
}

// ================================ launch / dispatch

template <typename QT, int D, int G>
int launch(const AttnArgs& a, hipStream_t stream) {
  const dim3 grid((uint32_t)a.max_parts, (uint32_t)a.cache.num_kv_heads, (uint32_t)a.num_seqs);
  if constexpr (sizeof(QT) == 4) {
    constexpr int GS = valu_heads(D, G);
    const dim3 vgrid(grid.x, grid.y * (G / GS), grid.z);
    hipLaunchKernelGGL((decode_valu_kernel<QT, D, G, GS>), vgrid, dim3(kWaves * kWave), 0, stream,
                       a);
  } else {
    hipLaunchKernelGGL((decode_mfma_kernel<QT, D, G, kStages>), grid, dim3(kWaves * kWave), 0,
                       stream, a);
  }
  if (a.max_parts > 1) {
    const int units = a.num_seqs * a.num_q_heads;
    hipLaunchKernelGGL((merge_kernel<QT, D>), dim3((units + kWaves - 1) / kWaves),
                       dim3(kWaves * kWave), 0, stream, a);
  }
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "paged_attention launch");
}

template <typename QT, int D>
int dispatch_group(const AttnArgs& a, int G, hipStream_t s) {
  switch (G) {
    case 1: return launch<QT, D, 1>(a, s);
    case 2: return launch<QT, D, 2>(a, s);
    case 4: return launch<QT, D, 4>(a, s);
    case 8: return launch<QT, D, 8>(a, s);
    case 16:  // fp32 queries: the VALU kernel's passes of 4 heads; f16/bf16 up to D = 128
      if constexpr (sizeof(QT) == 4 || D <= 128) return launch<QT, D, 16>(a, s);
      [[fallthrough]];
    default:
      return fail(ASTR_EUNSUPPORTED, "GQA group size %d not supported for this query dtype", G);
  }
}

template <typename QT>
int dispatch_dim(const AttnArgs& a, int G, hipStream_t s) {
  switch (a.cache.head_dim) {
    case 64: return dispatch_group<QT, 64>(a, G, s);
    case 128: return dispatch_group<QT, 128>(a, G, s);
    case 256: return dispatch_group<QT, 256>(a, G, s);
    default: return fail(ASTR_EUNSUPPORTED, "head_dim %d not in {64,128,256}", a.cache.head_dim);
  }
}

}  // namespace

template <>
int launch_partitioned_kf<KF>(const AttnArgs& a, int32_t q_dtype, hipStream_t stream) {
  const int G = a.num_q_heads / a.cache.num_kv_heads;
  switch (q_dtype) {
    case ASTR_F32: return dispatch_dim<float>(a, G, stream);
    case ASTR_F16: return dispatch_dim<_Float16>(a, G, stream);
    default: return dispatch_dim<bf16_t>(a, G, stream);
  }
}

}  // namespace attn
}  // namespace astr
