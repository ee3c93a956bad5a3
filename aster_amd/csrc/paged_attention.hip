// Ragged paged decode attention over the INT8 KV arena (gfx950).
//
// Work decomposition: one workgroup (4 waves) per (sequence, kv head, split-K
// partition). Every wave owns whole 16-token blocks of the partition
// (blocks w, w+4, ...) and serves all G query heads of the GQA group, so each
// K/V byte is read from HBM once per (sequence, kv head). The physical block ids
// of a wave are read once into a register and picked per block with readlane,
// so the loop issues no dependent vector loads and the next block's K/V loads
// stay in flight while the current block is processed.
//
// bf16/fp16 queries -> decode_mfma_kernel. Per 16-token block:
//   S^T[t][g] = K[t][:] . Q[g][:]  on 16x16x32 f16 MFMAs (A = K rows, B = Q^T),
//   O^T[d][g] += V^T[d][t] P^T[t][g] on 16x16x16 f16 MFMAs (A = V^T, B = P^T).
// INT8 codes are exact in f16: a byte permute builds 0x64xx halves (1024+u),
// the XOR with 0x80 makes u = c+128 and a packed f16 subtract of 1152 leaves c
// exactly. The MFMA output layout of S^T (lane l holds tokens 4*(l/16)+j of head
// l%16) is exactly the B-operand layout P^T needs, so softmax runs in registers
// with no transpose. Queries are rounded to f16 after an exact power-of-two
// rescale that keeps max|q| below 2^15 (the factor is folded into the score
// scale); probabilities (times the V scale) are rounded to f16 for PV.
//
// fp32 queries -> decode_valu_kernel: the same schedule in exact fp32 VALU
// arithmetic (int8 -> fp32 in registers, 16-wide dot products per lane reduced
// with DPP), used where f16 operands would lose query precision.
//
// Both fold dequantization into the score (q.(c*s) = s*(q.c)) and into the
// probability (p*s_v), and run the online softmax in base 2 with a lazily
// raised reference maximum: a block rescales the running (l, acc) only when one
// of its scores exceeds the reference by more than kRescaleSlack. The final
// state is the reference's SoftmaxState (online_attention.py:29-39) up to the
// exp -> exp2 change of base, which cancels in acc / l.
//
// Split-K: partitions of one (sequence, kv head) write (m, l, acc) partials and
// merge_kernel, launched next on the same stream, combines them with the
// merge_softmax rule (online_attention.py:42-63): non-finite maxima weigh 0,
// output = acc / max(l, FLT_MIN) (:35-39). (An in-kernel last-finisher merge
// needs agent-scope fences, which on gfx950 write back and invalidate the
// whole L2 of the XCD per workgroup; the kernel boundary is far cheaper.)
#include <cfloat>
#include <cmath>

#include "common.h"

namespace astr {
namespace {

constexpr int kBlockTokens = 16;
constexpr int kWaves = 4;
constexpr int kMaxBlocksPerWave = 64;  // partition <= 4096 tokens
constexpr int kStages = 2;             // LDS stages per wave in the MFMA kernel
constexpr float kRescaleSlack = 8.0f;  // p = exp2(s - m) <= 2^8 between rescales

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

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
  float* ws_o;          // [num_seqs][num_q_heads][max_parts][D]  unnormalised acc
  float* ws_ml;         // [num_seqs][num_q_heads][max_parts][2]  (m, l)
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

// Per-workgroup shared state: the 4 waves' (m, l, acc).
template <int G, int D>
struct Shared {
  float m[kWaves][G];
  float l[kWaves][G];
  float o[kWaves][G][D];
};

// Combine the 4 waves of the workgroup (already in `sh`) and write either the
// normalised output (single partition) or this partition's partial.
template <typename QT, int G, int D>
__device__ void finish_partition(const DecodeArgs& a, Shared<G, D>& sh, const RowPlan& row,
                                 int seq, int kvh, int part) {
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

// Physical block ids of this wave's blocks (pb0 + wave + 4*i), one per lane.
__device__ __forceinline__ int wave_block_ids(const DecodeArgs& a, int seq, int first, int nbw,
                                              int lane) {
  const int32_t* bt = a.block_tables + (int64_t)seq * a.bt_stride;
  return lane < nbw ? bt[first + kWaves * lane] : 0;
}

// ================================ MFMA kernel (bf16 / fp16 queries)

// One LDS stage holds a 16-token block of one kv head exactly as it sits in
// HBM: K codes (16 rows x D bytes), V codes, then 16 K and 16 V fp32 scales.
// Stages are filled with direct global->LDS loads (global_load_lds_dwordx4),
// so staging costs no VGPRs and a wave can keep NS blocks in flight.
template <int D>
struct Stage {
  static constexpr int kK = 0;
  static constexpr int kV = 16 * D;
  static constexpr int kS = 32 * D;
  static constexpr int kBytes = 32 * D + 128;
  static constexpr int kCodeLoads = 16 * D / 1024;   // 1 KiB wave-loads per K (and per V) tile
  static constexpr int kLoads = 2 * kCodeLoads + 1;  // VMEM instructions per stage
};

typedef __attribute__((address_space(3))) char lds_char_t;

// Byte address of an LDS location, as M0 expects it.
__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return (uint32_t)(uintptr_t)(const lds_char_t*)p;
}

// Direct global -> LDS loads. Each lane's 16 (or 4) bytes land at
// M0 + lane * 16 (or 4). Issued as inline asm so the compiler does not add its
// conservative "wait for every LDS DMA" before unrelated LDS reads; the stage
// pipeline waits for exactly the loads it needs with wait_vmcnt.
__device__ __forceinline__ void lds_dma_x4(const void* gptr, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(lds), "v"(gptr)
               : "memory", "m0");
}

__device__ __forceinline__ void lds_dma_x1(const void* gptr, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off"
               :
               : "s"(lds), "v"(gptr)
               : "memory", "m0");
}

// Wait until at most N vector-memory operations of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// Issue the direct-to-LDS loads of block `phys` (kv head kvh) into stage `st`:
// exactly Stage<D>::kLoads vector-memory instructions (waves are always full,
// so the 32-lane scale load always issues).
template <int D>
__device__ __forceinline__ void stage_block(const DecodeArgs& a, int phys, int kvh, int lane,
                                            char* st) {
  using S = Stage<D>;
  const int64_t off = (int64_t)phys * a.cache.code_block_stride +
                      (int64_t)kvh * a.cache.code_head_stride + lane * 16;
  const uint32_t base = lds_addr(st);
#pragma unroll
  for (int j = 0; j < S::kCodeLoads; ++j)
    lds_dma_x4(a.cache.k_codes + off + j * 1024, base + S::kK + j * 1024);
#pragma unroll
  for (int j = 0; j < S::kCodeLoads; ++j)
    lds_dma_x4(a.cache.v_codes + off + j * 1024, base + S::kV + j * 1024);
  const int64_t so = (int64_t)phys * a.cache.scale_block_stride +
                     (int64_t)kvh * a.cache.scale_head_stride;
  if (lane < 32) {
    const float* src = lane < 16 ? a.cache.k_scales + so + lane : a.cache.v_scales + so + lane - 16;
    lds_dma_x1(src, base + S::kS);
  }
}

// 4 int8 codes -> two f16 pairs holding exactly the codes.
__device__ __forceinline__ void codes_to_f16(uint32_t w, half2_t& lo, half2_t& hi) {
  const uint32_t u = w ^ 0x80808080u;                       // bytes c + 128
  const uint32_t l = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // 1024 + u0, 1024 + u1
  const uint32_t h = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // 1024 + u2, 1024 + u3
  const half2_t bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  lo = __builtin_bit_cast(half2_t, l) - bias;
  hi = __builtin_bit_cast(half2_t, h) - bias;
}

// Byte k of rows r0/r1 -> f16 pair (code[r0][k], code[r1][k]).
template <int K>
__device__ __forceinline__ half2_t column_pair(uint32_t r0, uint32_t r1) {
  constexpr uint32_t sel = 0x0C000C00u | ((4u + K) << 16) | K;
  const uint32_t p = __builtin_amdgcn_perm(r1, r0, sel) ^ 0x64806480u;  // 1152 + c
  const half2_t bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  return __builtin_bit_cast(half2_t, p) - bias;
}

template <int K>
__device__ __forceinline__ half4_t v_operand(const uint32_t (&v)[4]) {
  const half2_t a01 = column_pair<K>(v[0], v[1]);
  const half2_t a23 = column_pair<K>(v[2], v[3]);
  return half4_t{a01[0], a01[1], a23[0], a23[1]};
}

template <int D, int G>
constexpr int stage0_bytes() {
  constexpr int staging = kWaves * Stage<D>::kBytes;
  constexpr int merge = (int)sizeof(Shared<G, D>);
  return staging > merge ? staging : merge;
}

template <typename QT, int D, int G, int NS>
__global__ __launch_bounds__(256) void decode_mfma_kernel(DecodeArgs a) {
  static_assert(D == 64 || D == 128 || D == 256, "head_dim");
  static_assert(G >= 1 && G <= 16, "GQA group");
  static_assert(NS == 2 || NS == 3, "stages");
  using S = Stage<D>;
  constexpr int KCH = D / 64;  // 16-byte K chunks per lane per block
  constexpr int VB = D / 16;   // V bytes per lane per token row
  constexpr int NQK = D / 32;  // 16x16x32 MFMAs per block for S^T
  constexpr int NPV = D / 16;  // 16x16x16 MFMAs per block for O^T

  // One __shared__ object per stage: the compiler tracks outstanding LDS-DMA
  // writes per object, so reading stage s waits only for stage s's loads.
  __shared__ __attribute__((aligned(16))) char lds0[stage0_bytes<D, G>()];
  __shared__ __attribute__((aligned(16))) char lds1[kWaves * S::kBytes];
  __shared__ __attribute__((aligned(16))) char lds2[NS == 3 ? kWaves * S::kBytes : 16];
  const int part = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int r = lane & 15, qg = lane >> 4;
  const bool gvalid = r < G;

  // ---- prologue: query rows and (for window == 0) this wave's block ids do not
  // depend on the context length, so their loads issue together with it.
  uint4 qraw[KCH][2];
  {
    const QT* qp = static_cast<const QT*>(a.q) + seq * a.q_tok +
                   (int64_t)(kvh * G + (gvalid ? r : 0)) * a.q_head + 16 * qg;
#pragma unroll
    for (int h = 0; h < KCH; ++h) {
      const uint4* src = reinterpret_cast<const uint4*>(qp + 64 * h);
      qraw[h][0] = src[0];
      qraw[h][1] = src[1];
    }
  }
  const int32_t* bt = a.block_tables + (int64_t)seq * a.bt_stride;
  const int per_wave = (a.part_blocks + kWaves - 1) / kWaves;
  int spec = part * a.part_blocks + wave + kWaves * lane;  // block index if kv_begin == 0
  int ids = (a.window == 0 && lane < per_wave && spec < a.bt_stride) ? bt[spec] : 0;
  const RowPlan row = plan_row(a, seq, part == 0 && kvh == 0 && threadIdx.x == 0);
  if (part >= row.num_parts) return;
  const int pb0 = row.first_blk + part * a.part_blocks;
  const int pb1 = min(row.last_blk, pb0 + a.part_blocks);
  const int first = pb0 + wave;
  const int nbw = first < pb1 ? (pb1 - first + kWaves - 1) / kWaves : 0;
  if (a.window != 0) ids = lane < nbw ? bt[first + kWaves * lane] : 0;
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

  // ---- query operand: lane holds Q[g = r][d] for d in 16*qg + 64*h + [0, 16), as
  // f16 after an exact 2^-e rescale keeping max|q| < 2^15 (e folded into cf)
  half8_t qop[NQK];
  float cf;
  {
    float qv[KCH][16];
    float mx = 0.f;
#pragma unroll
    for (int h = 0; h < KCH; ++h) {
      const QT* e0 = reinterpret_cast<const QT*>(&qraw[h][0]);
      const QT* e1 = reinterpret_cast<const QT*>(&qraw[h][1]);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        qv[h][i] = gvalid ? to_float<QT>(e0[i]) : 0.f;
        qv[h][8 + i] = gvalid ? to_float<QT>(e1[i]) : 0.f;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fabsf(qv[h][i]));
    }
    mx = fmaxf(mx, shfl_xor(mx, 16));
    mx = fmaxf(mx, shfl_xor(mx, 32));
    int ex = 0;
    if (mx >= 32768.f) {
      frexpf(mx, &ex);
      ex -= 15;  // mx * 2^-ex < 2^15
    }
    const float down = ldexpf(1.f, -ex);
#pragma unroll
    for (int kk = 0; kk < NQK; ++kk)
#pragma unroll
      for (int e = 0; e < 8; ++e) qop[kk][e] = (_Float16)(qv[kk / 2][(kk % 2) * 8 + e] * down);
    cf = a.qk_scale_log2 * ldexpf(1.f, ex);
  }

  float4_t acc[NPV];
#pragma unroll
  for (int n = 0; n < NPV; ++n) acc[n] = float4_t{0.f, 0.f, 0.f, 0.f};
  float m = gvalid ? -INFINITY : 0.f;  // invalid head columns never contribute
  float l = 0.f;
  bool bad_score = false;

  auto step = [&](int i, char* st) {
    // wait until block i has landed: later stages (up to NS-1) may stay in flight
    const int later = min(NS - 1, nblk - 1 - i);
    if (later >= 3) wait_vmcnt<3 * S::kLoads>();
    else if (later == 2) wait_vmcnt<2 * S::kLoads>();
    else if (later == 1) wait_vmcnt<S::kLoads>();
    else wait_vmcnt<0>();

    // ---- S^T = K . Q^T (A = K rows from LDS)
    float4_t s4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int h = 0; h < KCH; ++h) {
      const uint4 c = *reinterpret_cast<const uint4*>(st + S::kK + r * D + 16 * qg + 64 * h);
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        half2_t p0, p1, p2, p3;
        codes_to_f16(sub ? c.z : c.x, p0, p1);
        codes_to_f16(sub ? c.w : c.y, p2, p3);
        const half8_t kop = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
        s4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop, qop[2 * h + sub], s4, 0, 0, 0);
      }
    }
    const float4_t ks = *reinterpret_cast<const float4_t*>(st + S::kS + 16 * qg);
    const float4_t vs = *reinterpret_cast<const float4_t*>(st + S::kS + 64 + 16 * qg);
    uint32_t vw[4][VB / 4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const char* rowp = st + S::kV + (4 * qg + j) * D + r * VB;
      if constexpr (VB == 4) {
        vw[j][0] = *reinterpret_cast<const uint32_t*>(rowp);
      } else if constexpr (VB == 8) {
        const uint2 w = *reinterpret_cast<const uint2*>(rowp);
        vw[j][0] = w.x;
        vw[j][1] = w.y;
      } else {
        const uint4 w = *reinterpret_cast<const uint4*>(rowp);
        vw[j][0] = w.x;
        vw[j][1] = w.y;
        vw[j][2] = w.z;
        vw[j][3] = w.w;
      }
    }

    // ---- scores of tokens 4*qg + j for head g = r (base-2, dequantised)
    const int blk = first + kWaves * i;
    const int tok0 = blk * kBlockTokens + 4 * qg;
    const bool edge = blk * kBlockTokens < row.kv_begin || (blk + 1) * kBlockTokens > row.ctx;
    float sc[4];
    bool need = false, nonfinite = false;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v = s4[j] * (ks[j] * cf);
      bool valid = gvalid;
      if (edge) valid = valid && tok0 + j >= row.kv_begin && tok0 + j < row.ctx;
      nonfinite |= valid && !__builtin_isfinite(v);
      v = valid ? v : -INFINITY;
      need |= v > m + kRescaleSlack;
      sc[j] = v;
    }
    if (__ballot(nonfinite) != 0) bad_score = true;
    if (__ballot(need) != 0) {
      float tmax = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
      tmax = fmaxf(tmax, shfl_xor(tmax, 16));
      tmax = fmaxf(tmax, shfl_xor(tmax, 32));
      const float mn = fmaxf(m, tmax);
      const float alpha = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mn);
      l *= alpha;
#pragma unroll
      for (int n = 0; n < NPV; ++n) acc[n] *= alpha;
      m = mn;
    }
    half4_t pop;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float p = __builtin_amdgcn_exp2f(sc[j] - m);
      l += p;
      pop[j] = (_Float16)(p * vs[j]);
    }
    // ---- O^T += V^T . P^T (row m of MFMA n is d = VB*m + n)
#pragma unroll
    for (int n = 0; n < NPV; ++n) {
      const uint32_t col[4] = {vw[0][n / 4], vw[1][n / 4], vw[2][n / 4], vw[3][n / 4]};
      half4_t vop;
      switch (n % 4) {
        case 0: vop = v_operand<0>(col); break;
        case 1: vop = v_operand<1>(col); break;
        case 2: vop = v_operand<2>(col); break;
        default: vop = v_operand<3>(col); break;
      }
      acc[n] = __builtin_amdgcn_mfma_f32_16x16x16f16(vop, pop, acc[n], 0, 0, 0);
    }
    // refill this stage with block i + NS (its LDS reads above have completed:
    // their values fed the MFMAs)
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
  l += shfl_xor(l, 16);
  l += shfl_xor(l, 32);
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
  finish_partition<QT, G, D>(a, sh, row, seq, kvh, part);
}

// ================================ exact fp32 VALU kernel (fp32 queries)

template <int NL>
struct ValuTile {
  uint4 k[NL];
  uint4 v[NL];
  float ks[NL];
  float vs[NL];
};

template <typename QT, int D, int G>
__global__ __launch_bounds__(256) void decode_valu_kernel(DecodeArgs a) {
  constexpr int LPT = D / 16;             // lanes per token row
  constexpr int TPL = kWave / LPT;        // token rows per load instruction
  constexpr int NL = kBlockTokens / TPL;  // load instructions per block
  constexpr int kLoadBytes = kWave * 16;
  static_assert(NL >= 1 && NL * TPL == kBlockTokens, "unsupported head_dim");

  __shared__ Shared<G, D> sh;
  const int part = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
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
    const QT* qp = static_cast<const QT*>(a.q) + seq * a.q_tok + (int64_t)kvh * G * a.q_head + d0;
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
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[g][i] = 0.f;
  }
  const int8_t* kbase = a.cache.k_codes + (int64_t)kvh * a.cache.code_head_stride + lane * 16;
  const int8_t* vbase = a.cache.v_codes + (int64_t)kvh * a.cache.code_head_stride + lane * 16;
  const float* ksbase = a.cache.k_scales + (int64_t)kvh * a.cache.scale_head_stride + lrow;
  const float* vsbase = a.cache.v_scales + (int64_t)kvh * a.cache.scale_head_stride + lrow;
  auto load = [&](int phys, ValuTile<NL>& t) {
    const int8_t* kp = kbase + (int64_t)phys * a.cache.code_block_stride;
    const int8_t* vp = vbase + (int64_t)phys * a.cache.code_block_stride;
    const float* ksp = ksbase + (int64_t)phys * a.cache.scale_block_stride;
    const float* vsp = vsbase + (int64_t)phys * a.cache.scale_block_stride;
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      t.k[j] = *reinterpret_cast<const uint4*>(kp + j * kLoadBytes);
      t.v[j] = *reinterpret_cast<const uint4*>(vp + j * kLoadBytes);
      t.ks[j] = ksp[j * TPL];
      t.vs[j] = vsp[j * TPL];
    }
  };

  const int ids = wave_block_ids(a, seq, first, nbw, lane);
  bool bad_index = false, bad_score = false;
  auto fetch = [&](int i, ValuTile<NL>& t) -> bool {
    const int phys = __builtin_amdgcn_readlane(ids, i);
    const bool ok = (unsigned)phys < (unsigned)a.cache.num_blocks;
    if (ok) load(phys, t);
    return ok;
  };
  auto process = [&](int i, const ValuTile<NL>& cur) {
    const int blk = first + kWaves * i;
    float s[NL][G];
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const uint32_t w[4] = {cur.k[j].x, cur.k[j].y, cur.k[j].z, cur.k[j].w};
      float kf[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) kf[e] = i8_to_f(w[e / 4], e % 4);
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
        for (int e = 0; e < 16; ++e) acc[g][e] *= alpha;
        m[g] = mn;
      }
    }
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const uint32_t w[4] = {cur.v[j].x, cur.v[j].y, cur.v[j].z, cur.v[j].w};
      float vf[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) vf[e] = i8_to_f(w[e / 4], e % 4);
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
  finish_partition<QT, G, D>(a, sh, row, seq, kvh, part);
}

// ================================ split-K merge

// One wave per (sequence, q head) with more than one partition: lanes load the
// partitions' (m, l) in parallel, take the wave max, and every lane then sums
// its d-slice over the partitions with the merge_softmax weights exp2(m_p - M).
template <typename QT, int D>
__global__ __launch_bounds__(256) void merge_kernel(DecodeArgs a) {
  constexpr int kPerLane = (D + kWave - 1) / kWave;
  const int lane = threadIdx.x % kWave;
  const int unit = blockIdx.x * kWaves + threadIdx.x / kWave;  // seq * Hq + h
  if (unit >= a.num_seqs * a.num_q_heads) return;
  const int seq = unit / a.num_q_heads, h = unit % a.num_q_heads;
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
  QT* out = static_cast<QT*>(a.out) + seq * a.o_tok + (int64_t)h * a.o_head;
  const float inv_l = 1.f / fmaxf(L, FLT_MIN);
#pragma unroll
  for (int e = 0; e < kPerLane; ++e) {
    const int d = lane + e * kWave;
    if (d < D) out[d] = from_float<QT>(O[e] * inv_l);
  }
}

// ================================ launch / dispatch

template <typename QT, int D, int G>
int launch_decode(const DecodeArgs& a, hipStream_t stream) {
  const dim3 grid((uint32_t)a.max_parts, (uint32_t)a.cache.num_kv_heads, (uint32_t)a.num_seqs);
  if constexpr (sizeof(QT) == 4) {
    hipLaunchKernelGGL((decode_valu_kernel<QT, D, G>), grid, dim3(kWaves * kWave), 0, stream, a);
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
int dispatch_group(const DecodeArgs& a, int G, hipStream_t s) {
  switch (G) {
    case 1: return launch_decode<QT, D, 1>(a, s);
    case 2: return launch_decode<QT, D, 2>(a, s);
    case 4: return launch_decode<QT, D, 4>(a, s);
    case 8: return launch_decode<QT, D, 8>(a, s);
    case 16:
      if constexpr (sizeof(QT) == 2 && D <= 128) return launch_decode<QT, D, 16>(a, s);
      [[fallthrough]];
    default:
      return fail(ASTR_EUNSUPPORTED, "GQA group size %d not supported for this query dtype", G);
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

bool valid_partition(int pt) {
  return pt > 0 && pt % (kBlockTokens * kWaves) == 0 &&
         pt <= kBlockTokens * kWaves * kMaxBlocksPerWave;
}

int64_t max_parts_for(int32_t max_context_len, int32_t partition_tokens) {
  const int64_t blocks = ((int64_t)max_context_len + kBlockTokens - 1) / kBlockTokens;
  const int64_t pb = partition_tokens / kBlockTokens;
  const int64_t parts = (blocks + pb - 1) / pb;
  return parts < 1 ? 1 : parts;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// [partial acc][partial (m, l)]
struct WorkspaceLayout {
  size_t o_bytes, ml_bytes;
  size_t total() const { return o_bytes + ml_bytes; }
};

WorkspaceLayout workspace_layout(int32_t num_seqs, int32_t num_q_heads, int32_t head_dim,
                                 int64_t parts) {
  WorkspaceLayout w{0, 0};
  if (parts <= 1) return w;
  const size_t rows = (size_t)num_seqs * num_q_heads * parts;
  w.o_bytes = align256(rows * head_dim * sizeof(float));
  w.ml_bytes = align256(rows * 2 * sizeof(float));
  return w;
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
  if (!valid_partition(pt)) return 0;
  return workspace_layout(num_seqs, num_q_heads, head_dim, max_parts_for(max_context_len, pt))
      .total();
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
  if (num_seqs > 65535) return fail(ASTR_EUNSUPPORTED, "more than 65535 sequences per launch");
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
  if (!valid_partition(pt))
    return fail(ASTR_EINVAL, "partition_tokens %d must be a positive multiple of %d up to %d", pt,
                kBlockTokens * kWaves, kBlockTokens * kWaves * kMaxBlocksPerWave);
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
      cache->code_block_stride % 16 || cache->code_head_stride % 16 ||
      !aligned16(cache->k_scales) || !aligned16(cache->v_scales) ||
      cache->scale_block_stride % 4 || cache->scale_head_stride % 4)
    return fail(ASTR_EINVAL, "cache code and scale blocks must be 16-byte aligned");
  const int64_t parts = max_parts_for(max_context_len, pt);
  if (parts > 65535)
    return fail(ASTR_EUNSUPPORTED, "too many split-K partitions (%lld)", (long long)parts);
  const WorkspaceLayout ws = workspace_layout(num_seqs, num_q_heads, cache->head_dim, parts);
  if (ws.total() > 0 && (workspace == nullptr || workspace_bytes < ws.total() ||
                         (reinterpret_cast<uintptr_t>(workspace) & 255u) != 0))
    return fail(ASTR_EINVAL, "a 256-byte aligned workspace of %zu bytes is required (%zu given)",
                ws.total(), workspace_bytes);

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
  if (ws.total() > 0) {
    char* base = static_cast<char*>(workspace);
    a.ws_o = reinterpret_cast<float*>(base);
    a.ws_ml = reinterpret_cast<float*>(base + ws.o_bytes);
  }
  a.err_flag = err_flag;
  const int G = num_q_heads / cache->num_kv_heads;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (q_dtype) {
    case ASTR_F32: return dispatch_dim<float>(a, G, s);
    case ASTR_F16: return dispatch_dim<_Float16>(a, G, s);
    default: return dispatch_dim<bf16_t>(a, G, s);
  }
}
