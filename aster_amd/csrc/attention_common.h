// Building blocks shared by the paged decode attention kernels (gfx950):
// launch arguments, the LDS block stage filled by direct global->LDS loads,
// exact int8 -> f16 operand conversion, the query operand and the per-block
// MFMA step (scores, online softmax, P.V).
#pragma once

#include <cfloat>
#include <cmath>

#include "common.h"

namespace astr {
namespace attn {

constexpr int kBlockTokens = 16;
constexpr int kWaves = 4;              // waves per workgroup
constexpr int kMaxBlocksPerWave = 64;  // block ids one wave keeps in a register
// stream-K: blocks one wave may stream (its block list goes in windows of 64)
constexpr int kMaxBlocksPerWaveSK = 1024;
// stream-K split costs: any block that is not a prefix pack's, and the start of a work
// row with blocks (its query load and the partial written when it ends). A pack
// block's cost is chosen per launch within [kSkPackCostMin, kSkPackCostMax]: at most
// the share that keeps the pack blocks' cost at half the total (SkSplit). The split
// gives every wave an equal share of the total; the host sizes the wave capacity from
// the same figures (the cheapest pack cost).
constexpr int kSkSeqCost = 50, kSkRowCost = 135;
constexpr int kSkPackCostMax = 32, kSkPackCostMin = 16;
constexpr float kRescaleSlack = 8.0f;  // p = exp2(s - m) <= 2^8 between rescales
// PV weights p * v_scale are rounded to f16: with p <= 2^8 (kRescaleSlack) and every
// v_scale <= kVWeightCap they stay below 2^15 (f16's largest finite value is 65504).
constexpr float kVWeightCap = 128.0f;

// Larger V scales in the decode kernels: the piece's running maximum m is the scores'
// running maximum plus koff (a non-negative integer), so every weight p = exp2(s - m)
// and the normaliser l carry 2^-koff, which cancels in acc / l and in the merge of
// (m, l, acc) partials. A block whose (weight-scaled) V scales exceed vlim =
// kVWeightCap * 2^koff grows koff by the exponent they need, through the same
// rescale of l and acc as a new score maximum. Every piece starts at {0, kVWeightCap}.
// `screen` is the lane's limit for the one staged scale it tests per block, so that a
// single compare and ballot per block finds the rare blocks (vrange_start).
struct VRange {
  float koff, vlim, screen;
};

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

struct AttnArgs {
  const void* q;
  int64_t q_tok, q_head;
  void* out;
  int64_t o_tok, o_head;
  astr_paged_kv cache;
  const int32_t* block_tables;
  int32_t bt_stride;
  const int32_t* context_lens;
  // Packed queries: sequence s owns query/output token rows [q_start[s], q_start[s+1]).
  // nullptr: one query token per sequence, at row s.
  const int32_t* q_start;
  int32_t num_q_tokens;  // rows of query/out (upper bound of q_start[num_seqs])
  int32_t max_q_len;     // host-declared bound of q_start[s+1] - q_start[s] (1 without q_start)
  int32_t causal;        // multi-token rows: key k is visible to query position p iff k <= p
  int32_t num_seqs, num_q_heads;
  float qk_scale_log2;  // softmax scale * log2(e)
  int32_t window;
  // fixed-size split-K partitions
  int32_t part_blocks;  // blocks per partition
  int32_t max_parts;
  // stream-K: equal contiguous block ranges per wave. The entry point passes the
  // workspace capacity in total_waves and the minimum in min_waves; the launcher
  // settles total_waves from the kernel's occupancy.
  int32_t total_waves;
  int32_t min_waves;
  int32_t pref_waves;  // stream-K: waves the GPU holds at once (set by the launcher)
  float* ws_o;          // partial acc (layout depends on the split mode)
  float* ws_ml;         // partial (m, l)
  int32_t* ws_seq;      // stream-K: block prefix over its work rows [num_packs + num_seqs + 1]
  int32_t* ws_ne;       // stream-K: work rows with blocks before each row [same]
  // stream-K prefix packs: num_packs records of 1 + pack_rows int32, [shared blocks,
  // member sequences (-1: empty)]; members read the pack's blocks in one MFMA tile,
  // query column p * G + g for member p, head g of the group (pack_rows * G <= 16)
  const int32_t* packs;
  int32_t num_packs, pack_rows;
  int32_t slot_cols;    // stream-K: columns of one partial slot (G, or pack_rows * G)
  int32_t* ws_pack;     // stream-K: per sequence, [pack column k * pack_rows + p or -1,
                        // the pack's first block, its end (the per-head order), the
                        // rows with blocks before the pack]
  // statistics mode (fp32 queries, fixed partitions): per (token row, query head) the
  // exact maximum score and the mass sum(exp(score - maximum)) at stats[(t * Hq + h) * 2
  // + {0, 1}], and out holds the unnormalised numerator; nullptr: normalised rows
  float* stats;
  // planned decode with the step's append: each decode row's newest token (position
  // ctx - 1) as key and value rows of the query dtype ([num_seqs, Hkv, D], strides in
  // elements) with its cache slot, quantized and written by the wave that streams the
  // block holding it; nullptr: the token was appended beforehand
  const void* new_k;
  const void* new_v;
  int64_t nk_tok, nk_head, nv_tok, nv_head;
  const int64_t* new_slots;
  int32_t* err_flag;
};

// Statistics of one row from its merged base-2 state (maximum m, mass l, numerator
// acc): the maximum back in score units; a row that saw no key keeps (-inf, 0)
// (online_attention.py:163-170 starts every row there).
__device__ __forceinline__ void store_row_stats(float* stats, int64_t row, float m, float l) {
  stats[row * 2] = l > 0.f ? m * (1.f / kLog2e) : -INFINITY;
  stats[row * 2 + 1] = l;
}

// Query/output token rows [begin, begin + count) of sequence `seq` (count is
// returned). A q_start entry that is negative, decreasing or beyond num_q_tokens
// gives count 0 and raises the index flag, so no kernel indexes outside query/out.
// So does a row longer than the declared max_q_len: the host launches the chunk
// kernel only when that bound is 2 or more, and no kernel may leave such a row's
// output unwritten without a flag.
//
// decode_token: the token row of `seq` when it carries exactly one query token
// (a decode row), else -1: sequences with several query tokens belong to the
// prefill kernel and sequences with none produce no output.
__device__ __forceinline__ int seq_queries(const AttnArgs& a, int seq, int& begin) {
  if (a.q_start == nullptr) {
    begin = seq;
    return 1;
  }
  const int b = a.q_start[seq], e = a.q_start[seq + 1];
  if (b < 0 || e < b || e > a.num_q_tokens || e - b > a.max_q_len) {  // no rows, flagged
    atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
    begin = 0;
    return 0;
  }
  begin = b;
  return e - b;
}

__device__ __forceinline__ int decode_token(const AttnArgs& a, int seq) {
  int begin;
  return seq_queries(a, seq, begin) == 1 ? begin : -1;
}

// Visible key range of a decode row: tokens [kv_begin, ctx), blocks [first, last).
struct RowSpan {
  int ctx, kv_begin, first_blk, last_blk;
};

__device__ __forceinline__ int clamp_ctx(const AttnArgs& a, int ctx, bool report) {
  const int cap = a.bt_stride * kBlockTokens;
  if (ctx < 0 || ctx > cap) {
    if (report) atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
    ctx = ctx < 0 ? 0 : cap;
  }
  return ctx;
}

__device__ __forceinline__ RowSpan row_span(const AttnArgs& a, int ctx) {
  RowSpan r;
  r.ctx = ctx;
  r.kv_begin = (a.window > 0 && ctx > a.window) ? ctx - a.window : 0;
  r.first_blk = r.kv_begin / kBlockTokens;
  r.last_blk = (ctx + kBlockTokens - 1) / kBlockTokens;
  return r;
}

// ---- LDS stage of one 16-token block of one kv head, as it sits in HBM:
// K codes (16 rows x D bytes), V codes, 16 K and 16 V fp32 scales, then the 16
// key-padding bytes of the block (loaded only when the arena has them).
template <int D>
struct Stage {
  static constexpr int kK = 0;
  static constexpr int kV = 16 * D;
  static constexpr int kS = 32 * D;
  static constexpr int kF = 32 * D + 128;
  static constexpr int kBytes = 32 * D + 144;
  static constexpr int kCodeLoads = 16 * D / 1024;   // 1 KiB wave-loads per K (and per V) tile
  static constexpr int kLoads = 2 * kCodeLoads + 1;  // vector-memory instructions per stage
};

typedef __attribute__((address_space(3))) char lds_char_t;

// Byte address of an LDS location, as M0 expects it.
__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return (uint32_t)(uintptr_t)(const lds_char_t*)p;
}

// Direct global -> LDS loads. Each lane's 16 (or 4) bytes land at
// M0 + lane * 16 (or 4). Issued as inline asm so the compiler does not add its
// conservative "wait for every LDS DMA" before unrelated LDS reads; the stage
// pipelines wait for exactly the loads they need with wait_vmcnt. Each helper
// declares M0 as an output operand (a definition of M0 in the compiler's view), so
// no value the compiler keeps in M0 (LDS DMA builtins, movrel indexing, M0
// initialisations it hoists) is assumed to live across one of them.
__device__ __forceinline__ void lds_dma_x4(const void* gptr, uint32_t lds) {
  int m0;
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, off"
               : "={m0}"(m0)
               : "s"(lds), "v"(gptr)
               : "memory");
}

__device__ __forceinline__ void lds_dma_x1(const void* gptr, uint32_t lds) {
  int m0;
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %2, off"
               : "={m0}"(m0)
               : "s"(lds), "v"(gptr)
               : "memory");
}

// The same with a wave-uniform 64-bit base in SGPRs and a 32-bit per-lane byte offset
// (the saddr form: no 64-bit per-lane address to hold). No instruction offset: the
// LDS destination is M0 + lane * 16 (or 4) exactly.
__device__ __forceinline__ void lds_dma_x4_s(const void* sbase, uint32_t voff, uint32_t lds) {
  int m0;
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, %3"
               : "={m0}"(m0)
               : "s"(lds), "v"(voff), "s"(sbase)
               : "memory");
}

__device__ __forceinline__ void lds_dma_x1_s(const void* sbase, uint32_t voff, uint32_t lds) {
  int m0;
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %2, %3"
               : "={m0}"(m0)
               : "s"(lds), "v"(voff), "s"(sbase)
               : "memory");
}

// Wait until at most N vector-memory operations of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// A wave-uniform pointer as the compiler's uniformity analysis sees it (values that
// came out of LDS count as per-lane there): the saddr operands need it in SGPRs.
template <typename T>
__device__ __forceinline__ const T* uniform_ptr(const T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const T*>(((uint64_t)hi << 32) | lo);
}

// K tiles are staged with the 16-byte chunks of each key row XOR-swizzled: chunk c of
// row r sits at chunk position c ^ k_swizzle<D>(r) of that row. Operand reads (lane
// (qg, r) reads chunk qg + 4h of row r) on rows D bytes apart otherwise meet LDS bank
// conflicts: 1.2x (D = 64, 128) to 1.45x (D = 256) the cycles of a contiguous
// 16-byte-per-lane read on gfx950. These swizzles, picked by timing every linear map
// of the row bits, read as fast as the contiguous pattern. The direct-to-LDS loads
// apply it through each lane's source chunk; every byte stays in its row, and each
// load still covers one contiguous KiB of the block.
template <int D>
__device__ __forceinline__ int k_swizzle(int r) {
  if constexpr (D == 64) return (r >> 1) & 2;
  else if constexpr (D == 128) return ((r << 1) & 4) | ((r >> 1) & 2);
  else return r & 15;
}
// Byte offset of d-chunk c (bytes 16c .. 16c+15) of key row r in a staged K tile (and,
// the swizzle being an involution, the source chunk of staging slot (r, c)).
template <int D>
__device__ __forceinline__ int k_chunk(int r, int c) {
  return r * D + 16 * (c ^ k_swizzle<D>(r));
}

// Issue the direct-to-LDS loads of block `phys` (kv head kvh) into stage `st`:
// Stage<D>::kLoads vector-memory instructions (waves are always full, so the
// 32-lane scale load always issues), plus one for the block's 16 key-padding bytes
// when the arena has them.
template <int D>
__device__ __forceinline__ void stage_block(const AttnArgs& a, int phys, int kvh, int lane,
                                            char* st) {
  using S = Stage<D>;
  const int64_t off = (int64_t)phys * a.cache.code_block_stride +
                      (int64_t)kvh * a.cache.code_head_stride;  // wave-uniform
  const uint32_t base = lds_addr(st);
  const int8_t* const kb = uniform_ptr(a.cache.k_codes + off);
  const int8_t* const vb = uniform_ptr(a.cache.v_codes + off);
#pragma unroll
  for (int j = 0; j < S::kCodeLoads; ++j)
    lds_dma_x4_s(kb, k_chunk<D>((64 * j + lane) / (D / 16), lane % (D / 16)),
                 base + S::kK + j * 1024);
#pragma unroll
  for (int j = 0; j < S::kCodeLoads; ++j)
    lds_dma_x4_s(vb, lane * 16 + j * 1024, base + S::kV + j * 1024);
  const int64_t so = (int64_t)phys * a.cache.scale_block_stride +
                     (int64_t)kvh * a.cache.scale_head_stride;
  if (lane < 32) {
    const float* src = lane < 16 ? a.cache.k_scales + so + lane : a.cache.v_scales + so + lane - 16;
    lds_dma_x1(src, base + S::kS);
  }
  // key padding bytes: one more instruction, issued last, only when the arena has
  // them. Stage pipelines count kLoads per stage: with this extra load their waits
  // let fewer loads stay in flight than allowed, never more, as loads complete in order.
  if (a.cache.key_valid != nullptr && lane < 4)
    lds_dma_x1_s(uniform_ptr(a.cache.key_valid + (int64_t)phys * kBlockTokens), lane * 4,
                 base + S::kF);
}

// ---- exact code -> f16 operands (int8; FP8 E4M3FN values times 2^-8; FP8 E5M2)

// 4 codes -> two f16 pairs. int8: a byte permute builds 0x64xx halves (1024 + u)
// with u = c + 128, then 1152 is subtracted. FP8: each code byte goes to the high
// byte of its half.
template <int KF = kInt8>
__device__ __forceinline__ void codes_to_f16(uint32_t w, half2_t& lo, half2_t& hi) {
  if constexpr (KF == kInt8) {
    const uint32_t u = w ^ 0x80808080u;                                      // bytes c + 128
    const uint32_t l = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // 1024 + u0, 1024 + u1
    const uint32_t h = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // 1024 + u2, 1024 + u3
    const half2_t bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    lo = __builtin_bit_cast(half2_t, l) - bias;
    hi = __builtin_bit_cast(half2_t, h) - bias;
  } else {
    lo = __builtin_bit_cast(half2_t, fp8_hi_bytes_to_f16<KF>(__builtin_amdgcn_perm(0u, w, 0x010C000Cu)));
    hi = __builtin_bit_cast(half2_t, fp8_hi_bytes_to_f16<KF>(__builtin_amdgcn_perm(0u, w, 0x030C020Cu)));
  }
}

// Byte k of rows r0/r1 -> f16 pair (code[r0][k], code[r1][k]).
template <int K, int KF = kInt8>
__device__ __forceinline__ half2_t column_pair(uint32_t r0, uint32_t r1) {
  if constexpr (KF == kInt8) {
    constexpr uint32_t sel = 0x0C000C00u | ((4u + K) << 16) | K;
    const uint32_t p = __builtin_amdgcn_perm(r1, r0, sel) ^ 0x64806480u;  // 1152 + c
    const half2_t bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    return __builtin_bit_cast(half2_t, p) - bias;
  } else {
    constexpr uint32_t sel = ((4u + K) << 24) | 0x000C0000u | (K << 8) | 0x0Cu;
    return __builtin_bit_cast(half2_t, fp8_hi_bytes_to_f16<KF>(__builtin_amdgcn_perm(r1, r0, sel)));
  }
}

// INT8 V operands of the decode kernels carry the code plus kVBias (exact in f16): the
// byte permute and XOR build 1152 + c directly, and the PV accumulators drop
// kVBias * sum_k(weight_k) once per piece (remove_v_bias) instead of every code paying
// for a subtraction.
constexpr float kVBias = 1152.f;
// Where the decode kernels use them: INT8 codes at D <= 128 (at D = 256 the weight-sum
// tile would take the partitioned kernel past 2 waves per SIMD).
template <int D, int KF>
constexpr bool biased_v() { return KF == kInt8 && D <= 128; }
template <int K>
__device__ __forceinline__ half2_t column_pair_biased(uint32_t r0, uint32_t r1) {
  constexpr uint32_t sel = 0x0C000C00u | ((4u + K) << 16) | K;
  return __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(r1, r0, sel) ^ 0x64806480u);  // 1152 + c
}
template <int K>
__device__ __forceinline__ half4_t v_operand_biased(const uint32_t (&v)[4]) {
  const half2_t a01 = column_pair_biased<K>(v[0], v[1]);
  const half2_t a23 = column_pair_biased<K>(v[2], v[3]);
  return half4_t{a01[0], a01[1], a23[0], a23[1]};
}

template <int K, int KF = kInt8>
__device__ __forceinline__ half4_t v_operand(const uint32_t (&v)[4]) {
  const half2_t a01 = column_pair<K, KF>(v[0], v[1]);
  const half2_t a23 = column_pair<K, KF>(v[2], v[3]);
  return half4_t{a01[0], a01[1], a23[0], a23[1]};
}

// ---- query operand: lane (qg = lane/16, r = lane%16) holds Q[g = r][d] for
// d in 16*qg + 64*h + [0, 16), h < D/64 (rows r >= G are zero).

template <int D>
struct QueryRaw {
  uint4 w[D / 64][2];
};

// Lane (qg, r)'s part of query row r of kv head kvh, token row tok (rows r >= G read
// row 0 and are zeroed where they are quantized).
template <typename QT, int G>
__device__ __forceinline__ const QT* query_lane_ptr(const AttnArgs& a, int tok, int kvh, int r,
                                                    int qg) {
  return static_cast<const QT*>(a.q) + (int64_t)tok * a.q_tok +
         (int64_t)(kvh * G + (r < G ? r : 0)) * a.q_head + 16 * qg;
}

// Lane (qg, r)'s part of query head `head`, token row tok (any column layout).
template <typename QT>
__device__ __forceinline__ const QT* query_col_ptr(const AttnArgs& a, int tok, int head, int qg) {
  return static_cast<const QT*>(a.q) + (int64_t)tok * a.q_tok + (int64_t)head * a.q_head + 16 * qg;
}

template <typename QT, int D>
__device__ __forceinline__ void load_query_at(const QT* qp, QueryRaw<D>& q) {
#pragma unroll
  for (int h = 0; h < D / 64; ++h) {
    const uint4* src = reinterpret_cast<const uint4*>(qp + 64 * h);
    q.w[h][0] = src[0];
    q.w[h][1] = src[1];
  }
}

template <typename QT, int D, int G>
__device__ __forceinline__ void load_query(const AttnArgs& a, int tok, int kvh, int r, int qg,
                                           QueryRaw<D>& q) {
  load_query_at<QT, D>(query_lane_ptr<QT, G>(a, tok, kvh, r, qg), q);
}

typedef int int4_t __attribute__((ext_vector_type(4)));

constexpr int kQRange = 127 * 128;  // |Q| bound: |hi| <= 127 and |lo| <= 64 fit int8

// NaN-propagating maximum and minimum (v_maximum_f32 / v_minimum_f32: no operand
// canonicalization).
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float vmin(float a, float b) { return __builtin_elementwise_minimum(a, b); }

// Byte 0 of each of four words, in order, as one word (v_perm_b32: selector 0x0c
// reads as zero).
__device__ __forceinline__ uint32_t low_bytes(const uint32_t (&v)[4]) {
  const uint32_t p01 = __builtin_amdgcn_perm(v[1], v[0], 0x0c0c0400u);
  const uint32_t p23 = __builtin_amdgcn_perm(v[3], v[2], 0x04000c0cu);
  return p01 | p23;
}

template <typename QT, int D>
struct QueryColumn {  // the lane's 16 elements of each 64-wide d chunk, as loaded
  uint4 w[D / 64][16 * sizeof(QT) / 16];
};

// The lane's part of one query column (qp: its first element, 16 * qg past the row's).
template <typename QT, int D>
__device__ __forceinline__ void load_query_column(const QT* qp, QueryColumn<QT, D>& raw) {
#pragma unroll
  for (int h = 0; h < D / 64; ++h)
#pragma unroll
    for (int c = 0; c < (int)(16 * sizeof(QT) / 16); ++c)
      raw.w[h][c] = reinterpret_cast<const uint4*>(qp + 64 * h)[c];
}

// Int8 B-operands of one query column for the QK MFMAs (lane r of its 16-lane group
// qg holds d = 16*qg + 64*h + [0, 16)): the column is quantized once to integers
// Q = 128 * hi + lo within 1/2 of q * kQRange / max|q|, hi and lo in int8, so that
// K.Q = 128 (K.hi) + K.lo is exact in int32 (a ~15-bit query, finer than f16's 11 bits
// for every element within 2^-4 of the column maximum).
// Returns the score factor max|q| / kQRange * qk_scale_log2 (NaN for a non-finite
// query, which makes every score of the column non-finite as in fp32 arithmetic).
// kTerms > 2: more terms for blocks whose scores are large enough that the 15-bit
// query's error would show. With x = q * kQRange / max|q| and r2 = x - Q (|r2| <= 1/2):
// lo2 = rint(128 r2), so that 128 Q + lo2 is within 1/2 of 128 x (a ~22-bit query);
// kTerms = 4 adds lo3 = rint(128 (128 r2 - lo2)), 2^14 Q + 2^7 lo2 + lo3 within 1/2 +
// 2^-11 of 2^14 x (~29 bits). Every term is in [-64, 64]; the same raw column always
// gives the same terms.
// Cross-lane: uniform control flow.
// The int8 terms of one query element xv (already lifted) at the column's inv, as floats
// whose low bytes are the terms' two's-complement bytes: adding kQRound (1.5 * 2^23, unit
// in the last place 1) to a value below 2^22 in magnitude rounds it to an integer held in
// the low mantissa bits. Each fma rounds once; hi = rint(xv * inv / 128) and
// lo = rint(xv * inv - 128 hi) (ties to even, |hi| <= 127, |lo| <= 64); with kTerms > 2,
// lo2 = rint(128 r2) where r2 = xv * inv - (128 hi + lo) (|r2| <= 1/2), and with
// kTerms > 3, lo3 = rint(128 (128 r2 - lo2)).
constexpr float kQRound = 12582912.f;
struct QueryTerms {
  float hi, lo, lo2, lo3;
};
template <int kTerms>
__device__ __forceinline__ QueryTerms query_terms(float xv, float inv) {
  QueryTerms t;
  t.hi = __builtin_fmaf(xv, inv * (1.f / 128.f), kQRound);  // inv / 128: exact
  const float hv = t.hi - kQRound;
  t.lo = __builtin_fmaf(xv, inv, __builtin_fmaf(hv, -128.f, kQRound));
  if constexpr (kTerms > 2) {
    // residual of Q = 128 hi + lo (exact integers), one rounding: |r2| <= 1/2
    const float q2 = __builtin_fmaf(hv, 128.f, t.lo - kQRound);
    const float r2 = __builtin_fmaf(xv, inv, -q2);
    t.lo2 = __builtin_fmaf(r2, 128.f, kQRound);
    if constexpr (kTerms > 3) {
      const float r3 = __builtin_fmaf(r2, 128.f, kQRound - t.lo2);  // exact
      t.lo3 = __builtin_fmaf(r3, 128.f, kQRound);
    }
  }
  return t;
}

template <typename QT, int D, int kTerms = 2>
__device__ __forceinline__ float query_column_i8(const QueryColumn<QT, D>& raw, bool valid,
                                                 float qk_scale_log2, int4_t (&qhi)[D / 64],
                                                 int4_t (&qlo)[D / 64],
                                                 int4_t* qlo2 = nullptr, int4_t* qlo3 = nullptr,
                                                 float* inv_out = nullptr,
                                                 float* lift_out = nullptr) {
  static_assert(kTerms >= 2 && kTerms <= 4, "query terms");
  constexpr int kVec = 16 / (int)sizeof(QT);  // elements per 16-byte load
  float x[D / 64][16];
#pragma unroll
  for (int h = 0; h < D / 64; ++h) {
#pragma unroll
    for (int c = 0; c < 16 / kVec; ++c) {
      const uint4 w = raw.w[h][c];
      const QT* e = reinterpret_cast<const QT*>(&w);
#pragma unroll
      for (int i = 0; i < kVec; ++i) x[h][c * kVec + i] = to_float<QT>(e[i]);
    }
  }
  // NaN-propagating maximum of |q| over the column (lanes r, r+16, r+32, r+48): one
  // finiteness test covers every element
  float mx = 0.f;
#pragma unroll
  for (int h = 0; h < D / 64; ++h)
#pragma unroll
    for (int i = 0; i < 16; i += 2) mx = vmax(mx, vmax(fabsf(x[h][i]), fabsf(x[h][i + 1])));
  mx = vmax(mx, shfl_xor(mx, 16));
  mx = vmax(mx, shfl_xor(mx, 32));
  mx = valid ? mx : 0.f;  // an invalid column (its operands meet no output) quantizes with inv = 0
  const bool finite = __builtin_isfinite(mx);
  const float factor = finite ? qk_scale_log2 * (mx / (float)kQRange) : __builtin_nanf("");
  // kQRange / mx overflows for mx below 2^-114: columns under 2^-64 are lifted by 2^64
  // first (exact), which leaves Q unchanged
  const float up = mx > 0.f && mx < 0x1p-64f ? 0x1p64f : 1.f;
  if (__ballot(up != 1.f) != 0) {
#pragma unroll
    for (int h = 0; h < D / 64; ++h)
#pragma unroll
      for (int i = 0; i < 16; ++i) x[h][i] *= up;
    mx *= up;
  }
  const float inv = (finite && mx > 0.f) ? (float)kQRange / mx : 0.f;
  if (inv_out != nullptr) *inv_out = inv;
  if (lift_out != nullptr) *lift_out = up;
#pragma unroll
  for (int h = 0; h < D / 64; ++h)
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t hb[4], lb[4], fb[4], gb[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const QueryTerms t = query_terms<kTerms>(x[h][4 * w + e], inv);
        hb[e] = __builtin_bit_cast(uint32_t, t.hi);
        lb[e] = __builtin_bit_cast(uint32_t, t.lo);
        if constexpr (kTerms > 2) fb[e] = __builtin_bit_cast(uint32_t, t.lo2);
        if constexpr (kTerms > 3) gb[e] = __builtin_bit_cast(uint32_t, t.lo3);
      }
      qhi[h][w] = (int)low_bytes(hb);
      qlo[h][w] = (int)low_bytes(lb);
      if constexpr (kTerms > 2) qlo2[h][w] = (int)low_bytes(fb);
      if constexpr (kTerms > 3) qlo3[h][w] = (int)low_bytes(gb);
    }
  return factor;
}

// The G query rows of kv head kvh, token row tok, by direct-to-LDS loads into
// `dst` as [G][D] elements of QT (16 bytes per lane, D*sizeof(QT)/16 lanes per
// head): ceil(G*D*sizeof(QT)/1024) vector-memory instructions.
template <typename QT, int D, int G>
constexpr int stage_query_loads() {
  return (G + kWave / (D * (int)sizeof(QT) / 16) - 1) / (kWave / (D * (int)sizeof(QT) / 16));
}
template <typename QT, int D, int G>
__device__ __forceinline__ void stage_query(const AttnArgs& a, int tok, int kvh, int lane,
                                            char* dst) {
  constexpr int kLanesPerHead = D * (int)sizeof(QT) / 16;
  constexpr int kHeadsPerLoad = kWave / kLanesPerHead;
  constexpr int kLoads = (G + kHeadsPerLoad - 1) / kHeadsPerLoad;
  const QT* q0 = static_cast<const QT*>(a.q) + (int64_t)tok * a.q_tok;
  // the destination is wave-uniform: held in an SGPR before the lane-dependent branch
  const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr(dst));
#pragma unroll
  for (int k = 0; k < kLoads; ++k) {
    const int g = k * kHeadsPerLoad + lane / kLanesPerHead;
    if (g < G) {
      const char* src = reinterpret_cast<const char*>(q0 + (int64_t)(kvh * G + g) * a.q_head) +
                        (lane % kLanesPerHead) * 16;
      lds_dma_x4(src, base + k * 1024);
    }
  }
}

// Query row g of a stage_query buffer as the lane's column (the QueryColumn layout
// load_query_column gives; any query type).
template <typename QT, int D>
__device__ __forceinline__ void lds_query_column(const char* buf, int g, int qg,
                                                 QueryColumn<QT, D>& q) {
  const char* row = buf + (g * D + 16 * qg) * (int)sizeof(QT);
#pragma unroll
  for (int h = 0; h < D / 64; ++h)
#pragma unroll
    for (int c = 0; c < (int)(16 * sizeof(QT) / 16); ++c)
      q.w[h][c] = *reinterpret_cast<const uint4*>(row + 64 * h * (int)sizeof(QT) + 16 * c);
}

// Query row g of a stage_query buffer in the QueryRaw lane layout.
template <typename QT, int D>
__device__ __forceinline__ void lds_query(const char* buf, int g, int qg, QueryRaw<D>& q) {
  static_assert(sizeof(QT) == 2, "16-bit queries");
  const char* row = buf + (g * D + 16 * qg) * (int)sizeof(QT);
#pragma unroll
  for (int h = 0; h < D / 64; ++h) {
    q.w[h][0] = *reinterpret_cast<const uint4*>(row + 64 * h * (int)sizeof(QT));
    q.w[h][1] = *reinterpret_cast<const uint4*>(row + 64 * h * (int)sizeof(QT) + 16);
  }
}

// f16 B-operands of the QK MFMAs (FP8 codes) after an exact 2^-e rescale keeping
// max|q| below 2^15 (e folded into the returned score factor). Cross-lane: call in
// uniform control flow.
template <typename QT, int D>
__device__ __forceinline__ float query_operand(const QueryRaw<D>& q, bool gvalid,
                                               float qk_scale_log2, half8_t (&qop)[D / 32]) {
  // two passes over the raw words (max, then convert) keep the live set small
  float mx = 0.f;
#pragma unroll
  for (int h = 0; h < D / 64; ++h)
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const QT* e = reinterpret_cast<const QT*>(&q.w[h][c]);
#pragma unroll
      for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(to_float<QT>(e[i])));
    }
  mx = gvalid ? mx : 0.f;
  mx = fmaxf(mx, shfl_xor(mx, 16));
  mx = fmaxf(mx, shfl_xor(mx, 32));
  int ex = 0;
  if (mx >= 32768.f) {
    frexpf(mx, &ex);
    ex -= 15;  // mx * 2^-ex < 2^15
  }
  const float down = ldexpf(1.f, -ex);
#pragma unroll
  for (int kk = 0; kk < D / 32; ++kk) {
    const QT* e = reinterpret_cast<const QT*>(&q.w[kk / 2][kk % 2]);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      qop[kk][i] = gvalid ? (_Float16)(to_float<QT>(e[i]) * down) : (_Float16)0.f;
  }
  return qk_scale_log2 * ldexpf(1.f, ex);
}

// QK^T operands of one query row per lane for the decode kernels: int8 codes meet a
// three-term int8 query on v_mfma_i32_16x16x64_i8 (the K codes need no conversion); FP8
// codes, converted to f16, meet an f16 query on v_mfma_f32_16x16x32_f16.
template <int D, int KF>
struct QkOperand {
  half8_t op[D / 32];
};
// INT8 codes: the query column as 128 Q + lo2 within 1/2 of 128 x (query_column_i8 with
// three terms, x = q * kQRange / max|q|), i.e. within 2^-8 of a ~15-bit step of q, about
// 2^-22 of max|q| per element: the score K.q carries, per unit of K, the error an fp32
// dot product's own rounding has. Every block takes all three terms (the third on a
// separate int32 accumulator: 128 (K.Q) + K.lo2 can exceed int32), so no key scale,
// however large, sees the coarser two-term query.
template <int D>
struct QkOperand<D, kInt8> {
  int4_t hi[D / 64], lo[D / 64], lo2[D / 64];
};

// Builds the operand of query row r (lane layout of QueryRaw; rows r >= G are zero)
// and returns its score factor, code scale included. Cross-lane: uniform control flow.
template <typename QT, int D, int KF>
__device__ __forceinline__ float qk_operand(const QueryRaw<D>& q, bool gvalid, float qk_scale_log2,
                                            QkOperand<D, KF>& op) {
  if constexpr (KF == kInt8) {
    static_assert(sizeof(QT) == 2, "16-bit queries (fp32 queries take the exact VALU kernel)");
    QueryColumn<QT, D> col;
#pragma unroll
    for (int h = 0; h < D / 64; ++h) {
      col.w[h][0] = q.w[h][0];
      col.w[h][1] = q.w[h][1];
    }
    return query_column_i8<QT, D, 3>(col, gvalid, qk_scale_log2, op.hi, op.lo, op.lo2);
  } else {
    return query_operand<QT, D>(q, gvalid, qk_scale_log2, op.op) * code_scale<KF>();
  }
}

// The same operand from a QueryColumn of any query type: int8 codes only for fp32
// queries (their three int8 terms keep ~22 bits of each element; an f16 query for the
// FP8 formats would keep 11).
template <typename QT, int D, int KF>
__device__ __forceinline__ float qk_operand_column(const QueryColumn<QT, D>& col, bool gvalid,
                                                   float qk_scale_log2, QkOperand<D, KF>& op) {
  if constexpr (KF == kInt8) {
    return query_column_i8<QT, D, 3>(col, gvalid, qk_scale_log2, op.hi, op.lo, op.lo2);
  } else {
    static_assert(sizeof(QT) == 2, "FP8 codes take 16-bit queries on the MFMA path");
    return query_operand<QT, D>(reinterpret_cast<const QueryRaw<D>&>(col), gvalid,
                                qk_scale_log2, op.op) *
           code_scale<KF>();
  }
}

// Screening of the rare blocks in mfma_block: every lane tests the staged V scale of
// token r against vlim (before the weight scale, a power of two, so the test is exact);
// the four lanes of each r test the same scale, so together the 16 lanes of a token
// group cover every V scale of the block, and a block with one above the limit takes
// the full test.
template <int KF>
__device__ __forceinline__ float screen_limit(float vlim) {
  return vlim * (1.f / v_weight_scale<KF>());
}
// A piece's starting VRange.
template <int KF>
__device__ __forceinline__ VRange vrange_start() {
  return VRange{0.f, kVWeightCap, screen_limit<KF>(kVWeightCap)};
}

// ---- one staged 16-token block through the MFMAs
//   S^T[t][g] = K[t][:] . Q[g][:]     INT8 codes: 3 (D/64) x v_mfma_i32_16x16x64_i8
//                                     (hi, then lo on the hi result shifted by 7, and
//                                     lo2 on its own accumulator);
//                                     FP8 codes: 4 (D/32) x v_mfma_f32_16x16x32_f16
//   O^T[d][g] += V^T[d][t] P^T[t][g]  8 (D/16) x v_mfma_f32_16x16x16_f16
// acc[D/16] is one more tile: with biased V operands (biased_v), a row of ones times
// P^T, whose row 0 sums the rounded weights for remove_v_bias.
// The S^T output layout (lane l: tokens 4*(l/16)+j of head l%16) is the B-operand
// layout P^T needs, so the online softmax stays in registers. Tokens outside
// [kv_begin, ctx) are masked; `tok_base` is the block's first token position.
// Cross-lane (ballots, shuffles): call in uniform control flow.
// `vr` keeps the PV weights p * v_scale in f16 range for large V scales (VRange).
// `gvalid`: this lane's query column feeds an output (its query operand is zero
// otherwise).
template <typename QT, int D, int KF = kInt8>
__device__ __forceinline__ void mfma_block(const char* st, const QkOperand<D, KF>& qop, float cf,
                                           int tok_base, int kv_begin, int ctx, bool gvalid, int r,
                                           int qg, float4_t (&acc)[D / 16 + 1], float& m, float& l,
                                           VRange& vr, bool& bad_score, bool masks = false) {
  using S = Stage<D>;
  constexpr int KCH = D / 64;
  constexpr int VB = D / 16;
  constexpr int NPV = D / 16;
  // V scales, times 2^8 for FP8 codes (E4M3FN operands carry 2^-8; E5M2 weights carry
  // 2^8, as does the normaliser of this format); finite, and the same on the 16 lanes
  // of a token group
  const float4_t vs = *reinterpret_cast<const float4_t*>(st + S::kS + 64 + 16 * qg) * v_weight_scale<KF>();
  const float4_t ks = *reinterpret_cast<const float4_t*>(st + S::kS + 16 * qg);
  // the one staged scale this lane screens against vr.screen (screen_limit): the V scale
  // of token r
  const float screened = *reinterpret_cast<const float*>(st + S::kS + 64 + 4 * r);
  // rare blocks, found by the screen: V scales beyond vr.vlim grow the running
  // maximum's offset, with its own rescale of l and acc, before the block's weights
  // are formed
  auto grow_vrange = [&]() __attribute__((always_inline)) {
    const float vsm = fmaxf(fmaxf(vs[0], vs[1]), fmaxf(vs[2], vs[3]));
    if (__ballot(vsm > vr.vlim) != 0) {
      float wm = fmaxf(vsm, shfl_xor(vsm, 16));
      wm = fmaxf(wm, shfl_xor(wm, 32));
      int x;
      frexpf(wm / vr.vlim, &x);  // in [2^(x-1), 2^x), x >= 1
      vr.koff += (float)x;
      vr.vlim = ldexpf(vr.vlim, x);
      vr.screen = screen_limit<KF>(vr.vlim);
      const float alpha = ldexpf(1.f, -x);  // m + x is the new maximum (with offset)
      m += (float)x;
      l *= alpha;
#pragma unroll
      for (int n = 0; n <= NPV; ++n) acc[n] *= alpha;
    }
  };
  // Up to D = 128 the screen follows the QK MFMAs, off their path; at D = 256 the V
  // range goes first, which keeps the registers of the PV accumulators free of the
  // scores while it rescales them
  constexpr bool kScreenLate = D <= 128;
  if constexpr (!kScreenLate) {
    if (__ballot(screened > vr.screen) != 0) grow_vrange();
  }
  // V code words of the PV operands. Up to D = 128 they are read with the K codes, so
  // that their LDS latency passes under the QK MFMAs; at D = 256 they would stay live
  // in too many registers, and are read after the QK MFMAs.
  uint32_t vw[4][VB / 4];
  auto read_v_words = [&]() __attribute__((always_inline)) {
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
  };
  if constexpr (kScreenLate) read_v_words();
  float4_t s4;
  if constexpr (KF == kInt8) {
    // exact int32 K.Q = 128 (K.hi) + K.lo and K.lo2 straight from the staged codes; the
    // score is K.Q + K.lo2 / 128 (one rounding each for the conversions and the fma)
    int4_t kop[KCH];
#pragma unroll
    for (int h = 0; h < KCH; ++h)
      kop[h] = *reinterpret_cast<const int4_t*>(st + S::kK + k_chunk<D>(r, qg + 4 * h));
    int4_t si = {0, 0, 0, 0}, sf = {0, 0, 0, 0};
#pragma unroll
    for (int h = 0; h < KCH; ++h) si = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop[h], qop.hi[h], si, 0, 0, 0);
#pragma unroll
    for (int h = 0; h < KCH; ++h) sf = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop[h], qop.lo2[h], sf, 0, 0, 0);
    si = si << 7;
#pragma unroll
    for (int h = 0; h < KCH; ++h) si = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop[h], qop.lo[h], si, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) s4[j] = __builtin_fmaf((float)sf[j], 1.f / 128.f, (float)si[j]);
    // keeps these conversions of MFMA results ahead of the branches below: sunk into
    // their blocks, they were issued without the wait states an MFMA result needs
    // (wrong scores at D = 64)
    asm volatile("" : "+v"(s4[0]), "+v"(s4[1]), "+v"(s4[2]), "+v"(s4[3]));
  } else {
    s4 = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int h = 0; h < KCH; ++h) {
      const uint4 c = *reinterpret_cast<const uint4*>(st + S::kK + k_chunk<D>(r, qg + 4 * h));
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        half2_t p0, p1, p2, p3;
        codes_to_f16<KF>(sub ? c.z : c.x, p0, p1);
        codes_to_f16<KF>(sub ? c.w : c.y, p2, p3);
        const half8_t kop = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
        s4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop, qop.op[2 * h + sub], s4, 0, 0, 0);
      }
    }
  }
  if constexpr (kScreenLate) {
    // one compare and ballot per block; the rare path is laid out away from the loop
    if (__builtin_expect(__ballot(screened > vr.screen) != 0, 0)) grow_vrange();
  } else {
    read_v_words();
  }
  // scores of tokens 4*qg + j for head g = r (base 2, dequantised)
  const int tok0 = tok_base + 4 * qg;
  // a block holding a padding key takes the edge path, which reads each key's byte
  bool padded = false;
  if (masks) padded = __ballot(*reinterpret_cast<const uint32_t*>(st + S::kF + 4 * qg) != 0x01010101u) != 0;
  const bool edge = tok_base < kv_begin || tok_base + kBlockTokens > ctx || padded;
  float sc[4];
  bool need = false, nonfinite = false;
  if (edge) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v = s4[j] * (ks[j] * cf);
      const bool valid = gvalid && tok0 + j >= kv_begin && tok0 + j < ctx &&
                         (!masks || st[S::kF + 4 * qg + j] != 0);
      nonfinite |= valid && !__builtin_isfinite(v);
      v = valid ? v : -INFINITY;
      need |= v > m + kRescaleSlack;
      sc[j] = v;
    }
  } else {
    // every key of the block is visible: a NaN-propagating maximum and minimum of the
    // four scores stand for the per-score finiteness and rescale tests. Columns
    // without an output (zero query, finite zero scores) test nothing.
#pragma unroll
    for (int j = 0; j < 4; ++j) sc[j] = s4[j] * (ks[j] * cf);
    const float hi = vmax(vmax(sc[0], sc[1]), vmax(sc[2], sc[3]));
    const float lo = vmin(vmin(sc[0], sc[1]), vmin(sc[2], sc[3]));
    nonfinite = gvalid && !(__builtin_isfinite(hi) && __builtin_isfinite(lo));
    need = gvalid && hi > m + kRescaleSlack;
  }
  if (__builtin_expect(__ballot(nonfinite) != 0, 0)) bad_score = true;
  if (__builtin_expect(__ballot(need) != 0, 0)) {
    float tmax = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
    tmax = fmaxf(tmax, shfl_xor(tmax, 16));
    tmax = fmaxf(tmax, shfl_xor(tmax, 32));
    const float mn = fmaxf(m, tmax + vr.koff);
    const float alpha = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mn);
    l *= alpha;
#pragma unroll
    for (int n = 0; n <= NPV; ++n) acc[n] *= alpha;
    m = mn;
  }
  half4_t pop;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float p = __builtin_amdgcn_exp2f(sc[j] - m);
    l += p;
    pop[j] = (_Float16)(p * vs[j]);
  }
  // O^T += V^T . P^T (row m of MFMA n is d = VB*m + n)
#pragma unroll
  for (int n = 0; n < NPV; ++n) {
    const uint32_t col[4] = {vw[0][n / 4], vw[1][n / 4], vw[2][n / 4], vw[3][n / 4]};
    half4_t vop;
    if constexpr (biased_v<D, KF>()) {
      switch (n % 4) {
        case 0: vop = v_operand_biased<0>(col); break;
        case 1: vop = v_operand_biased<1>(col); break;
        case 2: vop = v_operand_biased<2>(col); break;
        default: vop = v_operand_biased<3>(col); break;
      }
    } else {
      switch (n % 4) {
        case 0: vop = v_operand<0, KF>(col); break;
        case 1: vop = v_operand<1, KF>(col); break;
        case 2: vop = v_operand<2, KF>(col); break;
        default: vop = v_operand<3, KF>(col); break;
      }
    }
    acc[n] = __builtin_amdgcn_mfma_f32_16x16x16f16(vop, pop, acc[n], 0, 0, 0);
  }
  if constexpr (biased_v<D, KF>()) {
    const _Float16 one = r == 0 ? (_Float16)1.f : (_Float16)0.f;
    acc[NPV] = __builtin_amdgcn_mfma_f32_16x16x16f16(half4_t{one, one, one, one}, pop, acc[NPV], 0, 0, 0);
  }
}

// Lane (qg, r) holds, of head column r, the D/4 consecutive outputs
// d = (D/4) qg + t, t = VB j + k (VB = D/16), output t in acc[t % VB][t / VB].
// store_lane_f32 / store_lane_out write them with 16-byte stores from `dst`, the
// lane's first element (16-byte aligned).
template <int D>
__device__ __forceinline__ void store_lane_f32(float* dst, const float4_t (&acc)[D / 16 + 1]) {
  constexpr int VB = D / 16;
#pragma unroll
  for (int t = 0; t < D / 4; t += 4) {
    float4_t v;
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = acc[(t + u) % VB][(t + u) / VB];
    *reinterpret_cast<float4_t*>(dst + t) = v;
  }
}
template <typename QT, int D>
__device__ __forceinline__ void store_lane_out(QT* dst, const float4_t (&acc)[D / 16 + 1],
                                               float scale) {
  constexpr int VB = D / 16;
  constexpr int kVec = 16 / (int)sizeof(QT);  // elements per 16-byte store
#pragma unroll
  for (int t = 0; t < D / 4; t += kVec) {
    QT v[kVec];
#pragma unroll
    for (int u = 0; u < kVec; ++u) v[u] = from_float<QT>(acc[(t + u) % VB][(t + u) / VB] * scale);
    *reinterpret_cast<uint4*>(dst + t) = *reinterpret_cast<const uint4*>(v);
  }
}

// Ends a piece's accumulation: with biased V operands, subtracts kVBias times the
// weight sum of head r (row 0 of acc[D/16], held by lane (0, r)) from every output of
// that head. Cross-lane: call in uniform control flow.
template <int D, int KF>
__device__ __forceinline__ void end_piece(float4_t (&acc)[D / 16 + 1], int r) {
  if constexpr (biased_v<D, KF>()) {
    const float b = kVBias * __shfl(acc[D / 16][0], r, kWave);
#pragma unroll
    for (int n = 0; n < D / 16; ++n) acc[n] -= float4_t{b, b, b, b};
  }
}

// Launch arguments of the planned decode kernel: the attention arguments and the host
// plan (its int32 words in device memory, sizes and offsets in `info`).
struct PlanArgs {
  AttnArgs a;
  const int32_t* plan;
  astr_decode_plan_info info;
};

// Partial slots of a plan in the workspace, in columns of D floats (and (m, l) pairs):
// two per wave of the planned kernel, then G per chunk slot (rows cut across
// workgroups, and the ranges of shared prefixes).
__device__ __forceinline__ int64_t plan_chunk_slot(const PlanArgs& p, int64_t c, int G) {
  return ((int64_t)p.info.num_workgroups * p.info.waves_per_workgroup * 2 + c) * G;
}
// Column capacity of a prefix tile (decode_plan.cpp): the chunked-prefill kernel's
// columns per workgroup, the most tile_rows * G may be.
constexpr int prefix_tile_columns(int head_dim) { return head_dim == 256 ? 64 : 128; }

// Kernel entry points, one translation unit per code format KF (the source built
// with -DASTR_KF=KF), dispatched on query dtype, head dim and GQA group inside.
template <int KF> int launch_partitioned_kf(const AttnArgs& a, int32_t q_dtype, hipStream_t stream);
template <int KF> int launch_streamk_kf(const AttnArgs& a, int32_t q_dtype, hipStream_t stream);
// the stream-K launches without prefix packs (a unit of their own; launch_streamk_kf
// routes to it)
template <int KF>
int launch_streamk_plain_kf(const AttnArgs& a, int32_t q_dtype, hipStream_t stream);
// Rows with more than one query token (chunked prefill), one workgroup per
// (kv head, sequence, tile of query tokens); needs q_start.
template <int KF> int launch_prefill_kf(const AttnArgs& a, int32_t q_dtype, hipStream_t stream);
// Decode rows on a host plan (decode_planned.hip); with `resident` non-null nothing is
// launched and the kernel's resident workgroups per CU land there.
template <int KF>
int launch_planned_kf(const PlanArgs& p, int32_t q_dtype, hipStream_t stream, int* resident);
// The prefix tiles of a host plan (prefill.hip): partials for the chunk-merge kernel,
// which the planned launch runs after the decode kernel.
template <int KF>
int launch_prefix_tiles_kf(const PlanArgs& p, int32_t q_dtype, hipStream_t stream);
#define ASTR_DECLARE_LAUNCHERS(KF)                                                        \
  template <> int launch_partitioned_kf<KF>(const AttnArgs&, int32_t, hipStream_t);       \
  template <> int launch_streamk_kf<KF>(const AttnArgs&, int32_t, hipStream_t);           \
  template <> int launch_streamk_plain_kf<KF>(const AttnArgs&, int32_t, hipStream_t);     \
  template <> int launch_prefill_kf<KF>(const AttnArgs&, int32_t, hipStream_t);             \
  template <> int launch_planned_kf<KF>(const PlanArgs&, int32_t, hipStream_t, int*);     \
  template <> int launch_prefix_tiles_kf<KF>(const PlanArgs&, int32_t, hipStream_t);
ASTR_DECLARE_LAUNCHERS(kInt8)
ASTR_DECLARE_LAUNCHERS(kE4M3)
ASTR_DECLARE_LAUNCHERS(kE5M2)
#undef ASTR_DECLARE_LAUNCHERS

#define ASTR_BY_FORMAT(name)                                                     \
  inline int name(const AttnArgs& a, int32_t q_dtype, hipStream_t stream) {      \
    switch (a.cache.code_format) {                                               \
      case kInt8: return name##_kf<kInt8>(a, q_dtype, stream);                   \
      case kE4M3: return name##_kf<kE4M3>(a, q_dtype, stream);                   \
      default: return name##_kf<kE5M2>(a, q_dtype, stream);                     \
    }                                                                            \
  }
ASTR_BY_FORMAT(launch_partitioned)
ASTR_BY_FORMAT(launch_streamk)
ASTR_BY_FORMAT(launch_prefill)
#undef ASTR_BY_FORMAT
inline int launch_planned(const PlanArgs& p, int32_t q_dtype, hipStream_t stream, int* resident) {
  switch (p.a.cache.code_format) {
    case kInt8: return launch_planned_kf<kInt8>(p, q_dtype, stream, resident);
    case kE4M3: return launch_planned_kf<kE4M3>(p, q_dtype, stream, resident);
    default: return launch_planned_kf<kE5M2>(p, q_dtype, stream, resident);
  }
}
inline int launch_prefix_tiles(const PlanArgs& p, int32_t q_dtype, hipStream_t stream) {
  switch (p.a.cache.code_format) {
    case kInt8: return launch_prefix_tiles_kf<kInt8>(p, q_dtype, stream);
    case kE4M3: return launch_prefix_tiles_kf<kE4M3>(p, q_dtype, stream);
    default: return launch_prefix_tiles_kf<kE5M2>(p, q_dtype, stream);
  }
}

// Largest batch the stream-K kernel takes (its per-sequence table lives in LDS), the
// most prefix packs per launch and the largest batch that takes them, and the work
// rows of its block prefix (ws_seq and ws_ne hold one more entry each) for a head dim.
int stream_k_max_seqs();
int stream_k_max_packs();
int stream_k_max_pack_seqs();
int stream_k_work_rows(int head_dim);

}  // namespace attn
}  // namespace astr
