// Chunked-prefill paged attention over the INT8 arena (gfx950): the sequences of
// a step that carry more than one query token (a prompt chunk in
// PagedAttentionRunner.forward_batch, paged_attention.py:168-215), with the
// visibility rules of online_attention_statistics (online_attention.py:178-188):
// query token i of a sequence with n query tokens and context ctx (the chunk
// already appended) sits at position p = ctx - n + i and sees key k iff
//   k <= p (causal; else k < ctx)  and  k > p - window (window > 0).
//
// Work unit: (kv head, sequence, tile of TQ query tokens), TQ * G = 64 * NT
// (token, head) columns of one kv head, 16 * NT columns per wave. The unit's
// visible key range is streamed in steps of four 16-token blocks; each wave
// stages one block of the step into LDS with direct global->LDS loads and then
// all four waves run all four blocks through the MFMAs:
//   S^T[t][c]  = K[t][:] . Q[c][:]     v_mfma_i32_16x16x64_i8: the K codes as stored,
//                                        the query as two int8 terms (exact int32 dot),
//                                        three on steps with large key scales
//   O^T[d][c] += V^T[d][t] . P^T[t][c]  v_mfma_f32_16x16x32_f16 over two blocks (P^T
//                                        carries V's scales)
// so every K/V byte of the unit's range is read once per query tile and shared by
// the G heads and TQ tokens of the tile. Softmax statistics are per column, in
// base 2, with the lazy rescale of the decode kernels.
//
// Units of one (kv head, sequence) are consecutive, longest (latest) tile first,
// and the linear workgroup id is remapped so that each XCD (workgroups are dealt
// to the 8 XCDs round robin) runs one contiguous range of units: the tiles
// sharing a sequence's K/V then share that XCD's L2.
#include <climits>
#include <type_traits>

#include "attention_common.h"

namespace astr {
namespace attn {
namespace {

#ifndef ASTR_KF
#define ASTR_KF 0
#endif
constexpr int KF = ASTR_KF;  // this translation unit's code format

constexpr int kXcds = 8;
constexpr int kPrefillBuffers = 3;

// Per-wave timeline of the prefix-tile kernel (trace builds only, -DASTR_TRACE=1, built
// apart from the product library by `python -m aster_amd.build --trace`): wall-clock
// marks (100 MHz s_memrealtime) of each wave of the last launch, read back with
// astr_trace_read_tiles. Marks: 0 entry, 1 tile and members checked, 2 query columns
// quantized (the first steps' loads in flight), 3 first key step done, 4 key steps done,
// 5 partials stored. Info: key steps, XCC id, kv head, key range.
#ifndef ASTR_TRACE
#define ASTR_TRACE 0
#endif
constexpr bool kTrace = ASTR_TRACE != 0;
#if ASTR_TRACE
constexpr int kTileTraceWaves = 8192;
static __device__ long long g_ttrace[kTileTraceWaves][8];
static __device__ int g_ttrace_info[kTileTraceWaves][4];
#endif

template <int D>
struct PrefillShape {
  static constexpr int NT = D == 256 ? 1 : 2;     // 16-column MFMA tiles per wave
  static constexpr int kCols = kWaves * 16 * NT;  // (token, head) columns per workgroup
};

// Keys visible to query tile `tile` (tokens [t0, t1) of the sequence's n query tokens,
// context ctx): positions [lo, hi], blocks [b_lo, b_hi).
struct TileSpan {
  int pos0, t0, t1, lo, hi, b_lo, b_hi;
};

__device__ __forceinline__ TileSpan tile_span(const AttnArgs& a, int ctx, int n, int tile, int tq) {
  TileSpan t;
  t.pos0 = ctx - n;  // position of the sequence's first query token
  t.t0 = tile * tq;
  t.t1 = min(n, t.t0 + tq);
  t.lo = a.window > 0 ? max(0, t.pos0 + t.t0 - a.window + 1) : 0;
  t.hi = a.causal ? min(t.pos0 + t.t1 - 1, ctx - 1) : ctx - 1;
  t.b_lo = t.lo / kBlockTokens;
  t.b_hi = t.hi >= t.lo ? t.hi / kBlockTokens + 1 : t.b_lo;  // exclusive
  return t;
}

constexpr int kOrderMax = 256;  // chunk rows ordered longest first; beyond this, index order

__device__ __forceinline__ int query_tiles(const AttnArgs& a, int s, int tq) {
  int begin;
  const int n = seq_queries(a, s, begin);
  return n > 1 ? (n + tq - 1) / tq : 0;
}

// The dispatch plan, from one round of loads of the offsets and context lengths, in
// the LDS table `tab` (PlanTab::kInts ints): the chunk rows (sequences with more than
// one query token) with their sequence, query offset, query count and context length
// as loaded, and the rows in dispatch order, longest first (key: key blocks of the
// row's last tile, which sees the most keys; ties by index), with the inclusive prefix
// of their tile counts in that order. Returns the number of rows and the total tile
// count, or -1 when there are more than kOrderMax rows (then every sequence is taken
// in index order by scan_tiles). Every thread calls it.
struct PlanTab {
  enum { kSeq, kTiles, kKey, kQ0, kN, kCtx, kOrder, kIncl, kArrays };
  static constexpr int kInts = kArrays * kOrderMax;
  __device__ static int* at(int* tab, int array) { return tab + array * kOrderMax; }
};

__device__ int plan_rows(const AttnArgs& a, int tq, int* tab, int* s_wsum, int& total) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  int* const r_tiles = PlanTab::at(tab, PlanTab::kTiles);
  int* const r_key = PlanTab::at(tab, PlanTab::kKey);
  int* const o_row = PlanTab::at(tab, PlanTab::kOrder);
  int* const o_incl = PlanTab::at(tab, PlanTab::kIncl);
  int count = 0;
  for (int c0 = 0; c0 < a.num_seqs; c0 += kWaves * kWave) {
    const int s = c0 + (int)threadIdx.x;
    int key = -1, tiles = 0, q0 = 0, n = 0, ctx_raw = 0;
    if (s < a.num_seqs) {
      n = seq_queries(a, s, q0);
      if (n > 1) {
        ctx_raw = a.context_lens[s];
        const TileSpan sp = tile_span(a, clamp_ctx(a, ctx_raw, false), n, (n - 1) / tq, tq);
        key = sp.b_hi - sp.b_lo;
        tiles = (n + tq - 1) / tq;
      }
    }
    const uint64_t rows = __ballot(key >= 0);
    const int before = __builtin_popcountll(rows & ((1ull << lane) - 1));
    if (lane == 0) s_wsum[wave] = __builtin_popcountll(rows);
    __syncthreads();
    int idx = count + before;
    for (int w = 0; w < wave; ++w) idx += s_wsum[w];
    if (key >= 0 && idx < kOrderMax) {
      PlanTab::at(tab, PlanTab::kSeq)[idx] = s;
      PlanTab::at(tab, PlanTab::kQ0)[idx] = q0;
      PlanTab::at(tab, PlanTab::kN)[idx] = n;
      PlanTab::at(tab, PlanTab::kCtx)[idx] = ctx_raw;
      r_tiles[idx] = tiles;
      r_key[idx] = key;
    }
    count += s_wsum[0] + s_wsum[1] + s_wsum[2] + s_wsum[3];
    __syncthreads();
  }
  if (count > kOrderMax) return -1;
  static_assert(kOrderMax == kWaves * kWave, "one row per thread below");
  const int i = threadIdx.x;
  int tiles = 0;
  if (i < count) {
    const int k = r_key[i];
    int rank = 0;
    for (int j = 0; j < count; ++j) {
      const int kj = r_key[j];
      rank += (kj > k) | ((kj == k) & (j < i));
    }
    o_row[rank] = i;
    o_incl[rank] = r_tiles[i];
  }
  __syncthreads();
  if (i < count) tiles = o_incl[i];
  int incl = tiles;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int v = __shfl_up(incl, off, kWave);
    if (lane >= off) incl += v;
  }
  if (lane == kWave - 1) s_wsum[wave] = incl;
  __syncthreads();
  for (int w = 0; w < wave; ++w) incl += s_wsum[w];
  if (i < count) o_incl[i] = incl;
  total = s_wsum[0] + s_wsum[1] + s_wsum[2] + s_wsum[3];
  __syncthreads();
  return count;
}

// Workgroup-wide scan of the query-tile counts of all sequences in index order. Returns
// the total; when `unit` >= 0, the sequence holding that unit and the unit's index
// within the sequence land in found[0], found[1]. Every thread calls it.
__device__ int scan_tiles(const AttnArgs& a, int tq, int unit, int* s_wsum, int* found) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  int base = 0;
  for (int c0 = 0; c0 < a.num_seqs; c0 += kWaves * kWave) {
    const int s = c0 + (int)threadIdx.x;
    const int t = s < a.num_seqs ? query_tiles(a, s, tq) : 0;
    int incl = t;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int v = __shfl_up(incl, off, kWave);
      if (lane >= off) incl += v;
    }
    if (lane == kWave - 1) s_wsum[wave] = incl;
    __syncthreads();
    int wb = base;
    for (int w = 0; w < wave; ++w) wb += s_wsum[w];
    incl += wb;
    if (unit >= incl - t && unit < incl) {
      found[0] = s;
      found[1] = unit - (incl - t);
    }
    base += s_wsum[0] + s_wsum[1] + s_wsum[2] + s_wsum[3];
    __syncthreads();
  }
  return base;
}

// |S_int| <= 127 * kQRange * 256; a score factor below this keeps every score finite
constexpr float kSafeFactor = 1.0e29f;
// INT8 codes: the two-term query Q is within 1/2 of x = q * kQRange / max|q| per
// element, so a key with scale ks carries at most 1/2 * 127 D * ks * cf of score error
// (base 2; cf the column's score factor). A step in which any key scale times a
// column's cf exceeds kFineScoreError / (63.5 D) adds the third term, K.lo2 / 128 (lo2 =
// rint(128 (x - Q))), which divides that bound by 128. The worst case aligns every code
// at 127 with every rounding; the typical error is ~50 times smaller (the rounding
// errors are independent and codes average ~1/4 of 127), so steps without the term
// carry ~2e-4 nats of score error at most, well inside what moves an output by the
// north_star's 2e-3. Seeded N(0,1) queries and keys stay ~4x below the threshold.
constexpr float kFineScoreError = 1.f / 64.f;
// FP8 codes take the f16 QK path: |S| <= D * 2^15 * max|code as f16| (448 * 2^-8 for
// E4M3FN, 57344 for E5M2) with D <= 256, times a factor below these stays finite.
constexpr float kSafeFactorE4M3 = 1.0e31f;
constexpr float kSafeFactorE5M2 = 5.0e26f;
constexpr float safe_factor() {
  return KF == kInt8 ? kSafeFactor : KF == kE4M3 ? kSafeFactorE4M3 : kSafeFactorE5M2;
}

// Query operands of one column tile: two int8 terms per 64-wide d chunk for int8 codes
// (the int8 QK MFMA), f16 halves per 32-wide chunk for FP8 codes (the f16 QK MFMA).
template <int D>
struct QOpI8 {
  int4_t hi[D / 64], lo[D / 64];
};
template <int D>
struct QOpF16 {
  half8_t op[D / 32];
};
template <int D>
using QOp = typename std::conditional<KF == kInt8, QOpI8<D>, QOpF16<D>>::type;

// f16 B-operands of one query column for the f16 QK MFMAs (the FP8 path): chunk
// kk = 2h + sub holds d = 16 qg + 64 h + 8 sub + [0, 8), like the K operands. The
// column is scaled by an exact power of two 2^-ex that keeps max|q| < 2^15 before
// rounding to f16; returns qk_scale_log2 * 2^ex * code_scale (NaN for a non-finite
// query, which makes every score of the column non-finite as in fp32 arithmetic).
// Cross-lane: uniform control flow.
template <typename QT, int D>
__device__ __forceinline__ float query_column_f16(const QueryColumn<QT, D>& raw, bool valid,
                                                  float qk_scale_log2, half8_t (&qop)[D / 32]) {
  constexpr int kVec = 16 / (int)sizeof(QT);
  float mx = 0.f;
  bool finite = true;
#pragma unroll
  for (int h = 0; h < D / 64; ++h)
#pragma unroll
    for (int c = 0; c < 16 / kVec; ++c) {
      const QT* e = reinterpret_cast<const QT*>(&raw.w[h][c]);
#pragma unroll
      for (int i = 0; i < kVec; ++i) {
        const float x = to_float<QT>(e[i]);
        mx = fmaxf(mx, fabsf(x));
        finite = finite && __builtin_isfinite(x);
      }
    }
  mx = valid ? mx : 0.f;
  mx = fmaxf(mx, shfl_xor(mx, 16));
  mx = fmaxf(mx, shfl_xor(mx, 32));
  const uint64_t nonfinite_lanes = __ballot(valid && !finite);
  finite = ((nonfinite_lanes >> (threadIdx.x % 16)) & 0x0001000100010001ull) == 0;
  int ex = 0;
  if (finite && mx >= 32768.f) {
    frexpf(mx, &ex);
    ex -= 15;  // mx * 2^-ex < 2^15
  }
  const float down = ldexpf(1.f, -ex);
#pragma unroll
  for (int kk = 0; kk < D / 32; ++kk) {
    const int h = kk / 2, sub = kk % 2;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int el = 8 * sub + i;  // element of the lane's 16 in chunk h
      const QT* e = reinterpret_cast<const QT*>(&raw.w[h][el / kVec]);
      qop[kk][i] = valid ? (_Float16)(to_float<QT>(e[el % kVec]) * down) : (_Float16)0.f;
    }
  }
  if (!finite) return __builtin_nanf("");
  return qk_scale_log2 * ldexpf(1.f, ex) * code_scale<KF>();
}

// Dequantized V of one staged block as the f16 A-operands of the PV MFMAs, written
// once by the wave that loaded the block into the slab of its block pair: half `half`
// of entry n * 64 + lane holds, for that lane (qg, r) of every wave,
// V[4 qg + j][r * VB + n] * v_scale[4 qg + j] * 2^-e, j = 0..3, so that one 16-byte read
// at the reader's own lane index gives the pair's whole operand (conflict-free). The
// code is exact in f16 (FP8 codes times 2^-8) and multiplied by the f16-rounded scale
// times 2^8 (times 2^-e). A slab value is at most v_scale * format_max in magnitude; the
// block's exponent e (returned, wave-uniform) is the unit's current exponent `ve`, or
// more when a scale exceeds `vlim` = 2^(15 + ve) / format_max, so every value stays
// below 2^15. A block that was not loaded this step leaves stale codes and finite (or
// zeroed) scales: finite values, which meet p = 0 for its keys.
template <int D>
__device__ __forceinline__ int convert_v(const char* st, int lane, int half, uint2* vt, int ve,
                                         float vlim) {
  using S = Stage<D>;
  constexpr int VB = D / 16;
  const int r = lane & 15, qg = lane >> 4;
  const float4_t vsf = *reinterpret_cast<const float4_t*>(st + S::kS + 64 + 16 * qg);
  constexpr float cs = v_weight_scale<KF>();
  // the V code words go out with the scales, so that both LDS latencies overlap
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
  half4_t vsh;
  int e = ve;
  const float vsm = fmaxf(fmaxf(vsf[0], vsf[1]), fmaxf(vsf[2], vsf[3]));
  if (__ballot(vsm > vlim) != 0 || ve != 0) {
    if (__ballot(vsm > vlim) != 0) {
      float wm = fmaxf(vsm, shfl_xor(vsm, 16));
      wm = fmaxf(wm, shfl_xor(wm, 32));
      int x;
      frexpf(wm * (format_max<KF>() / 32768.f), &x);  // wm * M / 2^15 in [2^(x-1), 2^x)
      e = max(ve, __builtin_amdgcn_readfirstlane(x));
    }
    const float c = ldexpf(cs, -e);
    vsh = half4_t{(_Float16)(vsf[0] * c), (_Float16)(vsf[1] * c), (_Float16)(vsf[2] * c),
                  (_Float16)(vsf[3] * c)};
  } else {
    vsh = half4_t{(_Float16)(vsf[0] * cs), (_Float16)(vsf[1] * cs), (_Float16)(vsf[2] * cs),
                  (_Float16)(vsf[3] * cs)};
  }
#pragma unroll
  for (int n = 0; n < VB; ++n) {
    const uint32_t col[4] = {vw[0][n / 4], vw[1][n / 4], vw[2][n / 4], vw[3][n / 4]};
    half4_t v;
    switch (n % 4) {
      case 0: v = v_operand<0, KF>(col); break;
      case 1: v = v_operand<1, KF>(col); break;
      case 2: v = v_operand<2, KF>(col); break;
      default: v = v_operand<3, KF>(col); break;
    }
    if constexpr (KF == kE5M2) {
      constexpr _Float16 down = (_Float16)(1.f / 256.f);
      v = v * half4_t{down, down, down, down};  // exact: E5M2 values times 2^-8 fit f16
    }
    vt[2 * (n * kWave + lane) + half] = __builtin_bit_cast(uint2, v * vsh);
  }
  return e;
}

// The PV MFMAs of one step: weights p = exp2(u * cfe - m) rounded to f16 for the 32 keys
// of each block pair, against the slab of that pair, and the row sums from the same
// rounded weights. The weights of block b carry 2^(e_b - ve) (vf[b], at most 1, exact
// on f16; 1 unless the step's blocks were converted with different exponents) for the
// numerator only (scaled in place after the row sums), so that every block's products
// are in units of 2^-ve.
template <int D, int NT>
__device__ __forceinline__ void prefill_pv(const uint4* vt, const float (&u)[NT][16],
                                           const float (&cfe)[NT], const float (&m)[NT],
                                           int lane, const half8_t& ones, const half4_t& vf,
                                           float4_t (&acc)[NT][D / 16 + 1]) {
  constexpr int NPV = D / 16;
#pragma unroll
  for (int pp = 0; pp < 2; ++pp) {
    half8_t pop[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        pop[t][i] = (_Float16)__builtin_amdgcn_exp2f(fmaf(u[t][8 * pp + i], cfe[t], -m[t]));
    // row sums: a V^T row of ones (row 0 of the extra tile) gives sum_k f16(p_k), the
    // same rounded weights the numerator uses
#pragma unroll
    for (int t = 0; t < NT; ++t)
      acc[t][NPV] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pop[t], acc[t][NPV], 0, 0, 0);
    // (branch-free: vf is 1 but where the step mixes exponents, and a branch here would
    // split the exponentials from the PV MFMAs they overlap with)
    {
      const _Float16 f0 = vf[2 * pp], f1 = vf[2 * pp + 1];
#pragma unroll
      for (int t = 0; t < NT; ++t) pop[t] = pop[t] * half8_t{f0, f0, f0, f0, f1, f1, f1, f1};
    }
#pragma unroll
    for (int n = 0; n < NPV; ++n) {
      const half8_t vop = __builtin_bit_cast(half8_t, vt[pp * (NPV * kWave) + n * kWave + lane]);
#pragma unroll
      for (int t = 0; t < NT; ++t)
        acc[t][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop, pop[t], acc[t][n], 0, 0, 0);
    }
  }
}

// One key step: the four staged 16-token blocks w = 0..3 (first key position
// kb0 + 16 w) through the MFMAs for the wave's NT column tiles:
//   S^T = K . Q^T      v_mfma_i32_16x16x64_i8 twice per 64-wide d chunk (hi, then lo
//                      on the hi result shifted by 7): exact int32 dot products
//   O^T += V^T . P^T   v_mfma_f32_16x16x32_f16 over the 32 keys of block pair
//                      (0, 1) and (2, 3); V^T carries the V scales, one more tile
//                      with a row of ones accumulates the softmax row sums
// Score slot j = 4 w + i of lane group qg is key 4 qg + i of block w; in the PV
// operands, slots 8 p + [0, 8) of pair p match the interleaved V slab. The base-2
// score of a key is u * cf with u = S_int * k_scale, folded into the exponent as
// fma(u, cfe, -m) (cfe = cf, or FLT_MIN where cf = 0, so that a masked u = -inf stays
// -inf). Bit w of `use` (wave-uniform): block w holds keys some column of the wave
// sees; of `bounded`: the column bounds [lo, hi] cut into block w. `masks`: the
// stages carry the blocks' padding bytes (0 = padding key), and a step holding one
// takes the edge path.
// With every block used, none bounded and every key scale times query factor below
// kSafeFactor (no score can overflow) the step takes no per-score condition; otherwise
// the scores are masked to -inf outside the bounds, for padding keys and for unused
// blocks (whose stages hold stale but finite codes and scales) and checked for
// non-finite values.
// The query columns of a wave's NT tiles, for the third query term: column t of lane
// (qg, r) is head chead[t] of token row q0 + ctok[t] (token row q0 + t0 when it is not
// valid, as loaded for the first two terms).
template <int NT>
struct ColumnRefs {
  int q0, t0;
  const int (&ctok)[NT];
  const int (&chead)[NT];
  const bool (&cvalid)[NT];
};

// The third query term of a step (INT8 codes, every tile of the wave): per 64-wide d
// chunk, lo2 rebuilt from the query elements by the column's own quantization (the terms
// query_column_i8 gives for three terms), that chunk's K.lo2 exact in int32 on the
// staged codes, added to the dequantized scores as (K.lo2 / 128) * ks. One chunk of one
// tile is live at a time and the key scales are read again from LDS, so the path fits
// beside the step's accumulators.
template <typename QT, int D, int NT>
__device__ __forceinline__ void prefill_third_term(const char* cur, const AttnArgs& a,
                                                   const ColumnRefs<NT>& col, int r, int qg,
                                                   float (&u)[NT][4 * kWaves]) {
  using S = Stage<D>;
  constexpr int KCH = D / 64;
  constexpr int kVec = 16 / (int)sizeof(QT);
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const QT* qp = static_cast<const QT*>(a.q) +
                   (int64_t)(col.q0 + (col.cvalid[t] ? col.ctok[t] : col.t0)) * a.q_tok +
                   (int64_t)col.chead[t] * a.q_head + 16 * qg;
    // the column's quantization as query_column_i8 sets it: the NaN-propagating maximum
    // of |q| over the column (lanes r, r + 16, r + 32, r + 48), the exact lift of columns
    // below 2^-64 and inv = kQRange / max (a maximum does not depend on its order)
    float mx = 0.f;
#pragma nounroll
    for (int h = 0; h < KCH; ++h) {
      uint4 w[16 / kVec];
#pragma unroll
      for (int c = 0; c < 16 / kVec; ++c) w[c] = reinterpret_cast<const uint4*>(qp + 64 * h)[c];
      const QT* e = reinterpret_cast<const QT*>(w);
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = vmax(mx, fabsf(to_float<QT>(e[i])));
    }
    mx = vmax(mx, shfl_xor(mx, 16));
    mx = vmax(mx, shfl_xor(mx, 32));
    mx = col.cvalid[t] ? mx : 0.f;
    const bool finite = __builtin_isfinite(mx);
    const float up = mx > 0.f && mx < 0x1p-64f ? 0x1p64f : 1.f;
    mx *= up;
    const float inv = (finite && mx > 0.f) ? (float)kQRange / mx : 0.f;
#pragma nounroll
    for (int h = 0; h < KCH; ++h) {
      uint4 w[16 / kVec];
#pragma unroll
      for (int c = 0; c < 16 / kVec; ++c) w[c] = reinterpret_cast<const uint4*>(qp + 64 * h)[c];
      const QT* e = reinterpret_cast<const QT*>(w);
      int4_t lo2;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        uint32_t fb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          fb[i] = __builtin_bit_cast(
              uint32_t,
              query_terms<3>(to_float<QT>(e[4 * k + i]) * up, inv).lo2);
        lo2[k] = (int)low_bytes(fb);
      }
      // chunk h's share of K.lo2 (exact), added to each score on its own
#pragma unroll
      for (int b = 0; b < kWaves; ++b) {
        const char* st = cur + b * S::kBytes;
        const int4_t sf = __builtin_amdgcn_mfma_i32_16x16x64_i8(
            *reinterpret_cast<const int4_t*>(st + S::kK + k_chunk<D>(r, qg + 4 * h)), lo2,
            int4_t{0, 0, 0, 0}, 0, 0, 0);
        const float4_t ks = *reinterpret_cast<const float4_t*>(st + S::kS + 16 * qg);
#pragma unroll
        for (int k = 0; k < 4; ++k)
          u[t][4 * b + k] = __builtin_fmaf((float)sf[k], ks[k] * (1.f / 128.f), u[t][4 * b + k]);
      }
    }
  }
}

template <typename QT, int D, int NT>
__device__ __forceinline__ void prefill_step(const char* cur, const uint4* vt, uint32_t use,
                                             uint32_t bounded, bool masks, int kb0,
                                             const QOp<D> (&qop)[NT],
                                             const float (&cf)[NT], const float (&cfe)[NT],
                                             const int (&lo)[NT], const int (&hi)[NT], int r,
                                             int qg, const half8_t& ones,
                                             const half4_t& vf,
                                             float4_t (&acc)[NT][D / 16 + 1], float (&m)[NT],
                                             bool& bad_score, const AttnArgs& a,
                                             const ColumnRefs<NT>& cols) {
  using S = Stage<D>;
  constexpr int KCH = D / 64;
  constexpr int NPV = D / 16;
  constexpr int NBK = kWaves;  // blocks per step
  // a step holding a padding key takes the edge path (read ahead of the QK block)
  bool padded = false;
  if (masks) {
    uint32_t bad = 0;
#pragma unroll
    for (int b = 0; b < NBK; ++b)
      bad |= *reinterpret_cast<const uint32_t*>(cur + b * S::kBytes + S::kF + 4 * qg) ^ 0x01010101u;
    padded = __ballot(bad != 0) != 0;
  }
  // raw scores of key 4 qg + i of block b, column tile t: exact int32 (int8 codes) or
  // f32 (FP8 codes as f16 against the f16 query)
  using Acc = typename std::conditional<KF == kInt8, int4_t, float4_t>::type;
  Acc sacc[NBK][NT];
#pragma unroll
  for (int b = 0; b < NBK; ++b) {
    const char* st = cur + b * S::kBytes;
    if constexpr (KF == kInt8) {
      int4_t kop[KCH];
#pragma unroll
      for (int h = 0; h < KCH; ++h)
        kop[h] = *reinterpret_cast<const int4_t*>(st + S::kK + k_chunk<D>(r, qg + 4 * h));
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        sacc[b][t] = int4_t{0, 0, 0, 0};
#pragma unroll
        for (int h = 0; h < KCH; ++h)
          sacc[b][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop[h], qop[t].hi[h], sacc[b][t], 0, 0, 0);
        sacc[b][t] = sacc[b][t] << 7;
#pragma unroll
        for (int h = 0; h < KCH; ++h)
          sacc[b][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop[h], qop[t].lo[h], sacc[b][t], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int t = 0; t < NT; ++t) sacc[b][t] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int h = 0; h < KCH; ++h) {
        const uint4 c = *reinterpret_cast<const uint4*>(st + S::kK + k_chunk<D>(r, qg + 4 * h));
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
          half2_t p0, p1, p2, p3;
          codes_to_f16<KF>(sub ? c.z : c.x, p0, p1);
          codes_to_f16<KF>(sub ? c.w : c.y, p2, p3);
          const half8_t kop = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
#pragma unroll
          for (int t = 0; t < NT; ++t)
            sacc[b][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop, qop[t].op[2 * h + sub],
                                                                 sacc[b][t], 0, 0, 0);
        }
      }
    }
  }
  float4_t ks[NBK];
#pragma unroll
  for (int b = 0; b < NBK; ++b)
    ks[b] = *reinterpret_cast<const float4_t*>(cur + b * S::kBytes + S::kS + 16 * qg);
  // computed without a branch, so that the QK MFMAs and the conversions below share
  // one block: scales are finite and >= 0, their order is that of their bit patterns
  int kx = 0;
#pragma unroll
  for (int b = 0; b < NBK; ++b) {
    const int4_t kb = __builtin_bit_cast(int4_t, ks[b]);
    kx = max(kx, max(max(kb[0], kb[1]), max(kb[2], kb[3])));
  }
  const float kmax = __builtin_bit_cast(float, kx);
  bool ok = true, fine = false;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const float x = kmax * cf[t];
    ok = ok && x <= safe_factor();  // false for NaN
    if constexpr (KF == kInt8) fine = fine || x > kFineScoreError / (63.5f * D);
  }
  const bool unsafe = __ballot(!ok) != 0;
  float u[NT][4 * NBK];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int j = 0; j < 4 * NBK; ++j) u[t][j] = (float)sacc[j / 4][t][j % 4] * ks[j / 4][j % 4];
  if constexpr (KF == kInt8) {
    // steps whose key scales make the two-term query's error bound pass the budget
    if (__builtin_expect(__ballot(fine) != 0, 0)) prefill_third_term<QT, D, NT>(cur, a, cols, r, qg, u);
  }
  const bool edge = (use != (1u << NBK) - 1) | (bounded != 0) | unsafe | padded;
  if (edge) {
    asm volatile("");  // keeps this a branch: if-converted, the interior steps would pay for it
    // Per-score masks as all-ones/zero words in VGPRs (sign bits of differences, bit
    // selects), not as compare results: lane masks from 32 unrolled compares per tile
    // would stay live in SGPRs and push the loop's uniform values into spills.
    uint32_t nonfinite = 0;
#pragma unroll
    for (int b = 0; b < NBK; ++b) {
      // the padding bytes of this lane's four keys of block b (1 = real, 0 = padding)
      const uint32_t pad = masks ? *reinterpret_cast<const uint32_t*>(cur + b * S::kBytes + S::kF +
                                                                      4 * qg)
                                 : 0x01010101u;
      const bool used = (use >> b) & 1u, bnd = (bounded >> b) & 1u;  // wave-uniform
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int j = 4 * b + k;
        const int key = kb0 + 16 * b + 4 * qg + k;
        const int32_t padding = (int32_t)(((pad >> (8 * k)) & 0xffu) - 1u) >> 31;  // -1: padding
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          // -1 when key < lo or key > hi (either difference negative), else 0
          const int32_t outside = bnd ? ((key - lo[t]) | (hi[t] - key)) >> 31 : 0;
          const uint32_t hide = used ? (uint32_t)(outside | padding) : 0xffffffffu;
          const uint32_t ub = __builtin_bit_cast(uint32_t, u[t][j]);
          const uint32_t xb = __builtin_bit_cast(uint32_t, u[t][j] * cf[t]);
          // exponent field all ones (inf or NaN) -> bit 31 after the carry
          nonfinite |= ((xb & 0x7f800000u) + 0x00800000u) & ~hide;
          u[t][j] = __builtin_bit_cast(float, (ub & ~hide) | (0xff800000u & hide));  // -inf
        }
      }
    }
    if (__ballot((nonfinite >> 31) != 0) != 0) bad_score = true;
  }
  float tmax[NT];
  bool need = false;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    // NaN-propagating maximum (v_maximum3_f32: no operand canonicalization)
    float mu = u[t][0];
#pragma unroll
    for (int j = 1; j < 4 * NBK; ++j) mu = vmax(mu, u[t][j]);
    tmax[t] = mu * cfe[t];  // cfe > 0: the maximum of the scaled scores
    need |= tmax[t] > m[t] + kRescaleSlack;
  }
  if (__ballot(need) != 0) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      float x = fmaxf(tmax[t], shfl_xor(tmax[t], 16));
      x = fmaxf(x, shfl_xor(x, 32));
      const float mn = fmaxf(m[t], x);
      const float alpha = __builtin_amdgcn_exp2f(m[t] - mn);
#pragma unroll
      for (int n = 0; n <= NPV; ++n) acc[t][n] *= alpha;
      m[t] = mn;
    }
  }
  static_assert(NBK == 4, "two block pairs per step");
  const int lane = qg * 16 + r;
  prefill_pv<D, NT>(vt, u, cfe, m, lane, ones, vf, acc);
}

// N consecutive outputs from fp32, with 16-byte (or 8-byte) stores.
template <typename QT, int N>
__device__ __forceinline__ void store_run(QT* dst, const float (&v)[N]) {
  constexpr int kVec = 16 / (int)sizeof(QT);
  if constexpr (sizeof(QT) == 2 && N % 8 == 0) {
#pragma unroll
    for (int c = 0; c < N / 8; ++c) {
      const uint4 w = {pack2<QT>(v[8 * c], v[8 * c + 1]), pack2<QT>(v[8 * c + 2], v[8 * c + 3]),
                       pack2<QT>(v[8 * c + 4], v[8 * c + 5]), pack2<QT>(v[8 * c + 6], v[8 * c + 7])};
      reinterpret_cast<uint4*>(dst)[c] = w;
    }
  } else if constexpr (sizeof(QT) == 2 && N == 4) {
    *reinterpret_cast<uint2*>(dst) = uint2{pack2<QT>(v[0], v[1]), pack2<QT>(v[2], v[3])};
  } else if constexpr (N % kVec == 0) {
#pragma unroll
    for (int c = 0; c < N / kVec; ++c) {
      uint4 w;
      QT* e = reinterpret_cast<QT*>(&w);
#pragma unroll
      for (int i = 0; i < kVec; ++i) e[i] = from_float<QT>(v[c * kVec + i]);
      reinterpret_cast<uint4*>(dst)[c] = w;
    }
  } else if constexpr (N * (int)sizeof(QT) == 8) {
    uint2 w;
    QT* e = reinterpret_cast<QT*>(&w);
#pragma unroll
    for (int i = 0; i < N; ++i) e[i] = from_float<QT>(v[i]);
    *reinterpret_cast<uint2*>(dst) = w;
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) dst[i] = from_float<QT>(v[i]);
  }
}

// The LDS of one prefill workgroup: the key-step stages, the V operand slabs of the
// current step and the step's block exponents.
template <int D>
struct PrefillLds {
  static constexpr int NB = kPrefillBuffers;  // key steps in flight: NB - 1 ahead of the one computed
  __attribute__((aligned(16))) char stages[NB * kWaves * Stage<D>::kBytes];  // [step % NB][wave]
  uint4 vt[kWaves / 2][(D / 16) * kWave];  // the current step's V operands, one slab per pair
  __attribute__((aligned(16))) int vexp[kWaves];  // the step's block exponents
};

// A workgroup's columns: flat column f = (wave * NT + t) * 16 + r. The unit's columns
// read query token rows q0 + tok (an invalid column reads row q0 + t0 and is zeroed)
// and see keys [lo, hi]; per wave, the bounds of its columns' key ranges (lo_min ..
// hi_max: keys some column sees; lo_max .. hi_min: keys every valid column sees) and
// whether it has a valid column.
struct ColumnInfo {
  int tok, head, lo, hi;
  bool valid;
};
struct WaveBounds {
  int lo_min, lo_max, hi_min, hi_max;
  bool any;
};

// One unit of the chunked-prefill kernels: the key blocks [b_lo, b_hi) of kv head kvh
// (physical id of block b: blocks[b], a window of the arena's ids) against the
// workgroup's query columns (column_of(f), bounds_of(wave)), through the key steps
// described at the top of this file; store(t, acc, m, lt, ve, col) then takes column
// tile t of each wave (acc in units of 2^-ve, lt the row sums of lane (0, r)'s column).
// prologue() runs (in uniform control flow) once the stages are cleared and the first
// block ids are on their way, before any column is read: it returns false (uniformly)
// to end the unit there, with nothing stored. mark(k) is called at the unit's timeline
// marks 2-5 (the tile kernel's trace builds).
template <typename QT, int D, int G, typename ColumnOf, typename BoundsOf, typename Store,
          typename Prologue, typename Mark>
__device__ __forceinline__ void prefill_unit(const AttnArgs& a, PrefillLds<D>& L, int kvh,
                                             int b_lo, int b_hi, const int32_t* blocks, int q0,
                                             int t0, ColumnOf column_of, BoundsOf bounds_of,
                                             Store store, Prologue prologue, Mark mark) {
  using S = Stage<D>;
  constexpr int NT = PrefillShape<D>::NT;
  constexpr int NPV = D / 16;
  constexpr int NB = PrefillLds<D>::NB;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int r = lane & 15, qg = lane >> 4;
  char* const lds = L.stages;
  const int nsteps = (b_hi - b_lo + kWaves - 1) / kWaves;

  // The block ids of the first 64 steps go out first, so that their load overlaps the
  // clearing of the stages and the prologue. After each load the ids pass through an
  // empty asm that redefines them: the one wait for their load happens there (once per
  // 64 steps), and the compiler's wait tracking no longer treats them as a pending load
  // at every issue below (where it would wait for every stage in flight, vmcnt(0), each
  // step).
  int ids = 0;
  auto fetch_ids = [&](int s0) __attribute__((always_inline)) {
    const int blk = b_lo + (s0 + lane) * kWaves + wave;
    ids = (s0 + lane < nsteps && blk < b_hi) ? blocks[blk] : 0;
  };
  auto load_ids = [&](int s0) __attribute__((always_inline)) {
    fetch_ids(s0);
    asm volatile("" : "+v"(ids));
  };
  if (nsteps > 0) fetch_ids(0);

  // zero scales in every stage, once every wave is past its last read of what the
  // stages held before (the dispatch plan): a stage that no step writes (a block past
  // the range) then feeds finite products; stages written by loads only ever hold arena
  // scales, which are finite (the append writes no non-finite value). Every int8 and
  // E4M3FN byte is a finite code, but E5M2 bytes with all exponent bits set are Inf/NaN,
  // so there the codes are zeroed too.
  __syncthreads();
  for (int j = lane; j < NB * 32; j += kWave)
    reinterpret_cast<float*>(lds + (j / 32) * kWaves * S::kBytes + wave * S::kBytes + S::kS)[j % 32] = 0.f;
  if constexpr (KF == kE5M2) {
    for (int j = lane; j < NB * 2 * D; j += kWave)
      reinterpret_cast<uint4*>(lds + (j / (2 * D)) * kWaves * S::kBytes + wave * S::kBytes +
                               S::kK)[j % (2 * D)] = uint4{0u, 0u, 0u, 0u};
  }
  __syncthreads();
  if (!prologue()) {
    wait_vmcnt<0>();
    return;
  }

  // ---- this wave's columns: the query goes out, then the first steps' loads, before
  // the query is quantized.
  int lo[NT], hi[NT], ctok[NT], chead[NT];
  bool cvalid[NT];
  QueryColumn<QT, D> qraw[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const ColumnInfo c = column_of((wave * NT + t) * 16 + r);
    ctok[t] = c.tok;
    chead[t] = c.head;
    cvalid[t] = c.valid;
    lo[t] = c.valid ? c.lo : INT_MAX;
    hi[t] = c.valid ? c.hi : -1;
    // an invalid column reads token t0's row (in range) and is zeroed when quantized
    const QT* qp = static_cast<const QT*>(a.q) + (int64_t)(q0 + (c.valid ? c.tok : t0)) * a.q_tok +
                   (int64_t)c.head * a.q_head + 16 * qg;
    load_query_column<QT, D>(qp, qraw[t]);
  }

  // ---- key steps: block b_lo + 4*step + w is staged by wave w. Lane i of `ids`
  // holds the id for step (i + 64*k); reloaded every 64 steps.
  bool bad_index = false, bad_score = false;
  const bool masks = a.cache.key_valid != nullptr;  // the arena has key padding bytes
  auto issue = [&](int step, char* buf) __attribute__((always_inline)) -> bool {
    if (b_lo + step * kWaves + wave >= b_hi) return false;
    const int id = __builtin_amdgcn_readlane(ids, step % kWave);
    if ((unsigned)id >= (unsigned)a.cache.num_blocks) {
      bad_index = true;
      return false;
    }
    stage_block<D>(a, id, kvh, lane, buf + wave * S::kBytes);
    return true;
  };
  auto buffer = [&](int step) __attribute__((always_inline)) -> char* {
    return lds + (step % NB) * kWaves * S::kBytes;
  };
  asm volatile("" : "+v"(ids));  // the first ids have landed
  // bit (step % NB): this wave issued loads for that step (uniform over the wave)
  uint32_t inflight = 0;
  for (int j = 0; j < NB - 1 && j < nsteps; ++j)
    if (issue(j, buffer(j))) inflight |= 1u << (j % NB);

  QOp<D> qop[NT];
  float cf[NT], cfe[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if constexpr (KF == kInt8)
      cf[t] = query_column_i8<QT, D>(qraw[t], cvalid[t], a.qk_scale_log2, qop[t].hi, qop[t].lo);
    else
      cf[t] = query_column_f16<QT, D>(qraw[t], cvalid[t], a.qk_scale_log2, qop[t].op);
    cfe[t] = cf[t] > 0.f ? cf[t] : FLT_MIN;  // cf >= 0 or NaN (scale > 0)
  }
  const WaveBounds wb = bounds_of(wave);
  mark(2);

  const ColumnRefs<NT> cols{q0, t0, ctok, chead, cvalid};
  float4_t acc[NT][NPV + 1];  // [NPV]: row sums in row 0 (lanes qg = 0)
  const _Float16 one = r == 0 ? (_Float16)1.f : (_Float16)0.f;
  const half8_t ones = {one, one, one, one, one, one, one, one};  // A operand: row 0 all ones
  float m[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int k = 0; k <= NPV; ++k) acc[t][k] = float4_t{0.f, 0.f, 0.f, 0.f};
    m[t] = -FLT_MAX;  // finite start: fully masked blocks give exp2(-inf) = 0
  }
  // The PV accumulators are in units of 2^-ve: ve is the largest block exponent so far
  // (0 unless a block's V scales need more, see convert_v); vlim is its scale limit.
  int ve = 0;
  float vlim = 32768.f / format_max<KF>();

  for (int i = 0; i < nsteps; ++i) {
    const int ahead = i + NB - 1;
    if (ahead < nsteps) {
      if (ahead % kWave == 0) load_ids(ahead);
      // its buffer was last read in step i - 1 (barrier below)
      if (issue(ahead, buffer(ahead))) inflight |= 1u << (ahead % NB);
      else inflight &= ~(1u << (ahead % NB));
    }
    // wait for step i's loads; the later steps' loads stay in flight
    int younger = 0;
#pragma unroll
    for (int k = 1; k < NB; ++k)
      if (i + k < nsteps && (inflight >> ((i + k) % NB) & 1u)) ++younger;
    if (younger >= 3) wait_vmcnt<3 * S::kLoads>();
    else if (younger == 2) wait_vmcnt<2 * S::kLoads>();
    else if (younger == 1) wait_vmcnt<S::kLoads>();
    else wait_vmcnt<0>();
    char* const cur = buffer(i);
    // this wave's block of step i is in; its V operands go to the wave's slab (the
    // previous step's readers are past the barrier that ended that step)
    const int eb = convert_v<D>(cur + wave * S::kBytes, lane, wave % 2,
                                reinterpret_cast<uint2*>(L.vt[wave / 2]), ve, vlim);
    if (lane == 0) L.vexp[wave] = eb;
    __syncthreads();  // every wave's block of step i has landed and been converted
    // the step's block exponents (each at least ve): a larger one becomes the new ve
    // (the PV tiles, not the row sums, scale by the exact 2^(ve_old - ve)); blocks
    // converted below ve weigh their products by 2^(e_b - ve)
    bool vmix = false;
    half4_t vf = {(_Float16)1.f, (_Float16)1.f, (_Float16)1.f, (_Float16)1.f};
    {
      const int4_t ev = *reinterpret_cast<const int4_t*>(L.vexp);
      int e4[kWaves];
#pragma unroll
      for (int w = 0; w < kWaves; ++w) e4[w] = __builtin_amdgcn_readfirstlane(ev[w]);
      const int emax = max(max(e4[0], e4[1]), max(e4[2], e4[3]));
      if (emax != ve) {
        const float down = ldexpf(1.f, ve - emax);
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int n = 0; n < NPV; ++n) acc[t][n] *= down;
        ve = emax;
        vlim = ldexpf(32768.f / format_max<KF>(), ve);
      }
      vmix = e4[0] != ve || e4[1] != ve || e4[2] != ve || e4[3] != ve;
      if (vmix) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) vf[w] = (_Float16)ldexpf(1.f, e4[w] - ve);
      }
    }
    {
      const int kb0 = (b_lo + i * kWaves) * kBlockTokens;
      const int kend = b_hi * kBlockTokens;
      uint32_t use = 0, bounded = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const int kb = kb0 + w * kBlockTokens;
        if (wb.any && kb < kend && kb <= wb.hi_max && kb + kBlockTokens - 1 >= wb.lo_min)
          use |= 1u << w;
        if (!(kb >= wb.lo_max && kb + kBlockTokens - 1 <= wb.hi_min)) bounded |= 1u << w;
      }
      if (use != 0)
        prefill_step<QT, D, NT>(cur, L.vt[0], use, bounded & use, masks, kb0, qop, cf, cfe, lo, hi,
                                r, qg, ones, vf, acc, m, bad_score, a, cols);
    }
    __syncthreads();  // step i's stage may be refilled
    if (i == 0) mark(3);
  }
  mark(4);
  if (bad_index && lane == 0) atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
  if (bad_score && lane == 0) atomicOr(a.err_flag, ASTR_FLAG_NONFINITE_SCORE);

#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const float lt = __shfl(acc[t][NPV][0], r, kWave);  // row 0 of the sum tile: lane (0, r)
    store(t, acc[t], m[t], lt, ve, ColumnInfo{ctok[t], chead[t], lo[t], hi[t], cvalid[t]});
  }
  mark(5);
}

template <typename QT, int D, int G>
__global__ __launch_bounds__(256) void prefill_mfma_kernel(AttnArgs a) {
  static_assert(D == 64 || D == 128 || D == 256, "head_dim");
  constexpr int NT = PrefillShape<D>::NT;
  constexpr int TQ = PrefillShape<D>::kCols / G;
  constexpr int NPV = D / 16;
  constexpr int VB = D / 16;
  static_assert(PrefillShape<D>::kCols % G == 0, "GQA group must divide the column tile");

  __shared__ PrefillLds<D> L;
  __shared__ int s_wsum[kWaves];
  __shared__ int s_found[2];

  const int lane = threadIdx.x % kWave;
  const int qg = lane >> 4;
  const int hkv = a.cache.num_kv_heads;

  // ---- 1. this workgroup's unit (uniform over the workgroup). The plan lives in the
  // stage buffers until the first load.
  static_assert(PlanTab::kInts * sizeof(int) <= sizeof(L.stages), "the dispatch plan fits the stages");
  int* const tab = reinterpret_cast<int*>(L.stages);
  int per_kv = 0;
  const int nrows = plan_rows(a, TQ, tab, s_wsum, per_kv);
  if (nrows < 0) per_kv = scan_tiles(a, TQ, -1, s_wsum, s_found);
  const int64_t units = (int64_t)per_kv * hkv;
  const int64_t per_xcd = (units + kXcds - 1) / kXcds;
  const int64_t slot = blockIdx.x / kXcds;
  const int64_t logical = (int64_t)(blockIdx.x % kXcds) * per_xcd + slot;
  if (slot >= per_xcd || logical >= units) return;
  const int kvh = (int)(logical / per_kv);
  const int unit = (int)(logical % per_kv);
  int seq, within, q0, n, ctx_raw;
  if (nrows >= 0) {
    // the first row whose inclusive prefix exceeds the unit (prefixes strictly grow)
    const int* const o_incl = PlanTab::at(tab, PlanTab::kIncl);
    int lo_r = 0, hi_r = nrows - 1;
    while (lo_r < hi_r) {
      const int mid = (lo_r + hi_r) / 2;
      if (o_incl[mid] > unit) hi_r = mid;
      else lo_r = mid + 1;
    }
    // uniform values read from LDS: readfirstlane keeps them (and all they derive) scalar
    const int row = __builtin_amdgcn_readfirstlane(PlanTab::at(tab, PlanTab::kOrder)[lo_r]);
    within = __builtin_amdgcn_readfirstlane(unit - (lo_r > 0 ? o_incl[lo_r - 1] : 0));
    seq = __builtin_amdgcn_readfirstlane(PlanTab::at(tab, PlanTab::kSeq)[row]);
    q0 = __builtin_amdgcn_readfirstlane(PlanTab::at(tab, PlanTab::kQ0)[row]);
    n = __builtin_amdgcn_readfirstlane(PlanTab::at(tab, PlanTab::kN)[row]);
    ctx_raw = __builtin_amdgcn_readfirstlane(PlanTab::at(tab, PlanTab::kCtx)[row]);
  } else {
    if (threadIdx.x == 0) s_found[0] = -1;  // ordered before the scan's writes by its barriers
    scan_tiles(a, TQ, unit, s_wsum, s_found);
    seq = __builtin_amdgcn_readfirstlane(s_found[0]);
    within = __builtin_amdgcn_readfirstlane(s_found[1]);
    if (seq < 0) return;  // unreachable for unit < per_kv; keeps every index below in range
    n = seq_queries(a, seq, q0);
    ctx_raw = a.context_lens[seq];
  }
  const int ntq = (n + TQ - 1) / TQ;
  const int tile = ntq - 1 - within;  // latest (longest) tiles first
  const bool reporter = kvh == 0 && tile == ntq - 1 && threadIdx.x == 0;
  const int ctx = clamp_ctx(a, ctx_raw, reporter);
  if (ctx < n && reporter) atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);  // chunk longer than the context

  const TileSpan span = tile_span(a, ctx, n, tile, TQ);
  const int pos0 = span.pos0, t0 = span.t0, t1 = span.t1;

  // flat column f -> token t0 + f / G, head kvh * G + f % G, keys by its position
  auto column_of = [&](int f) __attribute__((always_inline)) -> ColumnInfo {
    const int tok = t0 + f / G;
    const int p = pos0 + tok;
    return ColumnInfo{tok, kvh * G + f % G, a.window > 0 ? max(0, p - a.window + 1) : 0,
                      a.causal ? p : ctx - 1, tok < t1};
  };
  // key bounds over the wave's valid columns (positions grow with f)
  auto bounds_of = [&](int wave) __attribute__((always_inline)) -> WaveBounds {
    const int tk_lo = t0 + (wave * NT * 16) / G;
    const int tk_hi = min(t1 - 1, t0 + ((wave + 1) * NT * 16 - 1) / G);
    return WaveBounds{a.window > 0 ? max(0, pos0 + tk_lo - a.window + 1) : 0,
                      a.window > 0 ? max(0, pos0 + tk_hi - a.window + 1) : 0,
                      a.causal ? pos0 + tk_lo : ctx - 1, a.causal ? pos0 + tk_hi : ctx - 1,
                      tk_lo < t1};
  };
  // normalise and store (fully masked columns: l = 0, acc = 0 -> 0)
  auto store = [&](int t, const float4_t (&acc)[NPV + 1], float, float lt, int ve,
                   const ColumnInfo& c) __attribute__((always_inline)) {
    if (!c.valid) return;
    const float inv = ldexpf(1.f, ve) / fmaxf(lt, FLT_MIN);  // the PV tiles carry 2^-ve
    QT* op = static_cast<QT*>(a.out) + (int64_t)(q0 + c.tok) * a.o_tok + (int64_t)c.head * a.o_head;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v[VB];
#pragma unroll
      for (int k = 0; k < NPV; ++k) v[k] = acc[k][j] * inv;
      store_run<QT, VB>(op + VB * (4 * qg + j), v);
    }
  };
  prefill_unit<QT, D, G>(a, L, kvh, span.b_lo, span.b_hi,
                         a.block_tables + (int64_t)seq * a.bt_stride, q0, t0, column_of,
                         bounds_of, store, []() { return true; }, [](int) {});
}

// Prefix tiles of a decode plan (decode_plan.cpp): the shared blocks of sequences whose
// block tables begin with the same blocks, every key visible to each, read once per
// tile of up to TQ member sequences (TQ * G columns: member j's head g is column
// j G + g) and key range, as the chunked-prefill kernel reads a chunk's keys against
// its query tokens, with no mask: each column's partial (m, l, acc) of the range goes to
// the member row's chunk slot, for the chunk-merge kernel (decode_planned.hip) to merge
// with the row's other ranges and its own blocks. Tiles reading the same blocks (one kv
// head and range) are consecutive and run on one XCD, whose L2 then serves their keys.
constexpr int kTileWords = 8, kMemberWords = 3;

template <typename QT, int D, int G>
__global__ __launch_bounds__(256) void prefix_tiles_kernel(PlanArgs p) {
  static_assert(D == 64 || D == 128 || D == 256, "head_dim");
  constexpr int TQ = PrefillShape<D>::kCols / G;
  constexpr int NPV = D / 16;
  constexpr int VB = D / 16;
  static_assert(PrefillShape<D>::kCols % G == 0, "GQA group must divide the column tile");
  const AttnArgs& a = p.a;

  __shared__ PrefillLds<D> L;
  __shared__ int s_row[TQ];      // member j's query token row
  __shared__ int s_slot[TQ];     // its chunk slot for this tile's kv head and range
  __shared__ int s_bad;

  const int lane = threadIdx.x % kWave;
  const int qg = lane >> 4;
  const int hkv = a.cache.num_kv_heads;
  long long tm[8] = {0, 0, 0, 0, 0, 0, 0, 0};  // trace marks (kTrace)
  if constexpr (kTrace) tm[0] = wall_clock64();
  const int64_t units = p.info.num_tiles;
  const int64_t per_xcd = (units + kXcds - 1) / kXcds;
  const int64_t slot = blockIdx.x / kXcds;
  const int64_t unit = (int64_t)(blockIdx.x % kXcds) * per_xcd + slot;
  if (slot >= per_xcd || unit >= units) return;

  // ---- the tile, every index checked (the plan is untrusted); its members are read and
  // checked in the unit's prologue, while the first block ids load
  const int32_t* rec = p.plan + p.info.off_tiles + unit * kTileWords;
  const int m0 = rec[0], n = rec[1], kvh = rec[2], range = rec[3];
  const int blk0 = rec[4], nblk = rec[5], ids_off = rec[6], lead = rec[7];
  if (!(m0 >= 0 && n >= 1 && n <= TQ && n <= p.info.num_tile_members - m0 && kvh >= 0 &&
        kvh < hkv && range >= 0 && range < p.info.tile_ranges && blk0 >= 0 && nblk >= 0 &&
        ids_off >= 0 && nblk <= p.info.num_ids - ids_off && lead >= 0 && lead < a.num_seqs)) {
    if (threadIdx.x == 0) atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
    return;  // the whole workgroup (every thread read the same record)
  }
  if (threadIdx.x == 0) s_bad = 0;  // ordered before the prologue by the unit's barriers
  int mctx = 0;  // thread j < n: member j's context length, checked after the unit
  auto prologue = [&]() __attribute__((always_inline)) -> bool {
    if ((int)threadIdx.x < n) {
      const int32_t* mem = p.plan + p.info.off_tile_members + (int64_t)(m0 + threadIdx.x) * kMemberWords;
      const int seq = mem[0], c0 = mem[1], span = mem[2];
      if (!(seq >= 0 && seq < a.num_seqs && c0 >= 0 && span > range &&
            (int64_t)c0 + (int64_t)hkv * span <= p.info.num_chunks)) {
        s_bad = 1;
      } else {
        s_row[threadIdx.x] = seq;  // decode rows: sequence s's query token is row s
        s_slot[threadIdx.x] = c0 + kvh * span + range;
        mctx = a.context_lens[seq];  // its wait falls after the key steps
      }
    }
    __syncthreads();
    if constexpr (kTrace) tm[1] = wall_clock64();
    return __builtin_amdgcn_readfirstlane(s_bad) == 0;
  };

  // an invalid column reads member 0's query row (and is zeroed when quantized)
  auto column_of = [&](int f) __attribute__((always_inline)) -> ColumnInfo {
    const int j = f / G;
    return ColumnInfo{s_row[j < n ? j : 0], kvh * G + f % G, 0, INT_MAX, j < n};
  };
  // every key of the range is visible to every column: no step is bounded
  auto bounds_of = [&](int wave) __attribute__((always_inline)) -> WaveBounds {
    return WaveBounds{0, 0, INT_MAX, INT_MAX, (wave * PrefillShape<D>::NT * 16) / G < n};
  };
  // the partial of column (member j, head g): m, l and acc into the member's chunk
  // slot, head g, with acc and l in the decode kernels' units (both times norm_scale,
  // as the decode partials they merge with). Lane (qg, r) holds elements
  // [D/4 qg, D/4 (qg + 1)) of column r: written as they are, every store instruction
  // would touch 64 cache lines. The tile goes through the wave's share of the stage
  // buffers (free after the last key step's barrier) instead, and each store
  // instruction then writes 1 KB of whole columns (4 to 16 cache lines).
  constexpr int kRow = D + 4;  // floats per staged column (padded against bank conflicts)
  static_assert(kWaves * 16 * kRow * (int)sizeof(float) <= (int)sizeof(L.stages),
                "a wave's column tile fits its share of the stages");
  auto store = [&](int t, const float4_t (&acc)[NPV + 1], float m, float lt, int ve,
                   const ColumnInfo& c) __attribute__((always_inline)) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int f0 = (wave * PrefillShape<D>::NT + t) * 16;  // the tile's first column
    float* const tile = reinterpret_cast<float*>(L.stages) + wave * 16 * kRow;
    const float up = ldexpf(norm_scale<KF>(), ve);  // the PV tiles carry 2^-ve
    __builtin_amdgcn_wave_barrier();  // after the previous tile's reads of this share
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v[VB];
#pragma unroll
      for (int k = 0; k < NPV; ++k) v[k] = acc[k][j] * up;
#pragma unroll
      for (int k = 0; k < VB / 4; ++k)
        *reinterpret_cast<float4_t*>(tile + (lane & 15) * kRow + VB * (4 * qg + j) + 4 * k) =
            float4_t{v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
    }
    __builtin_amdgcn_wave_barrier();  // a wave's LDS accesses complete in issue order
#pragma unroll
    for (int i = 0; i < D / 16; ++i) {
      const int e = i * kWave + lane;  // float4 e of the tile: column e / (D/4)
      const int cc = e / (D / 4), q = e % (D / 4);
      const int f = f0 + cc;
      const float4_t v = *reinterpret_cast<const float4_t*>(tile + cc * kRow + 4 * q);
      if (f / G < n) {
        // non-temporal: the decode kernel reads the partials only after streaming the
        // rows' own blocks, long after they would have left the cache, and dirty lines
        // left in the cache are written back at this kernel's end (measured: config 4's
        // call 69.2 -> 68.6 us)
        const int64_t col = plan_chunk_slot(p, s_slot[f / G], G) + f % G;
        __builtin_nontemporal_store(v, reinterpret_cast<float4_t*>(a.ws_o + col * D + 4 * q));
      }
    }
    if (c.valid && qg == 0) {
      const int f = f0 + (lane & 15);
      const int64_t col = plan_chunk_slot(p, s_slot[f / G], G) + f % G;
      a.ws_ml[col * 2] = m;
      a.ws_ml[col * 2 + 1] = lt * norm_scale<KF>();
    }
  };
  const int32_t* ids = p.plan + p.info.off_ids + ids_off - blk0;  // id of block b at ids[b]
  auto mark = [&](int k) __attribute__((always_inline)) {
    if constexpr (kTrace) tm[k] = wall_clock64();
  };
  prefill_unit<QT, D, G>(a, L, kvh, blk0, blk0 + nblk, ids, 0, 0, column_of, bounds_of, store,
                         prologue, mark);
  if (s_bad) {  // a member failed its checks: nothing was stored
    if (threadIdx.x == 0) atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
    return;
  }
  // every key of the range must be visible to each member (its length as planned)
  if ((int)threadIdx.x < n) {
    const RowSpan sp = row_span(a, mctx);
    if (sp.kv_begin > blk0 * kBlockTokens || (int64_t)sp.ctx < (int64_t)(blk0 + nblk) * kBlockTokens)
      atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
  }
#if ASTR_TRACE
  const int64_t tw = unit * kWaves + threadIdx.x / kWave;
  if (lane == 0 && tw < kTileTraceWaves) {
    for (int k = 0; k < 8; ++k) g_ttrace[tw][k] = tm[k];
    g_ttrace_info[tw][0] = (nblk + kWaves - 1) / kWaves;
    g_ttrace_info[tw][1] = (int)__builtin_amdgcn_s_getreg((20 << 0) | (0 << 6) | (3 << 11));  // XCC_ID
    g_ttrace_info[tw][2] = kvh;
    g_ttrace_info[tw][3] = range;
  }
#endif
}

template <typename QT, int D, int G>
int launch(const AttnArgs& a, hipStream_t stream) {
  constexpr int TQ = PrefillShape<D>::kCols / G;
  // Sum over sequences of ceil(n/TQ) for n >= 2 is at most tokens/TQ + sequences
  // (and at most tokens/2 sequences have n >= 2).
  const int64_t seqs = a.num_seqs < a.num_q_tokens / 2 ? a.num_seqs : a.num_q_tokens / 2;
  const int64_t max_units = ((int64_t)a.num_q_tokens + TQ - 1) / TQ + seqs;
  const int64_t total = max_units * a.cache.num_kv_heads;
  const int64_t grid = (total + kXcds - 1) / kXcds * kXcds;
  if (grid == 0) return 0;
  if (grid > INT32_MAX) return fail(ASTR_EUNSUPPORTED, "prefill grid too large");
  hipLaunchKernelGGL((prefill_mfma_kernel<QT, D, G>), dim3((uint32_t)grid), dim3(kWaves * kWave),
                     0, stream, a);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "paged_attention (prefill) launch");
}

template <typename QT, int D>
int dispatch_group(const AttnArgs& a, int G, hipStream_t s) {
  switch (G) {
    case 1: return launch<QT, D, 1>(a, s);
    case 2: return launch<QT, D, 2>(a, s);
    case 4: return launch<QT, D, 4>(a, s);
    case 8: return launch<QT, D, 8>(a, s);
    case 16: return launch<QT, D, 16>(a, s);
    default: return fail(ASTR_EUNSUPPORTED, "GQA group size %d not supported", G);
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

template <typename QT, int D, int G>
int launch_tiles(const PlanArgs& p, hipStream_t stream) {
  const int64_t grid = ((int64_t)p.info.num_tiles + kXcds - 1) / kXcds * kXcds;
  if (grid == 0) return 0;
  if (grid > INT32_MAX) return fail(ASTR_EUNSUPPORTED, "prefix tile grid too large");
  hipLaunchKernelGGL((prefix_tiles_kernel<QT, D, G>), dim3((uint32_t)grid), dim3(kWaves * kWave),
                     0, stream, p);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "paged_attention (prefix tiles) launch");
}

template <typename QT, int D>
int tiles_group(const PlanArgs& p, int G, hipStream_t s) {
  switch (G) {
    case 1: return launch_tiles<QT, D, 1>(p, s);
    case 2: return launch_tiles<QT, D, 2>(p, s);
    case 4: return launch_tiles<QT, D, 4>(p, s);
    case 8: return launch_tiles<QT, D, 8>(p, s);
    case 16: return launch_tiles<QT, D, 16>(p, s);
    default: return fail(ASTR_EUNSUPPORTED, "GQA group size %d not supported", G);
  }
}

template <typename QT>
int tiles_dim(const PlanArgs& p, int G, hipStream_t s) {
  switch (p.a.cache.head_dim) {
    case 64: return tiles_group<QT, 64>(p, G, s);
    case 128: return tiles_group<QT, 128>(p, G, s);
    case 256: return tiles_group<QT, 256>(p, G, s);
    default: return fail(ASTR_EUNSUPPORTED, "head_dim %d not in {64,128,256}", p.a.cache.head_dim);
  }
}

}  // namespace

#if ASTR_TRACE && ASTR_KF == 0
// Trace builds: copies the marks and info of the first `waves` waves of the last
// prefix-tile launch of the int8 format (8 int64 + 4 int32 per wave; wave w of tile
// unit u at u * 4 + w) to host memory.
extern "C" int astr_trace_read_tiles(void* marks, void* info, int waves) {
  if (waves < 0 || waves > kTileTraceWaves) return ASTR_EINVAL;
  hipError_t e = hipMemcpyFromSymbol(marks, HIP_SYMBOL(g_ttrace), (size_t)waves * 64);
  if (e == hipSuccess) e = hipMemcpyFromSymbol(info, HIP_SYMBOL(g_ttrace_info), (size_t)waves * 16);
  return e == hipSuccess ? 0 : (int)e;
}
#endif

template <>
int launch_prefix_tiles_kf<KF>(const PlanArgs& p, int32_t q_dtype, hipStream_t stream) {
  const int G = p.a.num_q_heads / p.a.cache.num_kv_heads;
  switch (q_dtype) {
    case ASTR_F32: return tiles_dim<float>(p, G, stream);
    case ASTR_F16: return tiles_dim<_Float16>(p, G, stream);
    default: return tiles_dim<bf16_t>(p, G, stream);
  }
}

template <>
int launch_prefill_kf<KF>(const AttnArgs& a, int32_t q_dtype, hipStream_t stream) {
  const int G = a.num_q_heads / a.cache.num_kv_heads;
  switch (q_dtype) {
    case ASTR_F32: return dispatch_dim<float>(a, G, stream);
    case ASTR_F16: return dispatch_dim<_Float16>(a, G, stream);
    default: return dispatch_dim<bf16_t>(a, G, stream);
  }
}

}  // namespace attn
}  // namespace astr
