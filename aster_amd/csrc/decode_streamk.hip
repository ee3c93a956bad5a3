// Stream-K paged decode attention (gfx950, bf16/fp16 queries).
//
// The visible 16-token blocks of all sequences are laid end to end (sequence,
// then block) and cut into Wr equal contiguous ranges; wave gw streams range
// gw / Hkv for kv head gw % Hkv, so the Hkv waves working on a range at the same
// time read the same blocks for different heads (all heads of a block sit in one
// contiguous stretch of the arena) and every wave streams the same number of
// blocks whatever the context lengths. Blocks go through a per-wave LDS ring
// filled by direct global->LDS loads and the MFMA step of attention_common.h.
// Where a range begins or ends inside a row (kv head, sequence), the wave writes
// a partial (m, l, acc) for that piece; rows a single wave covers entirely are
// normalised and written directly. A wave owns at most two partial slots (its
// first and its last piece), and merge_streamk_kernel combines the pieces of
// every split row with the merge_softmax rule (online_attention.py:42-63).
#include "attention_common.h"

namespace astr {
namespace attn {
namespace {

#ifndef ASTR_KF
#define ASTR_KF 0
#endif
constexpr int KF = ASTR_KF;  // this translation unit's code format

// Waves per workgroup and LDS stages per wave: 4-wave workgroups with a 4-block ring
// per wave (2 waves per SIMD) measured best among 4/8/16-wave workgroups with 2 or 4
// stages (all within 3 %); D = 256 stages are twice as large, so 8 waves x 2 stages.
template <int D>
constexpr int sk_waves() { return D == 256 ? 8 : 4; }
template <int D>
constexpr int sk_stages() { return D == 256 ? 2 : 4; }
constexpr int kMaxSeqsSK = 512;  // per-sequence table lives in LDS
constexpr int kFastPieces = 16;  // merge: rows split into at most this many pieces load at once

// Ranges per kv head over the Bh visible blocks of one head: the resident waves
// (one round, no tail), more only where that would put over kMaxBlocksPerWaveSK
// blocks on a wave, never more than launched, and at most one range per block (so
// every range owns at least one block and a row split over ranges r0..r1 has
// exactly one piece in each of them; the merge relies on it). The decode and the
// merge kernel both derive Wr from Bh with this function.
__device__ __forceinline__ int64_t streamk_ranges(const AttnArgs& a, int64_t Bh, int hkv) {
  int64_t w = (Bh + kMaxBlocksPerWaveSK - 1) / kMaxBlocksPerWaveSK;
  if (w < a.pref_waves / hkv) w = a.pref_waves / hkv;
  if (w > a.total_waves / hkv) w = a.total_waves / hkv;
  return w < Bh ? w : Bh;
}

// Range owning block b when range r owns [floor(Bh*r/Wr), floor(Bh*(r+1)/Wr)).
__device__ __forceinline__ int64_t range_of(int64_t b, int64_t Bh, int64_t Wr) {
  return ((b + 1) * Wr - 1) / Bh;
}

// Sequence owning block b of the per-head order (s_cu[s] <= b < s_cu[s + 1], the last
// such s where empty rows share an offset); wave-uniform.
__device__ __forceinline__ int seq_of_block(const int* s_cu, int nseq, int64_t b) {
  int lo = 0, hi = nseq;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (s_cu[mid] <= b) lo = mid;
    else hi = mid;
  }
  return lo;
}

template <typename QT>
__device__ __forceinline__ void store_row_zero(const AttnArgs& a, int tok, int D) {
  QT* orow = static_cast<QT*>(a.out) + (int64_t)tok * a.o_tok;
  for (int idx = threadIdx.x; idx < a.num_q_heads * D; idx += blockDim.x)
    orow[(int64_t)(idx / D) * a.o_head + idx % D] = from_float<QT>(0.f);
}

template <typename QT, int D, int G>
__global__ __launch_bounds__(sk_waves<D>() * kWave) void decode_streamk_kernel(AttnArgs a) {
  static_assert(D == 64 || D == 128 || D == 256, "head_dim");
  static_assert(G >= 1 && G <= 16, "GQA group");
  constexpr int NS = sk_stages<D>();
  static_assert(NS >= 2 && NS <= 4, "LDS stages per wave");
  using S = Stage<D>;
  constexpr int NPV = D / 16;
  constexpr int VB = D / 16;
  constexpr int NW = sk_waves<D>();
  constexpr int SPT = (kMaxSeqsSK + NW * kWave - 1) / (NW * kWave);  // sequences per thread

  // Per wave, besides its block ring: the next window's block ids (256 bytes), which
  // arrive by direct-to-LDS loads issued well before use.
  constexpr int kIdsBytes = 256;
  __shared__ __attribute__((aligned(16))) char lds[NS * NW * S::kBytes];  // [stage][wave]
  __shared__ __attribute__((aligned(16))) char id_slots[NW * kIdsBytes];   // [wave]
  __shared__ int s_ctx[kMaxSeqsSK];  // -1: not a decode row
  __shared__ int s_tok[kMaxSeqsSK];  // query/output token row
  __shared__ int s_cu[kMaxSeqsSK + 1];
  __shared__ int s_wsum[NW];

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int r = lane & 15, qg = lane >> 4;
  const bool gvalid = r < G;
  const int nseq = a.num_seqs;
  const int hkv = a.cache.num_kv_heads;

  // ---- 1. visible blocks per sequence -> exclusive prefix s_cu (thread t owns
  // sequences SPT*t .. SPT*t + SPT-1); sequences without exactly one query token take
  // no blocks
  int nb[SPT];
#pragma unroll
  for (int k = 0; k < SPT; ++k) {
    nb[k] = 0;
    const int s = SPT * threadIdx.x + k;
    if (s < nseq) {
      const int tok = decode_token(a, s);
      s_tok[s] = tok;
      if (tok >= 0) {
        const int ctx = clamp_ctx(a, a.context_lens[s], blockIdx.x == 0);
        s_ctx[s] = ctx;
        const RowSpan sp = row_span(a, ctx);
        nb[k] = sp.last_blk - sp.first_blk;
      } else {
        s_ctx[s] = -1;
      }
    }
  }
  int local = 0;
#pragma unroll
  for (int k = 0; k < SPT; ++k) local += nb[k];
  int incl = local;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int v = __shfl_up(incl, off, kWave);
    if (lane >= off) incl += v;
  }
  if (lane == kWave - 1) s_wsum[wave] = incl;
  __syncthreads();
  int wbase = 0;
  for (int w = 0; w < wave; ++w) wbase += s_wsum[w];
  int excl = wbase + incl - local;
#pragma unroll
  for (int k = 0; k < SPT; ++k) {
    if (SPT * (int)threadIdx.x + k < nseq) s_cu[SPT * threadIdx.x + k] = excl;
    excl += nb[k];
  }
  int bseq = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) bseq += s_wsum[w];
  if (threadIdx.x == 0) s_cu[nseq] = bseq;
  __syncthreads();
  if (blockIdx.x == 0)
    for (int s = threadIdx.x; s <= nseq; s += blockDim.x) a.ws_seq[s] = s_cu[s];
  // rows with nothing visible (ctx == 0) are zero (online_attention.py:37)
  for (int s = blockIdx.x; s < nseq; s += gridDim.x)
    if (s_cu[s + 1] == s_cu[s] && s_ctx[s] >= 0) store_row_zero<QT>(a, s_tok[s], D);

  // ---- 2. this wave's head, block range and block ids / rows (lane j <-> block b0 + j);
  // waves from Wr * Hkv on have nothing to do
  const int64_t Wr = streamk_ranges(a, bseq, hkv);
  const int64_t gw = (int64_t)blockIdx.x * NW + wave;
  const int kv = (int)(gw % hkv);
  const int64_t rg = gw / hkv;
  int64_t b0 = 0;
  int n = 0;
  if (rg < Wr) {
    b0 = (int64_t)bseq * rg / Wr;
    n = (int)((int64_t)bseq * (rg + 1) / Wr - b0);
  }
  const bool too_long = n > kMaxBlocksPerWaveSK;  // contexts beyond the declared maximum
  if (too_long) n = kMaxBlocksPerWaveSK;
  // Block list in windows of 64: lane j of window w holds block b0 + 64 w + j of the
  // per-head order, as its physical id and its row id (kv_head * nseq + seq).
  // Window 0 is read here; the ids of window w + 1 go by direct-to-LDS loads into the
  // wave's id slot when window w starts, before block 64 w + NS is issued: direct-to-LDS
  // loads complete in issue order, so once a block issued after them has landed, they
  // have too (the block ring relies on the same), 64 - 2 NS blocks before they are read.
  auto window_rows = [&](int w, int& row_id) __attribute__((always_inline)) -> const int32_t* {
    const int j = 64 * w + lane;
    if (j >= n) return nullptr;
    const int64_t rem = b0 + j;
    const int sq = seq_of_block(s_cu, nseq, rem);
    row_id = kv * nseq + sq;
    return a.block_tables + (int64_t)sq * a.bt_stride + row_span(a, s_ctx[sq]).first_blk +
           (rem - s_cu[sq]);
  };
  int rows = 0, ids = 0, rows_nx = 0, ids_nx = 0;
  char* const id_slot = id_slots + wave * kIdsBytes;
  auto request_ids = [&](int w) __attribute__((always_inline)) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // earlier reads of the slot are done
    if (const int32_t* t = window_rows(w, rows_nx)) lds_dma_x1(t, lds_addr(id_slot));
  };
  if (const int32_t* t = window_rows(0, rows)) ids = *t;
  const int row0 = __builtin_amdgcn_readfirstlane(rows);
  bool bad_index =
      too_long || __ballot(lane < n && (unsigned)ids >= (unsigned)a.cache.num_blocks) != 0;
  int nblk = bad_index ? 0 : n;
  int cw = 0;  // window of `ids` / `rows`; `ids_nx` / `rows_nx` hold window cw + 1

  auto stage = [&](int j) __attribute__((always_inline)) -> char* {
    return lds + ((j % NS) * NW + wave) * S::kBytes;
  };
  auto issue = [&](int j) __attribute__((always_inline)) {
    const bool cur = (j >> 6) == cw;
    const int id = cur ? __builtin_amdgcn_readlane(ids, j & 63)
                       : __builtin_amdgcn_readlane(ids_nx, j & 63);
    const int rid = cur ? __builtin_amdgcn_readlane(rows, j & 63)
                        : __builtin_amdgcn_readlane(rows_nx, j & 63);
    stage_block<D>(a, __builtin_amdgcn_readfirstlane(id), __builtin_amdgcn_readfirstlane(rid) / nseq,
                   lane, stage(j));
  };
  // Wait until block j has landed; the blocks after it (up to NS - 1) stay in flight.
  // Loads the compiler does not count only add to what is outstanding: never too few.
  auto wait_block = [&](int j) __attribute__((always_inline)) {
    const int later = min(NS - 1, nblk - 1 - j);
    if (NS > 3 && later >= 3) wait_vmcnt<3 * S::kLoads>();
    else if (NS > 2 && later >= 2) wait_vmcnt<2 * S::kLoads>();
    else if (later >= 1) wait_vmcnt<S::kLoads>();
    else wait_vmcnt<0>();
  };
  // First row's query: its G head rows go by direct-to-LDS loads into the last
  // stage, issued before blocks 0 .. NS-2, so the block stream starts without
  // waiting for it; block NS-1 takes that stage once the query has been read out.
  QueryRaw<D> qr;
  QkOperand<D, KF> qop;
  float cf = 0.f;
  if (nblk > 0) {
    stage_query<QT, D, G>(a, s_tok[row0 % nseq], row0 / nseq, lane, stage(NS - 1));
    const int first = min(NS - 1, nblk);
    for (int j = 0; j < first; ++j) issue(j);
    if (first == 3) wait_vmcnt<3 * S::kLoads>();  // the query has landed
    else if (first == 2) wait_vmcnt<2 * S::kLoads>();
    else wait_vmcnt<S::kLoads>();
    lds_query<QT, D>(stage(NS - 1), gvalid ? r : 0, qg, qr);
    cf = qk_operand<QT, D, KF>(qr, gvalid, a.qk_scale_log2, qop,
                               query_lane_ptr<QT, G>(a, s_tok[row0 % nseq], row0 / nseq, r, qg));
    if (NS - 1 < nblk) issue(NS - 1);  // after the query reads above (their values are consumed)
    if (64 < nblk) request_ids(1);
  }

  // ---- 3. stream the blocks, one piece (the run of one row's blocks) at a time;
  // block i sits in stage i % NS and block i + NS is issued into it once consumed
  float4_t acc[NPV + 1];  // [NPV]: weight sums (INT8)
  float m = 0.f, l = 0.f;
  bool bad_score = false;
  const bool masks = a.cache.key_valid != nullptr;
  int i = 0;
  while (i < nblk) {
    const int crid = __builtin_amdgcn_readlane(rows, i & 63);  // this piece's row
    const int pstart = i;
    const int pseq = crid % nseq, pkvh = crid / nseq;
    const RowSpan psp = row_span(a, s_ctx[pseq]);
    const int64_t pfb = s_cu[pseq];  // first block of the row in the per-head order
    if (i > 0) {  // a new row starts inside this wave's range
      load_query<QT, D, G>(a, s_tok[pseq], pkvh, r, qg, qr);
      cf = qk_operand<QT, D, KF>(qr, gvalid, a.qk_scale_log2, qop,
                                 query_lane_ptr<QT, G>(a, s_tok[pseq], pkvh, r, qg));
    }
#pragma unroll
    for (int k = 0; k <= NPV; ++k) acc[k] = float4_t{0.f, 0.f, 0.f, 0.f};
    // invalid head columns never contribute; a finite start makes a block whose keys
    // are all masked (padding) give exp2(-inf) = 0, not exp2(-inf + inf)
    m = gvalid ? -FLT_MAX : 0.f;
    l = 0.f;
    VRange vr = {0.f, kVWeightCap};
    const int pos0 = (psp.first_blk + (int)(b0 + i - pfb)) * kBlockTokens;
    for (;;) {
      // the row's blocks in the current window: up to the first lane with another row
      const int wend = min(64 * (cw + 1), nblk);
      const uint64_t beyond =
          __ballot(lane >= (i & 63) && 64 * cw + lane < wend && rows != crid);
      const int iend = beyond ? 64 * cw + (int)__builtin_ctzll(beyond) : wend;
      for (; i < iend; ++i) {
        wait_block(i);
        mfma_block<QT, D, G, KF>(stage(i), qop, cf, pos0 + (i - pstart) * kBlockTokens,
                             psp.kv_begin, psp.ctx, r, qg, acc, m, l, vr, bad_score, masks);
        const int nx = i + NS;
        if (nx < nblk && (nx & 63) == 0) {
          // first block of window cw + 1: its ids were requested before block
          // nx - 64 + NS <= i was issued, which has landed; check them before use
          ids_nx = reinterpret_cast<const int*>(id_slot)[lane];
          if (__ballot(lane < min(64, nblk - nx) &&
                       (unsigned)ids_nx >= (unsigned)a.cache.num_blocks) != 0) {
            bad_index = true;
            nblk = nx;  // stop after the blocks already issued
          }
        }
        if (nx < nblk) issue(nx);
      }
      if (i == wend && i < nblk) {  // into the next window of the block list
        ids = ids_nx;
        rows = rows_nx;
        ++cw;
        if (64 * (cw + 1) < nblk) request_ids(cw + 1);
        if (__builtin_amdgcn_readlane(rows, 0) == crid) continue;  // the row goes on
      }
      break;
    }
    // write the piece [pstart, i): the final output when the whole row is in this
    // wave, else a partial in slot 0 (the piece starts the wave's range) or 1 (it
    // ends it)
    const int iend = i;
    end_piece<D, KF>(acc, r);
    float lt = l + shfl_xor(l, 16);
    lt += shfl_xor(lt, 32);
    lt *= norm_scale<KF>();  // the factor the PV weights carry
    const int64_t pfe = pfb + (s_cu[pseq + 1] - s_cu[pseq]) - 1;
    if (b0 + pstart == pfb && b0 + iend - 1 == pfe) {
      if (gvalid) {
        const float inv = 1.f / fmaxf(lt, FLT_MIN);
        QT* op = static_cast<QT*>(a.out) + (int64_t)s_tok[pseq] * a.o_tok +
                 (int64_t)(pkvh * G + r) * a.o_head;
#pragma unroll
        for (int k = 0; k < NPV; ++k)
#pragma unroll
          for (int j = 0; j < 4; ++j) op[VB * (4 * qg + j) + k] = from_float<QT>(acc[k][j] * inv);
      }
    } else if (gvalid) {
      const int64_t slot = (gw * 2 + (pstart == 0 ? 0 : 1)) * G + r;
      float* o = a.ws_o + slot * D;
#pragma unroll
      for (int k = 0; k < NPV; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) o[VB * (4 * qg + j) + k] = acc[k][j];
      if (qg == 0) {
        a.ws_ml[slot * 2] = m;
        a.ws_ml[slot * 2 + 1] = lt;
      }
    }
  }
  if (bad_index && lane == 0) atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
  if (bad_score && lane == 0) atomicOr(a.err_flag, ASTR_FLAG_NONFINITE_SCORE);
}

// One wave per (sequence, q head): merge the pieces of rows split across waves.
template <typename QT, int D>
__global__ __launch_bounds__(256) void merge_streamk_kernel(AttnArgs a) {
  constexpr int kPerLane = (D + kWave - 1) / kWave;
  const int lane = threadIdx.x % kWave;
  const int unit = blockIdx.x * kWaves + threadIdx.x / kWave;  // seq * Hq + h
  if (unit >= a.num_seqs * a.num_q_heads) return;
  const int seq = unit / a.num_q_heads, h = unit % a.num_q_heads;
  const int G = a.num_q_heads / a.cache.num_kv_heads;
  const int kvh = h / G, g = h % G;
  const int cu0 = a.ws_seq[seq], cu1 = a.ws_seq[seq + 1], bseq = a.ws_seq[a.num_seqs];
  if (cu1 == cu0) return;  // empty or not a decode row: nothing to merge
  const int hkv = a.cache.num_kv_heads;
  const int64_t Wr = streamk_ranges(a, bseq, hkv);
  const int64_t fb = cu0, fe = cu1 - 1;  // the row's blocks in the per-head order
  const int64_t r0 = range_of(fb, bseq, Wr), r1 = range_of(fe, bseq, Wr);
  if (r0 == r1) return;  // written whole by one wave
  const int pieces = (int)(r1 - r0 + 1);
  const bool first_is_tail = (int64_t)bseq * r0 / Wr < fb;  // the row is r0's last piece (slot 1)
  auto slot_of = [&](int p) __attribute__((always_inline)) -> int64_t {
    const int64_t w = (r0 + p) * hkv + kvh;  // the wave that streamed range r0 + p for this head
    return (w * 2 + (p == 0 && first_is_tail ? 1 : 0)) * G + g;
  };
  float L = 0.f, O[kPerLane];
#pragma unroll
  for (int e = 0; e < kPerLane; ++e) O[e] = 0.f;
  if (pieces <= kFastPieces) {
    // common case: every load (statistics and partial rows) issues before the first use
    float mp = -INFINITY, lp = 0.f;
    if (lane < pieces) {
      mp = a.ws_ml[slot_of(lane) * 2];
      lp = a.ws_ml[slot_of(lane) * 2 + 1];
    }
    float v[kFastPieces][kPerLane];
#pragma unroll
    for (int u = 0; u < kFastPieces; ++u) {
      const float* op = a.ws_o + slot_of(u < pieces ? u : 0) * D;
#pragma unroll
      for (int e = 0; e < kPerLane; ++e) {
        const int d = lane + e * kWave;
        v[u][e] = (u < pieces && d < D) ? op[d] : 0.f;
      }
    }
    const float M = wave_max(mp);
    const float w = mp == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mp - M);
    L = wave_sum(lp * w);
#pragma unroll
    for (int u = 0; u < kFastPieces; ++u) {
      const float wq = __shfl(w, u, kWave);
#pragma unroll
      for (int e = 0; e < kPerLane; ++e) O[e] = fmaf(v[u][e], wq, O[e]);
    }
  } else {
    float M = -INFINITY;
    for (int p = lane; p < pieces; p += kWave) M = fmaxf(M, a.ws_ml[slot_of(p) * 2]);
    M = wave_max(M);
    for (int p0 = 0; p0 < pieces; p0 += kWave) {
      const int p = p0 + lane;
      float w = 0.f, lw = 0.f;
      if (p < pieces) {
        const float mp = a.ws_ml[slot_of(p) * 2];
        w = mp == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mp - M);
        lw = a.ws_ml[slot_of(p) * 2 + 1] * w;
      }
      L += wave_sum(lw);
      const int np = min(kWave, pieces - p0);
      for (int q0 = 0; q0 < np; q0 += 8) {
        float v[8][kPerLane], wq[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int q = min(q0 + u, np - 1);
          wq[u] = q0 + u < np ? __shfl(w, q, kWave) : 0.f;
          const float* op = a.ws_o + slot_of(p0 + q) * D;
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
  }
  QT* out = static_cast<QT*>(a.out) + (int64_t)decode_token(a, seq) * a.o_tok +
            (int64_t)h * a.o_head;
  const float inv_l = 1.f / fmaxf(L, FLT_MIN);
#pragma unroll
  for (int e = 0; e < kPerLane; ++e) {
    const int d = lane + e * kWave;
    if (d < D) out[d] = from_float<QT>(O[e] * inv_l);
  }
}

// Workgroups of `kernel` one CU holds at once (queried once per kernel).
template <typename Kernel>
int resident_per_cu(Kernel kernel, int threads) {
  static int cached = 0;
  if (cached == 0) {
    int n = 0;
    cached = (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0) ==
                  hipSuccess && n > 0)
                 ? n
                 : 1;
  }
  return cached;
}

int device_cus() {
  int dev = 0, v = 0;
  if (hipGetDevice(&dev) == hipSuccess &&
      hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
    return v;
  return 256;
}

template <typename QT, int D, int G>
int launch(AttnArgs a, hipStream_t stream) {
  auto kernel = decode_streamk_kernel<QT, D, G>;
  constexpr int NW = sk_waves<D>();
  // launch one wave per resident slot (whole workgroups) and at least min_waves (the
  // host-side bound), at most the workspace capacity passed in total_waves; the
  // kernels settle the waves they use from the actual block count
  const int64_t resident = (int64_t)device_cus() * resident_per_cu(kernel, NW * kWave) * NW;
  int64_t waves = resident;
  if (waves < a.min_waves) waves = (a.min_waves + NW - 1) / NW * NW;
  if (waves > a.total_waves) waves = a.total_waves / NW * NW;
  a.total_waves = (int32_t)waves;
  a.pref_waves = (int32_t)(resident < waves ? resident : waves);
  const int wgs = (int)(waves / NW);
  hipLaunchKernelGGL(kernel, dim3(wgs), dim3(NW * kWave), 0, stream, a);
  const int units = a.num_seqs * a.num_q_heads;
  hipLaunchKernelGGL((merge_streamk_kernel<QT, D>), dim3((units + kWaves - 1) / kWaves),
                     dim3(kWaves * kWave), 0, stream, a);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "paged_attention (stream-K) launch");
}

template <typename QT, int D>
int dispatch_group(const AttnArgs& a, int G, hipStream_t s) {
  switch (G) {
    case 1: return launch<QT, D, 1>(a, s);
    case 2: return launch<QT, D, 2>(a, s);
    case 4: return launch<QT, D, 4>(a, s);
    case 8: return launch<QT, D, 8>(a, s);
    case 16:
      if constexpr (D <= 128) return launch<QT, D, 16>(a, s);
      [[fallthrough]];
    default:
      return fail(ASTR_EUNSUPPORTED, "GQA group size %d not supported", G);
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
int launch_streamk_kf<KF>(const AttnArgs& a, int32_t q_dtype, hipStream_t stream) {
  if (a.min_waves > a.total_waves)
    return fail(ASTR_EINVAL, "stream-K workspace too small for this launch");
  const int G = a.num_q_heads / a.cache.num_kv_heads;
  if (q_dtype == ASTR_F16) return dispatch_dim<_Float16>(a, G, stream);
  if (q_dtype == ASTR_BF16) return dispatch_dim<bf16_t>(a, G, stream);
  return fail(ASTR_EUNSUPPORTED, "stream-K decode takes bf16/fp16 queries");
}

#if ASTR_KF == 0
int stream_k_max_seqs() { return kMaxSeqsSK; }
#endif

}  // namespace attn
}  // namespace astr
