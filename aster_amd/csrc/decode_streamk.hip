// Stream-K paged decode attention (gfx950, bf16/fp16 queries).
//
// Work rows: the prefix packs of the call (host plan: sequences whose block tables
// begin with the same blocks, read once for up to 16/G sequences, one query column
// per member head), then the sequences (the blocks of a packed sequence after its
// pack's). The blocks of all work rows are laid end to end and cut into Wr equal
// contiguous ranges; wave gw streams range gw / Hkv for kv head gw % Hkv, so the Hkv
// waves working on a range at the same time read the same blocks for different
// heads (all heads of a block sit in one contiguous stretch of the arena) and every
// wave streams the same number of blocks whatever the context lengths. Blocks go
// through a per-wave LDS ring filled by direct global->LDS loads and the MFMA step
// of attention_common.h. Where a range begins or ends inside a work row, the wave
// writes a partial (m, l, acc) for that piece into one of its two slots (its first
// and its last piece); a sequence row a single wave covers entirely is normalised
// and written directly, unless it is packed: then that piece, like a pack's whole
// piece, goes to the row's own slot. merge_streamk_kernel combines the pieces of a
// sequence (its pack's column and its own) with the merge_softmax rule
// (online_attention.py:42-63).
#include "attention_common.h"

namespace astr {
namespace attn {
namespace {

#ifndef ASTR_KF
#define ASTR_KF 0
#endif
constexpr int KF = ASTR_KF;  // this translation unit's code format

// The product build compiles this source twice per code format: the launches with
// prefix packs, the entry point and the shared tables (ASTR_SK_PART 1), and the
// launches without packs (ASTR_SK_PART 2), a unit scheduled for instruction-level
// parallelism (measured faster for sequence rows, slower for pack rows). Trace builds
// compile it once (ASTR_SK_PART 0), so that one set of trace marks serves every launch.
#ifndef ASTR_SK_PART
#define ASTR_SK_PART 0
#endif

// Per-wave timeline (trace builds only, -DASTR_TRACE=1, built apart from the product
// library by `python -m aster_amd.build --trace`): wall-clock marks (100 MHz
// s_memrealtime) of each wave of the last stream-K launch, read back with
// astr_trace_read. Marks: 0 entry, 1 block prefix done, 2 block ids in hand, 3 first
// block landed, 4 exit; of the wave's second piece: 5 end of the first piece's blocks,
// 6 its query loaded and quantised, 7 its first block landed. Info: blocks, pieces,
// pack blocks, XCC id.
#ifndef ASTR_TRACE
#define ASTR_TRACE 0
#endif
constexpr bool kTrace = ASTR_TRACE != 0;
#if ASTR_TRACE
constexpr int kTraceWaves = 16384;
static __device__ long long g_trace[kTraceWaves][8];
static __device__ int g_trace_info[kTraceWaves][4];
#endif

// Waves per workgroup and LDS stages per wave: 4-wave workgroups with a 4-block ring
// per wave (2 waves per SIMD) measured best among 4/8/16-wave workgroups with 2 or 4
// stages (all within 3 %); D = 256 stages are twice as large, so 8 waves x 2 stages.
template <int D>
constexpr int sk_waves() { return D == 256 ? 8 : 4; }
template <int D>
constexpr int sk_stages() { return D == 256 ? 2 : 4; }
constexpr int kMaxSeqsSK = 512;   // per-sequence tables live in LDS
// With prefix packs the tables hold fewer sequences (their LDS goes to the pack
// tables): at most kMaxPackSeqsSK sequences and kMaxPacksSK packs (thread k of a
// workgroup owns pack k).
constexpr int kMaxPackSeqsSK = 256;
constexpr int kMaxPacksSK = 128;
constexpr int kMaxRowsSK = kMaxSeqsSK + 1;  // block prefix entries over work rows (+ 1)
constexpr int kFastPieces = 16;   // merge: sequences in at most this many pieces load at once


// Work rows of one kv head: packs 0 .. npk-1, then sequence s as row npk + s.
// row_seq: the sequence of row x, or -1 - k for pack k.
__device__ __forceinline__ int row_seq(int x, int npk) { return x < npk ? -1 - x : x - npk; }

// The split of one kv head's Bh blocks (the PB blocks of the packs first) into Wr
// contiguous ranges of equal cost. A pack block costs KP and any other block kSeqCost
// (pack blocks are shared by all rows of the call and hit in cache, so they are bound
// by the waves' own work, while a sequence's own blocks stream from HBM), and every
// work row with blocks costs kRowCost more, charged to its first block: block b of a
// row with ne rows with blocks before it starts at cost c(b) = wcost(b) +
// kRowCost (ne + 1), wcost(b) the block costs before b. Range r owns the blocks whose
// start lies in [T r / Wr, T (r + 1) / Wr), T = wcost(Bh) + kRowCost * (rows with
// blocks). The costs were fitted to per-wave timelines of the config2 and config4
// workloads (a row start measured ~3.4 us against ~1.27 us per streamed block; pack
// blocks ~0.85 us). KP is 32 (against 50 per sequence block) unless the pack blocks
// would then take over half of T: each CU holds the workgroups of ranges r and
// r + Wr / 2, and two compute-bound pack waves on one CU run ~25 % slower per block
// (config 4 with packs: 72.8 us at KP 32, 78.9 at 33, where the packs pass one half).
// Wr: the resident waves per head (one round,
// no tail), more where a range could otherwise hold over kMaxBlocksPerWaveSK
// blocks, never more than launched, and ranges no shorter than a block's cost, so
// that a row split over ranges r0..r1 has exactly one piece in each of them (the
// merge relies on it; a range between two rows may own no block, its wave then
// has nothing to do). The decode and the merge kernel both derive the split with
// this type.
constexpr int kSeqCost = kSkSeqCost, kRowCost = kSkRowCost;
// pack block cost: the pack blocks' cost at most the rest of the split's
__device__ __forceinline__ int64_t sk_pack_cost(int64_t bh, int64_t pb, int64_t rows) {
  if (pb <= 0) return kSkPackCostMax;
  const int64_t even = (kSeqCost * (bh - pb) + kRowCost * rows) / pb;
  return even < kSkPackCostMin ? kSkPackCostMin : even > kSkPackCostMax ? kSkPackCostMax : even;
}
struct SkSplit {
  int64_t PB, KP, T, Wr;
  __device__ SkSplit(const AttnArgs& a, int64_t bh, int64_t pb, int64_t rows_with_blocks,
                     int hkv)
      : PB(pb), KP(sk_pack_cost(bh, pb, rows_with_blocks)),
        T(KP * pb + kSeqCost * (bh - pb) + kRowCost * rows_with_blocks) {
    // the resident waves, or more where a range would pass kMaxBlocksPerWaveSK pack
    // blocks (divided only then: KP is not a constant)
    int64_t w = a.pref_waves / hkv;
    if (T > w * KP * kMaxBlocksPerWaveSK)
      w = (T + KP * kMaxBlocksPerWaveSK - 1) / (KP * kMaxBlocksPerWaveSK);
    if (w > a.total_waves / hkv) w = a.total_waves / hkv;
    const int64_t most = T / kSeqCost > 1 ? T / kSeqCost : 1;
    Wr = w < most ? w : most;
  }
  __device__ int64_t wcost(int64_t b) const {
    return b < PB ? KP * b : KP * PB + kSeqCost * (b - PB);
  }
  // start of block b of a row with `ne` rows with blocks before it
  __device__ int64_t cost(int64_t b, int ne) const { return wcost(b) + kRowCost * (ne + 1); }
  // 32-bit quotients where the products fit (every launch up to ~2^31 / Wr cost)
  __device__ bool narrow() const { return T * (Wr + 1) < ((int64_t)1 << 31); }
  __device__ int64_t range_at(int64_t c) const {
    return narrow() ? (int64_t)((uint32_t)(c * Wr) / (uint32_t)T) : c * Wr / T;
  }
  __device__ int64_t range_of(int64_t b, int ne) const { return range_at(cost(b, ne)); }
  // the least cost range r may start at: ceil(T r / Wr)
  __device__ int64_t target(int64_t r) const {
    return narrow() ? (int64_t)((uint32_t)(T * r + Wr - 1) / (uint32_t)Wr)
                    : (T * r + Wr - 1) / Wr;
  }
};

// First block of ranges r and r + 1 (wave-uniform): the first block whose start
// cost reaches the range's target. A lane-parallel search over the work rows' start
// costs (monotone; a row without blocks shares the next row's): lane l tests rows
// l * S (S = ceil(nrow / 64)), then the S rows after the last passing one, for both
// targets at once (lanes 0-31 and 32-63 in the second round).
__device__ __forceinline__ void range_bounds(const SkSplit& sp, int64_t r, const int* s_cu,
                                            const short* s_ne, int nrow, int npk, int lane,
                                            int64_t& b0, int64_t& b1) {
  const int64_t c0 = sp.target(r), c1 = sp.target(r + 1);
  auto start = [&](int x) __attribute__((always_inline)) -> int64_t {
    return sp.cost(s_cu[x], s_ne[x]);
  };
  const int S = (nrow + kWave - 1) / kWave;
  const int xa = lane * S;
  const int64_t ca = xa < nrow ? start(xa) : INT64_MAX;
  const int la = __popcll(__ballot(ca <= c0)) - 1, lb = __popcll(__ballot(ca <= c1)) - 1;
  const int half = lane >> 5, j = lane & 31;
  const int base = (half == 0 ? la : lb) * S;
  const int xb = base + j;
  const int64_t cb = base >= 0 && j < S && xb < nrow ? start(xb) : INT64_MAX;
  const uint64_t pass = __ballot(cb <= (half == 0 ? c0 : c1));
  const int x0 = la < 0 ? -1 : la * S + __popcll(pass & 0xffffffffull) - 1;
  const int x1 = lb < 0 ? -1 : lb * S + __popcll(pass >> 32) - 1;
  auto first_at = [&](int x, int64_t c) __attribute__((always_inline)) -> int64_t {
    if (x < 0) return 0;  // before the first row's start
    const int64_t w = x < npk ? sp.KP : kSeqCost;
    const int64_t k = (c - start(x) + w - 1) / w;
    const int64_t b = s_cu[x] + k;
    return b < s_cu[x + 1] ? b : s_cu[x + 1];
  };
  b0 = first_at(x0, c0);
  b1 = first_at(x1, c1);
}

// Work row owning block b of the per-head order (s_cu[x] <= b < s_cu[x + 1], the last
// such x where empty rows share an offset); wave-uniform.
__device__ __forceinline__ int row_of_block(const int* s_cu, int nrow, int64_t b) {
  int lo = 0, hi = nrow;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (s_cu[mid] <= b) lo = mid;
    else hi = mid;
  }
  return lo;
}

// Partial slots, counted in columns of D floats (and (m, l) pairs): two per wave
// (slot_cols columns each) for pieces cut by a range boundary, then the slots of
// work rows that one wave streams whole but that still merge: pack k of kv head kvh
// (pack_rows * G columns), then packed sequence at pack column pc (G columns).
__device__ __forceinline__ int64_t wave_slot(const AttnArgs& a, int64_t wave, int which, int col) {
  return (wave * 2 + which) * a.slot_cols + col;
}
__device__ __forceinline__ int64_t pack_slot(const AttnArgs& a, int G, int kvh, int k, int col) {
  const int64_t base = (int64_t)a.total_waves * 2 * a.slot_cols;
  return base + ((int64_t)kvh * a.num_packs + k) * a.pack_rows * G + col;
}
__device__ __forceinline__ int64_t packed_seq_slot(const AttnArgs& a, int G, int hkv, int kvh,
                                                   int pc, int g) {
  const int64_t base = (int64_t)a.total_waves * 2 * a.slot_cols +
                       (int64_t)hkv * a.num_packs * a.pack_rows * G;
  return base + ((int64_t)kvh * a.num_packs * a.pack_rows + pc) * G + g;
}

template <typename QT>
__device__ __forceinline__ void store_row_zero(const AttnArgs& a, int tok, int D) {
  QT* orow = static_cast<QT*>(a.out) + (int64_t)tok * a.o_tok;
  for (int idx = threadIdx.x; idx < a.num_q_heads * D; idx += blockDim.x)
    orow[(int64_t)(idx / D) * a.o_head + idx % D] = from_float<QT>(0.f);
}

// kPacks: the launch carries prefix packs (a separate instantiation, so that batches
// without them run none of the pack code).
template <typename QT, int D, int G, bool kPacks>
__global__ __launch_bounds__(sk_waves<D>() * kWave) void decode_streamk_kernel(AttnArgs a) {
  static_assert(D == 64 || D == 128 || D == 256, "head_dim");
  static_assert(G >= 1 && G <= 16, "GQA group");
  constexpr int NS = sk_stages<D>();
  static_assert(NS >= 2 && NS <= 4, "LDS stages per wave");
  using S = Stage<D>;
  constexpr int NPV = D / 16;
  constexpr int NW = sk_waves<D>();
  constexpr int SEQS = kPacks ? kMaxPackSeqsSK : kMaxSeqsSK;
  constexpr int PACKS = kPacks ? kMaxPacksSK : 1;
  constexpr int SPT = (SEQS + NW * kWave - 1) / (NW * kWave);  // sequences per thread
  constexpr int kPackRowsMax = 16 / G;
  static_assert(NW * kWave >= kMaxPacksSK, "one pack per thread");

  // Per wave, besides its block ring: the next window's block ids (256 bytes), which
  // arrive by direct-to-LDS loads issued well before use.
  constexpr int kIdsBytes = 256;
  __shared__ __attribute__((aligned(16))) char lds[NS * NW * S::kBytes];  // [stage][wave]
  __shared__ __attribute__((aligned(16))) char id_slots[NW * kIdsBytes];   // [wave]
  __shared__ int s_ctx[SEQS];   // -1: not a decode row
  __shared__ int s_tok[SEQS];   // query/output token row
  __shared__ int s_cu[SEQS + PACKS + 1];
  __shared__ short s_ne[SEQS + PACKS + 1];  // work rows with blocks before row x
  __shared__ int s_wsum[4 * NW];  // per wave: pack blocks, sequence blocks, and their rows
  __shared__ int s_pcol[kPacks ? SEQS : 1];  // pack column k * pack_rows + p of a member, else INT_MAX
  __shared__ short s_pmem[kPacks ? SEQS : 1];  // [k * pack_rows + p]: member sequence or -1
  __shared__ int s_pblk[PACKS];               // shared blocks of pack k (0: no member left)
  __shared__ short s_plead[PACKS];            // first member of pack k: its table holds the blocks

  long long tm[8] = {0, 0, 0, 0, 0, 0, 0, 0};  // trace marks (kTrace)
  if constexpr (kTrace) tm[0] = wall_clock64();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int r = lane & 15, qg = lane >> 4;
  const int nseq = a.num_seqs;
  const int hkv = a.cache.num_kv_heads;
  const int npk = kPacks ? a.num_packs : 0, P = kPacks ? a.pack_rows : 1;
  const int nrow = npk + nseq;

  // ---- 0. this thread's pack record (thread k: pack k), loaded with the lengths below
  int mem[kPackRowsMax];
  int shared = 0;
  const bool mine = kPacks && (int)threadIdx.x < npk;
  if constexpr (kPacks) {
    const int32_t* rec = a.packs + (int64_t)threadIdx.x * (1 + P);
    shared = mine ? rec[0] : 0;
#pragma unroll
    for (int p = 0; p < kPackRowsMax; ++p) mem[p] = (mine && p < P) ? rec[1 + p] : -1;
  }

  // ---- 1. per sequence: token row and visible context (thread t owns sequences
  // SPT*t .. SPT*t + SPT-1); sequences without exactly one query token take no blocks
  int nb[SPT];
#pragma unroll
  for (int k = 0; k < SPT; ++k) {
    nb[k] = 0;
    const int s = SPT * threadIdx.x + k;
    if (s < nseq) {
      const int tok = decode_token(a, s);
      s_tok[s] = tok;
      if constexpr (kPacks) s_pcol[s] = INT_MAX;
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
  if constexpr (kPacks) {
    // the pack record is needed after the barrier below: take it now, while the
    // context lengths arrive, so that it is not loaded only then
#pragma unroll
    for (int p = 0; p < kPackRowsMax; ++p) asm volatile("" ::"v"(mem[p]));
    asm volatile("" ::"v"(shared));
  }
  // ---- 1b. packs (thread k checks pack k): a member must be a decode row listed once
  // whose first shared-blocks * 16 tokens are all visible (no window); a member that
  // fails is dropped from its pack (and the plan reported as bad), a pack without
  // members streams nothing
  int pack_blocks = 0;
  bool bad_plan = false;
  if constexpr (kPacks) if (npk > 0) {
    __syncthreads();
    // all members' LDS entries first (independent reads), then the tests
    int mtok[kPackRowsMax], mctx[kPackRowsMax];
#pragma unroll
    for (int p = 0; p < kPackRowsMax; ++p) {
      const int sm = mem[p] >= 0 && mem[p] < nseq ? mem[p] : 0;
      mtok[p] = s_tok[sm];
      mctx[p] = s_ctx[sm];
    }
#pragma unroll
    for (int p = 0; p < kPackRowsMax; ++p) {
      if (mem[p] == -1) continue;
      const int sm = mem[p];
      const bool ok = sm >= 0 && sm < nseq && shared >= 1 && a.window == 0 && mtok[p] >= 0 &&
                      (int64_t)shared * kBlockTokens <= mctx[p];
      if (ok) {
        atomicMin(&s_pcol[sm], (int)threadIdx.x * P + p);
      } else {
        bad_plan = true;
        mem[p] = -1;
      }
    }
    __syncthreads();
    int lead = -1, won[kPackRowsMax];
#pragma unroll
    for (int p = 0; p < kPackRowsMax; ++p) won[p] = s_pcol[mem[p] >= 0 ? mem[p] : 0];
#pragma unroll
    for (int p = 0; p < kPackRowsMax; ++p) {
      if (mem[p] >= 0 && won[p] != (int)threadIdx.x * P + p) {  // listed twice
        bad_plan = true;
        mem[p] = -1;
      }
      if (mine && p < P) s_pmem[threadIdx.x * P + p] = (short)mem[p];
      if (lead < 0) lead = mem[p];
    }
    if (mine) {
      pack_blocks = lead >= 0 ? shared : 0;
      s_pblk[threadIdx.x] = pack_blocks;
      s_plead[threadIdx.x] = (short)lead;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < SPT; ++k) {  // a packed sequence's own row starts after the pack's
      const int s = SPT * threadIdx.x + k;
      if (s < nseq && s_pcol[s] < npk * P) nb[k] -= s_pblk[s_pcol[s] / P];
    }
  }
  auto pack_col = [&](int s) __attribute__((always_inline)) -> int {
    if constexpr (kPacks) return npk > 0 && s_pcol[s] < npk * P ? s_pcol[s] : -1;
    return -1;
  };

  // ---- 2. block prefix over work rows: the packs' blocks (pack t on thread t) and
  // the sequences' blocks scanned side by side, the sequences placed after every
  // pack; beside them the counts of rows with blocks (the split's row costs)
  int lseq = 0, lrows = 0;
#pragma unroll
  for (int k = 0; k < SPT; ++k) {
    lseq += nb[k];
    lrows += nb[k] > 0;
  }
  int ip = pack_blocks, is = lseq, ipr = pack_blocks > 0, isr = lrows;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int vq = __shfl_up(is, off, kWave);
    const int vqr = __shfl_up(isr, off, kWave);
    if constexpr (kPacks) {
      const int vp = __shfl_up(ip, off, kWave);
      const int vpr = __shfl_up(ipr, off, kWave);
      if (lane >= off) {
        ip += vp;
        ipr += vpr;
      }
    }
    if (lane >= off) {
      is += vq;
      isr += vqr;
    }
  }
  if (lane == kWave - 1) {
    if constexpr (kPacks) {
      s_wsum[wave] = ip;
      s_wsum[2 * NW + wave] = ipr;
    }
    s_wsum[NW + wave] = is;
    s_wsum[3 * NW + wave] = isr;
  }
  __syncthreads();
  int bp = 0, bs = 0, pack_total = 0, bseq = 0;
  int rp = 0, rs = 0, pack_rows_total = 0, rows_total = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    if (w < wave) {
      if constexpr (kPacks) {
        bp += s_wsum[w];
        rp += s_wsum[2 * NW + w];
      }
      bs += s_wsum[NW + w];
      rs += s_wsum[3 * NW + w];
    }
    if constexpr (kPacks) {
      pack_total += s_wsum[w];
      pack_rows_total += s_wsum[2 * NW + w];
    }
    bseq += s_wsum[NW + w];
    rows_total += s_wsum[3 * NW + w];
  }
  bseq += pack_total;
  rows_total += pack_rows_total;
  if (kPacks && (int)threadIdx.x < npk) {
    s_cu[threadIdx.x] = bp + ip - pack_blocks;
    s_ne[threadIdx.x] = (short)(rp + ipr - (pack_blocks > 0));
  }
  int excl = pack_total + bs + is - lseq;
  int rexcl = pack_rows_total + rs + isr - lrows;
#pragma unroll
  for (int k = 0; k < SPT; ++k) {
    const int s = SPT * threadIdx.x + k;
    if (s < nseq) {
      s_cu[npk + s] = excl;
      s_ne[npk + s] = (short)rexcl;
    }
    excl += nb[k];
    rexcl += nb[k] > 0;
  }
  if (threadIdx.x == 0) {
    s_cu[nrow] = bseq;
    s_ne[nrow] = (short)rows_total;
  }
  __syncthreads();
  if (blockIdx.x == 0) {
    for (int x = threadIdx.x; x <= nrow; x += blockDim.x) {
      a.ws_seq[x] = s_cu[x];
      a.ws_ne[x] = s_ne[x];
    }
    if (npk > 0)
      for (int s = threadIdx.x; s < nseq; s += blockDim.x) {
        const int pc = pack_col(s);
        a.ws_pack[4 * s] = pc;
        a.ws_pack[4 * s + 1] = pc >= 0 ? s_cu[pc / P] : 0;
        a.ws_pack[4 * s + 2] = pc >= 0 ? s_cu[pc / P + 1] : 0;
        a.ws_pack[4 * s + 3] = pc >= 0 ? s_ne[pc / P] : 0;
      }
    if (bad_plan) atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
  }
  // rows with nothing visible (ctx == 0) are zero (online_attention.py:37)
  for (int s = blockIdx.x; s < nseq; s += gridDim.x) {
    const int x = npk + s;
    if (s_cu[x + 1] == s_cu[x] && s_ctx[s] >= 0 && pack_col(s) < 0)
      store_row_zero<QT>(a, s_tok[s], D);
  }

  if constexpr (kTrace) tm[1] = wall_clock64();
  // ---- 3. this wave's head, block range and block ids / rows (lane j <-> block b0 + j);
  // waves from Wr * Hkv on have nothing to do
  const SkSplit split(a, bseq, npk > 0 ? s_cu[npk] : 0, rows_total, hkv);
  const int64_t gw = (int64_t)blockIdx.x * NW + wave;
  const int kv = (int)(gw % hkv);
  const int64_t rg = gw / hkv;
  int64_t b0 = 0;
  int n = 0;
  if (rg < split.Wr) {
    int64_t b1;
    range_bounds(split, rg, s_cu, s_ne, nrow, npk, lane, b0, b1);
    n = (int)(b1 - b0);
  }
  const bool too_long = n > kMaxBlocksPerWaveSK;  // contexts beyond the declared maximum
  if (too_long) n = kMaxBlocksPerWaveSK;
  // First block of work row x within its sequence's block table (packs: the first
  // member's table from block 0; sequences: after the window start and the pack).
  auto row_table = [&](int x) __attribute__((always_inline)) -> const int32_t* {
    const int s = row_seq(x, npk);
    if (s < 0) return a.block_tables + (int64_t)s_plead[-1 - s] * a.bt_stride;
    const int pc = pack_col(s);
    return a.block_tables + (int64_t)s * a.bt_stride + row_span(a, s_ctx[s]).first_blk +
           (pc >= 0 ? s_pblk[pc / P] : 0);
  };
  // Block list in windows of 64: lane j of window w holds block b0 + 64 w + j of the
  // per-head order, as its physical id and its row id (kv_head * nrow + work row).
  // Window 0 is read here; the ids of window w + 1 go by direct-to-LDS loads into the
  // wave's id slot when window w starts, before block 64 w + NS is issued: direct-to-LDS
  // loads complete in issue order, so once a block issued after them has landed, they
  // have too (the block ring relies on the same), 64 - 2 NS blocks before they are read.
  auto window_rows = [&](int w, int& row_id) __attribute__((always_inline)) -> const int32_t* {
    const int j = 64 * w + lane;
    if (j >= n) return nullptr;
    const int64_t rem = b0 + j;
    const int x = row_of_block(s_cu, nrow, rem);
    row_id = kv * nrow + x;
    return row_table(x) + (rem - s_cu[x]);
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
  // `ids` has landed (the test above read it); redefine it here so that the compiler's
  // wait tracking stops treating it as a pending load inside the block loop (where it
  // would add waits of its own; the loop's waits are the explicit ones below)
  asm volatile("" : "+v"(ids));
  int nblk = bad_index ? 0 : n;
  int cw = 0;  // window of `ids` / `rows`; `ids_nx` / `rows_nx` hold window cw + 1

  auto stage = [&](int j) __attribute__((always_inline)) -> char* {
    return lds + ((j % NS) * NW + wave) * S::kBytes;
  };
  // row id of block j (in window cw or cw + 1); wave-uniform
  auto row_at = [&](int j) __attribute__((always_inline)) -> int {
    const bool cur = (j >> 6) == cw;
    return __builtin_amdgcn_readfirstlane(cur ? __builtin_amdgcn_readlane(rows, j & 63)
                                              : __builtin_amdgcn_readlane(rows_nx, j & 63));
  };
  auto issue = [&](int j) __attribute__((always_inline)) {
    const bool cur = (j >> 6) == cw;
    const int id = cur ? __builtin_amdgcn_readlane(ids, j & 63)
                       : __builtin_amdgcn_readlane(ids_nx, j & 63);
    stage_block<D>(a, __builtin_amdgcn_readfirstlane(id), row_at(j) / nrow, lane, stage(j));
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
  // This lane's query column in work row x of kv head kvh: a sequence row's column r
  // is head r of the group (r < G); a pack's column r = p G + g is head g of member p.
  // Columns without an output read a valid row and are zeroed by qk_operand.
  struct Column {
    const QT* q;
    bool valid;
  };
  auto column = [&](int x, int kvh) __attribute__((always_inline)) -> Column {
    const int s = row_seq(x, npk);
    if (s >= 0)
      return {query_col_ptr<QT>(a, s_tok[s], kvh * G + (r < G ? r : 0), qg), r < G};
    const int k = -1 - s;
    const int sm = r < P * G ? s_pmem[k * P + r / G] : -1;
    const int tok = s_tok[sm >= 0 ? sm : s_plead[k]];
    return {query_col_ptr<QT>(a, tok, kvh * G + (sm >= 0 ? r % G : 0), qg), sm >= 0};
  };
  // First row's query: a sequence row's G head rows go by direct-to-LDS loads into the
  // last stage, issued before blocks 0 .. NS-2, so the block stream starts without
  // waiting for it; block NS-1 takes that stage once the query has been read out. A
  // pack's columns come from several token rows and load into registers first.
  QueryRaw<D> qr;
  QkOperand<D, KF> qop;
  float cf = 0.f;
  if constexpr (kTrace) tm[2] = wall_clock64();
  int pieces_seen = 0, pack_seen = 0;  // trace info
  if (nblk > 0) {
    const int x0 = row0 % nrow, kvh0 = row0 / nrow;
    const Column c0 = column(x0, kvh0);
    if (row_seq(x0, npk) >= 0) {
      stage_query<QT, D, G>(a, s_tok[row_seq(x0, npk)], kvh0, lane, stage(NS - 1));
      const int first = min(NS - 1, nblk);
      for (int j = 0; j < first; ++j) issue(j);
      if (first == 3) wait_vmcnt<3 * S::kLoads>();  // the query has landed
      else if (first == 2) wait_vmcnt<2 * S::kLoads>();
      else wait_vmcnt<S::kLoads>();
      lds_query<QT, D>(stage(NS - 1), r < G ? r : 0, qg, qr);
      cf = qk_operand<QT, D, KF>(qr, c0.valid, a.qk_scale_log2, qop);
      if (NS - 1 < nblk) issue(NS - 1);  // after the query reads above (their values are consumed)
    } else {
      load_query_at<QT, D>(c0.q, qr);
      const int first = min(NS, nblk);
      for (int j = 0; j < first; ++j) issue(j);
      cf = qk_operand<QT, D, KF>(qr, c0.valid, a.qk_scale_log2, qop);
    }
    if (64 < nblk) request_ids(1);
  }

  // ---- 4. stream the blocks, one piece (the run of one row's blocks) at a time;
  // block i sits in stage i % NS and block i + NS is issued into it once consumed
  float4_t acc[NPV + 1];  // [NPV]: weight sums (INT8)
  float m = 0.f, l = 0.f;
  bool bad_score = false;
  const bool masks = a.cache.key_valid != nullptr;
  int i = 0;
  while (i < nblk) {
    if constexpr (kTrace) ++pieces_seen;
    const int crid = __builtin_amdgcn_readlane(rows, i & 63);  // this piece's row
    const int pstart = i;
    const int px = crid % nrow, pkvh = crid / nrow;
    const int ps = row_seq(px, npk);  // sequence, or -1 - pack
    const Column col = column(px, pkvh);
    // visible keys: a pack's blocks are whole and visible to every member
    RowSpan psp;
    int pblk0;  // block index of the row's first block within the sequence
    if (ps >= 0) {
      psp = row_span(a, s_ctx[ps]);
      const int pc = pack_col(ps);
      pblk0 = psp.first_blk + (pc >= 0 ? s_pblk[pc / P] : 0);
    } else {
      psp.kv_begin = 0;
      psp.ctx = s_pblk[-1 - ps] * kBlockTokens;
      pblk0 = 0;
    }
    const bool merged = ps < 0 || pack_col(ps) >= 0;  // the row's output goes through the merge
    const int64_t pfb = s_cu[px];  // first block of the row in the per-head order
    if (i > 0) {  // a new row starts inside this wave's range
      load_query_at<QT, D>(col.q, qr);
      cf = qk_operand<QT, D, KF>(qr, col.valid, a.qk_scale_log2, qop);
      if (kTrace && pieces_seen == 2) tm[6] = wall_clock64();
    }
#pragma unroll
    for (int k = 0; k <= NPV; ++k) acc[k] = float4_t{0.f, 0.f, 0.f, 0.f};
    // invalid head columns never contribute; a finite start makes a block whose keys
    // are all masked (padding) give exp2(-inf) = 0, not exp2(-inf + inf)
    m = col.valid ? -FLT_MAX : 0.f;
    l = 0.f;
    VRange vr = vrange_start<KF>();
    const int pos0 = (pblk0 + (int)(b0 + i - pfb)) * kBlockTokens;
    for (;;) {
      // the row's blocks in the current window: up to the first lane with another row
      const int wend = min(64 * (cw + 1), nblk);
      const uint64_t beyond =
          __ballot(lane >= (i & 63) && 64 * cw + lane < wend && rows != crid);
      const int iend = beyond ? 64 * cw + (int)__builtin_ctzll(beyond) : wend;
      for (; i < iend; ++i) {
        wait_block(i);
        if constexpr (kTrace) {
          if (i == 0) tm[3] = wall_clock64();
          if (i == pstart && pieces_seen == 2) tm[7] = wall_clock64();
          if (ps < 0) ++pack_seen;
        }
        mfma_block<QT, D, KF>(stage(i), qop, cf, pos0 + (i - pstart) * kBlockTokens,
                              psp.kv_begin, psp.ctx, col.valid, r, qg, acc, m, l, vr, bad_score,
                              masks);
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
        if (nx < nblk) {
          // one block in flight per wave: every earlier block has landed before the next
          // one is issued (the ring then holds landed blocks ahead of the MFMAs). With
          // 2 048 resident waves streaming from HBM this measured best: 2 or 3 blocks in
          // flight per wave took config 2 from 70.7 to 71.6 / 71.9 us and config 5 from
          // 202 to 212 / 216 us (more outstanding 4 KiB gathers, less HBM throughput)
          if (kPacks && ps < 0) wait_vmcnt<(NS - 2) * S::kLoads>();  // pack blocks: cache hits
          else wait_vmcnt<0>();
          issue(nx);
        }
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
    if (kTrace && pieces_seen == 1) tm[5] = wall_clock64();
    // write the piece [pstart, i): the final output when a sequence row is whole in
    // this wave and merges with nothing, else a partial: in the row's own slot when
    // whole, in wave slot 0 (the piece starts the wave's range) or 1 (it ends it)
    const int iend = i;
    end_piece<D, KF>(acc, r);
    float lt = l + shfl_xor(l, 16);
    lt += shfl_xor(lt, 32);
    lt *= norm_scale<KF>();  // the factor the PV weights carry
    const int64_t pfe = s_cu[px + 1] - 1;
    const bool whole = b0 + pstart == pfb && b0 + iend - 1 == pfe;
    if (whole && !merged) {
      if (col.valid) {
        const float inv = 1.f / fmaxf(lt, FLT_MIN);
        store_lane_out<QT, D>(static_cast<QT*>(a.out) + (int64_t)s_tok[ps] * a.o_tok +
                                  (int64_t)(pkvh * G + r) * a.o_head + qg * (D / 4),
                              acc, inv);
      }
    } else if (col.valid) {
      const int64_t slot =
          !whole ? wave_slot(a, gw, pstart == 0 ? 0 : 1, r)
          : ps < 0 ? pack_slot(a, G, pkvh, -1 - ps, r)
                   : packed_seq_slot(a, G, hkv, pkvh, pack_col(ps), r);
      store_lane_f32<D>(a.ws_o + slot * D + qg * (D / 4), acc);
      if (qg == 0) {
        a.ws_ml[slot * 2] = m;
        a.ws_ml[slot * 2 + 1] = lt;
      }
    }
  }
  if (bad_index && lane == 0) atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
  if (bad_score && lane == 0) atomicOr(a.err_flag, ASTR_FLAG_NONFINITE_SCORE);
#if ASTR_TRACE
  tm[4] = wall_clock64();
  if (lane == 0 && gw < kTraceWaves) {
    for (int k = 0; k < 8; ++k) g_trace[gw][k] = tm[k];
    g_trace_info[gw][0] = nblk;
    g_trace_info[gw][1] = pieces_seen;
    g_trace_info[gw][2] = pack_seen;
    g_trace_info[gw][3] = (int)__builtin_amdgcn_s_getreg((20 << 0) | (0 << 6) | (3 << 11));  // XCC_ID
  }
#endif
}

// The pieces of one work row of kv head kvh over the per-head order [fb, fe]: their
// count, and where piece p (0 <= p < count) keeps its partial for query column col.
// A row within one range is one piece in the row's own slot (`own`, or -1 when the
// wave wrote it as output); a longer row has one piece per range r0..r1, the first in
// slot 1 of its wave when the row starts inside r0's range (it is that range's last
// piece), every other in slot 0.
struct RowPieces {
  int64_t r0, own;
  int count;
  bool first_is_tail;
};
// ne: the rows with blocks before this one. Block fb - 1 ends the previous row with
// blocks, which starts kRowCost + its own cost earlier than fb.
__device__ __forceinline__ RowPieces row_pieces(int64_t fb, int64_t fe, int ne, const SkSplit& sp,
                                                int64_t own) {
  RowPieces rp{0, own, 0, false};
  if (fe < fb) return rp;  // no blocks
  const int64_t cf = sp.cost(fb, ne);
  rp.r0 = sp.range_at(cf);
  const int64_t r1 = sp.range_of(fe, ne);
  rp.count = (int)(r1 - rp.r0 + 1);
  rp.first_is_tail =
      fb > 0 && sp.range_at(cf - kRowCost - (fb - 1 < sp.PB ? sp.KP : kSeqCost)) == rp.r0;
  return rp;
}
__device__ __forceinline__ int64_t piece_slot(const AttnArgs& a, const RowPieces& rp, int p,
                                              int hkv, int kvh, int col) {
  const int64_t w = (rp.r0 + p) * hkv + kvh;  // the wave that streamed range r0 + p
  const int64_t split = wave_slot(a, w, p == 0 && rp.first_is_tail ? 1 : 0, col);
  return rp.count == 1 ? rp.own : split;
}

// Heads of a GQA group that one merge wave takes: at most 4, so that a wave holds the
// partials of up to kFastPieces pieces at once (groups of 8 and 16 split over 2 and 4
// waves).
template <int G>
constexpr int merge_heads() { return G < 4 ? G : 4; }

// One wave per (sequence, kv head, GS heads of the group): merge the pieces of
// sequences that no single wave wrote: rows split across waves, and packed sequences
// (their pack's pieces, columns p G .. p G + G-1 for member p, then their own). The
// heads' rows of one piece sit in consecutive slot columns (G x D contiguous floats);
// the wave takes heads h0 .. h0 + GS-1, lane L elements [L E, L E + E) of them
// (E = GS D / 64), of head h0 + hl, hl = L E / D. Statistics go lane-parallel: in a
// round of R = min(64 / GS, kFast) pieces, lane u GS + h holds (m, l) of piece u, head
// h0 + h, and the maxima and weight sums reduce over the lanes of one head. The
// merge_softmax rule (online_attention.py:42-63) and SoftmaxState.output (:35-39).
template <typename QT, int D, int G, int GS>
__global__ __launch_bounds__(kWave) void merge_streamk_kernel(AttnArgs a) {
  constexpr int E = GS * D / kWave;  // floats per lane
  static_assert(G % GS == 0 && E >= 1 && GS * D % kWave == 0, "lanes cover the heads' rows");
  constexpr int HS = G / GS;  // waves per (sequence, kv head)
  constexpr int V = E >= 4 ? 4 : E;  // floats per load
  constexpr int kRegs = 128 / E > 0 ? 128 / E : 1;  // partial rows held at once
  constexpr int R0 = kWave / GS < kFastPieces ? kWave / GS : kFastPieces;
  constexpr int R = R0 < kRegs ? R0 : kRegs;  // pieces per round
  typedef float vec_t __attribute__((ext_vector_type(V)));
  const int lane = threadIdx.x;
  const int hkv = a.cache.num_kv_heads;
  const int seq = blockIdx.x / (hkv * HS), kvh = blockIdx.x / HS % hkv;
  const int h0 = blockIdx.x % HS * GS;  // first head of the group this wave takes
  const int hl = lane * E / D;
  const int xs = a.num_packs + seq;
  const int cu0 = a.ws_seq[xs], cu1 = a.ws_seq[xs + 1];
  const int bseq = a.ws_seq[a.num_packs + a.num_seqs];
  const int pb = a.ws_seq[a.num_packs];  // blocks of the packs
  // a packed sequence: its pack column, the pack's block range and the rows with
  // blocks before the pack, in one record
  int pc = -1, pk0 = 0, pk1 = 0, pne = 0;
  if (a.num_packs > 0) {
    pc = a.ws_pack[4 * seq];
    pk0 = a.ws_pack[4 * seq + 1];
    pk1 = a.ws_pack[4 * seq + 2];
    pne = a.ws_pack[4 * seq + 3];
  }
  const SkSplit split(a, bseq, pb, a.ws_ne[a.num_packs + a.num_seqs], hkv);
  RowPieces own = row_pieces(cu0, cu1 - 1, a.ws_ne[xs], split, -1);
  RowPieces pack{0, -1, 0, false};
  int pcol0 = 0;  // the pack column of this sequence's head 0
  if (pc >= 0) {
    const int k = pc / a.pack_rows;
    pcol0 = (pc % a.pack_rows) * G;
    pack = row_pieces(pk0, pk1 - 1, pne, split, pack_slot(a, G, kvh, k, pcol0));
    own.own = packed_seq_slot(a, G, hkv, kvh, pc, 0);
  } else if (own.count <= 1) {
    return;  // empty (zeroed) or written whole by one wave
  }
  const int pieces = pack.count + own.count;
  // slot (column of head 0) of piece p, the pack's pieces first
  auto slot_of = [&](int p) __attribute__((always_inline)) -> int64_t {
    const bool in_pack = p < pack.count;
    const RowPieces& rp = in_pack ? pack : own;
    return piece_slot(a, rp, in_pack ? p : p - pack.count, hkv, kvh, in_pack ? pcol0 : 0);
  };
  const int su = lane / GS, sh = lane % GS;  // the (piece in round, head) of this lane's statistics
  auto head_max = [&](float x) __attribute__((always_inline)) -> float {
#pragma unroll
    for (int off = GS; off < kWave; off <<= 1) x = fmaxf(x, shfl_xor(x, off));
    return x;
  };
  auto head_sum = [&](float x) __attribute__((always_inline)) -> float {
#pragma unroll
    for (int off = GS; off < kWave; off <<= 1) x += shfl_xor(x, off);
    return x;
  };
  // one round: pieces [p0, p0 + R); returns this lane's slot and loads its statistics
  auto stats = [&](int p0, int64_t& sl, float& mp, float& lp) __attribute__((always_inline)) {
    const int p = p0 + su;
    const bool live = su < R && p < pieces;
    sl = slot_of(live ? p : p0);
    mp = live ? a.ws_ml[(sl + h0 + sh) * 2] : -INFINITY;
    lp = live ? a.ws_ml[(sl + h0 + sh) * 2 + 1] : 0.f;
  };
  float M = -INFINITY;  // of head sh (lane-parallel layout)
  if (pieces > R) {     // several rounds: the maxima first
    for (int p0 = 0; p0 < pieces; p0 += R) {
      int64_t sl;
      float mp, lp;
      stats(p0, sl, mp, lp);
      M = fmaxf(M, head_max(mp));
    }
  }
  float L = 0.f, O[E];
#pragma unroll
  for (int e = 0; e < E; ++e) O[e] = 0.f;
  for (int p0 = 0; p0 < pieces; p0 += R) {
    int64_t sl;
    float mp, lp;
    stats(p0, sl, mp, lp);
    float v[R][E];
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const int64_t s_u = ((int64_t)__builtin_amdgcn_readlane((int)(sl >> 32), u * GS) << 32) |
                          (uint32_t)__builtin_amdgcn_readlane((int)sl, u * GS);
      const float* src = a.ws_o + (s_u + h0) * D + lane * E;
      const bool live = p0 + u < pieces;
#pragma unroll
      for (int e = 0; e < E; e += V) {
        const vec_t x = live ? *reinterpret_cast<const vec_t*>(src + e) : vec_t{};
#pragma unroll
        for (int c = 0; c < V; ++c) v[u][e + c] = x[c];
      }
    }
    const float mx = pieces > R ? M : head_max(mp);
    const float w = mp == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mp - mx);
    L += head_sum(lp * w);
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const float wu = __shfl(w, u * GS + hl, kWave);
#pragma unroll
      for (int e = 0; e < E; ++e) O[e] = fmaf(v[u][e], wu, O[e]);
    }
  }
  const float inv_l = 1.f / fmaxf(__shfl(L, hl, kWave), FLT_MIN);
  QT* out = static_cast<QT*>(a.out) + (int64_t)decode_token(a, seq) * a.o_tok +
            (int64_t)(kvh * G + h0 + hl) * a.o_head + lane * E % D;
  QT r[E];
#pragma unroll
  for (int e = 0; e < E; ++e) r[e] = from_float<QT>(O[e] * inv_l);
  if constexpr (E % 8 == 0) {
#pragma unroll
    for (int e = 0; e < E; e += 8)
      *reinterpret_cast<uint4*>(out + e) = *reinterpret_cast<const uint4*>(r + e);
  } else if constexpr (E == 4) {
    *reinterpret_cast<uint2*>(out) = *reinterpret_cast<const uint2*>(r);
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) out[e] = r[e];
  }
}

// Workgroups of `kernel` one CU holds at once.
template <typename Kernel>
int query_resident_per_cu(Kernel kernel, int threads) {
  int n = 0;
  return (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0) == hipSuccess &&
          n > 0)
             ? n
             : 1;
}

int device_cus() {
  int dev = 0, v = 0;
  if (hipGetDevice(&dev) == hipSuccess &&
      hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
    return v;
  return 256;
}

template <typename QT, int D, int G, bool kPacks>
int launch(AttnArgs a, hipStream_t stream) {
  auto kernel = decode_streamk_kernel<QT, D, G, kPacks>;
  constexpr int NW = sk_waves<D>();
  // queried once per instantiation (each has its own registers and LDS tables)
  static const int per_cu = query_resident_per_cu(kernel, NW * kWave);
  // launch one wave per resident slot (whole workgroups) and at least min_waves (the
  // host-side bound), at most the workspace capacity passed in total_waves; the
  // kernels settle the waves they use from the actual block count
  const int64_t resident = (int64_t)device_cus() * per_cu * NW;
  int64_t waves = resident;
  if (waves < a.min_waves) waves = (a.min_waves + NW - 1) / NW * NW;
  if (waves > a.total_waves) waves = a.total_waves / NW * NW;
  a.total_waves = (int32_t)waves;
  a.pref_waves = (int32_t)(resident < waves ? resident : waves);
  const int wgs = (int)(waves / NW);
  hipLaunchKernelGGL(kernel, dim3(wgs), dim3(NW * kWave), 0, stream, a);
  constexpr int GS = merge_heads<G>();
  hipLaunchKernelGGL((merge_streamk_kernel<QT, D, G, GS>),
                     dim3(a.num_seqs * a.cache.num_kv_heads * (G / GS)), dim3(kWave), 0, stream, a);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "paged_attention (stream-K) launch");
}

template <typename QT, int D, bool kP>
int dispatch_group(const AttnArgs& a, int G, hipStream_t s) {
  switch (G) {
    case 1: return launch<QT, D, 1, kP>(a, s);
    case 2: return launch<QT, D, 2, kP>(a, s);
    case 4: return launch<QT, D, 4, kP>(a, s);
    case 8: return launch<QT, D, 8, kP>(a, s);
    case 16:
      if constexpr (D <= 128 && !kP) return launch<QT, D, 16, false>(a, s);  // 16 columns: no packs
      [[fallthrough]];
    default:
      return fail(ASTR_EUNSUPPORTED, "GQA group size %d not supported", G);
  }
}

// kDims: the head dims this unit launches (bits: 1 = 64, 2 = 128, 4 = 256)
template <typename QT, bool kP, int kDims>
int dispatch_dim(const AttnArgs& a, int G, hipStream_t s) {
  const int d = a.cache.head_dim;
  if constexpr ((kDims & 1) != 0) if (d == 64) return dispatch_group<QT, 64, kP>(a, G, s);
  if constexpr ((kDims & 2) != 0) if (d == 128) return dispatch_group<QT, 128, kP>(a, G, s);
  if constexpr ((kDims & 4) != 0) if (d == 256) return dispatch_group<QT, 256, kP>(a, G, s);
  return fail(ASTR_EUNSUPPORTED, "head_dim %d not in {64,128,256}", d);
}

template <bool kP, int kDims>
int dispatch_dtype(const AttnArgs& a, int G, int32_t q_dtype, hipStream_t s) {
  if (q_dtype == ASTR_F16) return dispatch_dim<_Float16, kP, kDims>(a, G, s);
  if (q_dtype == ASTR_BF16) return dispatch_dim<bf16_t, kP, kDims>(a, G, s);
  return fail(ASTR_EUNSUPPORTED, "stream-K decode takes bf16/fp16 queries");
}

}  // namespace

#if ASTR_SK_PART != 1
// head dim 256 stays with the entry point's unit: under the max-ilp scheduler its
// kernels spill to scratch
template <>
int launch_streamk_plain_kf<KF>(const AttnArgs& a, int32_t q_dtype, hipStream_t stream) {
  constexpr int kDims = ASTR_SK_PART == 2 ? 1 | 2 : 1 | 2 | 4;
  return dispatch_dtype<false, kDims>(a, a.num_q_heads / a.cache.num_kv_heads, q_dtype, stream);
}
#endif

#if ASTR_SK_PART != 2
template <>
int launch_streamk_kf<KF>(const AttnArgs& a, int32_t q_dtype, hipStream_t stream) {
  if (a.min_waves > a.total_waves)
    return fail(ASTR_EINVAL, "stream-K workspace too small for this launch");
  const int G = a.num_q_heads / a.cache.num_kv_heads;
  // a group of 16 fills the 16 query columns alone: no packs
  if (a.num_packs == 0 || G == 16) {
    if constexpr (ASTR_SK_PART == 1)
      if (a.cache.head_dim == 256) return dispatch_dtype<false, 4>(a, G, q_dtype, stream);
    return launch_streamk_plain_kf<KF>(a, q_dtype, stream);
  }
  return dispatch_dtype<true, 1 | 2 | 4>(a, G, q_dtype, stream);
}

#if ASTR_KF == 0
int stream_k_max_seqs() { return kMaxSeqsSK; }
#if ASTR_TRACE
// Trace builds: copies the marks and info of the first `waves` waves of the last
// stream-K launch of the int8 format (8 int64 + 4 int32 per wave) to host memory.
extern "C" int astr_trace_read(void* marks, void* info, int waves) {
  if (waves < 0 || waves > kTraceWaves) return ASTR_EINVAL;
  hipError_t e = hipMemcpyFromSymbol(marks, HIP_SYMBOL(g_trace), (size_t)waves * 64);
  if (e == hipSuccess) e = hipMemcpyFromSymbol(info, HIP_SYMBOL(g_trace_info), (size_t)waves * 16);
  return e == hipSuccess ? 0 : (int)e;
}
#endif
int stream_k_max_packs() { return kMaxPacksSK; }
int stream_k_max_pack_seqs() { return kMaxPackSeqsSK; }
int stream_k_work_rows(int) { return kMaxRowsSK; }
#endif
#endif  // ASTR_SK_PART != 2

}  // namespace attn
}  // namespace astr
