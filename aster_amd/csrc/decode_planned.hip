// Planned paged decode attention (gfx950, bf16/fp16 queries): the decode rows of a
// batch on a schedule built on the host (decode_plan.cpp).
//
// One workgroup of kPlanWaves waves per resident slot of the GPU. The plan gives each
// workgroup its items ((sequence, kv head) rows, or chunks of long rows) and each wave a
// contiguous range of the workgroup's flat block list, with the physical block ids in
// it, so a wave starts streaming after one round trip for its block ids. Blocks go
// through a per-wave LDS ring filled by direct global->LDS loads and the MFMA step of
// attention_common.h, piece by piece (a piece is the run of one item's blocks in the
// wave's range), as in the stream-K kernel. A piece that is a whole row is normalised
// and written; the other pieces write (m, l, acc) partials. When every wave of the
// workgroup is done, the workgroup merges the pieces of each of its rows that several
// of its waves hold (the merge_softmax rule, online_attention.py:42-63, and
// SoftmaxState.output, :35-39) and writes the row; rows the plan cut across
// workgroups leave one partial per chunk for merge_chunks_kernel.
#include <type_traits>

#include "attention_common.h"

namespace astr {
namespace attn {
namespace {

#ifndef ASTR_KF
#define ASTR_KF 0
#endif
constexpr int KF = ASTR_KF;  // this translation unit's code format

constexpr int kPlanWaves = 8;           // waves per workgroup
constexpr int kMaxItems = 64;           // items per workgroup (the planner's limit)
constexpr int kItemWords = 8;           // seq, kv head, first block, blocks, ctx, out, position, ids offset
constexpr int kChunkedWords = 4;        // seq, kv head, first chunk slot, chunks
constexpr int kIdsBytes = 256;          // per wave: the next window's block ids
constexpr int kWaveWords = 6;           // first piece's sequence and kv head, prefetch count, ids
constexpr int kPrefetchBlocks = 3;

template <int D>
constexpr int pl_stages() { return D == 256 ? 2 : 4; }
// Where the partials the workgroup merges wait for the merge. The last piece of a wave
// stays in its accumulators and goes to the freed ring after the streaming (head dims up
// to 128). The first piece, when more follow it, stays in registers at head dim 128
// (4 (D / 16 + 1) + 2 more, within the budget of two waves per SIMD); at 64 they would
// cost a wave per SIMD, and it goes to the workspace, as both pieces do at 256 (where
// the ring holds only two stages and the accumulators twice the registers).
template <int D>
constexpr bool first_in_registers() { return D == 128; }
template <int D>
constexpr bool last_in_ring() { return D <= 128; }

// Per-wave timeline (trace builds only, -DASTR_TRACE=1, built apart from the product
// library by `python -m aster_amd.build --trace`): wall-clock marks (100 MHz
// s_memrealtime) of each wave of the last planned launch, read back with
// astr_trace_read_planned. Marks: 0 entry, 1 items in LDS, 2 block ids in hand, 3 first
// block landed, 4 streaming done, 5 every wave of the workgroup done, 6 exit (merges
// written). Info: blocks, pieces, items of the workgroup, XCC id.
#ifndef ASTR_TRACE
#define ASTR_TRACE 0
#endif
constexpr bool kTrace = ASTR_TRACE != 0;
#if ASTR_TRACE
constexpr int kTraceWaves = 16384;
static __device__ long long g_ptrace[kTraceWaves][8];
static __device__ int g_ptrace_info[kTraceWaves][4];
#endif

struct Item {
  int seq, kvh, blk0, nblk, ctx, out, pos, ids_off;
};

__device__ __forceinline__ Item item_at(const int* s_item, int k) {
  const int* v = s_item + k * kItemWords;
  return Item{v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]};
}

// Partial slots in the workspace (plan_chunk_slot): two per wave (at D = 256 its first
// piece's), then the chunk slots.
__device__ __forceinline__ int64_t wave_slot(int64_t gw, int which, int G) {
  return (gw * 2 + which) * G;
}
__device__ __forceinline__ int64_t chunk_slot(const PlanArgs& p, int c, int G) {
  return plan_chunk_slot(p, c, G);
}

// Where a partial of G heads lies: acc rows (head h at o + h * D) and (m, l) pairs
// (head h at ml + 2 h), in LDS or in the workspace (generic pointers).
struct Partial {
  const float* o;
  const float* ml;
};

// Merges the partials src_of(k) (k < count; o == nullptr for no piece) of the G heads of
// one row with the merge_softmax rule in base 2, and writes the normalised row to
// `orow` (head h at orow + h * o_head), or, when orow is null, the merged partial to
// workspace slot `dest`. One wave; lane L takes elements [L E, L E + E) of the G x D
// floats, of head L E / D. Pieces go in groups of MAXK whose loads are all issued
// together; between groups the running (M, L, O) is rescaled to the new maximum.
// Pieces with maximum -inf weigh 0 (a row with no visible key has l = 0 and acc = 0 in
// every piece, and comes out 0).
// Pieces merge_pieces loads at once: up to a wave's share of 64 floats per lane.
template <int D, int G>
constexpr int merge_group() {
  return 64 / (G * D / kWave) < 1 ? 1 : 64 / (G * D / kWave) > 8 ? 8 : 64 / (G * D / kWave);
}

template <typename QT, int D, int G, int MAXK, typename SrcOf>
__device__ __forceinline__ void merge_pieces(const AttnArgs& a, SrcOf src_of, int count,
                                             QT* orow, int64_t dest, int lane) {
  constexpr int E = G * D / kWave;
  static_assert(E >= 1 && G * D % kWave == 0, "lanes cover the row");
  constexpr int V = E >= 4 ? 4 : E;
  typedef float vec_t __attribute__((ext_vector_type(V)));
  const int h = lane * E / D, d0 = lane * E % D;
  float M = -INFINITY, L = 0.f, O[E];
#pragma unroll
  for (int e = 0; e < E; ++e) O[e] = 0.f;
  for (int k0 = 0; k0 < count; k0 += MAXK) {
    const float* po[MAXK];
    float mp[MAXK], lp[MAXK];
#pragma unroll
    for (int j = 0; j < MAXK; ++j) {
      const Partial pk = k0 + j < count ? src_of(k0 + j) : Partial{nullptr, nullptr};
      po[j] = pk.o == nullptr ? nullptr : pk.o + h * D + d0;
      mp[j] = pk.o == nullptr ? -INFINITY : pk.ml[2 * h];
      lp[j] = pk.o == nullptr ? 0.f : pk.ml[2 * h + 1];
    }
    float Mn = M;
#pragma unroll
    for (int j = 0; j < MAXK; ++j) Mn = fmaxf(Mn, mp[j]);
    if (Mn != M) {  // the running merge moves to the new maximum
      const float f = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - Mn);
      L *= f;
#pragma unroll
      for (int e = 0; e < E; ++e) O[e] *= f;
      M = Mn;
    }
    float w[MAXK];
#pragma unroll
    for (int j = 0; j < MAXK; ++j) {
      w[j] = mp[j] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mp[j] - M);
      L += lp[j] * w[j];
    }
#pragma unroll
    for (int e = 0; e < E; e += V) {
      vec_t x[MAXK];
#pragma unroll
      for (int j = 0; j < MAXK; ++j)
        x[j] = po[j] == nullptr ? vec_t{} : *reinterpret_cast<const vec_t*>(po[j] + e);
#pragma unroll
      for (int j = 0; j < MAXK; ++j)
#pragma unroll
        for (int c = 0; c < V; ++c) O[e + c] = fmaf(x[j][c], w[j], O[e + c]);
    }
  }
  if (orow == nullptr) {
    float* dst = a.ws_o + (dest + h) * D + d0;
#pragma unroll
    for (int e = 0; e < E; e += V) {
      vec_t x;
#pragma unroll
      for (int c = 0; c < V; ++c) x[c] = O[e + c];
      *reinterpret_cast<vec_t*>(dst + e) = x;
    }
    if (d0 == 0) {
      a.ws_ml[(dest + h) * 2] = M;
      a.ws_ml[(dest + h) * 2 + 1] = L;
    }
    return;
  }
  const float inv = 1.f / fmaxf(L, FLT_MIN);
  QT r[E];
#pragma unroll
  for (int e = 0; e < E; ++e) r[e] = from_float<QT>(O[e] * inv);
  QT* o = orow + (int64_t)h * a.o_head + d0;
  constexpr int kVec = 16 / (int)sizeof(QT);  // elements per 16-byte store
  if constexpr (E % kVec == 0) {
#pragma unroll
    for (int e = 0; e < E; e += kVec)
      *reinterpret_cast<uint4*>(o + e) = *reinterpret_cast<const uint4*>(r + e);
  } else if constexpr (E * sizeof(QT) == 8) {
    *reinterpret_cast<uint2*>(o) = *reinterpret_cast<const uint2*>(r);
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) o[e] = r[e];
  }
}

// The step's append inside the decode (AttnArgs::new_k): the newest token of a row sits
// at position ctx - 1, in the row's last visible block, which one wave of the plan
// streams. That wave stages the token's key and value rows and the slot the caller
// reserved for it right before the block (so they have landed once the block has),
// quantizes them as quantize_kv does (kv_quantization.py:71-94, the same arithmetic as
// quantize_append_kernel), writes the codes and scales into the block's LDS stage before
// the attention reads it, and into the arena. Bytes per stage and wave: both rows, then
// the slot.
template <typename QT, int D>
constexpr int new_token_bytes() { return 2 * D * (int)sizeof(QT) + 16; }

template <typename QT, int D>
__device__ __forceinline__ void stage_new_token(const AttnArgs& a, int seq, int kvh, int lane,
                                                char* dst) {
  constexpr int kRow = D * (int)sizeof(QT);
  static_assert(kRow % 128 == 0, "rows of whole 4-byte lanes");
  const char* k = static_cast<const char*>(a.new_k) +
                  ((int64_t)seq * a.nk_tok + (int64_t)kvh * a.nk_head) * (int64_t)sizeof(QT);
  const char* v = static_cast<const char*>(a.new_v) +
                  ((int64_t)seq * a.nv_tok + (int64_t)kvh * a.nv_head) * (int64_t)sizeof(QT);
  const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr(dst));
#pragma unroll
  for (int j = 0; j * 256 < kRow; ++j)
    if (j * 256 + lane * 4 < kRow) lds_dma_x1(k + j * 256 + lane * 4, base + j * 256);
#pragma unroll
  for (int j = 0; j * 256 < kRow; ++j)
    if (j * 256 + lane * 4 < kRow) lds_dma_x1(v + j * 256 + lane * 4, base + kRow + j * 256);
  if (lane < 2)
    lds_dma_x1(reinterpret_cast<const char*>(a.new_slots + seq) + lane * 4, base + 2 * kRow);
}

// Quantizes the staged token of row (seq, kvh) whose position ctx - 1 lies in block
// `phys` (staged at `st`; its rows and slot at `nb`) and writes it into the stage and
// into the arena. The caller's slot must be the plan's position of the token (else the
// index flag is raised and only the arena copy is written, at the caller's slot); a
// token holding a non-finite value raises the input flag and is written nowhere.
template <typename QT, int D, int KF>
__device__ __forceinline__ void append_token(const AttnArgs& a, int kvh, int ctx, int phys,
                                             char* st, const char* nb, int lane) {
  using S = Stage<D>;
  constexpr int E = D / kWave;  // elements per lane
  constexpr int kRow = D * (int)sizeof(QT);
  struct alignas(E * sizeof(QT)) Elems {
    QT e[E];
  };
  const Elems wk = *reinterpret_cast<const Elems*>(nb + lane * E * (int)sizeof(QT));
  const Elems wv = *reinterpret_cast<const Elems*>(nb + kRow + lane * E * (int)sizeof(QT));
  const int64_t slot = *reinterpret_cast<const int64_t*>(nb + 2 * kRow);
  bool bad = false;
  float ak = 0.f, av = 0.f;
  float xk[E], xv[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    xk[e] = to_float<QT>(wk.e[e]);
    xv[e] = to_float<QT>(wv.e[e]);
    bad |= !__builtin_isfinite(xk[e]) || !__builtin_isfinite(xv[e]);
    ak = fmaxf(ak, fabsf(xk[e]));
    av = fmaxf(av, fabsf(xv[e]));
  }
  if (__ballot(bad) != 0) {
    if (lane == 0) atomicOr(a.err_flag, ASTR_FLAG_NONFINITE_INPUT);
    return;
  }
  const float sk = quant_scale<KF>(wave_max(ak)), sv = quant_scale<KF>(wave_max(av));
  typedef typename std::conditional<E == 1, uint8_t,
                                    typename std::conditional<E == 2, uint16_t, uint32_t>::type>::type
      Codes;
  Codes ck = 0, cv = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    ck |= (Codes)((uint32_t)(uint8_t)quant_code<KF>(xk[e], sk) << (8 * e));
    cv |= (Codes)((uint32_t)(uint8_t)quant_code<KF>(xv[e], sv) << (8 * e));
  }
  const int t = (ctx - 1) % kBlockTokens;
  const int d = lane * E;
  if (slot == (int64_t)phys * kBlockTokens + t) {
    *reinterpret_cast<Codes*>(st + S::kK + k_chunk<D>(t, d / 16) + d % 16) = ck;
    *reinterpret_cast<Codes*>(st + S::kV + t * D + d) = cv;
    if (lane == 0) {
      *reinterpret_cast<float*>(st + S::kS + 4 * t) = sk;
      *reinterpret_cast<float*>(st + S::kS + 64 + 4 * t) = sv;
    }
  } else if (lane == 0) {
    atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
  }
  if (slot >= 0 && slot < (int64_t)a.cache.num_blocks * kBlockTokens) {
    const int64_t blk = slot / kBlockTokens, off = slot % kBlockTokens;
    const int64_t co = blk * a.cache.code_block_stride + (int64_t)kvh * a.cache.code_head_stride +
                       off * D + d;
    *reinterpret_cast<Codes*>(a.cache.k_codes + co) = ck;
    *reinterpret_cast<Codes*>(a.cache.v_codes + co) = cv;
    if (lane == 0) {
      const int64_t so = blk * a.cache.scale_block_stride +
                         (int64_t)kvh * a.cache.scale_head_stride + off;
      a.cache.k_scales[so] = sk;
      a.cache.v_scales[so] = sv;
    }
  } else if (lane == 0) {
    atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
  }
}

template <typename QT, int D, int G, bool kAppend>
__global__ __launch_bounds__(kPlanWaves * kWave) void decode_planned_kernel(PlanArgs p) {
  static_assert(D == 64 || D == 128 || D == 256, "head_dim");
  static_assert(G >= 1 && G <= 16, "GQA group");
  constexpr int NW = kPlanWaves;
  constexpr int NS = pl_stages<D>();
  using S = Stage<D>;
  constexpr int NPV = D / 16;
  constexpr bool kFirstInRegs = first_in_registers<D>();
  constexpr bool kLastInRing = last_in_ring<D>();
  // the G query rows of a piece travel by direct-to-LDS load into a ring stage
  constexpr bool kStagedQuery = G * D * (int)sizeof(QT) <= S::kBytes;
  const AttnArgs& a = p.a;

  // the block ring; once every wave is done streaming, the workgroup's partials
  // ([wave][first | last piece][column] acc rows, then (m, l) pairs)
  __shared__ __attribute__((aligned(16))) char lds[NS * NW * S::kBytes];
  static_assert(!kLastInRing || NW * 2 * G * (D + 2) * sizeof(float) <= sizeof(lds),
                "partials fit the ring");
  __shared__ __attribute__((aligned(16))) char id_slots[NW * kIdsBytes];   // [wave]
  __shared__ __attribute__((aligned(16))) int s_item[kMaxItems * kItemWords];
  __shared__ __attribute__((aligned(16))) int s_rec[NW + 3];  // first item, end item, wave bounds
  __shared__ int s_bad;
  __shared__ bool s_first_ring[NW];  // the wave's slot 0 partial is in the ring
  // the step's append: per stage and wave, the newest token staged with its block
  static_assert(!kAppend || sizeof(QT) == 2, "appends of 2-byte rows");
  constexpr int kNewBytes = new_token_bytes<QT, D>();
  __shared__ __attribute__((aligned(16))) char s_new[kAppend ? NS * NW * kNewBytes : 16];

  long long tm[8] = {0, 0, 0, 0, 0, 0, 0, 0};  // trace marks (kTrace)
  if constexpr (kTrace) tm[0] = wall_clock64();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int r = lane & 15, qg = lane >> 4;
  const int g = blockIdx.x;
  const int hkv = a.cache.num_kv_heads;
  const int32_t* const ids_tab = p.plan + p.info.off_ids;
  const bool valid = r < G;

  // ---- 0. in one round trip: this wave's entry (its first piece and the ids of its
  // first blocks) with its bounds, and (wave 0) the workgroup's record and items (at a
  // fixed stride) by direct-to-LDS loads; the query and the entry's blocks go out as
  // soon as the entry is in, after the record and items (loads complete in issue
  // order). The entry is checked against the items below.
  int went = 0;
  if (lane < kWaveWords)
    went = p.plan[p.info.off_waves + ((int64_t)g * NW + wave) * kWaveWords + lane];
  else if (lane < kWaveWords + 2)
    went = p.plan[p.info.off_workgroups + (int64_t)g * (NW + 3) + 2 + wave + lane - kWaveWords];
  const int stride = p.info.item_stride;  // checked on the host: 1..kMaxItems
  if (wave == 0) {
    if (lane < NW + 3)
      lds_dma_x1(p.plan + p.info.off_workgroups + (int64_t)g * (NW + 3) + lane,
                 __builtin_amdgcn_readfirstlane(lds_addr(reinterpret_cast<const char*>(s_rec))));
    const int32_t* src = p.plan + p.info.off_items + (int64_t)g * stride * kItemWords;
    const uint32_t dst = __builtin_amdgcn_readfirstlane(lds_addr(reinterpret_cast<const char*>(s_item)));
    for (int k = 0; k * kWave < stride * kItemWords; ++k)
      if (k * kWave + lane < stride * kItemWords) lds_dma_x1(src + k * kWave + lane, dst + k * kWave * 4);
  }
  if (threadIdx.x == 0) s_bad = 0;
  asm volatile("" : "+v"(went));  // the entry has landed
  const int pseq = __builtin_amdgcn_readlane(went, 0), pkvh = __builtin_amdgcn_readlane(went, 1);
  int pre = __builtin_amdgcn_readlane(went, 2);  // blocks issued here
  const int pn = __builtin_amdgcn_readlane(went, kWaveWords + 1) - __builtin_amdgcn_readlane(went, kWaveWords);
  int pid[kPrefetchBlocks];
#pragma unroll
  for (int j = 0; j < kPrefetchBlocks; ++j) pid[j] = __builtin_amdgcn_readlane(went, 3 + j);
  bool pre_ok = pn > 0 && pre >= 1 && pre <= kPrefetchBlocks && pre <= pn && pseq >= 0 &&
                pseq < a.num_seqs && pkvh >= 0 && pkvh < hkv;
#pragma unroll
  for (int j = 0; j < kPrefetchBlocks; ++j)
    pre_ok = pre_ok && (j >= pre || (unsigned)pid[j] < (unsigned)a.cache.num_blocks);
  const bool bad_entry = pre != 0 && !pre_ok;  // raised with the wave's index flag below
  // the wave starts after its items without a (valid) entry; it issues at most NS - 1
  // blocks here (the last stage takes the query). Queries whose G rows do not fit a stage
  // (fp32 at G D > 1024 for D = 128) load into registers and start after the items: their
  // register loads would wait behind the blocks (measured slower).
  pre = pre_ok && kStagedQuery ? min(pre, NS - 1) : 0;
  QueryColumn<QT, D> qr;
  if (pre > 0) {
    if constexpr (kStagedQuery)
      stage_query<QT, D, G>(a, pseq, pkvh, lane, lds + ((NS - 1) * NW + wave) * S::kBytes);
#pragma unroll
    for (int j = 0; j < kPrefetchBlocks; ++j)
      if (j < pre) stage_block<D>(a, pid[j], pkvh, lane, lds + (j * NW + wave) * S::kBytes);
  }
  if (wave == 0) {  // the record and items have landed (the loads issued after them may not)
    constexpr int QL = kStagedQuery ? stage_query_loads<QT, D, G>() : 0;
    if (pre == 3) wait_vmcnt<QL + 3 * S::kLoads>();
    else if (pre == 2) wait_vmcnt<QL + 2 * S::kLoads>();
    else if (pre == 1) wait_vmcnt<QL + S::kLoads>();
    else wait_vmcnt<0>();
  }
  __syncthreads();

  // ---- 1. the record and items, every index checked
  const int ib = s_rec[0], ie = s_rec[1];
  const int total = s_rec[2 + NW];  // blocks of the workgroup's list
  const int ni = ie - ib;
  bool bad = !(ib == g * stride && ib <= ie && ie - ib <= stride && s_rec[2] == 0 &&
               total <= p.info.num_blocks);
  if (threadIdx.x < NW)  // wave bounds: non-decreasing
    bad |= s_rec[3 + threadIdx.x] < s_rec[2 + threadIdx.x];
  const Item mine = !bad && (int)threadIdx.x < ni ? item_at(s_item, threadIdx.x) : Item{};
  if (!bad && (int)threadIdx.x < ni)
    bad = !(mine.seq >= 0 && mine.seq < a.num_seqs && mine.kvh >= 0 && mine.kvh < hkv &&
            mine.nblk >= 0 && mine.blk0 >= 0 && mine.pos >= 0 &&
            (int64_t)mine.pos + mine.nblk <= total && mine.ids_off >= 0 &&
            (int64_t)mine.ids_off + mine.nblk <= p.info.num_ids && mine.ctx >= 0 &&
            ((mine.out >= -1 && mine.out < p.info.num_chunks) ||
             (mine.out <= -2 && p.info.tile_ranges >= 1 &&
              -2 - (int64_t)mine.out + p.info.tile_ranges < p.info.num_chunks)));
  if (bad) s_bad = 1;
  __syncthreads();
  if (s_bad) {
    if (threadIdx.x == 0) atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
    wait_vmcnt<0>();  // the blocks issued above land before the wave ends
    return;  // the whole workgroup: nothing below runs
  }
  if constexpr (kTrace) tm[1] = wall_clock64();

  // ---- 2. this wave's range of the workgroup's list and its first window of ids
  const int64_t gw = (int64_t)g * NW + wave;
  const int b0 = s_rec[2 + wave];
  int n = s_rec[3 + wave] - b0;
  bool bad_index = n > kMaxBlocksPerWaveSK || bad_entry;
  if (bad_index) n = 0;
  // block b0 + j of the list: its item (the last whose first block is at or before it)
  // and the offset of its id; false when no item holds it
  // (appends: whether it holds its row's newest token, position ctx - 1)
  auto locate = [&](int j, int& k, int64_t& off, bool& fin) __attribute__((always_inline)) -> bool {
    const int v = b0 + j;
    int lo = 0;
#pragma unroll
    for (int step = kMaxItems / 2; step > 0; step >>= 1)
      if (lo + step < ni && s_item[(lo + step) * kItemWords + 6] <= v) lo += step;
    k = lo;
    const int* it = s_item + lo * kItemWords;
    off = (int64_t)it[7] + (v - it[6]);
    fin = kAppend && it[4] > 0 && it[2] + (v - it[6]) == (it[4] - 1) / kBlockTokens;
    return ni > 0 && v >= it[6] && v < it[6] + it[3];
  };
  int ids = 0, rows = 0, ids_nx = 0, rows_nx = 0;
  uint64_t fmask = 0, fmask_nx = 0;  // appends: the windows' blocks that hold a newest token
  bool ok0 = true, fin0 = false;
  if (lane < n) {
    int64_t off;
    ok0 = locate(lane, rows, off, fin0);
    if (ok0) ids = ids_tab[off];
  }
  bad_index |= __ballot(lane < n && !ok0) != 0;
  if constexpr (kAppend) fmask = __ballot(lane < n && ok0 && fin0);
  int nblk = bad_index ? 0 : n;
  // The first window's ids, when first used (a wave with an entry first processes its
  // query): every one in the arena; and the entry's piece and blocks the items'. Else
  // the wave stops there, flagged.
  auto check_ids = [&](const Item& it0) __attribute__((always_inline)) {
    bool bad_ids = __ballot(lane < n && (unsigned)ids >= (unsigned)a.cache.num_blocks) != 0;
    asm volatile("" : "+v"(ids));  // landed (tested here): no pending load below
    if (pre > 0) {
      bool same = it0.seq == pseq && it0.kvh == pkvh;
#pragma unroll
      for (int j = 0; j < kPrefetchBlocks; ++j)
        same = same && (j >= pre || (__builtin_amdgcn_readlane(ids, j) == pid[j] &&
                                     __builtin_amdgcn_readlane(rows, j) == __builtin_amdgcn_readlane(rows, 0)));
      bad_ids |= !same;
      // appends: the entry's blocks never hold a newest token (its rows are staged with
      // the block, once the wave has its items)
      if constexpr (kAppend) bad_ids |= (fmask & ((1ull << pre) - 1)) != 0;
    }
    if (bad_ids) {
      bad_index = true;
      nblk = 0;
    }
    if constexpr (kTrace) tm[2] = wall_clock64();
  };
  int cw = 0;  // window of ids / rows; ids_nx / rows_nx hold window cw + 1
  char* const id_slot = id_slots + wave * kIdsBytes;
  bool ok_nx = true;
  // the ids of window w + 1 by direct-to-LDS loads when window w starts (their items by
  // the search, into rows_nx): they complete in issue order, so once a block issued
  // after them has landed, they have too
  auto request_ids = [&](int w) __attribute__((always_inline)) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // earlier reads of the slot are done
    const int j = 64 * w + lane;
    ok_nx = true;
    bool fin = false;
    if (j < n) {
      int64_t off;
      ok_nx = locate(j, rows_nx, off, fin);
      if (ok_nx) lds_dma_x1(ids_tab + off, lds_addr(id_slot));
    }
    if constexpr (kAppend) fmask_nx = __ballot(j < n && ok_nx && fin);
  };

  auto stage = [&](int j) __attribute__((always_inline)) -> char* {
    return lds + ((j % NS) * NW + wave) * S::kBytes;
  };
  auto row_at = [&](int j) __attribute__((always_inline)) -> int {
    const bool cur = (j >> 6) == cw;
    return __builtin_amdgcn_readfirstlane(cur ? __builtin_amdgcn_readlane(rows, j & 63)
                                              : __builtin_amdgcn_readlane(rows_nx, j & 63));
  };
  auto new_token = [&](int j) __attribute__((always_inline)) -> char* {
    return s_new + ((j % NS) * NW + wave) * kNewBytes;
  };
  auto issue = [&](int j) __attribute__((always_inline)) {
    const bool cur = (j >> 6) == cw;
    const int id = cur ? __builtin_amdgcn_readlane(ids, j & 63)
                       : __builtin_amdgcn_readlane(ids_nx, j & 63);
    const int k = row_at(j);
    if constexpr (kAppend) {  // the token goes out right before its block
      if (((cur ? fmask : fmask_nx) >> (j & 63)) & 1)
        stage_new_token<QT, D>(a, s_item[k * kItemWords], s_item[k * kItemWords + 1], lane,
                               new_token(j));
    }
    stage_block<D>(a, __builtin_amdgcn_readfirstlane(id), s_item[k * kItemWords + 1], lane,
                   stage(j));
  };
  // Wait until block j has landed; the blocks after it (up to NS - 1) stay in flight.
  auto wait_block = [&](int j) __attribute__((always_inline)) {
    const int later = min(NS - 1, nblk - 1 - j);
    if (NS > 3 && later >= 3) wait_vmcnt<3 * S::kLoads>();
    else if (NS > 2 && later >= 2) wait_vmcnt<2 * S::kLoads>();
    else if (later >= 1) wait_vmcnt<S::kLoads>();
    else wait_vmcnt<0>();
  };
  // this lane's query column of an item: head r of the group (r < G)
  auto column_ptr = [&](const Item& it) __attribute__((always_inline)) -> const QT* {
    return query_col_ptr<QT>(a, it.seq, it.kvh * G + (r < G ? r : 0), qg);
  };

  // The first item's query rows go by direct-to-LDS loads into the last stage, issued
  // before blocks 0 .. NS-2, so the block stream starts without waiting for them (at
  // the top, with the blocks of the wave's entry, when it has one). Queries whose rows
  // do not fit a stage load into registers before the first blocks are issued.
  QkOperand<D, KF> qop;
  float cf = 0.f;
  if (nblk > 0) {
    const Item it0 = item_at(s_item, __builtin_amdgcn_readfirstlane(rows));
    if (pre == 0) check_ids(it0);
    if constexpr (kStagedQuery) {
      if (pre == 0 && nblk > 0) stage_query<QT, D, G>(a, it0.seq, it0.kvh, lane, stage(NS - 1));
      const int first = min(NS - 1, nblk);
      if (pre > 0 && pre < first) check_ids(it0);
      for (int j = pre; j < first && j < nblk; ++j) issue(j);
      // the query has landed: at least `first` stages' loads were issued after it
      if (nblk == 0) wait_vmcnt<0>();  // stopped by check_ids: fewer loads
      else if (first == 3) wait_vmcnt<3 * S::kLoads>();
      else if (first == 2) wait_vmcnt<2 * S::kLoads>();
      else if (first == 1) wait_vmcnt<S::kLoads>();
      else wait_vmcnt<0>();
      lds_query_column<QT, D>(stage(NS - 1), r < G ? r : 0, qg, qr);
      cf = qk_operand_column<QT, D, KF>(qr, valid, a.qk_scale_log2, qop);
      if (pre > 0 && pre >= first) check_ids(it0);
      if (NS - 1 < nblk) issue(NS - 1);  // after the query reads above (values consumed)
    } else {
      if (pre == 0 && nblk > 0) load_query_column<QT, D>(column_ptr(it0), qr);
      cf = qk_operand_column<QT, D, KF>(qr, valid, a.qk_scale_log2, qop);
      if (pre > 0) check_ids(it0);
      const int first = min(NS, nblk);
      for (int j = pre; j < first; ++j) issue(j);
    }
    if (64 < nblk) request_ids(1);
  }

  // ---- 3. stream the blocks, one piece at a time; block i sits in stage i % NS and
  // block i + NS is issued into it once consumed
  float4_t acc[NPV + 1];  // [NPV]: weight sums (INT8)
  float m = 0.f, l = 0.f, lt = 0.f;
  // the wave's first piece, when it is a partial and more pieces follow (kFirstInRegs)
  float4_t acc0[kFirstInRegs ? NPV + 1 : 1];
  float m0 = 0.f, lt0 = 0.f;
  // partials the workgroup merges: the wave's first piece (kept in acc0, or in the
  // workspace at D = 256) or its only piece (left in acc), and its last piece (in acc)
  bool first_saved = false, first_in_acc = false, last_in_acc = false;
  bool bad_score = false;
  const bool masks = a.cache.key_valid != nullptr;
  const int tail = p.info.tail_blocks;
  int pieces_seen = 0;  // trace info
  int i = 0;
  while (i < nblk) {
    if constexpr (kTrace) ++pieces_seen;
    const int crid = __builtin_amdgcn_readlane(rows, i & 63);  // this piece's item
    const int pstart = i;
    const Item it = item_at(s_item, crid);
    const RowSpan psp = row_span(a, it.ctx);
    if (i > 0) {  // a new item starts inside this wave's range
      load_query_column<QT, D>(column_ptr(it), qr);
      cf = qk_operand_column<QT, D, KF>(qr, valid, a.qk_scale_log2, qop);
    }
#pragma unroll
    for (int k = 0; k <= NPV; ++k) acc[k] = float4_t{0.f, 0.f, 0.f, 0.f};
    // a finite start makes a block whose keys are all masked give exp2(-inf) = 0
    m = valid ? -FLT_MAX : 0.f;
    l = 0.f;
    VRange vr = vrange_start<KF>();
    const int pos0 = (it.blk0 + (b0 + i - it.pos)) * kBlockTokens;
    for (;;) {
      // the item's blocks in the current window: up to the first lane with another item
      const int wend = min(64 * (cw + 1), nblk);
      const uint64_t beyond =
          __ballot(lane >= (i & 63) && 64 * cw + lane < wend && rows != crid);
      const int iend = beyond ? 64 * cw + (int)__builtin_ctzll(beyond) : wend;
      for (; i < iend; ++i) {
        wait_block(i);
        if constexpr (kTrace) {
          if (i == 0) tm[3] = wall_clock64();
        }
        if constexpr (kAppend) {
          if ((fmask >> (i & 63)) & 1)
            append_token<QT, D, KF>(a, it.kvh, it.ctx,
                                    __builtin_amdgcn_readlane(ids, i & 63), stage(i),
                                    new_token(i), lane);
        }
        mfma_block<QT, D, KF>(stage(i), qop, cf, pos0 + (i - pstart) * kBlockTokens,
                              psp.kv_begin, psp.ctx, valid, r, qg, acc, m, l, vr, bad_score,
                              masks);
        const int nx = i + NS;
        if (nx < nblk && (nx & 63) == 0) {
          // first block of window cw + 1: its ids were requested before block
          // nx - 64 + NS <= i was issued, which has landed; check them before use
          ids_nx = reinterpret_cast<const int*>(id_slot)[lane];
          if (__ballot(lane < min(64, nblk - nx) &&
                       (!ok_nx || (unsigned)ids_nx >= (unsigned)a.cache.num_blocks)) != 0) {
            bad_index = true;
            nblk = nx;  // stop after the blocks already issued
          }
        }
        if (nx < nblk) {
          // one block in flight per wave (every earlier block has landed before the
          // next is issued), two in the last `tail` blocks of the range
          if (nblk - nx > tail) wait_vmcnt<0>();
          else wait_vmcnt<S::kLoads>();
          issue(nx);
        }
      }
      if (i == wend && i < nblk) {  // into the next window of the block list
        ids = ids_nx;
        rows = rows_nx;
        fmask = fmask_nx;
        ++cw;
        if (64 * (cw + 1) < nblk) request_ids(cw + 1);
        if (__builtin_amdgcn_readlane(rows, 0) == crid) continue;  // the item goes on
      }
      break;
    }
    // the piece [pstart, i): a whole row's output, a whole chunk's partial, or a partial
    // the workgroup merges (the wave's first piece, or its last)
    end_piece<D, KF>(acc, r);
    lt = l + shfl_xor(l, 16);
    lt += shfl_xor(lt, 32);
    lt *= norm_scale<KF>();  // the factor the PV weights carry
    const bool whole = b0 + pstart == it.pos && b0 + i == it.pos + it.nblk;
    if (whole && it.out == -1) {
      if (valid) {
        const float inv = 1.f / fmaxf(lt, FLT_MIN);
        store_lane_out<QT, D>(static_cast<QT*>(a.out) + (int64_t)it.seq * a.o_tok +
                                  (int64_t)(it.kvh * G + r) * a.o_head + qg * (D / 4),
                              acc, inv);
      }
    } else if (whole) {
      // a chunk's partial; or a row after shared-prefix ranges: its own partial, in the
      // slot after theirs, for the workgroup's merge below
      if (valid) {
        const int own = it.out >= 0 ? it.out : -2 - it.out + p.info.tile_ranges;
        const int64_t slot = chunk_slot(p, own, G) + r;
        store_lane_f32<D>(a.ws_o + slot * D + qg * (D / 4), acc);
        if (qg == 0) {
          a.ws_ml[slot * 2] = m;
          a.ws_ml[slot * 2 + 1] = lt;
        }
      }
    } else {
      // a partial the workgroup merges: slot 1 for a last piece that began inside the
      // range, slot 0 for the first piece (the only one included)
      const int which = pstart > 0 ? 1 : 0;
      const bool in_ring = which == 1 ? kLastInRing : (kFirstInRegs || kLastInRing) && i == nblk;
      if (in_ring) {
        (which == 1 ? last_in_acc : first_in_acc) = true;
      } else if (kFirstInRegs && which == 0) {
        first_saved = true;
#pragma unroll
        for (int k = 0; k <= NPV; ++k) acc0[k] = acc[k];
        m0 = m;
        lt0 = lt;
      } else if (valid) {
        const int64_t slot = wave_slot(gw, which, G) + r;
        store_lane_f32<D>(a.ws_o + slot * D + qg * (D / 4), acc);
        if (qg == 0) {
          a.ws_ml[slot * 2] = m;
          a.ws_ml[slot * 2 + 1] = lt;
        }
      }
    }
  }
  if (bad_index && lane == 0) atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
  if (bad_score && lane == 0) atomicOr(a.err_flag, ASTR_FLAG_NONFINITE_SCORE);
  if constexpr (kTrace) tm[4] = wall_clock64();
  // The plan's lengths must be the device's and its blocks visible to them (a mismatch
  // raises the index flag; the rows' outputs are then not to be used).
  if ((int)threadIdx.x < ni) {
    const int ctx = a.context_lens[mine.seq];
    const RowSpan sp = row_span(a, ctx);
    if (ctx != mine.ctx || mine.blk0 < sp.first_blk || mine.blk0 + mine.nblk > sp.last_blk)
      atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
  }

  // ---- 4. every wave is done streaming: the ring takes the workgroup's partials, then
  // the workgroup merges its rows that several of its waves hold (wave w takes items
  // w, w + NW, ...)
  float* const lo_ = reinterpret_cast<float*>(lds);            // [NW][2][G][D]
  float* const lml = lo_ + NW * 2 * G * D;                      // [NW][2][G][2]
  wait_vmcnt<0>();  // no load into the ring is left (a wave stopped early may have some)
  __syncthreads();
  if constexpr (kTrace) tm[5] = wall_clock64();
  auto put = [&](int which, const float4_t (&v)[NPV + 1], float mv, float lv)
      __attribute__((always_inline)) {
    if (!kLastInRing || !valid) return;
    const int col = (wave * 2 + which) * G + r;
    store_lane_f32<D>(lo_ + col * D + qg * (D / 4), v);
    if (qg == 0) {
      lml[col * 2] = mv;
      lml[col * 2 + 1] = lv;
    }
  };
  if (last_in_acc) put(1, acc, m, lt);
  if (first_in_acc) put(0, acc, m, lt);
  if (lane == 0) s_first_ring[wave] = first_in_acc;
  if constexpr (kFirstInRegs) {
    if (first_saved) put(0, acc0, m0, lt0);
  }
  __syncthreads();
  for (int k = wave; k < ni; k += NW) {
    const Item it = item_at(s_item, k);
    QT* const orow = it.out < 0 ? static_cast<QT*>(a.out) + (int64_t)it.seq * a.o_tok +
                                      (int64_t)it.kvh * G * a.o_head
                                : nullptr;
    // a row after shared-prefix ranges: their partials (chunk slots tb .. tb + R - 1)
    // join its own pieces
    const int tb = it.out <= -2 ? -2 - it.out : 0;
    const int ranges = it.out <= -2 ? p.info.tile_ranges : 0;
    auto range_src = [&](int j) __attribute__((always_inline)) -> Partial {
      const int64_t slot = chunk_slot(p, tb + j, G);
      return Partial{a.ws_o + slot * D, a.ws_ml + slot * 2};
    };
    if (it.nblk == 0 && ranges == 0) {  // no visible key (online_attention.py:37): zero
      if (orow != nullptr)
        for (int e = lane; e < G * D; e += kWave)
          orow[(int64_t)(e / D) * a.o_head + e % D] = from_float<QT>(0.f);
      continue;
    }
    // the waves whose ranges hold the item's first and last block
    int w0 = 0, w1 = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      if (s_rec[2 + w] <= it.pos) w0 = w;
      if (s_rec[2 + w] <= it.pos + it.nblk - 1) w1 = w;
    }
    if (w0 == w1) {  // whole in one wave: written there, or (after ranges) in its slot
      if (ranges > 0)
        merge_pieces<QT, D, G, merge_group<D, G>()>(a, range_src, ranges + 1, orow, 0, lane);
      continue;
    }
    // the piece of wave w0 + j: its last piece when the item begins inside w0's range
    // after another item, else its first; an empty range holds none
    auto src_of = [&](int j) __attribute__((always_inline)) -> Partial {
      const int w = w0 + j;
      if (s_rec[2 + w] == s_rec[3 + w]) return Partial{nullptr, nullptr};
      const int which = j == 0 && it.pos > s_rec[2 + w] ? 1 : 0;
      // in the ring: slot 1 when the ring takes last pieces; slot 0 when the first
      // piece stayed in registers or was the wave's only piece (s_first_ring)
      const bool ring = kLastInRing && (which == 1 || kFirstInRegs || s_first_ring[w]);
      if (!ring) {
        const int64_t slot = wave_slot((int64_t)g * NW + w, which, G);
        return Partial{a.ws_o + slot * D, a.ws_ml + slot * 2};
      }
      const int col = (w * 2 + which) * G;
      return Partial{lo_ + col * D, lml + col * 2};
    };
    const int nw = w1 - w0 + 1;
    auto all_src = [&](int j) __attribute__((always_inline)) -> Partial {
      return j < nw ? src_of(j) : range_src(j - nw);
    };
    merge_pieces<QT, D, G, merge_group<D, G>()>(a, all_src, nw + ranges, orow,
                                                it.out < 0 ? 0 : chunk_slot(p, it.out, G), lane);
  }
#if ASTR_TRACE
  tm[6] = wall_clock64();
  if (lane == 0 && gw < kTraceWaves) {
    for (int k = 0; k < 8; ++k) g_ptrace[gw][k] = tm[k];
    g_ptrace_info[gw][0] = n;
    g_ptrace_info[gw][1] = pieces_seen;
    g_ptrace_info[gw][2] = ni;
    g_ptrace_info[gw][3] = (int)__builtin_amdgcn_s_getreg((20 << 0) | (0 << 6) | (3 << 11));  // XCC_ID
  }
#endif
}

// One wave per row the plan cut across workgroups: merges its chunks' partials.
template <typename QT, int D, int G>
__global__ __launch_bounds__(kWave) void merge_chunks_kernel(PlanArgs p) {
  const AttnArgs& a = p.a;
  const int32_t* rec = p.plan + p.info.off_chunked + (int64_t)blockIdx.x * kChunkedWords;
  const int seq = rec[0], kvh = rec[1], c0 = rec[2], count = rec[3];
  if (seq < 0 || seq >= a.num_seqs || kvh < 0 || kvh >= a.cache.num_kv_heads || c0 < 0 ||
      count < 1 || count > p.info.num_chunks - c0) {
    if (threadIdx.x == 0) atomicOr(a.err_flag, ASTR_FLAG_BAD_INDEX);
    return;
  }
  auto src_of = [&](int c) __attribute__((always_inline)) -> Partial {
    const int64_t slot = chunk_slot(p, c0 + c, G);
    return Partial{a.ws_o + slot * D, a.ws_ml + slot * 2};
  };
  QT* orow = static_cast<QT*>(a.out) + (int64_t)seq * a.o_tok + (int64_t)kvh * G * a.o_head;
  merge_pieces<QT, D, G, merge_group<D, G>()>(a, src_of, count, orow, 0, threadIdx.x);
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

template <typename QT, int D, int G>
int launch(const PlanArgs& p, hipStream_t stream, int* resident) {
  auto kernel = decode_planned_kernel<QT, D, G, false>;
  static const int per_cu = query_resident_per_cu(kernel, kPlanWaves * kWave);
  if (resident != nullptr) {
    *resident = per_cu;
    return 0;
  }
  if (p.a.new_k != nullptr) {  // the step's append in the decode (2-byte rows)
    // at head dim 64 the token rows would take the LDS of the second workgroup per CU
    if constexpr (sizeof(QT) == 2 && D >= 128) {
      auto append = decode_planned_kernel<QT, D, G, true>;
      static const int append_per_cu = query_resident_per_cu(append, kPlanWaves * kWave);
      if (append_per_cu < per_cu)  // the plan counts on the plain kernel's residency
        return fail(ASTR_EUNSUPPORTED, "the appending decode holds fewer workgroups per CU");
      kernel = append;
    } else {
      return fail(ASTR_EUNSUPPORTED, "the decode appends bf16/fp16 rows at head dims 128 and "
                  "256 only");
    }
  }
  hipLaunchKernelGGL(kernel, dim3(p.info.num_workgroups), dim3(kPlanWaves * kWave), 0, stream, p);
  if (p.info.num_chunked > 0)
    hipLaunchKernelGGL((merge_chunks_kernel<QT, D, G>), dim3(p.info.num_chunked), dim3(kWave), 0,
                       stream, p);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "paged_attention (planned) launch");
}

template <typename QT, int D>
int dispatch_group(const PlanArgs& p, int G, hipStream_t s, int* resident) {
  switch (G) {
    case 1: return launch<QT, D, 1>(p, s, resident);
    case 2: return launch<QT, D, 2>(p, s, resident);
    case 4: return launch<QT, D, 4>(p, s, resident);
    case 8: return launch<QT, D, 8>(p, s, resident);
    case 16:
      if constexpr (D <= 128) return launch<QT, D, 16>(p, s, resident);
      [[fallthrough]];
    default:
      return fail(ASTR_EUNSUPPORTED, "GQA group size %d not supported", G);
  }
}

template <typename QT>
int dispatch_dim(const PlanArgs& p, int G, hipStream_t s, int* resident) {
  switch (p.a.cache.head_dim) {
    case 64: return dispatch_group<QT, 64>(p, G, s, resident);
    case 128: return dispatch_group<QT, 128>(p, G, s, resident);
    case 256: return dispatch_group<QT, 256>(p, G, s, resident);
    default: return fail(ASTR_EUNSUPPORTED, "head_dim %d not in {64,128,256}", p.a.cache.head_dim);
  }
}

}  // namespace

// The planned decode launch (resident == nullptr), or the resident workgroups per CU of
// its kernel in *resident (nothing is launched), for this unit's code format.
#if ASTR_TRACE && ASTR_KF == 0
// Trace builds: copies the marks and info of the first `waves` waves of the last planned
// launch of the int8 format (8 int64 + 4 int32 per wave) to host memory.
extern "C" int astr_trace_read_planned(void* marks, void* info, int waves) {
  if (waves < 0 || waves > kTraceWaves) return ASTR_EINVAL;
  hipError_t e = hipMemcpyFromSymbol(marks, HIP_SYMBOL(g_ptrace), (size_t)waves * 64);
  if (e == hipSuccess) e = hipMemcpyFromSymbol(info, HIP_SYMBOL(g_ptrace_info), (size_t)waves * 16);
  return e == hipSuccess ? 0 : (int)e;
}
#endif

template <>
int launch_planned_kf<KF>(const PlanArgs& p, int32_t q_dtype, hipStream_t stream, int* resident) {
  const int G = p.a.num_q_heads / p.a.cache.num_kv_heads;
  if (q_dtype == ASTR_F16) return dispatch_dim<_Float16>(p, G, stream, resident);
  if (q_dtype == ASTR_BF16) return dispatch_dim<bf16_t>(p, G, stream, resident);
  if constexpr (KF == kInt8)
    if (q_dtype == ASTR_F32) return dispatch_dim<float>(p, G, stream, resident);
  return fail(ASTR_EUNSUPPORTED, "planned decode takes bf16/fp16 queries (fp32 with int8 codes)");
}

}  // namespace attn
}  // namespace astr
