// C ABI of the paged attention: argument checks, workspace layout and kernel
// choice. Decode rows (one query token) run the stream-K kernel (bf16/fp16
// queries, partition_tokens == 0, up to 512 sequences) or fixed-size split-K
// partitions (every other case); rows with several query tokens (chunked
// prefill, varlen entry point only) run the prefill kernel after them on the same
// stream. Kernels: decode_streamk.hip, decode_partition.hip, prefill.hip.
#include <mutex>

#include "attention_common.h"

namespace astr {
namespace attn {
namespace {

constexpr int kDefaultPartitionTokens = 512;
constexpr int kMaxResidentWavesPerCU = 32;  // gfx950: 8 waves per SIMD

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

// Compute units of the current device (256 when no device is visible).
int device_cus() {
  static std::mutex mu;
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (cus[dev] == 0) {
    int v = 0;
    cus[dev] = (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) ==
                    hipSuccess && v > 0)
                   ? v
                   : 256;
  }
  return cus[dev];
}

// Upper bound of the visible blocks of all rows of one launch.
int64_t max_total_blocks(int32_t num_seqs, int32_t num_kv_heads, int32_t max_context_len,
                         int32_t window) {
  int64_t per_row = ((int64_t)max_context_len + kBlockTokens - 1) / kBlockTokens;
  if (window > 0) {
    const int64_t w = ((int64_t)window + kBlockTokens - 1) / kBlockTokens + 1;
    per_row = per_row < w ? per_row : w;
  }
  return per_row * num_seqs * num_kv_heads;
}

// Fewest stream-K waves that keep every wave at kMaxBlocksPerWaveSK blocks or less:
// the split's ranges hold an equal share of the block and row costs, so a range of
// pack blocks only (the cheapest) sets the bound. rows: work rows of one kv head.
int64_t streamk_need_waves(int64_t total_blocks, int32_t num_kv_heads, int64_t rows) {
  const int64_t per_head = (total_blocks + num_kv_heads - 1) / num_kv_heads;
  const int64_t cost = kSkSeqCost * per_head + kSkRowCost * rows;
  const int64_t unit = (int64_t)kSkPackCostMin * kMaxBlocksPerWaveSK;
  return num_kv_heads * ((cost + unit - 1) / unit);
}

bool use_streamk(int32_t q_dtype, int32_t partition_tokens, int32_t num_seqs) {
  return partition_tokens == 0 && q_dtype != ASTR_F32 && num_seqs <= stream_k_max_seqs();
}

// Workspace layouts. Partitioned: [acc][(m,l)] per (seq, q head, partition).
// Stream-K: [block prefix over work rows, rows with blocks before each row,
// per-sequence pack record][acc][(m,l)] per column of the partial slots: (wave, 2
// slots, slot columns) sized for every wave the GPU can hold, then with prefix packs
// the packs' and packed sequences' own slots.
size_t seq_table_bytes(int32_t head_dim, int32_t num_seqs) {
  return (2 * ((size_t)stream_k_work_rows(head_dim) + 1) + 4 * (size_t)num_seqs) *
         sizeof(int32_t);
}
struct Layout {
  size_t seq_bytes, o_bytes, ml_bytes;
  int64_t waves;  // stream-K wave count of the launch (0 for partitioned)
  size_t total() const { return seq_bytes + o_bytes + ml_bytes; }
};

Layout partitioned_layout(int32_t num_seqs, int32_t num_q_heads, int32_t head_dim,
                          int64_t parts) {
  Layout w{0, 0, 0, 0};
  if (parts <= 1) return w;
  const size_t rows = (size_t)num_seqs * num_q_heads * parts;
  w.o_bytes = align256(rows * head_dim * sizeof(float));
  w.ml_bytes = align256(rows * 2 * sizeof(float));
  return w;
}

// max_waves > 0 limits the capacity (the allocation-free entry point's fixed scratch);
// the layout never holds fewer waves than the block count needs.
Layout streamk_layout(int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                      int32_t head_dim, int32_t max_context_len, int32_t window,
                      int64_t max_waves, int32_t num_packs = 0, int32_t pack_rows = 0) {
  const int64_t need =
      streamk_need_waves(max_total_blocks(num_seqs, num_kv_heads, max_context_len, window),
                         num_kv_heads, (int64_t)num_seqs + num_packs);
  int64_t cap = (int64_t)device_cus() * kMaxResidentWavesPerCU;
  if (max_waves > 0 && cap > max_waves) cap = max_waves / kWaves * kWaves;
  cap = cap > need ? cap : need;
  cap = (cap + kWaves - 1) / kWaves * kWaves;
  const int64_t group = num_q_heads / num_kv_heads;
  const int64_t cols = num_packs > 0 ? (int64_t)pack_rows * group : group;
  const int64_t row_cols = num_packs > 0 ? 2 * (int64_t)num_kv_heads * num_packs * pack_rows * group : 0;
  const size_t slots = (size_t)(cap * 2 * cols + row_cols);
  Layout w;
  w.seq_bytes = align256(seq_table_bytes(head_dim, num_seqs));
  w.o_bytes = align256(slots * head_dim * sizeof(float));
  w.ml_bytes = align256(slots * 2 * sizeof(float));
  w.waves = cap;
  return w;
}

// Bytes of one stream-K wave's partials (two slots of the group's rows) and the most
// waves whose partials fit in `bytes` beside the per-sequence table.
int64_t streamk_waves_in(size_t bytes, int32_t num_seqs, int32_t num_q_heads,
                         int32_t num_kv_heads, int32_t head_dim) {
  const size_t group = (size_t)(num_q_heads / num_kv_heads);
  const size_t per_wave = 2 * group * ((size_t)head_dim + 2) * sizeof(float);
  const size_t fixed = align256(seq_table_bytes(head_dim, num_seqs)) + 2 * 256;
  return bytes > fixed ? (int64_t)((bytes - fixed) / per_wave) : 0;
}

// streamk_need_waves in whole workgroups.
int64_t streamk_min_waves(int64_t total_blocks, int32_t num_kv_heads, int64_t rows) {
  const int64_t need = streamk_need_waves(total_blocks, num_kv_heads, rows);
  return (need + kWaves - 1) / kWaves * kWaves;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace attn
}  // namespace astr

namespace astr {
namespace attn {
namespace {

size_t required_workspace(int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                          int32_t head_dim, int32_t max_context_len, int32_t partition_tokens,
                       int32_t num_packs, int32_t pack_rows) {
  if (num_seqs < 0 || num_q_heads < 1 || num_kv_heads < 1 || head_dim < 1 ||
      max_context_len < 0 || partition_tokens < 0 || num_q_heads % num_kv_heads ||
      num_packs < 0 || (num_packs > 0 && pack_rows < 1))
    return 0;
  if (num_seqs == 0) return 0;
  // stream-K is chosen per query dtype at launch; size for it whenever it may run
  if (partition_tokens == 0 && num_seqs <= stream_k_max_seqs()) {
    const Layout sk = streamk_layout(num_seqs, num_q_heads, num_kv_heads, head_dim,
                                     max_context_len, 0, 0, num_packs, pack_rows);
    const Layout pt = partitioned_layout(num_seqs, num_q_heads, head_dim,
                                         max_parts_for(max_context_len, kDefaultPartitionTokens));
    return sk.total() > pt.total() ? sk.total() : pt.total();
  }
  const int pt = partition_tokens == 0 ? kDefaultPartitionTokens : partition_tokens;
  if (!valid_partition(pt)) return 0;
  return partitioned_layout(num_seqs, num_q_heads, head_dim, max_parts_for(max_context_len, pt))
      .total();
}

}  // namespace
}  // namespace attn
}  // namespace astr

extern "C" size_t astr_paged_attention_i8_workspace_bytes(int32_t num_seqs, int32_t num_q_heads,
                                                          int32_t num_kv_heads, int32_t head_dim,
                                                          int32_t max_context_len,
                                                          int32_t partition_tokens) {
  return astr::attn::required_workspace(num_seqs, num_q_heads, num_kv_heads, head_dim,
                                     max_context_len, partition_tokens, 0, 0);
}

extern "C" size_t astr_paged_attention_i8_shared_workspace_bytes(
    int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t max_context_len, int32_t num_packs, int32_t rows_per_pack) {
  return astr::attn::required_workspace(num_seqs, num_q_heads, num_kv_heads, head_dim,
                                     max_context_len, 0, num_packs, rows_per_pack);
}

namespace {

int paged_attention(const astr_paged_kv* cache, const void* query, int32_t q_dtype,
                    int64_t q_token_stride, int64_t q_head_stride, void* out,
                    int64_t out_token_stride, int64_t out_head_stride,
                    const int32_t* query_start_loc, int32_t num_query_tokens,
                    int32_t max_query_len, int32_t causal, const int32_t* block_tables,
                    int32_t block_table_stride, const int32_t* context_lens, int32_t num_seqs,
                    int32_t num_q_heads, int32_t max_context_len, float scale, int32_t window,
                    int32_t partition_tokens, void* workspace, size_t workspace_bytes,
                    int32_t* err_flag, void* stream, bool fixed_scratch = false,
                    const int32_t* packs = nullptr, int32_t num_packs = 0,
                    int32_t pack_rows = 0, float* stats = nullptr) {
  using namespace astr;
  using namespace astr::attn;
  if (cache == nullptr || err_flag == nullptr)
    return fail(ASTR_EINVAL, "cache descriptor and err_flag are required");
  if (num_seqs < 0 || num_q_heads < 1 || max_context_len < 0 || block_table_stride < 0)
    return fail(ASTR_EINVAL, "num_seqs/max_context_len/block_table_stride must be >= 0 and "
                             "num_q_heads >= 1");
  if (num_seqs == 0) return 0;
  if (num_seqs > 65535) return fail(ASTR_EUNSUPPORTED, "more than 65535 sequences per launch");
  if (query_start_loc != nullptr && (num_query_tokens < 0 || max_query_len < 0))
    return fail(ASTR_EINVAL, "num_query_tokens and max_query_len must be >= 0");
  if (query_start_loc != nullptr && num_query_tokens == 0) return 0;
  if (query == nullptr || out == nullptr || block_tables == nullptr || context_lens == nullptr)
    return fail(ASTR_EINVAL, "query, out, block_tables and context_lens are required");
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(ASTR_EINVAL, "attention scale must be finite and positive");
  if (window < 0) return fail(ASTR_EINVAL, "window must be >= 0 (0 = no window)");
  if (cache->block_size != kBlockTokens)
    return fail(ASTR_EUNSUPPORTED, "block_size %d != 16", cache->block_size);
  if (cache->code_format != ASTR_KV_INT8 && cache->code_format != ASTR_KV_FP8_E4M3FN &&
      cache->code_format != ASTR_KV_FP8_E5M2)
    return fail(ASTR_EUNSUPPORTED, "code format %d is not int8 / fp8 e4m3fn / fp8 e5m2",
                cache->code_format);
  if (cache->num_kv_heads < 1 || num_q_heads % cache->num_kv_heads != 0)
    return fail(ASTR_EINVAL, "num_q_heads %d must be a multiple of num_kv_heads %d", num_q_heads,
                cache->num_kv_heads);
  if (cache->num_blocks < 1) return fail(ASTR_EINVAL, "cache has no blocks");
  if (partition_tokens < 0 || (partition_tokens != 0 && !valid_partition(partition_tokens)))
    return fail(ASTR_EINVAL, "partition_tokens %d must be 0 (auto) or a positive multiple of %d "
                "up to %d", partition_tokens, kBlockTokens * kWaves,
                kBlockTokens * kWaves * kMaxBlocksPerWave);
  // statistics come from the fixed-partition kernels (fp32 queries, exact VALU)
  const bool streamk = stats == nullptr && use_streamk(q_dtype, partition_tokens, num_seqs);
  const int group = num_q_heads / cache->num_kv_heads;
  if (num_packs < 0) return fail(ASTR_EINVAL, "num_packs must be >= 0");
  if (num_packs > 0) {
    if (packs == nullptr || (reinterpret_cast<uintptr_t>(packs) & 3u) != 0)
      return fail(ASTR_EINVAL, "a 4-byte aligned pack table is required for %d packs", num_packs);
    if (pack_rows < 2 || pack_rows * group > 16)
      return fail(ASTR_EINVAL, "rows_per_pack %d must be in [2, 16 / G = %d]", pack_rows,
                  16 / group);
    if (num_packs > stream_k_max_packs() ||
        (int64_t)num_packs * pack_rows > stream_k_max_pack_seqs())
      return fail(ASTR_EUNSUPPORTED, "%d packs of %d rows: at most %d packs and %d pack rows",
                  num_packs, pack_rows, stream_k_max_packs(), stream_k_max_pack_seqs());
    if (window != 0)
      return fail(ASTR_EUNSUPPORTED, "prefix packs need window == 0 (the packed blocks are "
                  "visible to every member)");
    // the partitioned kernels read every row's blocks themselves, and batches beyond
    // the pack tables run the stream-K kernel without them
    if (!streamk || num_seqs > stream_k_max_pack_seqs()) num_packs = 0;
  }
  const int pt = partition_tokens == 0 ? kDefaultPartitionTokens : partition_tokens;
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
  if (cache->key_valid != nullptr && !aligned16(cache->key_valid))
    return fail(ASTR_EINVAL, "cache key_valid must be 16-byte aligned");
  const int64_t parts = max_parts_for(max_context_len, pt);
  if (!streamk && parts > 65535)
    return fail(ASTR_EUNSUPPORTED, "too many split-K partitions (%lld)", (long long)parts);
  // a caller's workspace is sized by astr_paged_attention_i8_workspace_bytes; the fixed
  // scratch of the allocation-free entry point caps the stream-K capacity instead
  const int64_t sk_limit = fixed_scratch ? streamk_waves_in(workspace_bytes, num_seqs,
                                                            num_q_heads, cache->num_kv_heads,
                                                            cache->head_dim) : 0;
  if (fixed_scratch && streamk && sk_limit < kWaves)
    return fail(ASTR_EINVAL, "the allocation-free entry point's %zu-byte scratch holds too few "
                "stream-K partials for %d sequences x %d query heads", workspace_bytes, num_seqs,
                num_q_heads);
  const Layout ws = streamk ? streamk_layout(num_seqs, num_q_heads, cache->num_kv_heads,
                                             cache->head_dim, max_context_len, 0, sk_limit,
                                             num_packs, pack_rows)
                            : partitioned_layout(num_seqs, num_q_heads, cache->head_dim, parts);
  const size_t need = fixed_scratch ? ws.total()
                                    : required_workspace(num_seqs, num_q_heads, cache->num_kv_heads,
                                                         cache->head_dim, max_context_len,
                                                         partition_tokens, num_packs, pack_rows);
  if (fixed_scratch && need > workspace_bytes)
    return fail(ASTR_EINVAL, "this launch needs %zu bytes of split-K scratch, more than the "
                "%zu bytes the allocation-free entry point holds", need, workspace_bytes);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need ||
                   (reinterpret_cast<uintptr_t>(workspace) & 255u) != 0))
    return fail(ASTR_EINVAL, "a 256-byte aligned workspace of %zu bytes is required (%zu given)",
                need, workspace_bytes);

  AttnArgs a{};
  a.q_start = query_start_loc;
  a.num_q_tokens = query_start_loc != nullptr ? num_query_tokens : num_seqs;
  a.max_q_len = query_start_loc != nullptr ? max_query_len : 1;
  a.causal = causal != 0;
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
  a.total_waves = (int32_t)ws.waves;  // capacity; the stream-K launcher settles the count
  a.min_waves = (int32_t)streamk_min_waves(
      max_total_blocks(num_seqs, cache->num_kv_heads, max_context_len, window),
      cache->num_kv_heads, (int64_t)num_seqs + (num_packs > 0 ? num_packs : 0));
  a.packs = num_packs > 0 ? packs : nullptr;
  a.num_packs = num_packs;
  a.pack_rows = num_packs > 0 ? pack_rows : 1;
  a.slot_cols = a.pack_rows * group;
  if (ws.total() > 0) {
    char* base = static_cast<char*>(workspace);
    a.ws_seq = reinterpret_cast<int32_t*>(base);
    if (streamk) {
      a.ws_ne = a.ws_seq + stream_k_work_rows(cache->head_dim) + 1;
      a.ws_pack = a.ws_ne + stream_k_work_rows(cache->head_dim) + 1;
    }
    a.ws_o = reinterpret_cast<float*>(base + ws.seq_bytes);
    a.ws_ml = reinterpret_cast<float*>(base + ws.seq_bytes + ws.o_bytes);
  }
  a.stats = stats;
  a.err_flag = err_flag;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int rc = streamk ? launch_streamk(a, q_dtype, s) : launch_partitioned(a, q_dtype, s);
  if (rc != 0 || query_start_loc == nullptr || max_query_len < 2) return rc;
  return launch_prefill(a, q_dtype, s);
}

}  // namespace

extern "C" int astr_paged_attention_i8(const astr_paged_kv* cache, const void* query,
                                       int32_t q_dtype, int64_t q_token_stride,
                                       int64_t q_head_stride, void* out, int64_t out_token_stride,
                                       int64_t out_head_stride, const int32_t* block_tables,
                                       int32_t block_table_stride, const int32_t* context_lens,
                                       int32_t num_seqs, int32_t num_q_heads,
                                       int32_t max_context_len, float scale, int32_t window,
                                       int32_t partition_tokens, void* workspace,
                                       size_t workspace_bytes, int32_t* err_flag, void* stream) {
  astr::CallRange range("astr_paged_attention_i8");
  return paged_attention(cache, query, q_dtype, q_token_stride, q_head_stride, out,
                         out_token_stride, out_head_stride, nullptr, num_seqs, 1, 1, block_tables,
                         block_table_stride, context_lens, num_seqs, num_q_heads, max_context_len,
                         scale, window, partition_tokens, workspace, workspace_bytes, err_flag,
                         stream);
}

extern "C" int astr_paged_attention_varlen_i8(
    const astr_paged_kv* cache, const void* query, int32_t q_dtype, int64_t q_token_stride,
    int64_t q_head_stride, void* out, int64_t out_token_stride, int64_t out_head_stride,
    const int32_t* query_start_loc, int32_t num_query_tokens, int32_t max_query_len,
    int32_t causal, const int32_t* block_tables, int32_t block_table_stride,
    const int32_t* context_lens, int32_t num_seqs, int32_t num_q_heads, int32_t max_context_len,
    float scale, int32_t window, int32_t partition_tokens, void* workspace, size_t workspace_bytes,
    int32_t* err_flag, void* stream) {
  astr::CallRange range("astr_paged_attention_varlen_i8");
  if (query_start_loc == nullptr)
    return astr::fail(ASTR_EINVAL, "query_start_loc is required (int32 [num_seqs + 1])");
  return paged_attention(cache, query, q_dtype, q_token_stride, q_head_stride, out,
                         out_token_stride, out_head_stride, query_start_loc, num_query_tokens,
                         max_query_len, causal, block_tables, block_table_stride, context_lens,
                         num_seqs, num_q_heads, max_context_len, scale, window, partition_tokens,
                         workspace, workspace_bytes, err_flag, stream);
}

extern "C" int astr_paged_attention_i8_shared(
    const astr_paged_kv* cache, const void* query, int32_t q_dtype, int64_t q_token_stride,
    int64_t q_head_stride, void* out, int64_t out_token_stride, int64_t out_head_stride,
    const int32_t* block_tables, int32_t block_table_stride, const int32_t* context_lens,
    int32_t num_seqs, int32_t num_q_heads, int32_t max_context_len, float scale, int32_t window,
    const int32_t* packs, int32_t num_packs, int32_t rows_per_pack, void* workspace,
    size_t workspace_bytes, int32_t* err_flag, void* stream) {
  astr::CallRange range("astr_paged_attention_i8_shared");
  return paged_attention(cache, query, q_dtype, q_token_stride, q_head_stride, out,
                         out_token_stride, out_head_stride, nullptr, num_seqs, 1, 1, block_tables,
                         block_table_stride, context_lens, num_seqs, num_q_heads, max_context_len,
                         scale, window, 0, workspace, workspace_bytes, err_flag, stream, false,
                         packs, num_packs, rows_per_pack);
}

extern "C" int astr_paged_attention_i8_statistics(
    const astr_paged_kv* cache, const float* query, int64_t q_token_stride,
    int64_t q_head_stride, float* weighted, int64_t w_token_stride, int64_t w_head_stride,
    float* stats, const int32_t* block_tables, int32_t block_table_stride,
    const int32_t* context_lens, int32_t num_seqs, int32_t num_q_heads, int32_t max_context_len,
    float scale, int32_t window, int32_t partition_tokens, void* workspace,
    size_t workspace_bytes, int32_t* err_flag, void* stream) {
  astr::CallRange range("astr_paged_attention_i8_statistics");
  if (stats == nullptr || (reinterpret_cast<uintptr_t>(stats) & 7u) != 0)
    return astr::fail(ASTR_EINVAL, "an 8-byte aligned stats array [num_seqs, num_q_heads, 2] "
                      "is required");
  return paged_attention(cache, query, ASTR_F32, q_token_stride, q_head_stride, weighted,
                         w_token_stride, w_head_stride, nullptr, num_seqs, 1, 1, block_tables,
                         block_table_stride, context_lens, num_seqs, num_q_heads, max_context_len,
                         scale, window, partition_tokens, workspace, workspace_bytes, err_flag,
                         stream, false, nullptr, 0, 0, stats);
}

// ---- allocation-free decode entry point: split-K partials in a fixed device array

namespace {

// Scratch of astr_paged_attention_i8_noalloc, one copy per GPU for the life of the
// process. In host code `scratch` only names the symbol: its device address comes from
// hipGetSymbolAddress, once per device (scratch_on_current_device).
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;

// The address of `scratch` on the current device in *ptr, looked up with that device
// current the first time and kept per device. Returns 0, or an error code with
// astr_last_error set.
int scratch_on_current_device(void** ptr) {
  static std::mutex mu;
  static void* addr[kMaxDevices] = {nullptr};
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return astr::hip_fail(err, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices)
    return astr::fail(ASTR_EUNSUPPORTED, "device %d beyond the %d the scratch table holds", dev,
                      kMaxDevices);
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return astr::hip_fail(err, "hipGetSymbolAddress(scratch)");
    if (p == nullptr) return astr::fail(ASTR_EINVAL, "hipGetSymbolAddress(scratch) gave NULL");
    addr[dev] = p;
  }
  *ptr = addr[dev];
  return 0;
}

}  // namespace

extern "C" int astr_paged_attention_i8_noalloc(
    const astr_paged_kv* cache, const void* query, int32_t q_dtype, int64_t q_token_stride,
    int64_t q_head_stride, void* out, int64_t out_token_stride, int64_t out_head_stride,
    const int32_t* block_tables, int32_t block_table_stride, const int32_t* context_lens,
    int32_t num_seqs, int32_t num_q_heads, int32_t max_context_len, float scale, int32_t window,
    int32_t partition_tokens, int32_t* err_flag, void* stream) {
  astr::CallRange range("astr_paged_attention_i8_noalloc");
  if (num_seqs <= 0) return num_seqs == 0 ? 0 : astr::fail(ASTR_EINVAL, "num_seqs must be >= 0");
  void* ws = nullptr;
  const int rc = scratch_on_current_device(&ws);
  if (rc != 0) return rc;
  return paged_attention(cache, query, q_dtype, q_token_stride, q_head_stride, out,
                         out_token_stride, out_head_stride, nullptr, num_seqs, 1, 1, block_tables,
                         block_table_stride, context_lens, num_seqs, num_q_heads, max_context_len,
                         scale, window, partition_tokens, ws, kNoAllocScratchBytes, err_flag,
                         stream, true);
}

// ---- decode rows on a host plan (decode_plan.cpp, decode_planned.hip)

namespace {

constexpr int kPlanWavesPerWorkgroup = 8;  // the planned kernel's workgroup

// Partial slots of a plan: two per wave, G per chunk; bytes of their (acc, (m, l)).
size_t planned_workspace(const astr_decode_plan_info& info, int32_t num_q_heads, int32_t head_dim) {
  using astr::attn::align256;
  if (info.num_kv_heads < 1 || num_q_heads % info.num_kv_heads) return 0;
  const size_t group = (size_t)(num_q_heads / info.num_kv_heads);
  const size_t slots = ((size_t)info.num_workgroups * info.waves_per_workgroup * 2 +
                        (size_t)info.num_chunks) * group;
  return align256(slots * head_dim * sizeof(float)) + align256(slots * 2 * sizeof(float));
}

}  // namespace

extern "C" int astr_decode_plan_workgroups(int32_t head_dim, int32_t num_q_heads,
                                           int32_t num_kv_heads, int32_t q_dtype,
                                           int32_t code_format, int32_t* num_workgroups,
                                           int32_t* waves_per_workgroup) {
  using namespace astr;
  using namespace astr::attn;
  if (num_workgroups == nullptr || waves_per_workgroup == nullptr || num_kv_heads < 1 ||
      num_q_heads < 1 || num_q_heads % num_kv_heads)
    return fail(ASTR_EINVAL, "plan workgroups: invalid arguments");
  if (code_format != ASTR_KV_INT8 && code_format != ASTR_KV_FP8_E4M3FN &&
      code_format != ASTR_KV_FP8_E5M2)
    return fail(ASTR_EUNSUPPORTED, "code format %d", code_format);
  PlanArgs p{};
  p.a.cache.head_dim = head_dim;
  p.a.cache.num_kv_heads = num_kv_heads;
  p.a.cache.code_format = code_format;
  p.a.num_q_heads = num_q_heads;
  int per_cu = 0;
  const int rc = launch_planned(p, q_dtype, nullptr, &per_cu);
  if (rc != 0) return rc;
  *num_workgroups = device_cus() * per_cu;
  *waves_per_workgroup = kPlanWavesPerWorkgroup;
  return 0;
}

extern "C" size_t astr_paged_attention_i8_planned_workspace_bytes(
    const astr_decode_plan_info* info, int32_t num_q_heads, int32_t head_dim) {
  if (info == nullptr || head_dim < 1 || num_q_heads < 1) return 0;
  return planned_workspace(*info, num_q_heads, head_dim);
}

namespace {

// The step's newest tokens for the appending decode (AttnArgs::new_k), or none.
struct NewTokens {
  const void* key = nullptr;
  const void* value = nullptr;
  int64_t k_tok = 0, k_head = 0, v_tok = 0, v_head = 0;
  const int64_t* slots = nullptr;
};

int planned_attention(const astr_paged_kv* cache, const void* query, int32_t q_dtype,
                      int64_t q_token_stride, int64_t q_head_stride, void* out,
                      int64_t out_token_stride, int64_t out_head_stride,
                      const int32_t* context_lens, int32_t num_q_heads, float scale,
                      const int32_t* plan, const astr_decode_plan_info* info, void* workspace,
                      size_t workspace_bytes, int32_t* err_flag, void* stream,
                      const NewTokens& nt) {
  using namespace astr;
  using namespace astr::attn;
  if (cache == nullptr || err_flag == nullptr || info == nullptr)
    return fail(ASTR_EINVAL, "cache descriptor, plan info and err_flag are required");
  const astr_decode_plan_info& pi = *info;
  if (pi.num_seqs == 0) return 0;
  if (pi.num_seqs < 0 || pi.num_workgroups < 1 || pi.waves_per_workgroup != kPlanWavesPerWorkgroup ||
      pi.num_items < 0 || pi.num_blocks < 0 || pi.num_chunks < 0 || pi.num_chunked < 0 ||
      pi.window < 0 || pi.tail_blocks < 0 || pi.num_kv_heads != cache->num_kv_heads)
    return fail(ASTR_EINVAL, "plan info does not describe a plan for this arena");
  const int64_t wg_words = (int64_t)pi.num_workgroups * (pi.waves_per_workgroup + 3);
  const bool layout =
      pi.off_workgroups == 0 && pi.off_waves == wg_words &&
      pi.off_items == wg_words + (int64_t)pi.num_workgroups * pi.waves_per_workgroup * 6 &&
      pi.num_ids >= 0 &&
      pi.item_stride >= 1 && pi.item_stride <= 64 &&
      pi.num_items == (int64_t)pi.num_workgroups * pi.item_stride &&
      pi.off_ids == pi.off_items + (int64_t)pi.num_items * 8 &&
      pi.off_chunked == pi.off_ids + pi.num_ids &&
      pi.off_tiles == pi.off_chunked + (int64_t)pi.num_chunked * 4 &&
      pi.off_tile_members == pi.off_tiles + (int64_t)pi.num_tiles * 8 &&
      pi.plan_words == pi.off_tile_members + (int64_t)pi.num_tile_members * 3;
  if (!layout) return fail(ASTR_EINVAL, "plan info offsets are inconsistent");
  if (pi.num_tiles < 0 || pi.num_tile_members < 0 ||
      (pi.num_tiles > 0 && (pi.tile_ranges < 1 || pi.tile_ranges > 16 || pi.tile_rows < 2)))
    return fail(ASTR_EINVAL, "plan info describes invalid prefix tiles");

  if (plan == nullptr || (reinterpret_cast<uintptr_t>(plan) & 3u) != 0)
    return fail(ASTR_EINVAL, "a 4-byte aligned device plan is required");
  if (query == nullptr || out == nullptr || context_lens == nullptr)
    return fail(ASTR_EINVAL, "query, out and context_lens are required");
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(ASTR_EINVAL, "attention scale must be finite and positive");
  if (cache->block_size != kBlockTokens)
    return fail(ASTR_EUNSUPPORTED, "block_size %d != 16", cache->block_size);
  if (cache->code_format != ASTR_KV_INT8 && cache->code_format != ASTR_KV_FP8_E4M3FN &&
      cache->code_format != ASTR_KV_FP8_E5M2)
    return fail(ASTR_EUNSUPPORTED, "code format %d", cache->code_format);
  if (cache->num_kv_heads < 1 || num_q_heads % cache->num_kv_heads != 0)
    return fail(ASTR_EINVAL, "num_q_heads %d must be a multiple of num_kv_heads %d", num_q_heads,
                cache->num_kv_heads);
  if (pi.num_tiles > 0 &&
      (int64_t)pi.tile_rows * (num_q_heads / cache->num_kv_heads) > prefix_tile_columns(cache->head_dim))
    return fail(ASTR_EINVAL, "prefix tiles of %d rows exceed the %d query columns of a tile",
                pi.tile_rows, prefix_tile_columns(cache->head_dim));
  if (cache->num_blocks < 1) return fail(ASTR_EINVAL, "cache has no blocks");
  if (q_dtype != ASTR_F16 && q_dtype != ASTR_BF16 &&
      !(q_dtype == ASTR_F32 && cache->code_format == ASTR_KV_INT8))
    return fail(ASTR_EUNSUPPORTED, "the planned decode takes bf16/fp16 queries, or fp32 "
                "queries with int8 codes");
  const int64_t esize = q_dtype == ASTR_F32 ? 4 : 2;
  if (!aligned16(query) || !aligned16(out) || (q_token_stride * esize) % 16 ||
      (q_head_stride * esize) % 16 || (out_token_stride * esize) % 16 ||
      (out_head_stride * esize) % 16)
    return fail(ASTR_EINVAL, "query/out rows must be 16-byte aligned");
  if (!aligned16(cache->k_codes) || !aligned16(cache->v_codes) ||
      cache->code_block_stride % 16 || cache->code_head_stride % 16 ||
      !aligned16(cache->k_scales) || !aligned16(cache->v_scales) ||
      cache->scale_block_stride % 4 || cache->scale_head_stride % 4)
    return fail(ASTR_EINVAL, "cache code and scale blocks must be 16-byte aligned");
  if (cache->key_valid != nullptr && !aligned16(cache->key_valid))
    return fail(ASTR_EINVAL, "cache key_valid must be 16-byte aligned");
  const size_t need = planned_workspace(pi, num_q_heads, cache->head_dim);
  if (workspace == nullptr || workspace_bytes < need ||
      (reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
    return fail(ASTR_EINVAL, "a 256-byte aligned workspace of %zu bytes is required (%zu given)",
                need, workspace_bytes);
  const size_t group = (size_t)(num_q_heads / cache->num_kv_heads);
  const size_t slots = ((size_t)pi.num_workgroups * pi.waves_per_workgroup * 2 +
                        (size_t)pi.num_chunks) * group;
  PlanArgs p{};
  AttnArgs& a = p.a;
  a.q = query;
  a.q_tok = q_token_stride;
  a.q_head = q_head_stride;
  a.out = out;
  a.o_tok = out_token_stride;
  a.o_head = out_head_stride;
  a.cache = *cache;
  // the block tables are not read (the plan holds the block ids); bt_stride bounds the
  // context lengths as the plan's tables did
  a.bt_stride = INT32_MAX / kBlockTokens;
  a.context_lens = context_lens;
  a.num_q_tokens = pi.num_seqs;
  a.max_q_len = 1;
  a.num_seqs = pi.num_seqs;
  a.num_q_heads = num_q_heads;
  a.qk_scale_log2 = scale * kLog2e;
  a.window = pi.window;
  a.ws_o = static_cast<float*>(workspace);
  a.ws_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                     align256(slots * cache->head_dim * sizeof(float)));
  a.err_flag = err_flag;
  a.new_k = nt.key;
  a.new_v = nt.value;
  a.nk_tok = nt.k_tok;
  a.nk_head = nt.k_head;
  a.nv_tok = nt.v_tok;
  a.nv_head = nt.v_head;
  a.new_slots = nt.slots;
  p.plan = plan;
  p.info = pi;
  // the prefix tiles' partials, then the decode kernel and the chunk merge that reads them
  if (pi.num_tiles > 0) {
    const int rc = launch_prefix_tiles(p, q_dtype, static_cast<hipStream_t>(stream));
    if (rc != 0) return rc;
  }
  return launch_planned(p, q_dtype, static_cast<hipStream_t>(stream), nullptr);
}

}  // namespace

extern "C" int astr_paged_attention_i8_planned(
    const astr_paged_kv* cache, const void* query, int32_t q_dtype, int64_t q_token_stride,
    int64_t q_head_stride, void* out, int64_t out_token_stride, int64_t out_head_stride,
    const int32_t* context_lens, int32_t num_q_heads, float scale, const int32_t* plan,
    const astr_decode_plan_info* info, void* workspace, size_t workspace_bytes,
    int32_t* err_flag, void* stream) {
  astr::CallRange range("astr_paged_attention_i8_planned");
  return planned_attention(cache, query, q_dtype, q_token_stride, q_head_stride, out,
                           out_token_stride, out_head_stride, context_lens, num_q_heads, scale,
                           plan, info, workspace, workspace_bytes, err_flag, stream,
                           NewTokens{});
}

extern "C" int astr_paged_attention_i8_planned_append(
    const astr_paged_kv* cache, const void* query, int32_t q_dtype, int64_t q_token_stride,
    int64_t q_head_stride, void* out, int64_t out_token_stride, int64_t out_head_stride,
    const void* key, const void* value, int64_t key_token_stride, int64_t key_head_stride,
    int64_t value_token_stride, int64_t value_head_stride, const int64_t* slot_mapping,
    const int32_t* context_lens, int32_t num_q_heads, float scale, const int32_t* plan,
    const astr_decode_plan_info* info, void* workspace, size_t workspace_bytes,
    int32_t* err_flag, void* stream) {
  astr::CallRange range("astr_paged_attention_i8_planned_append");
  using astr::fail;
  if (info != nullptr && info->num_seqs > 0) {
    if (key == nullptr || value == nullptr || slot_mapping == nullptr)
      return fail(ASTR_EINVAL, "key, value and slot_mapping are required");
    if (q_dtype != ASTR_BF16 && q_dtype != ASTR_F16)
      return fail(ASTR_EUNSUPPORTED, "the appending decode takes bf16/fp16 queries and rows");
    // 4-byte lanes of each row (the rows' direct-to-LDS loads), 8-byte slots
    if ((reinterpret_cast<uintptr_t>(key) | reinterpret_cast<uintptr_t>(value)) & 3u ||
        (key_token_stride | key_head_stride | value_token_stride | value_head_stride) & 1 ||
        (reinterpret_cast<uintptr_t>(slot_mapping) & 7u))
      return fail(ASTR_EINVAL, "key/value rows must be 4-byte aligned and slot_mapping 8-byte "
                  "aligned");
  }
  NewTokens nt;
  nt.key = key;
  nt.value = value;
  nt.k_tok = key_token_stride;
  nt.k_head = key_head_stride;
  nt.v_tok = value_token_stride;
  nt.v_head = value_head_stride;
  nt.slots = slot_mapping;
  return planned_attention(cache, query, q_dtype, q_token_stride, q_head_stride, out,
                           out_token_stride, out_head_stride, context_lens, num_q_heads, scale,
                           plan, info, workspace, workspace_bytes, err_flag, stream, nt);
}
