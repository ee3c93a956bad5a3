/*
 * aster_kv.h -- C ABI of the MI355X (gfx950) INT8 paged-KV decode path.
 *
 * Plain pointers and sizes only: every pointer except `cache` and the
 * `astr_*_workspace_bytes` arguments is a DEVICE pointer owned by the caller
 * (the torch allocator in the Python host layer); the library never allocates
 * or frees device memory. `stream` is a hipStream_t passed as void*; work is
 * stream-ordered and the calls return without synchronising.
 *
 * Return codes (all entry points):
 *    0  success (launched)
 *   -1  ASTR_EINVAL       invalid argument (Python raises ValueError)
 *   -2  ASTR_EUNSUPPORTED configuration this build has no kernel for
 *                         (Python raises UnsupportedAttentionBackend)
 *   >0  hipError_t from the launch
 * astr_last_error() returns a thread-local message for the last failure.
 *
 * Device error flag (int32, caller-zeroed, sticky until the caller clears it):
 *   bit 0 ASTR_FLAG_NONFINITE_INPUT  a K/V input value was NaN/Inf: the
 *                                    append wrote NO slot (all-or-nothing; the
 *                                    reserved-slot appends: none of the
 *                                    non-finite rows)
 *   bit 1 ASTR_FLAG_NONFINITE_SCORE  an attention score was NaN/Inf
 *   bit 2 ASTR_FLAG_BAD_INDEX        a slot / block-table entry / context
 *                                    length pointed outside the arena or
 *                                    the block table (the access was skipped)
 */
#ifndef ASTER_KV_H
#define ASTER_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ASTR_EINVAL (-1)
#define ASTR_EUNSUPPORTED (-2)

#define ASTR_FLAG_NONFINITE_INPUT 1
#define ASTR_FLAG_NONFINITE_SCORE 2
#define ASTR_FLAG_BAD_INDEX 4

/* Element types of queries, outputs and K/V inputs. */
enum astr_dtype { ASTR_F32 = 0, ASTR_F16 = 1, ASTR_BF16 = 2 };

/*
 * Code formats of the arena (KVQuantization.format, kv_quantization.py:7-25): one byte
 * per element, with maximum 127 (int8), 448 (OCP FP8 E4M3FN) or 57344 (OCP FP8 E5M2).
 */
enum astr_kv_format { ASTR_KV_INT8 = 0, ASTR_KV_FP8_E4M3FN = 1, ASTR_KV_FP8_E5M2 = 2 };

/*
 * One layer of the paged KV arena (device memory, caller-owned).
 * Codes: a block holds num_kv_heads x block_size token rows of head_dim one-byte
 * codes in `code_format` (int8, or FP8 E4M3FN / E5M2 bit patterns); a token row is
 * contiguous (token stride = head_dim bytes).
 * Scales: one fp32 per (block, head, token); token stride = 1 float.
 * Physical block b, kv head h, token slot s lives at
 *   k_codes + b*code_block_stride + h*code_head_stride + s*head_dim
 *   k_scales + b*scale_block_stride + h*scale_head_stride + s
 * (same for v_*). This is the reference's per-page [1,Hkv,bs,D] codes and
 * [1,Hkv,bs,1] scales (kv_quantization.py:97-110, state.py:319-327) stacked
 * into one arena indexed by PageRef.index.
 * Key padding: key_valid + b*block_size + s is 0 when that slot holds a padding
 * token, which no query attends (the page's padding leaf [1,1,bs,1] of
 * state.py:319-327, applied as a key mask by online_attention.py:185-186), and
 * nonzero for a real token. One byte per slot, shared by every layer and head;
 * NULL means every key is real (the attention kernels then skip the mask).
 */
typedef struct astr_paged_kv {
  int8_t* k_codes;
  int8_t* v_codes;
  float* k_scales;
  float* v_scales;
  int64_t code_block_stride;  /* bytes  */
  int64_t code_head_stride;   /* bytes  */
  int64_t scale_block_stride; /* floats */
  int64_t scale_head_stride;  /* floats */
  int32_t num_blocks;
  int32_t block_size;   /* must be 16 */
  int32_t num_kv_heads;
  int32_t head_dim;     /* 64, 128 or 256 for attention; any 1..512 for append */
  uint8_t* key_valid;   /* [num_blocks * block_size] or NULL; 16-byte aligned */
  int32_t code_format;  /* astr_kv_format */
} astr_paged_kv;

/*
 * Quantize new K and V token rows to the arena's code format + fp32
 * per-(token, head) scales and write them into their cache slots.
 * Replaces quantize_kv (src/aster/optimization/kv_quantization.py:71-94) as
 * called from PagedStatePool._append_leaves (src/aster/inference/state.py:292)
 * plus its per-token raw copy_kv into page slot divmod(offset, block_size)
 * (state.py:339-344, kv_quantization.py:113-127).
 *   key/value: [num_tokens, num_kv_heads, head_dim] elements of `in_dtype`,
 *              strides in elements (last dim contiguous). value may be NULL
 *              to quantize key rows only (into k_codes/k_scales).
 *   slot_mapping: int64 [num_tokens], slot = block*block_size + offset;
 *              slot < 0 skips the token (padding).
 * Bit-exact with the reference: scale = amax==0 ? 1 : max(amax/M, FLT_MIN) and
 * c = clamp(x/scale, -M, M) with IEEE fp32 division (M the format's maximum); the
 * code is rint(c) (half to even) for int8, and c rounded to nearest-even FP8
 * (subnormals kept, -0 for negative underflow) for the FP8 formats, as torch's
 * float32 -> float8 conversion does.
 * All-or-nothing: a NaN/Inf anywhere in key/value sets
 * ASTR_FLAG_NONFINITE_INPUT and no slot is written (kv_quantization.py:77-81).
 * A set input-flag bit also suppresses later appends until cleared.
 */
int astr_kv_quantize_append_i8(const astr_paged_kv* cache, const void* key, const void* value,
                               int32_t in_dtype, int64_t num_tokens, int64_t key_token_stride,
                               int64_t key_head_stride, int64_t value_token_stride,
                               int64_t value_head_stride, const int64_t* slot_mapping,
                               int32_t* err_flag, void* stream);

/*
 * astr_kv_quantize_append_i8 in one launch instead of two, for slots the caller has
 * reserved and rolls back when the call is flagged: the same quantizer
 * (kv_quantization.py:71-94) and slot placement (state.py:339-344), with the
 * all-or-nothing rule of kv_quantization.py:77-81 / state.py:292 kept at the level
 * of the caller's transaction instead of the slots. Each (token, head, K|V) row
 * checks itself: a row holding a NaN/Inf sets ASTR_FLAG_NONFINITE_INPUT and is not
 * written; the call's other rows may be written. A set input-flag bit at launch
 * suppresses the rows that read it. The runner's step appends this way and aborts
 * every reservation of a flagged step, so the pool's visible state is unchanged, as
 * PagedStatePool.append_delta leaves it when quantize_kv raises.
 */
int astr_kv_quantize_append_i8_reserved(const astr_paged_kv* cache, const void* key,
                                        const void* value, int32_t in_dtype,
                                        int64_t num_tokens, int64_t key_token_stride,
                                        int64_t key_head_stride, int64_t value_token_stride,
                                        int64_t value_head_stride,
                                        const int64_t* slot_mapping, int32_t* err_flag,
                                        void* stream);

/*
 * Write the key-padding bytes of new tokens: key_valid[slot_mapping[i]] =
 * token_valid[i] != 0 (1 for every token when token_valid is NULL); slots < 0
 * are skipped, slots outside the arena raise ASTR_FLAG_BAD_INDEX. The padding
 * leaf of PagedStatePool._append_leaves (state.py:292, 339-344) as the runner
 * appends it (paged_attention.py:228-229), written once per step for all
 * layers. cache->key_valid must be set.
 */
int astr_kv_write_key_valid(const astr_paged_kv* cache, const int64_t* slot_mapping,
                            const uint8_t* token_valid, int64_t num_tokens, int32_t* err_flag,
                            void* stream);

/*
 * Ragged paged attention over the INT8 arena, one query token per sequence
 * (decode). Replaces the per-row online_attention call of
 * PagedAttentionRunner.forward_batch (src/aster/inference/paged_attention.py:168-215),
 * i.e. online_attention_statistics (src/aster/optimization/online_attention.py:74-214),
 * merge_softmax (:42-63) and SoftmaxState.output (:35-39), for all rows in one launch.
 *   query/out: [num_seqs, num_q_heads, head_dim] of q_dtype (out has the query
 *              dtype, online_attention.py:219); strides in elements.
 *   block_tables: int32 [num_seqs, block_table_stride] physical block ids.
 *   context_lens: int32 [num_seqs]; the query sits at position ctx-1 and sees
 *              keys 0..ctx-1 (ctx-window..ctx-1 when window > 0).
 *   GQA: query head h reads kv head h / (num_q_heads / num_kv_heads).
 *   max_context_len: host-side upper bound of context_lens (sizes the split-K grid).
 *   partition_tokens: 0 = automatic: bf16/fp16 queries with at most 512
 *              sequences use stream-K (equal block ranges per wave across
 *              rows, partials merged afterwards), everything else 512-token
 *              split-K partitions; > 0 forces fixed partitions of that many
 *              tokens (a multiple of 64, at most 4096).
 *   workspace: >= astr_paged_attention_i8_workspace_bytes(...) bytes of
 *              scratch for split-K partials, 256-byte aligned (NULL allowed
 *              when that size is 0); no initialisation needed. Calls sharing
 *              one workspace must be stream-ordered (concurrent calls race).
 * Launches the decode kernel and, when any row can span more than one
 * partition, the split-K merge kernel after it on the same stream.
 * Output rows with ctx == 0 are zero (fully-masked rows, online_attention.py:37).
 */
int astr_paged_attention_i8(const astr_paged_kv* cache, const void* query, int32_t q_dtype,
                            int64_t q_token_stride, int64_t q_head_stride, void* out,
                            int64_t out_token_stride, int64_t out_head_stride,
                            const int32_t* block_tables, int32_t block_table_stride,
                            const int32_t* context_lens, int32_t num_seqs, int32_t num_q_heads,
                            int32_t max_context_len, float scale, int32_t window,
                            int32_t partition_tokens, void* workspace, size_t workspace_bytes,
                            int32_t* err_flag, void* stream);

/*
 * The unnormalised softmax state of each decode row instead of its output: replaces
 * online_attention_statistics (src/aster/optimization/online_attention.py:74-214),
 * whose SoftmaxState (:29-39) is (maximum, mass, weighted) per query row and head.
 *   query: fp32 [num_seqs, num_q_heads, head_dim] (strides in elements).
 *   weighted: fp32 [num_seqs, num_q_heads, head_dim], sum over visible keys of
 *              exp(score - maximum) * value.
 *   stats: fp32 [num_seqs, num_q_heads, 2], 8-byte aligned: (maximum, mass) with
 *              maximum the largest visible score q.k * scale and mass the sum of
 *              exp(score - maximum); a row with no visible key gets (-inf, 0) and
 *              weighted 0 (the reference's initial state, online_attention.py:163-170).
 *   Other arguments as astr_paged_attention_i8, whose fixed-partition kernels in exact
 *   fp32 arithmetic serve this call (workspace sized by
 *   astr_paged_attention_i8_workspace_bytes).
 * weighted / max(mass, FLT_MIN) is the astr_paged_attention_i8 output up to the
 * rounding of the division; maximum + log(mass) is the row's log-sum-exp.
 */
int astr_paged_attention_i8_statistics(const astr_paged_kv* cache, const float* query,
                                       int64_t q_token_stride, int64_t q_head_stride,
                                       float* weighted, int64_t w_token_stride,
                                       int64_t w_head_stride, float* stats,
                                       const int32_t* block_tables, int32_t block_table_stride,
                                       const int32_t* context_lens, int32_t num_seqs,
                                       int32_t num_q_heads, int32_t max_context_len,
                                       float scale, int32_t window, int32_t partition_tokens,
                                       void* workspace, size_t workspace_bytes,
                                       int32_t* err_flag, void* stream);

/*
 * astr_paged_attention_i8 without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid allocation): no counterpart in the reference. The split-K partials live
 * in a 32 MiB device array that the library holds on every GPU it runs on until the
 * process ends; its address is looked up once per device, with that device current,
 * on the first call (make that first call outside graph capture). Same arguments,
 * kernels and results as astr_paged_attention_i8; a launch whose partials do not fit
 * returns ASTR_EINVAL (the stream-K path uses at most the waves that fit). Calls
 * on one GPU share the array and the last call's contents stay in it: calls that
 * overlap on one GPU (different streams without ordering) race. Nothing is allocated.
 */
int astr_paged_attention_i8_noalloc(const astr_paged_kv* cache, const void* query,
                                    int32_t q_dtype, int64_t q_token_stride,
                                    int64_t q_head_stride, void* out, int64_t out_token_stride,
                                    int64_t out_head_stride, const int32_t* block_tables,
                                    int32_t block_table_stride, const int32_t* context_lens,
                                    int32_t num_seqs, int32_t num_q_heads,
                                    int32_t max_context_len, float scale, int32_t window,
                                    int32_t partition_tokens, int32_t* err_flag, void* stream);

/*
 * Ragged paged attention for a continuous-batching step that mixes prompt
 * chunks (several query tokens per sequence, chunked prefill) with decode rows.
 * Replaces the same per-row online_attention calls of
 * PagedAttentionRunner.forward_batch (paged_attention.py:168-215) for chunks of
 * any length, with the visibility rules of online_attention_statistics
 * (online_attention.py:178-188).
 *   query/out: [num_query_tokens, num_q_heads, head_dim] packed by sequence.
 *   query_start_loc: int32 [num_seqs + 1] device offsets (cu_seqlens):
 *              sequence s owns token rows [qsl[s], qsl[s+1]); an entry that is
 *              negative, decreasing or beyond num_query_tokens raises
 *              ASTR_FLAG_BAD_INDEX and that sequence produces nothing.
 *   max_query_len: host-side upper bound of qsl[s+1]-qsl[s]; <= 1 launches the
 *              decode kernels only. A sequence with more query tokens than this
 *              bound raises ASTR_FLAG_BAD_INDEX and produces nothing.
 *   context_lens: int32 [num_seqs], counting the step's own tokens (the chunk
 *              is appended before attention). Query token i of a sequence with
 *              n query tokens sits at position ctx-n+i and sees key k iff
 *              k <= position (causal != 0; else k < ctx) and, when window > 0,
 *              k > position - window. ctx < n raises ASTR_FLAG_BAD_INDEX.
 *   Other arguments as astr_paged_attention_i8 (workspace sized by
 *   astr_paged_attention_i8_workspace_bytes for num_seqs rows; chunk rows need none).
 * Sequences with one query token take the decode kernels (the query sees every
 * key, as for astr_paged_attention_i8), longer ones the MFMA prefill kernel
 * (bf16/fp16/fp32 queries; with int8 codes a query column enters the int8 QK
 * MFMAs as integers within 1/2 of q * 16256 / max|q|, with FP8 codes it is
 * rounded to f16 after an exact power-of-two rescale), launched after the
 * decode kernels on the same stream.
 */
int astr_paged_attention_varlen_i8(const astr_paged_kv* cache, const void* query,
                                   int32_t q_dtype, int64_t q_token_stride,
                                   int64_t q_head_stride, void* out, int64_t out_token_stride,
                                   int64_t out_head_stride, const int32_t* query_start_loc,
                                   int32_t num_query_tokens, int32_t max_query_len,
                                   int32_t causal, const int32_t* block_tables,
                                   int32_t block_table_stride, const int32_t* context_lens,
                                   int32_t num_seqs, int32_t num_q_heads, int32_t max_context_len,
                                   float scale, int32_t window, int32_t partition_tokens,
                                   void* workspace, size_t workspace_bytes, int32_t* err_flag,
                                   void* stream);

/*
 * Workspace bytes astr_paged_attention_i8 needs for its split-K partials on
 * the current device (0 when no row can span more than one partition).
 * Analogue of KernelSpec.workspace_bytes (src/aster/core/contracts.py:102-134).
 */
size_t astr_paged_attention_i8_workspace_bytes(int32_t num_seqs, int32_t num_q_heads,
                                               int32_t num_kv_heads, int32_t head_dim,
                                               int32_t max_context_len,
                                               int32_t partition_tokens);

/*
 * astr_paged_attention_i8 (automatic split) for a decode batch whose block tables
 * alias shared prefix pages: the reference reads such pages once per row, as
 * PagedAttentionRunner.forward_batch does for the PrefixCache's shared page refs
 * (paged_attention.py:168-215 over state.py:599-625). `packs` is a host-built plan
 * of num_packs records of 1 + rows_per_pack int32 in device memory:
 *   [shared_blocks, member_0, ..., member_{rows_per_pack-1}]  (member -1: empty)
 * Every member's block table must begin with the same shared_blocks physical ids
 * (those of the first member), all of them visible (shared_blocks * 16 <= ctx).
 * The stream-K kernel reads each pack's blocks once for all its members, query
 * column p * G + g for head g of member p (2 <= rows_per_pack, rows_per_pack * G <=
 * 16), then each member's remaining blocks as its own row, and merges the two with
 * the split-K rule. Outputs are those of astr_paged_attention_i8 on the same
 * tables. At most 128 packs and 256 pack rows; window must be 0. A member that is
 * not a decode row, is listed twice or sees fewer than shared_blocks * 16 tokens
 * raises ASTR_FLAG_BAD_INDEX and is dropped from its pack. fp32 queries, batches
 * beyond 256 sequences and num_packs == 0 run astr_paged_attention_i8's kernels
 * without the plan. workspace: >=
 * astr_paged_attention_i8_shared_workspace_bytes(...) bytes, 256-byte aligned.
 */
int astr_paged_attention_i8_shared(const astr_paged_kv* cache, const void* query,
                                   int32_t q_dtype, int64_t q_token_stride,
                                   int64_t q_head_stride, void* out, int64_t out_token_stride,
                                   int64_t out_head_stride, const int32_t* block_tables,
                                   int32_t block_table_stride, const int32_t* context_lens,
                                   int32_t num_seqs, int32_t num_q_heads,
                                   int32_t max_context_len, float scale, int32_t window,
                                   const int32_t* packs, int32_t num_packs,
                                   int32_t rows_per_pack, void* workspace,
                                   size_t workspace_bytes, int32_t* err_flag, void* stream);

/* Workspace bytes of astr_paged_attention_i8_shared (no reference counterpart: the
 * pack plan is this library's). */
size_t astr_paged_attention_i8_shared_workspace_bytes(int32_t num_seqs, int32_t num_q_heads,
                                                      int32_t num_kv_heads, int32_t head_dim,
                                                      int32_t max_context_len,
                                                      int32_t num_packs,
                                                      int32_t rows_per_pack);

/*
 * A host-built schedule of a decode batch (astr_decode_plan): sizes and word offsets of
 * its int32 arrays. The plan itself is copied to device memory by the caller; this
 * struct stays on the host and is passed by pointer to the planned entry points.
 */
typedef struct astr_decode_plan_info {
  int32_t num_workgroups;       /* grid of the planned launch (one per resident slot) */
  int32_t waves_per_workgroup;
  int32_t num_items;            /* entries of the item table: (sequence, kv head) rows
                                   and row chunks, item_stride per workgroup */
  int32_t num_blocks;           /* blocks the plan streams (over all kv heads) */
  int32_t num_ids;              /* block ids it holds (each sequence's, once) */
  int32_t num_chunks;           /* chunk partial slots (rows split across workgroups) */
  int32_t num_chunked;          /* rows split across workgroups */
  int32_t num_seqs;
  int32_t num_kv_heads;
  int32_t window;
  int32_t tail_blocks;          /* blocks at the end of each wave's range that it loads
                                   two at a time (0: one at a time throughout) */
  int32_t item_stride;          /* item-table entries per workgroup */
  int32_t num_tiles;            /* prefix tiles: (shared prefix, kv head, key range) */
  int32_t tile_rows;            /* sequences per prefix tile at most */
  int32_t tile_ranges;          /* key ranges of each shared prefix */
  int32_t num_tile_members;     /* sequences read through a prefix tile */
  int64_t off_workgroups, off_waves, off_items, off_ids, off_chunked, off_tiles,
      off_tile_members;
  int64_t plan_words;           /* int32 words of the plan */
} astr_decode_plan_info;

/*
 * Resident workgroups of the planned decode kernel on the current device (the
 * num_workgroups to plan for) and its waves per workgroup, for this head dim, GQA
 * group, query dtype and code format. No reference counterpart: the reference has no
 * device schedule.
 */
int astr_decode_plan_workgroups(int32_t head_dim, int32_t num_q_heads, int32_t num_kv_heads,
                                int32_t q_dtype, int32_t code_format, int32_t* num_workgroups,
                                int32_t* waves_per_workgroup);

/* Upper bound of the int32 words of a plan (visible_blocks: sum over sequences;
 * tile_rows as passed to astr_decode_plan). */
int64_t astr_decode_plan_words_bound(int32_t num_seqs, int32_t num_kv_heads,
                                     int64_t visible_blocks, int32_t num_workgroups,
                                     int32_t waves_per_workgroup, int32_t tile_rows);

/*
 * Builds, on the host, the schedule of a decode batch: the same work as
 * astr_paged_attention_i8 over these HOST block tables and context lengths (the
 * per-row online_attention calls of PagedAttentionRunner.forward_batch,
 * paged_attention.py:168-215, as the runner holds the rows' page lists on the host,
 * state.py:358-390). Each (sequence, kv head) row's visible blocks become an item;
 * items go to workgroups longest first onto the least loaded (rows costing more than
 * a workgroup's share are cut into chunks), and each workgroup's blocks are cut into
 * equal-cost ranges, one per wave. A plan holds the physical block ids, so it is
 * valid for these tables and lengths only (one plan per decode step serves every
 * layer). plan == NULL only sizes it (info->plan_words). Host memory only; nothing
 * is launched.
 * Shared prefixes (the pages PrefixCache hands to several sequences, state.py:547-640,
 * forked at state.py:210-216): with tile_rows >= 2, sequences whose tables begin with
 * the same min_shared_blocks blocks or more, all of them visible, are read in prefix
 * tiles of up to tile_rows sequences (tile_rows * G <= the prefix-tile kernel's
 * columns: 128 at head dims up to 128, 64 at 256), each kv head's shared blocks cut
 * into tile_ranges key ranges (0: chosen from the workgroup count); the rows' own
 * blocks remain items. tile_rows = 0 plans no tiles.
 */
int astr_decode_plan(const int32_t* block_tables, int32_t block_table_stride,
                     const int32_t* context_lens, int32_t num_seqs, int32_t num_kv_heads,
                     int32_t window, int32_t num_workgroups, int32_t waves_per_workgroup,
                     int32_t tile_rows, int32_t tile_ranges, int32_t min_shared_blocks,
                     int32_t* plan, int64_t plan_words, astr_decode_plan_info* info);

/* Workspace bytes of astr_paged_attention_i8_planned for this plan. */
size_t astr_paged_attention_i8_planned_workspace_bytes(const astr_decode_plan_info* info,
                                                       int32_t num_q_heads, int32_t head_dim);

/*
 * astr_paged_attention_i8 (decode rows, bf16/fp16 queries) on a plan from
 * astr_decode_plan: no device-side split, and the pieces of a row that several waves
 * of one workgroup hold are merged by that workgroup after its waves finish, so no
 * merge kernel runs unless the plan cut a row across workgroups. Same outputs as
 * astr_paged_attention_i8 on the tables the plan was built from.
 *   plan: the plan's int32 words in device memory (info->plan_words, 4-byte aligned);
 *         info: its host record. The plan is untrusted: every index read from it is
 *         checked (block ids against the arena, items against the batch, context
 *         lengths against context_lens); a workgroup whose part fails a check writes
 *         nothing and raises ASTR_FLAG_BAD_INDEX.
 *   context_lens: int32 [num_seqs] device lengths, which the plan's must equal.
 *   query/out: [num_seqs, num_q_heads, head_dim], strides in elements (token row s is
 *         sequence s).
 *   workspace: >= astr_paged_attention_i8_planned_workspace_bytes(info, ...) bytes,
 *         256-byte aligned.
 */
int astr_paged_attention_i8_planned(const astr_paged_kv* cache, const void* query,
                                    int32_t q_dtype, int64_t q_token_stride,
                                    int64_t q_head_stride, void* out, int64_t out_token_stride,
                                    int64_t out_head_stride, const int32_t* context_lens,
                                    int32_t num_q_heads, float scale, const int32_t* plan,
                                    const astr_decode_plan_info* info, void* workspace,
                                    size_t workspace_bytes, int32_t* err_flag, void* stream);

/*
 * astr_kv_quantize_append_i8_reserved and astr_paged_attention_i8_planned in one
 * launch: the decode step of PagedAttentionRunner.forward_batch with its chunk's
 * quantize-then-append (paged_attention.py:185-192, 226-229; quantize_kv,
 * kv_quantization.py:71-94) folded into the attention. Each sequence's newest token
 * (position ctx - 1, one per decode row) comes as key/value rows of the query dtype
 * (bf16/fp16): [num_seqs, num_kv_heads, head_dim], strides in elements (even), rows
 * 4-byte aligned; slot_mapping: int64 [num_seqs] device slots the caller reserved
 * (8-byte aligned). The wave that streams the block holding the token quantizes it
 * (the quantizer's arithmetic, bit for bit), writes the codes and scales into the
 * arena at slot_mapping[s] and into its copy of the block, so the call's outputs and
 * the arena after it equal the two calls'. A slot that is not the plan's position of
 * the token (block id of position ctx - 1 times 16 plus (ctx - 1) mod 16) raises
 * ASTR_FLAG_BAD_INDEX (the token is still written at slot_mapping[s] when that lies in
 * the arena); a token holding a NaN/Inf raises ASTR_FLAG_NONFINITE_INPUT and is not
 * written, the call's other tokens may be: the caller rolls back reserved slots on a
 * flagged call, as for astr_kv_quantize_append_i8_reserved. Plans from
 * astr_decode_plan keep each newest token's block out of prefix tiles and out of the
 * blocks a wave issues from its entry. Each newest token's block must be its own
 * sequence's (no other row's table holds it), as the runner's copy-on-write
 * reservations make it (state.py:306-310, 330-337): another row reading that block
 * would see it as it was before the call. Other arguments as
 * astr_paged_attention_i8_planned.
 */
int astr_paged_attention_i8_planned_append(
    const astr_paged_kv* cache, const void* query, int32_t q_dtype, int64_t q_token_stride,
    int64_t q_head_stride, void* out, int64_t out_token_stride, int64_t out_head_stride,
    const void* key, const void* value, int64_t key_token_stride, int64_t key_head_stride,
    int64_t value_token_stride, int64_t value_head_stride, const int64_t* slot_mapping,
    const int32_t* context_lens, int32_t num_q_heads, float scale, const int32_t* plan,
    const astr_decode_plan_info* info, void* workspace, size_t workspace_bytes,
    int32_t* err_flag, void* stream);

/*
 * Bit-exact copy of whole blocks: block i of `num_blocks` goes from
 *   src + (src_index ? src_index[i] : i) * src_stride
 * to
 *   dst + (dst_index ? dst_index[i] : i) * dst_stride   (block_bytes bytes each).
 * Replaces the raw page copies of copy_kv (src/aster/optimization/kv_quantization.py:113-127)
 * as used for copy-on-write of a shared tail page (src/aster/inference/state.py:330-337)
 * and for page transfers in restore_pages / PagedStateArchive (state.py:427-493,
 * src/aster/inference/offload.py:140-190): one launch per array (codes, scales)
 * moves every block of a step; gather (src_index) into a staging buffer and
 * scatter (dst_index) out of one are the two halves of host swap.
 *   src_index/dst_index: int32 device arrays of num_blocks entries, or NULL for
 *              identity; an entry outside [0, src_blocks) / [0, dst_blocks) raises
 *              ASTR_FLAG_BAD_INDEX and that block is not copied.
 *   Blocks of one call must not overlap between source and destination.
 * 16-byte vector copies when pointers, strides and block_bytes are multiples of 16.
 */
int astr_kv_copy_blocks(const void* src, int64_t src_stride, const int32_t* src_index,
                        int32_t src_blocks, void* dst, int64_t dst_stride,
                        const int32_t* dst_index, int32_t dst_blocks, int64_t block_bytes,
                        int32_t num_blocks, int32_t* err_flag, void* stream);

/*
 * merge_softmax of two fp32 softmax states over disjoint key partitions of the same
 * queries (src/aster/optimization/online_attention.py:42-63): maximum M = max(m_l, m_r)
 * (NaN propagates), weights exp(m - M) for finite m and 0 otherwise (M replaced by 0
 * when it is not finite), mass and weighted numerator summed under those weights.
 *   *_max, *_mass: [rows] contiguous; *_weighted: [rows, width] contiguous, device
 *   memory. The outputs must not overlap any input or each other (ASTR_EINVAL): the
 *   threads of a row read both maxima while one of them writes the merged maximum.
 */
int astr_merge_softmax_f32(const float* left_max, const float* left_mass,
                           const float* left_weighted, const float* right_max,
                           const float* right_mass, const float* right_weighted,
                           float* out_max, float* out_mass, float* out_weighted, int64_t rows,
                           int32_t width, void* stream);

/* Thread-local description of the last non-zero return code. */
const char* astr_last_error(void);

/* Library version string ("aster_kv <semver> gfx950"). */
const char* astr_version(void);

#ifdef __cplusplus
}
#endif

#endif /* ASTER_KV_H */
