// Host-side schedule of a decode batch for decode_planned_kernel (decode_planned.hip).
//
// The work of a decode step is one item per (sequence, kv head): the row's visible
// blocks. The planner knows every row's length on the host (the runner built the block
// tables there) and settles the whole split before the launch, so that no workgroup
// spends the start of the kernel on it:
//   * items whose cost passes the per-workgroup share are cut into equal chunks;
//   * items and chunks go to workgroups longest first, each to the least loaded one
//     (LPT), one workgroup per resident slot of the GPU (a single round);
//   * inside a workgroup the items' blocks are laid end to end and cut into one equal
//     range per wave. Pieces of an item that two or more of the workgroup's waves hold
//     are merged in that workgroup after its waves finish; chunks of an item that two
//     or more workgroups hold are merged by the chunk-merge kernel.
// The cost model: 50 per block and 200 per row start (a row's query load, the partial
// it writes when it ends and, in a step that appends, its newest token; measured on the
// planned kernel, config 2 and config 4 steps ran 0.5 and 0.9 us faster at 200 than at
// the stream-K kernel's 135, with the attention-only calls unchanged, and 260 slower).
//
// Shared prefixes (tile_rows >= 2): sequences whose block tables begin with the same
// blocks, every key of them visible to each, are read together by the prefix-tile
// kernel (prefill.hip): a tile holds up to tile_rows such sequences (tile_rows * G
// query columns, one MFMA column tile of the chunked-prefill kernel) and covers, per kv
// head, one of tile_ranges equal ranges of their shared blocks. Each member row's
// partials (one per range, then its own blocks' chunks) take consecutive chunk slots;
// its own blocks are an item like any row's. Where they are one item, that item's
// workgroup merges its partial (the slot after the ranges') with the ranges' (the tile
// kernel runs first) into the row's output (out = -2 - the first range's slot); else
// the chunk-merge kernel does.
//
// Plan layout (int32 words, offsets in astr_decode_plan_info):
//   workgroups  [num_workgroups][waves + 3]: first item, end item, then waves + 1 bounds
//               of the workgroup's block list: wave w streams its blocks [bound[w],
//               bound[w + 1]) (positions counted from the workgroup's first block)
//   waves       [num_workgroups * waves][6]: the wave's first piece (sequence, kv head),
//               how many of its first blocks follow (up to 2, all of that piece) and
//               their physical ids, so that the wave issues them before it reads its
//               items
//   items       [num_workgroups][item_stride][8] (workgroup g's items at g * item_stride,
//               so a workgroup loads them without its record): sequence, kv head, first
//               block within the sequence's
//               block table, blocks, context length, output (-1: the output row; c >= 0:
//               the chunk slot of its partial; -2 - c: the output row, through the
//               tile_ranges + 1 chunk slots from c: the ranges' partials, then its own),
//               position of its first block in the workgroup's list, offset of its first
//               block id in `ids`
//   ids         [num_ids]: the physical ids of every sequence's visible blocks, once per
//               sequence (the items of its kv heads and chunks point into them)
//   chunked     [num_chunked][4]: sequence, kv head, first chunk slot, chunks
//   tiles       [num_tiles][8]: first member (index into tile members), members, kv
//               head, range, first block, blocks, offset of the first block's id in
//               `ids`, the sequence whose ids those are
//   tile members [num_tile_members][3]: sequence, its first chunk slot (kv head h,
//               range r: slot + h * span + r), span (slots per kv head: ranges, then
//               the chunks of its own blocks)
#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <vector>

#include "aster_kv.h"

namespace astr {
int fail(int code, const char* fmt, ...);

namespace plan {

constexpr int kBlockTokens = 16;
constexpr int64_t kBlockCost = 50, kRowCost = 200;
constexpr int kItemWords = 8, kChunkedWords = 4, kTileWords = 8, kMemberWords = 3;
constexpr int kWaveWords = 6;
// first blocks a wave issues from its entry (of the entry's 3 id slots): two measured
// as fast as three on configs 2 and 5 (62.0-62.6 against 62.9 us on config 2), with a
// smaller burst at the kernel's start
constexpr int kPrefetchBlocks = 2;
constexpr int kMaxItemsPerWorkgroup = 64;  // the kernel's LDS item table
constexpr int kMaxBlocksPerWave = 1024;    // the kernel's block list windows
constexpr int kMaxTileRanges = 16;
constexpr int kMinTileRangeBlocks = 8;     // automatic ranges: at least two key steps each

struct Unit {
  int seq, kvh, blk_begin, nblk, ctx, out, ids_off;
  int64_t cost;
  bool member;  // the row's shared prefix is a tile's
};

int64_t words_for(int64_t workgroups, int waves, int64_t items, int64_t ids, int64_t chunked,
                  int64_t tiles, int64_t members) {
  return workgroups * (waves + 3) + workgroups * waves * kWaveWords + items * kItemWords + ids +
         chunked * kChunkedWords +
         tiles * kTileWords + members * kMemberWords;
}

}  // namespace plan
}  // namespace astr

using namespace astr::plan;

extern "C" int64_t astr_decode_plan_words_bound(int32_t num_seqs, int32_t num_kv_heads,
                                                int64_t visible_blocks, int32_t num_workgroups,
                                                int32_t waves_per_workgroup, int32_t tile_rows) {
  if (num_seqs < 0 || num_kv_heads < 1 || visible_blocks < 0 || num_workgroups < 1 ||
      waves_per_workgroup < 1 || tile_rows < 0)
    return 0;
  // items: at most kMaxItemsPerWorkgroup per workgroup, at a common stride; every row
  // may be chunked; a tile holds two sequences at least, and each sequence is a member
  // of one tile at most
  const int64_t rows = (int64_t)num_seqs * num_kv_heads;
  const int64_t items = (int64_t)num_workgroups * kMaxItemsPerWorkgroup;
  const int64_t tiles = tile_rows >= 2 ? (int64_t)(num_seqs / 2) * num_kv_heads * kMaxTileRanges : 0;
  const int64_t members = tile_rows >= 2 ? num_seqs : 0;
  return words_for(num_workgroups, waves_per_workgroup, items, visible_blocks, rows, tiles,
                   members);
}

extern "C" int astr_decode_plan(const int32_t* block_tables, int32_t block_table_stride,
                                const int32_t* context_lens, int32_t num_seqs,
                                int32_t num_kv_heads, int32_t window, int32_t num_workgroups,
                                int32_t waves_per_workgroup, int32_t tile_rows,
                                int32_t tile_ranges, int32_t min_shared_blocks, int32_t* plan,
                                int64_t plan_words, astr_decode_plan_info* info) {
  using astr::fail;
  if (info == nullptr || (num_seqs > 0 && (block_tables == nullptr || context_lens == nullptr)))
    return fail(ASTR_EINVAL, "plan: block_tables, context_lens and info are required");
  if (num_seqs < 0 || num_kv_heads < 1 || block_table_stride < 0 || window < 0 ||
      num_workgroups < 1 || waves_per_workgroup < 1 || waves_per_workgroup > 16 ||
      tile_rows < 0 || tile_ranges < 0 || tile_ranges > kMaxTileRanges || min_shared_blocks < 0)
    return fail(ASTR_EINVAL, "plan: invalid sizes");
  std::memset(info, 0, sizeof(*info));
  const int NW = waves_per_workgroup;
  // ---- rows: visible blocks of every sequence (the kernels' row_span)
  std::vector<int64_t> row_ids(num_seqs);  // offset of sequence s's visible ids
  std::vector<int> first_blk(num_seqs), last_blk(num_seqs);
  int64_t visible = 0;
  for (int s = 0; s < num_seqs; ++s) {
    const int ctx = context_lens[s];
    if (ctx < 0 || (int64_t)ctx > (int64_t)block_table_stride * kBlockTokens)
      return fail(ASTR_EINVAL, "plan: context length %d of sequence %d outside its block table",
                  ctx, s);
    const int kv_begin = (window > 0 && ctx > window) ? ctx - window : 0;
    first_blk[s] = kv_begin / kBlockTokens;
    last_blk[s] = (ctx + kBlockTokens - 1) / kBlockTokens;
    row_ids[s] = visible;
    visible += last_blk[s] - first_blk[s];
  }
  if (visible > INT32_MAX / 2) return fail(ASTR_EUNSUPPORTED, "plan: batch too large");
  // ---- shared prefixes: sequences that see every key of their first blocks, grouped
  // by their first block's id; within a group, each sequence's run of leading blocks
  // equal to the group leader's (the first sequence of the group), longest runs first,
  // cut into tiles of tile_rows; a tile shares the shortest run of its members (a tile
  // sharing fewer than min_shared_blocks ends its group)
  struct Tile {
    int lead, shared, m0, n;
  };
  std::vector<Tile> tiles;
  std::vector<int> tile_seqs;           // members of tile t at [m0, m0 + n)
  std::vector<int> shared_of(num_seqs, 0);
  if (tile_rows >= 2 && min_shared_blocks >= 1 && block_table_stride > 0) {
    std::vector<int> cand;
    for (int s = 0; s < num_seqs; ++s)
      if (first_blk[s] == 0 && context_lens[s] / kBlockTokens >= min_shared_blocks) cand.push_back(s);
    std::stable_sort(cand.begin(), cand.end(), [&](int x, int y) {
      return block_tables[(int64_t)x * block_table_stride] < block_tables[(int64_t)y * block_table_stride];
    });
    std::vector<int> common(num_seqs, 0);
    for (size_t g0 = 0; g0 < cand.size();) {
      const int32_t id0 = block_tables[(int64_t)cand[g0] * block_table_stride];
      size_t g1 = g0 + 1;
      while (g1 < cand.size() && block_tables[(int64_t)cand[g1] * block_table_stride] == id0) ++g1;
      if (g1 - g0 >= 2) {
        const int lead = cand[g0];
        const int32_t* lt = block_tables + (int64_t)lead * block_table_stride;
        const int lead_full = context_lens[lead] / kBlockTokens;
        std::vector<int> group(cand.begin() + g0, cand.begin() + g1);
        for (int s : group) {
          const int32_t* st = block_tables + (int64_t)s * block_table_stride;
          // whole blocks before the one of the newest token (position ctx - 1), which
          // stays the row's own (an appending decode writes it in that row's block)
          const int reach = std::min((context_lens[s] - 1) / kBlockTokens, lead_full);
          common[s] = (int)(std::mismatch(st, st + reach, lt).first - st);
        }
        std::stable_sort(group.begin(), group.end(), [&](int x, int y) { return common[x] > common[y]; });
        for (size_t t0 = 0; t0 + 1 < group.size(); t0 += tile_rows) {
          const size_t t1 = std::min(group.size(), t0 + (size_t)tile_rows);
          int shared = INT32_MAX;
          for (size_t i = t0; i < t1; ++i) shared = std::min(shared, common[group[i]]);
          if (shared < min_shared_blocks) break;  // later tiles share even less
          tiles.push_back(Tile{lead, shared, (int)tile_seqs.size(), (int)(t1 - t0)});
          for (size_t i = t0; i < t1; ++i) {
            tile_seqs.push_back(group[i]);
            shared_of[group[i]] = shared;
          }
        }
      }
      g0 = g1;
    }
  }
  int ranges = 0;
  if (!tiles.empty()) {
    int least = INT32_MAX;  // the shortest shared run: every range holds a block at least
    for (const Tile& t : tiles) least = std::min(least, t.shared);
    if (tile_ranges > 0) {
      ranges = std::min(tile_ranges, least);
    } else {  // about one tile per resident workgroup of the decode kernel
      const int64_t per_range = (int64_t)tiles.size() * num_kv_heads;
      ranges = (int)std::max<int64_t>(1, num_workgroups / per_range);
      ranges = std::min({ranges, kMaxTileRanges, std::max(1, least / kMinTileRangeBlocks)});
    }
  }
  // ---- items: every row's visible blocks after its shared prefix
  std::vector<Unit> units;
  units.reserve((size_t)num_seqs * num_kv_heads);
  int64_t total_cost = 0;
  for (int s = 0; s < num_seqs; ++s) {
    const int b0 = first_blk[s] + shared_of[s], nb = last_blk[s] - b0;
    for (int h = 0; h < num_kv_heads; ++h) {
      const int64_t cost = nb > 0 ? kBlockCost * nb + kRowCost : 0;
      units.push_back(Unit{s, h, b0, nb, context_lens[s], -1, (int)(row_ids[s] + shared_of[s]),
                           cost, shared_of[s] > 0});
      total_cost += cost;
    }
  }
  // ---- chunks: an item costing more than the per-workgroup share is cut evenly; a
  // member row's slots are its ranges' partials, then its chunks (all its kv heads'
  // slots together, span per head)
  const double share = std::max(1.0, (double)total_cost / num_workgroups);
  std::vector<Unit> work;
  work.reserve(units.size());
  std::vector<int32_t> chunked;  // [seq, kvh, first slot, chunks]
  std::vector<int> member_c0(num_seqs, -1), member_span(num_seqs, 0);
  int64_t chunk_slots = 0;
  for (const Unit& u : units) {
    int k = 1;
    if (u.nblk > 1 && (double)u.cost > share) {
      k = (int)std::ceil((double)u.cost / share);
      k = std::min(k, u.nblk);
    }
    if (!u.member && k == 1) {
      work.push_back(u);
      continue;
    }
    int64_t c0 = chunk_slots;
    int lead_slots = 0;  // the ranges' slots before the chunks
    if (u.member) {
      if (u.nblk == 0) k = 0;  // the prefix is the whole row
      if (u.kvh == 0) {
        member_c0[u.seq] = (int)chunk_slots;
        member_span[u.seq] = ranges + k;
        chunk_slots += (int64_t)num_kv_heads * (ranges + k);
      }
      c0 = member_c0[u.seq] + (int64_t)u.kvh * member_span[u.seq];
      lead_slots = ranges;
      if (k == 1) {  // merged by its workgroup: no chunk-merge record
        Unit whole = u;
        whole.out = (int)(-2 - c0);
        work.push_back(whole);
        continue;
      }
    } else {
      chunk_slots += k;
    }
    chunked.insert(chunked.end(), {u.seq, u.kvh, (int32_t)c0, lead_slots + k});
    for (int c = 0; c < k; ++c) {
      const int b0 = (int)((int64_t)u.nblk * c / k), b1 = (int)((int64_t)u.nblk * (c + 1) / k);
      Unit part = u;
      part.blk_begin = u.blk_begin + b0;
      part.nblk = b1 - b0;
      part.ids_off = u.ids_off + b0;
      part.out = (int)(c0 + lead_slots + c);
      part.cost = kBlockCost * part.nblk + kRowCost;
      work.push_back(part);
    }
    if (chunk_slots > INT32_MAX / 2) return fail(ASTR_EUNSUPPORTED, "plan: batch too large");
  }
  // ---- LPT: longest first onto the least loaded workgroup (ties: lowest index); the
  // units then laid out per workgroup in that order (placed[off[g] .. off[g + 1]))
  std::vector<std::pair<int64_t, int>> order(work.size());  // (-cost, index): stable
  for (size_t i = 0; i < work.size(); ++i) order[i] = {-work[i].cost, (int)i};
  std::sort(order.begin(), order.end());
  // a binary min-heap of (cost, workgroup): the top takes the unit, then sinks
  typedef std::pair<int64_t, int> Load;
  std::vector<Load> heap(num_workgroups);
  for (int g = 0; g < num_workgroups; ++g) heap[g] = Load{0, g};  // already a heap
  std::vector<int> owner(work.size());
  std::vector<int64_t> off(num_workgroups + 1, 0);
  const size_t nh = heap.size();
  for (const auto& o : order) {
    owner[o.second] = heap[0].second;
    ++off[heap[0].second + 1];
    heap[0].first += work[o.second].cost;
    for (size_t i = 0;;) {
      const size_t l = 2 * i + 1;
      if (l >= nh) break;
      const size_t c = l + 1 < nh && heap[l + 1] < heap[l] ? l + 1 : l;
      if (!(heap[c] < heap[i])) break;
      std::swap(heap[c], heap[i]);
      i = c;
    }
  }
  int64_t stride = 1;  // items of the fullest workgroup
  for (int g = 0; g < num_workgroups; ++g) {
    stride = std::max(stride, off[g + 1]);
    off[g + 1] += off[g];
  }
  std::vector<Unit> placed(work.size());
  {
    std::vector<int64_t> next(off.begin(), off.end() - 1);
    for (const auto& o : order) placed[next[owner[o.second]]++] = work[o.second];
  }
  // ---- sizes and layout
  const int64_t num_items = stride * num_workgroups;
  int64_t num_blocks = 0;
  for (const Unit& u : work) num_blocks += u.nblk;
  const int64_t num_chunked = (int64_t)chunked.size() / kChunkedWords;
  const int64_t num_tiles = (int64_t)tiles.size() * num_kv_heads * ranges;
  const int64_t num_members = (int64_t)tile_seqs.size();
  const int64_t need = words_for(num_workgroups, NW, num_items, visible, num_chunked, num_tiles,
                                 num_members);
  if (num_items > INT32_MAX / kItemWords || num_blocks > INT32_MAX / 4)
    return fail(ASTR_EUNSUPPORTED, "plan: batch too large");
  if (stride > kMaxItemsPerWorkgroup)
    return fail(ASTR_EUNSUPPORTED, "plan: %lld items on one workgroup (at most %d)",
                (long long)stride, kMaxItemsPerWorkgroup);
  info->num_workgroups = num_workgroups;
  info->waves_per_workgroup = NW;
  info->num_items = (int32_t)num_items;
  info->item_stride = (int32_t)stride;
  info->num_blocks = (int32_t)num_blocks;
  info->num_ids = (int32_t)visible;
  info->num_chunks = chunk_slots;
  info->num_chunked = (int32_t)num_chunked;
  info->num_seqs = num_seqs;
  info->num_kv_heads = num_kv_heads;
  info->window = window;
  info->off_workgroups = 0;
  info->off_waves = (int64_t)num_workgroups * (NW + 3);
  info->off_items = info->off_waves + (int64_t)num_workgroups * NW * kWaveWords;
  info->off_ids = info->off_items + num_items * kItemWords;
  info->off_chunked = info->off_ids + visible;
  info->num_tiles = (int32_t)num_tiles;
  info->tile_rows = num_tiles > 0 ? tile_rows : 0;
  info->tile_ranges = ranges;
  info->num_tile_members = (int32_t)num_members;
  info->off_tiles = info->off_chunked + num_chunked * kChunkedWords;
  info->off_tile_members = info->off_tiles + num_tiles * kTileWords;
  info->plan_words = need;
  if (plan == nullptr) return 0;  // sizing call
  if (plan_words < need)
    return fail(ASTR_EINVAL, "plan: %lld words given, %lld needed", (long long)plan_words,
                (long long)need);
  int32_t* wgt = plan + info->off_workgroups;
  int32_t* items = plan + info->off_items;
  int32_t* ids = plan + info->off_ids;
  std::memset(items, 0, (size_t)num_items * kItemWords * sizeof(int32_t));
  for (int s = 0; s < num_seqs; ++s) {  // every sequence's visible ids, once
    const int ctx = context_lens[s];
    const int kv_begin = (window > 0 && ctx > window) ? ctx - window : 0;
    const int first = kv_begin / kBlockTokens, last = (ctx + kBlockTokens - 1) / kBlockTokens;
    if (last > first)
      std::memcpy(ids + row_ids[s], block_tables + (int64_t)s * block_table_stride + first,
                  (size_t)(last - first) * sizeof(int32_t));
  }
  int64_t most_per_wave = 0;
  for (int g = 0; g < num_workgroups; ++g) {
    int32_t* rec = wgt + (int64_t)g * (NW + 3);
    int64_t item = g * stride;
    rec[0] = (int32_t)item;
    int64_t pos = 0, g_cost = 0;
    const Unit* const mine = placed.data() + off[g];
    const size_t cnt = (size_t)(off[g + 1] - off[g]);
    for (size_t q = 0; q < cnt; ++q) {
      const Unit& u = mine[q];
      int32_t* it = items + item * kItemWords;
      it[0] = u.seq;
      it[1] = u.kvh;
      it[2] = u.blk_begin;
      it[3] = u.nblk;
      it[4] = u.ctx;
      it[5] = u.out;
      it[6] = (int32_t)pos;
      it[7] = u.ids_off;
      pos += u.nblk;
      g_cost += u.cost;
      ++item;
    }
    rec[1] = (int32_t)item;
    // equal-cost wave ranges: block b of an item starts at the cost of the items before
    // it, plus a row start, plus b blocks; wave w takes the blocks whose start lies in
    // [C w / NW, C (w + 1) / NW). Bound w is the first block starting at or after
    // ceil(C w / NW).
    int32_t* bound = rec + 2;
    bound[0] = 0;
    bound[NW] = (int32_t)pos;
    size_t k = 0;
    int64_t k_cost = 0, k_pos = 0;  // cost and position at the start of member k
    for (int w = 1; w < NW; ++w) {
      const int64_t target = (g_cost * w + NW - 1) / NW;
      // skip members whose last block starts before the target
      while (k < cnt) {
        const Unit& u = mine[k];
        if (u.nblk > 0 && k_cost + kRowCost + kBlockCost * (u.nblk - 1) >= target) break;
        k_cost += u.cost;
        k_pos += u.nblk;
        ++k;
      }
      int64_t b = k_pos;
      if (k < cnt) {
        const int64_t over = target - k_cost - kRowCost;
        b += over <= 0 ? 0 : (over + kBlockCost - 1) / kBlockCost;
      }
      bound[w] = (int32_t)b;
    }
    for (int w = 0; w < NW; ++w) most_per_wave = std::max<int64_t>(most_per_wave, bound[w + 1] - bound[w]);
    // each wave's first piece and the ids of its first blocks
    int32_t* went = plan + info->off_waves + (int64_t)g * NW * kWaveWords;
    std::memset(went, 0, (size_t)NW * kWaveWords * sizeof(int32_t));
    size_t m = 0;
    int64_t m_pos = 0;  // position of member m's first block
    for (int w = 0; w < NW; ++w, went += kWaveWords) {
      const int64_t b0 = bound[w], b1 = bound[w + 1];
      if (b1 <= b0) continue;
      while (m < cnt && m_pos + mine[m].nblk <= b0) {
        m_pos += mine[m].nblk;
        ++m;
      }
      const Unit& u = mine[m];
      int64_t c = std::min<int64_t>({kPrefetchBlocks, b1 - b0, m_pos + u.nblk - b0});
      // not the block of the row's newest token: an appending decode stages the token
      // with that block, after the wave has its items
      const int64_t newest = u.ctx > 0 ? (u.ctx - 1) / kBlockTokens - (u.blk_begin + b0 - m_pos) : -1;
      if (newest >= 0) c = std::min(c, newest);
      went[0] = u.seq;
      went[1] = u.kvh;
      went[2] = (int32_t)c;
      for (int64_t j = 0; j < c; ++j) went[3 + j] = ids[u.ids_off + (b0 - m_pos) + j];
    }
  }
  if (most_per_wave > kMaxBlocksPerWave)
    return fail(ASTR_EUNSUPPORTED, "plan: %lld blocks on one wave (at most %d): launch more "
                "workgroups", (long long)most_per_wave, kMaxBlocksPerWave);
  std::memcpy(plan + info->off_chunked, chunked.data(), chunked.size() * sizeof(int32_t));
  // tiles by (kv head, range, tile): the tiles reading the same blocks are consecutive
  // (the tile kernel runs consecutive tiles on one XCD)
  int32_t* trec = plan + info->off_tiles;
  for (int h = 0; h < num_kv_heads; ++h)
    for (int r = 0; r < ranges; ++r)
      for (const Tile& t : tiles) {
        const int b0 = (int)((int64_t)t.shared * r / ranges);
        const int b1 = (int)((int64_t)t.shared * (r + 1) / ranges);
        const int32_t rec[kTileWords] = {t.m0, t.n, h, r, b0, b1 - b0,
                                         (int32_t)(row_ids[t.lead] + b0), t.lead};
        std::memcpy(trec, rec, sizeof(rec));
        trec += kTileWords;
      }
  int32_t* mrec = plan + info->off_tile_members;
  for (int s : tile_seqs) {
    mrec[0] = s;
    mrec[1] = member_c0[s];
    mrec[2] = member_span[s];
    mrec += kMemberWords;
  }
  return 0;
}
