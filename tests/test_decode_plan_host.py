"""The host planner of the planned decode kernel (astr_decode_plan, C++): on random
batches its plan covers every visible block of every (sequence, kv head) row exactly
once with the row's physical ids (through a prefix tile for the shared blocks of
sequences whose tables begin alike), cuts only rows costing more than a workgroup's
share, balances workgroups within one item of the mean (LPT) and waves within one block
and one row start, gives every partial its own chunk slot, and refuses what the kernel
cannot take. No GPU: host memory only."""

import ctypes

import numpy as np
import pytest

from aster_amd import _native
from aster_amd.decode_plan import DecodePlanInfo

I32P = ctypes.POINTER(ctypes.c_int32)
BLOCK_COST, ROW_COST = 50, 200  # the planner's cost model (decode_plan.cpp)


def _plan(tables, lens, hkv, window, wg, nw=8, tile_rows=0, tile_ranges=0, min_shared=8):
    lib = _native.lib()
    tables = np.ascontiguousarray(tables, np.int32)
    lens = np.ascontiguousarray(lens, np.int32)
    ctx = lens.astype(np.int64)
    first = np.where((window > 0) & (ctx > window), ctx - window, 0) // 16
    visible = int(np.maximum(-(-ctx // 16) - first, 0).sum())
    bound = lib.astr_decode_plan_words_bound(len(lens), hkv, visible, wg, nw, tile_rows)
    buf = np.zeros(max(bound, 1), np.int32)
    info = DecodePlanInfo()
    rc = lib.astr_decode_plan(tables.ctypes.data_as(I32P), tables.shape[1],
                              lens.ctypes.data_as(I32P), len(lens), hkv, window, wg, nw,
                              tile_rows, tile_ranges, min_shared,
                              buf.ctypes.data_as(I32P), buf.size, ctypes.byref(info))
    return rc, info, buf


def _batch(rng, seqs, max_ctx, pool_extra=7):
    lens = rng.integers(0, max_ctx + 1, seqs).astype(np.int32)
    need = (lens + 15) // 16
    width = max(int(need.max()), 1)
    pool = int(need.sum()) + pool_extra
    perm = rng.permutation(pool).astype(np.int32)
    tables = np.full((seqs, width), -1, np.int32)
    cur = 0
    for s, n in enumerate(need):
        tables[s, :n] = perm[cur:cur + n]
        cur += n
    return tables, lens


def _check(tables, lens, hkv, window, wg, nw=8, tile_rows=0, tile_ranges=0, min_shared=8):
    rc, info, buf = _plan(tables, lens, hkv, window, wg, nw, tile_rows, tile_ranges, min_shared)
    assert rc == 0, _native.last_error()
    n_items = info.num_items
    wgt = buf[info.off_workgroups:info.off_waves].reshape(wg, nw + 3)
    wents = buf[info.off_waves:info.off_items].reshape(wg, nw, 6)
    items = buf[info.off_items:info.off_ids].reshape(n_items, 8)
    stride = info.item_stride
    assert n_items == wg * stride and 1 <= stride <= 64
    ids = buf[info.off_ids:info.off_chunked]
    chunked = buf[info.off_chunked:info.off_tiles].reshape(info.num_chunked, 4)
    tiles = buf[info.off_tiles:info.off_tile_members].reshape(info.num_tiles, 8)
    members = buf[info.off_tile_members:info.plan_words].reshape(info.num_tile_members, 3)
    assert info.off_tiles == info.off_chunked + 4 * info.num_chunked
    assert info.plan_words == info.off_tile_members + 3 * info.num_tile_members
    assert info.num_ids == ids.size
    # prefix tiles: members share the tile's blocks (the lead's ids), see all of them,
    # and write slot c0 + h * span + range of their own slots
    tiled = {}  # (seq, kvh) -> list of (blk0, nblk, slot)
    ranges = info.tile_ranges
    if info.num_tiles:
        assert 2 <= info.tile_rows <= max(tile_rows, 2) and 1 <= ranges <= 16
    for m0, n, h, r, b0, nb, off, lead in tiles:
        assert 2 <= n <= tile_rows and 0 <= h < hkv and 0 <= r < ranges and nb >= 1
        assert (ids[off:off + nb] == tables[lead, b0:b0 + nb]).all()
        for seq, c0, span in members[m0:m0 + n]:
            assert (tables[seq, b0:b0 + nb] == tables[lead, b0:b0 + nb]).all()
            # whole blocks before the newest token's (position ctx - 1), which stays
            # the row's own (an appending decode writes it in the row's own block)
            assert (lens[seq] - 1) // 16 >= b0 + nb and not (window and lens[seq] > window)
            assert span > r
            tiled.setdefault((int(seq), int(h)), []).append((int(b0), int(nb), int(c0 + h * span + r)))
    # workgroup g's items start at g * stride; each one's list starts at 0
    assert (wgt[:, 0] == np.arange(wg) * stride).all()
    assert (wgt[:, 1] - wgt[:, 0] <= stride).all() and (wgt[:, 1] >= wgt[:, 0]).all()
    assert (wgt[:, 2] == 0).all()
    assert (np.diff(wgt[:, 2:], axis=1) >= 0).all()
    assert int(wgt[:, 2 + nw].sum()) == info.num_blocks
    # items: laid end to end in their workgroup's list, their ids the rows' ids
    covered = {}
    loads = []
    for g in range(wg):
        cost, pos = 0, 0
        for k in range(wgt[g, 0], wgt[g, 1]):
            seq, kvh, blk0, nb, ctx, out, ipos, off = items[k]
            assert ctx == lens[seq] and 0 <= kvh < hkv and ipos == pos
            assert (ids[off:off + nb] == tables[seq, blk0:blk0 + nb]).all()
            covered.setdefault((seq, kvh), []).append((blk0, nb, out))
            cost += BLOCK_COST * nb + (ROW_COST if nb else 0)
            pos += nb
        assert pos == wgt[g, 2 + nw]
        loads.append(cost)
        # waves: equal shares of the workgroup's cost, within one block and a row start
        starts = []
        c = 0
        for k in range(wgt[g, 0], wgt[g, 1]):
            for b in range(items[k, 3]):
                c += ROW_COST if b == 0 else 0
                starts.append(c)
                c += BLOCK_COST
        for w in range(nw):
            lo, hi = wgt[g, 2 + w], wgt[g, 3 + w]
            if hi > lo:
                assert starts[lo] >= cost * w / nw - 1e-9
                assert starts[hi - 1] < cost * (w + 1) / nw
            # the wave's entry: its first piece and the ids of up to 2 of its blocks
            seq, kvh, count = wents[g, w, :3]
            if hi <= lo:
                assert count == 0
                continue
            k = next(k for k in range(wgt[g, 0], wgt[g, 1])
                     if items[k, 6] <= lo < items[k, 6] + items[k, 3])
            assert (seq, kvh) == (items[k, 0], items[k, 1])
            first = items[k, 2] + lo - items[k, 6]
            # never the block of the row's newest token (an appending decode stages the
            # token with it, once the wave has its items)
            newest = (items[k, 4] - 1) // 16 - first if items[k, 4] > 0 else -1
            assert count == min(2, hi - lo, items[k, 6] + items[k, 3] - lo,
                                newest if newest >= 0 else 2)
            assert (wents[g, w, 3:3 + count] == tables[seq, first:first + count]).all()
    # every row covered once; rows in several items or with tiles are chunked, with
    # consecutive slots (a member's tile ranges first)
    chunk_rows = {(int(s), int(h)): (int(c0), int(n)) for s, h, c0, n in chunked}
    assert len(chunk_rows) == info.num_chunked
    slots = []
    total = 0
    for s, ctx in enumerate(lens.tolist()):
        kv0 = ctx - window if window and ctx > window else 0
        first, last = kv0 // 16, (ctx + 15) // 16
        for h in range(hkv):
            tparts = sorted(tiled.get((s, h), []))
            own = sorted(covered.get((s, h), []))
            parts = tparts + own
            assert parts[0][0] == first and sum(p[1] for p in parts) == last - first
            for (a0, an, _), (b0, _, _) in zip(parts, parts[1:]):
                assert a0 + an == b0
            if len(parts) == 1 and not tparts:
                assert parts[0][2] == -1 and (s, h) not in chunk_rows
            elif len(own) == 1 and own[0][2] <= -2:
                # a member row whose own blocks are one item: its workgroup merges the
                # ranges' slots and its own (the next one)
                tb = -2 - own[0][2]
                assert (s, h) not in chunk_rows and len(tparts) == ranges
                assert [p[2] for p in tparts] == list(range(tb, tb + ranges))
                slots += list(range(tb, tb + ranges + 1))
            else:
                c0, n = chunk_rows[(s, h)]
                assert n == len(parts) and len(tparts) in (0, ranges)
                assert [p[2] for p in tparts] == list(range(c0, c0 + len(tparts)))
                assert sorted(p[2] for p in own) == list(range(c0 + len(tparts), c0 + n))
                slots += list(range(c0, c0 + n))
            nown = sum(p[1] for p in own)
            total += BLOCK_COST * nown + (ROW_COST if nown else 0)
    assert sorted(slots) == list(range(info.num_chunks))
    # LPT: no workgroup beyond the mean plus one item (a chunk is at most a share)
    share = total / wg
    biggest = max(BLOCK_COST * it[3] + ROW_COST for it in items) if n_items else 0
    assert max(loads) <= share + biggest + 1e-9
    return info, loads


@pytest.mark.parametrize("seed", range(6))
def test_random_batches_are_covered_and_balanced(seed):
    rng = np.random.default_rng(seed)
    seqs = int(rng.integers(1, 80))
    tables, lens = _batch(rng, seqs, int(rng.choice([40, 700, 5000])))
    window = int(rng.choice([0, 0, 100, 1000]))
    hkv = int(rng.choice([1, 2, 8]))
    wg = max(int(rng.choice([4, 16, 64])), -(-seqs * hkv // 40))  # <= 64 items per workgroup
    _check(tables, lens, hkv, window, wg)


def test_config2_needs_no_chunks_and_balances():
    from aster_amd import workloads as wl

    w = wl.config2()
    info, loads = _check(w.block_tables, w.context_lens, w.num_kv_heads, 0, 256)
    assert info.num_chunked == 0  # every row fits one workgroup: no merge kernel
    assert max(loads) / np.mean(loads) < 1.05


def test_long_rows_are_cut_into_chunks():
    from aster_amd import workloads as wl

    w = wl.config5()
    info, loads = _check(w.block_tables, w.context_lens, w.num_kv_heads, 0, 256)
    assert info.num_chunked == 16 * 8 and info.num_chunks == 16 * 8 * 2
    assert max(loads) / np.mean(loads) < 1.01


def test_empty_rows_and_single_row():
    tables = np.arange(8, dtype=np.int32).reshape(2, 4)
    info, _ = _check(tables, np.array([0, 50], np.int32), 2, 0, 4)
    assert info.num_items >= 4  # the empty row still has an item per head (zero output)
    _check(tables[:1], np.array([64], np.int32), 1, 0, 3)


def test_refusals():
    tables = np.zeros((2, 4), np.int32)
    rc, _, _ = _plan(tables, np.array([65, 3], np.int32), 1, 0, 4)  # 65 > 4 blocks
    assert rc == _native.ASTR_EINVAL and "outside" in _native.last_error()
    rc, _, _ = _plan(tables, np.array([-1, 3], np.int32), 1, 0, 4)
    assert rc == _native.ASTR_EINVAL
    rc, _, _ = _plan(tables, np.array([3, 3], np.int32), 1, 0, 4, nw=17)
    assert rc == _native.ASTR_EINVAL
    # more than 64 items on one workgroup
    many = np.zeros((130, 1), np.int32)
    rc, _, _ = _plan(many, np.full(130, 16, np.int32), 1, 0, 2)
    assert rc == _native.ASTR_EUNSUPPORTED and "items" in _native.last_error()
    # a sizing call writes nothing and reports the words
    info = DecodePlanInfo()
    lens = np.array([33, 3], np.int32)
    rc = _native.lib().astr_decode_plan(tables.ctypes.data_as(I32P), 4, lens.ctypes.data_as(I32P),
                                        2, 1, 0, 4, 8, 0, 0, 8, None, 0, ctypes.byref(info))
    assert rc == 0 and info.plan_words > 0
    rc, _, _ = _plan(tables, np.array([3, 3], np.int32), 1, 0, 4, tile_rows=2, tile_ranges=17)
    assert rc == _native.ASTR_EINVAL


def _shared_batch(rng, groups, seqs_per_group, shared_blocks, own_max, hkv_pool_extra=5):
    """Tables whose rows begin with their group's shared blocks, then blocks of their own."""
    rows, lens = [], []
    nxt = 0
    for g in range(groups):
        prefix = list(range(nxt, nxt + shared_blocks[g]))
        nxt += shared_blocks[g]
        for _ in range(seqs_per_group[g]):
            own = int(rng.integers(0, own_max + 1))
            ctx = shared_blocks[g] * 16 + own
            nb = -(-ctx // 16)
            row = prefix + list(range(nxt, nxt + nb - shared_blocks[g]))
            nxt += nb - shared_blocks[g]
            rows.append(row)
            lens.append(ctx)
    width = max(len(r) for r in rows)
    tables = np.full((len(rows), width), 0, np.int32)
    perm = rng.permutation(nxt + hkv_pool_extra).astype(np.int32)
    for i, r in enumerate(rows):
        tables[i, :len(r)] = perm[r]
    order = rng.permutation(len(rows))  # groups interleaved in the batch
    return tables[order], np.asarray(lens, np.int32)[order]


@pytest.mark.parametrize("seed", range(4))
def test_shared_prefixes_become_tiles(seed):
    rng = np.random.default_rng(100 + seed)
    groups = int(rng.integers(1, 4))
    per = [int(rng.integers(2, 40)) for _ in range(groups)]
    shared = [int(rng.integers(8, 40)) for _ in range(groups)]
    tables, lens = _shared_batch(rng, groups, per, shared, int(rng.choice([0, 100, 700])))
    hkv = int(rng.choice([1, 2, 8]))
    rows = int(rng.choice([2, 4, 8, 32]))
    wg = max(16, -(-len(lens) * hkv // 40))
    info, _ = _check(tables, lens, hkv, 0, wg, tile_rows=rows,
                     tile_ranges=int(rng.choice([0, 1, 3])))
    # every group's sequences in tiles of `rows`, but for a last tile of one
    assert info.num_tiles > 0
    assert info.num_tile_members == sum(n - (n % rows == 1) for n in per)


def test_config4_prefix_tiles():
    from aster_amd import workloads as wl

    w = wl.config4()
    info, loads = _check(w.block_tables, w.context_lens, w.num_kv_heads, 0, 256, tile_rows=32)
    assert info.num_tile_members == 256 and info.tile_ranges >= 1
    assert info.num_tiles == 8 * (256 // 32) * info.tile_ranges
    # the shared prefix is a windowed row's only when every key of it is visible
    _check(w.block_tables[:40], w.context_lens[:40], w.num_kv_heads, 4096, 64, tile_rows=32)
    info, _ = _check(w.block_tables[:40], w.context_lens[:40], w.num_kv_heads, 1000, 64,
                     tile_rows=32)
    assert info.num_tiles == 0
