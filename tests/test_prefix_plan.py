"""Host planning of prefix packs (aster_amd/prefix_plan.py): decode rows whose block
tables begin with the same physical blocks (the PrefixCache's shared page refs,
state.py:599-625) are grouped into packs of 16 // G rows that share a stated number
of whole, visible blocks. Every plan is checked against the tables it describes."""

import numpy as np
import pytest

from aster_amd.prefix_plan import MAX_PACK_ROWS, MAX_PACKS, plan_prefix_packs


def _check_plan(plan, tables, lens, min_blocks=4):
    """Each pack's members hold the same first `shared` blocks, all of them visible;
    no row is in two packs."""
    rec = plan.records()
    seen = set()
    for shared, *members in rec:
        live = [m for m in members if m >= 0]
        assert len(live) >= 2 and shared >= min_blocks
        for m in live:
            assert m not in seen
            seen.add(m)
            assert shared * 16 <= lens[m]
            assert (tables[m, :shared] == tables[live[0], :shared]).all()
    assert plan.packed_rows == len(seen)
    assert plan.shared_blocks == int(rec[:, 0].sum())
    return rec


def _prefix_batch(rows, prefix_blocks, seed, suffix=(64, 512)):
    """Config-4 shape: every row aliases one prefix, then private blocks."""
    rng = np.random.default_rng(seed)
    lens = prefix_blocks * 16 + rng.integers(suffix[0], suffix[1] + 1, rows)
    width = int(-(-lens.max() // 16))
    tables = np.full((rows, width), -1, np.int64)
    nxt = prefix_blocks
    for r in range(rows):
        n = -(-int(lens[r]) // 16)
        tables[r, :prefix_blocks] = np.arange(prefix_blocks)
        tables[r, prefix_blocks:n] = np.arange(nxt, nxt + n - prefix_blocks)
        nxt += n - prefix_blocks
    return tables, lens


def test_config4_shape_packs_every_row():
    tables, lens = _prefix_batch(256, 128, seed=4)
    plan = plan_prefix_packs(tables, lens, 32, 8, device="cpu")
    assert plan.rows_per_pack == 4 and plan.num_packs == 64
    rec = _check_plan(plan, tables, lens)
    assert (rec[:, 0] == 128).all() and plan.packed_rows == 256
    assert plan.saved_block_reads == 64 * 128 * 3


@pytest.mark.parametrize("hq,hkv,width", [(8, 8, 16), (16, 8, 8), (64, 8, 2)])
def test_pack_width_follows_the_group(hq, hkv, width):
    tables, lens = _prefix_batch(40, 10, seed=hq)
    plan = plan_prefix_packs(tables, lens, hq, hkv, device="cpu")
    assert plan.rows_per_pack == width
    _check_plan(plan, tables, lens)
    assert plan_prefix_packs(tables, lens, 128, 8, device="cpu") is None  # G = 16


def test_partial_blocks_groups_and_thresholds():
    # rows 0-2 share 6 blocks; row 3 shares only 3; rows 4-5 share another first block;
    # row 6's context ends inside block 5: only 5 whole blocks visible
    t = np.arange(7 * 12).reshape(7, 12) + 1000
    t[0:4, :6] = np.arange(6)
    t[3, 3:] = 500 + np.arange(9)
    t[4:6, :8] = 50 + np.arange(8)
    t[6, :6] = np.arange(6)
    lens = np.array([190, 96, 120, 180, 130, 150, 90])
    plan = plan_prefix_packs(t, lens, 8, 2, device="cpu")  # G = 4: 4 rows per pack
    rec = _check_plan(plan, t, lens)
    packs = sorted((int(s), sorted(int(m) for m in ms if m >= 0)) for s, *ms in rec)
    # row 3 (3 shared blocks) falls below the threshold with the others of its group
    assert packs == [(5, [0, 1, 2, 6]), (8, [4, 5])]
    assert plan_prefix_packs(t, lens, 8, 2, device="cpu", min_shared_blocks=9) is None
    assert plan_prefix_packs(t[:1], lens[:1], 8, 2, device="cpu") is None


def test_longest_prefixes_pack_together():
    # 8 rows with the same first block; rows diverge after 20, 20, 20, 20, 6, 6, 6, 6 blocks
    t = np.arange(8 * 24).reshape(8, 24) + 1000
    t[:, :6] = np.arange(6)
    t[:4, 6:20] = 100 + np.arange(14)
    lens = np.full(8, 24 * 16)
    plan = plan_prefix_packs(t, lens, 4, 1, device="cpu", rows_per_pack=4)
    rec = _check_plan(plan, t, lens)
    assert sorted(map(int, rec[:, 0])) == [6, 20]


def test_limits_and_arguments():
    tables, lens = _prefix_batch(256, 8, seed=1, suffix=(16, 32))
    plan = plan_prefix_packs(tables, lens, 8, 8, device="cpu", rows_per_pack=2)
    assert plan.num_packs == MAX_PACKS and plan.num_packs * plan.rows_per_pack <= MAX_PACK_ROWS
    _check_plan(plan, tables, lens)
    big, big_lens = _prefix_batch(MAX_PACK_ROWS + 1, 8, seed=1)
    assert plan_prefix_packs(big, big_lens, 32, 8, device="cpu") is None
    with pytest.raises(ValueError):
        plan_prefix_packs(tables, lens, 32, 8, device="cpu", rows_per_pack=5)
    with pytest.raises(ValueError):
        plan_prefix_packs(tables, lens[:-1], 32, 8, device="cpu")
    with pytest.raises(ValueError):
        plan_prefix_packs(tables, lens, 30, 8, device="cpu")
    with pytest.raises(ValueError):
        plan_prefix_packs(tables.astype(float), lens, 32, 8, device="cpu")
