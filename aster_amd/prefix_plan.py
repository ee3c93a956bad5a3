"""Prefix packs: a host-built plan that lets decode rows whose block tables alias the
same shared prefix pages read those pages once per pack instead of once per row.

The reference's prefix reuse hands several sequences the same physical pages
(``PrefixCache.lookup`` returns shared page refs, state.py:599-625), and its row
loop reads those pages once per row (paged_attention.py:168-215). The scheduler
builds the step's block tables on the host anyway, so it can also see which rows
begin with the same pages: ``plan_prefix_packs`` groups decode rows by their first
block, measures each row's common prefix with the group's first row (whole blocks
only, every token of them visible), and cuts each group, longest prefixes first,
into packs of ``16 // G`` rows (G = query heads per kv head), the rows whose query
columns fill one MFMA tile. A pack's shared length is the shortest common prefix
among its rows; packs shorter than ``min_shared_blocks`` are dropped.

The plan travels to the kernels as one int32 device vector of ``num_packs``
records ``[shared_blocks, member_0, ..., member_{P-1}]`` (member -1: empty), the
``packs`` argument of ``astr_paged_attention_i8_shared``.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

MAX_PACKS = 128       # packs per launch
MAX_PACK_ROWS = 256   # pack rows per launch, and the largest batch that takes packs


@dataclass(frozen=True)
class PrefixPacks:
    """A prefix-pack plan for one step's decode rows (see module docstring)."""

    table: torch.Tensor  # int32 [num_packs * (1 + rows_per_pack)] on the cache device
    num_packs: int
    rows_per_pack: int
    num_seqs: int        # rows of the block tables the plan describes
    shared_blocks: int   # sum over packs of shared blocks: blocks read once, not per row
    packed_rows: int     # rows that are members of a pack
    saved_block_reads: int  # per kv head: block reads saved against reading per row

    def records(self):
        """The plan as a host array ``[num_packs, 1 + rows_per_pack]``."""
        return self.table.cpu().view(self.num_packs, 1 + self.rows_per_pack).numpy()


def _host_ints(x, name):
    arr = x.detach().cpu().numpy() if isinstance(x, torch.Tensor) else np.asarray(x)
    if not np.issubdtype(arr.dtype, np.integer):
        raise ValueError(f"{name} must hold integers")
    return arr.astype(np.int64)


def plan_prefix_packs(block_tables, context_lens, num_q_heads, num_kv_heads, *, device,
                      block_size=16, min_shared_blocks=4, rows_per_pack=None):
    """Prefix packs of a decode step, or None when no two rows share enough blocks.

    ``block_tables`` ``[S, max_blocks]`` and ``context_lens`` ``[S]`` as host arrays
    or tensors (a device tensor is copied to the host: plan where the tables are
    built). ``rows_per_pack`` defaults to ``16 // G``; it must be in ``[2, 16 // G]``."""
    tables = _host_ints(block_tables, "block_tables")
    lens = _host_ints(context_lens, "context_lens")
    if tables.ndim != 2 or lens.shape != (tables.shape[0],):
        raise ValueError("block_tables [S, max_blocks] and context_lens [S] are required")
    if num_kv_heads < 1 or num_q_heads % num_kv_heads:
        raise ValueError("Query heads must divide into KV groups")
    group = num_q_heads // num_kv_heads
    width = rows_per_pack if rows_per_pack is not None else 16 // group
    if type(width) is not int or width < 2 or width * group > 16:
        if rows_per_pack is not None:
            raise ValueError(f"rows_per_pack must be in [2, {16 // group}]")
        return None  # G = 16: one row fills the MFMA tile already
    if type(min_shared_blocks) is not int or min_shared_blocks < 1:
        raise ValueError("min_shared_blocks must be a positive int")
    if tables.shape[0] > MAX_PACK_ROWS:
        return None  # the kernels take packs for batches up to MAX_PACK_ROWS rows
    full = np.minimum(lens // block_size, tables.shape[1])  # blocks with every token visible
    rows = np.nonzero(full >= min_shared_blocks)[0]
    if rows.size < 2:
        return None
    first = tables[rows, 0]
    order = np.lexsort((rows, first))
    rows, first = rows[order], first[order]
    bounds = np.flatnonzero(np.diff(first)) + 1
    records, packed, shared_total = [], 0, 0
    for group_rows in np.split(rows, bounds):
        if group_rows.size < 2:
            continue
        leader = group_rows[0]
        reach = np.minimum(full[group_rows], full[leader])
        k = int(reach.max())
        same = tables[group_rows, :k] == tables[leader, :k]
        same &= np.arange(k)[None, :] < reach[:, None]
        common = np.cumprod(same, axis=1).sum(axis=1)  # leading blocks equal to the leader's
        by_prefix = np.argsort(-common, kind="stable")
        for start in range(0, group_rows.size, width):
            take = by_prefix[start:start + width]
            if take.size < 2:
                break
            shared = int(common[take].min())
            if shared < min_shared_blocks:
                break  # later chunks share even less
            if len(records) == MAX_PACKS or (len(records) + 1) * width > MAX_PACK_ROWS:
                break
            members = list(group_rows[take]) + [-1] * (width - take.size)
            records.append([shared] + [int(m) for m in members])
            packed += take.size
            shared_total += shared
    if not records:
        return None
    table = torch.tensor(np.asarray(records, np.int32).reshape(-1)).to(device)
    saved = sum(r[0] * (sum(m >= 0 for m in r[1:]) - 1) for r in records)
    return PrefixPacks(table, len(records), width, tables.shape[0], shared_total, packed, saved)
