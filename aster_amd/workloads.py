"""Seeded synthetic workloads: the INT8 paged-decode configurations of the benchmark.

Each builder returns a :class:`DecodeWorkload` with host-side metadata (context
lengths, block tables as numpy arrays); :func:`materialize` fills a
``PagedKVCache`` on the device through the HIP quantize-and-append kernel from
seeded N(0,1) K/V and draws the queries. Nothing here reads files.

  config1  tiny ragged decode (CPU-runnable): ctx {17,64,129,300}, 4q/4kv, D 64,
           fp32 Q, block tables = seeded permutation of a 64-block pool.
  config2  Llama-3-8B-shaped GQA decode: 64 seqs, 32q/8kv, D 128, ctx U[128,4096],
           bf16 Q, shuffled pool sized to the total context; the step appends one
           new token per sequence (64 tokens) before attending.
  config3  continuous-batching mixed step: 8 prefill chunks of 512 query tokens
           (prior context U[0,2048]) packed with 120 decode rows (ctx U[256,4096]);
           32q/8kv, D 128, bf16 Q, causal within chunks.
  config4  prefix-shared decode: 256 seqs aliasing one 2048-token prefix (128
           blocks) + private suffixes U[64,512]; 32q/8kv, D 128, bf16 Q.
  config5  long context: 16 x 32768, 64q/8kv, D 128, bf16 Q, 10% of K rows x8.
"""

from __future__ import annotations

from dataclasses import dataclass, field
import math

import numpy as np
import torch

BLOCK = 16


@dataclass
class DecodeWorkload:
    name: str
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    context_lens: np.ndarray          # int32 [S], committed length incl. the new token
    block_tables: np.ndarray          # int32 [S, max_blocks]
    num_blocks: int
    q_dtype: torch.dtype
    seed: int
    scale: float
    k_outlier_fraction: float = 0.0   # fraction of K rows multiplied by 8
    shared_prefix_blocks: int = 0     # leading blocks aliased by every row
    query_lens: np.ndarray = None     # int32 [S] query tokens per row (None: 1 each)
    meta: dict = field(default_factory=dict)

    @property
    def num_seqs(self):
        return int(self.context_lens.shape[0])

    @property
    def q_lens(self):
        if self.query_lens is None:
            return np.ones(self.num_seqs, dtype=np.int32)
        return self.query_lens

    @property
    def num_query_tokens(self):
        return int(self.q_lens.sum())

    @property
    def max_query_len(self):
        return int(self.q_lens.max()) if self.num_seqs else 0

    def query_start_loc(self):
        return np.concatenate([[0], np.cumsum(self.q_lens)]).astype(np.int32)

    def prefill_flops(self):
        """QK^T + PV flops of the rows with more than one query token under the
        causal mask: 4*Hq*D per visible (query, key) pair."""
        pairs = 0
        for n, ctx in zip(self.q_lens.tolist(), self.context_lens.tolist()):
            if n > 1:
                prior = ctx - n
                pairs += n * prior + n * (n + 1) // 2
        return 4 * self.num_q_heads * self.head_dim * pairs

    @property
    def max_context_len(self):
        return int(self.context_lens.max()) if self.num_seqs else 0

    @property
    def attended_tokens(self):
        return int(self.context_lens.astype(np.int64).sum())

    def algorithmic_bytes(self):
        """HBM bytes one decode-attention call must move: K/V codes + fp32 scales of
        every attended token, Q in, O out, block-table entries and lengths."""
        q_bytes = torch.tensor([], dtype=self.q_dtype).element_size()
        kv = self.attended_tokens * self.num_kv_heads * (2 * self.head_dim + 8)
        qo = self.num_query_tokens * self.num_q_heads * self.head_dim * 2 * q_bytes
        tables = 4 * int(np.ceil(self.context_lens / BLOCK).sum()) + 4 * self.num_seqs
        return kv + qo + tables

    def unique_kv_bytes(self):
        """K/V bytes of distinct physical blocks touched (prefix sharing reads the
        shared blocks once from HBM at best)."""
        used = set()
        for row, ctx in zip(self.block_tables, self.context_lens):
            used.update(row[: math.ceil(int(ctx) / BLOCK)].tolist())
        return len(used) * BLOCK * self.num_kv_heads * (2 * self.head_dim + 8)


def _tables_from_lengths(lengths, rng, spare_blocks=0):
    need = [math.ceil(int(c) / BLOCK) for c in lengths]
    pool = int(sum(need)) + spare_blocks
    perm = rng.permutation(pool).astype(np.int32)
    width = max(need) if need else 1
    tables = np.zeros((len(lengths), max(width, 1)), dtype=np.int32)
    cursor = 0
    for i, n in enumerate(need):
        tables[i, :n] = perm[cursor : cursor + n]
        cursor += n
    return tables, pool


def config1(seed=1):
    rng = np.random.default_rng(seed)
    lengths = np.array([17, 64, 129, 300], dtype=np.int32)
    need = [math.ceil(int(c) / BLOCK) for c in lengths]
    perm = rng.permutation(64).astype(np.int32)
    tables = np.zeros((4, max(need)), dtype=np.int32)
    cursor = 0
    for i, n in enumerate(need):
        tables[i, :n] = perm[cursor : cursor + n]
        cursor += n
    return DecodeWorkload("config1_tiny_ragged", 4, 4, 64, lengths, tables, 64, torch.float32,
                          seed, 64 ** -0.5)


def config2(seed=2):
    rng = np.random.default_rng(seed)
    lengths = rng.integers(128, 4096, size=64, endpoint=True).astype(np.int32)
    tables, pool = _tables_from_lengths(lengths, rng, spare_blocks=64)
    return DecodeWorkload("config2_llama3_8b_decode", 32, 8, 128, lengths, tables, pool,
                          torch.bfloat16, seed, 128 ** -0.5)


def config3(seed=3, num_prefill=8, chunk=512, max_prior=2048, num_decode=120,
            decode_range=(256, 4096)):
    """Prefill rows first (chunk tokens on top of a prior context), then decode rows;
    context lengths count the step's own tokens."""
    rng = np.random.default_rng(seed)
    prior = rng.integers(0, max_prior, size=num_prefill, endpoint=True)
    dec = rng.integers(decode_range[0], decode_range[1], size=num_decode, endpoint=True)
    lengths = np.concatenate([prior + chunk, dec]).astype(np.int32)
    qlens = np.concatenate([np.full(num_prefill, chunk), np.ones(num_decode)]).astype(np.int32)
    tables, pool = _tables_from_lengths(lengths, rng, spare_blocks=16)
    return DecodeWorkload("config3_mixed_prefill_decode", 32, 8, 128, lengths, tables, pool,
                          torch.bfloat16, seed, 128 ** -0.5, query_lens=qlens)


def config4(seed=4):
    rng = np.random.default_rng(seed)
    prefix = 2048
    suffix = rng.integers(64, 512, size=256, endpoint=True).astype(np.int32)
    lengths = (prefix + suffix).astype(np.int32)
    pblocks = prefix // BLOCK
    need = [math.ceil(int(s) / BLOCK) for s in suffix]
    pool = pblocks + int(sum(need))
    perm = rng.permutation(pool).astype(np.int32)
    shared, private = perm[:pblocks], perm[pblocks:]
    tables = np.zeros((256, pblocks + max(need)), dtype=np.int32)
    cursor = 0
    for i, n in enumerate(need):
        tables[i, :pblocks] = shared
        tables[i, pblocks : pblocks + n] = private[cursor : cursor + n]
        cursor += n
    return DecodeWorkload("config4_prefix_shared", 32, 8, 128, lengths, tables, pool,
                          torch.bfloat16, seed, 128 ** -0.5, shared_prefix_blocks=pblocks)


def config5(seed=5):
    rng = np.random.default_rng(seed)
    lengths = np.full(16, 32768, dtype=np.int32)
    tables, pool = _tables_from_lengths(lengths, rng)
    return DecodeWorkload("config5_long_context_splitk", 64, 8, 128, lengths, tables, pool,
                          torch.bfloat16, seed, 128 ** -0.5, k_outlier_fraction=0.1)


def scaled(workload, num_seqs=None, max_len=None, seed=None):
    """A smaller copy of ``workload`` (first ``num_seqs`` rows, lengths clipped to
    ``max_len``) with re-packed block tables, for oracle-sized parity tests."""
    rng = np.random.default_rng(workload.seed if seed is None else seed)
    lengths = workload.context_lens[: num_seqs or workload.num_seqs].copy()
    if max_len is not None:
        lengths = np.minimum(lengths, max_len).astype(np.int32)
    if workload.shared_prefix_blocks:
        pb = min(workload.shared_prefix_blocks, int(lengths.min()) // BLOCK)
        need = [math.ceil(int(c) / BLOCK) - pb for c in lengths]
        pool = pb + int(sum(need))
        perm = rng.permutation(pool).astype(np.int32)
        tables = np.zeros((len(lengths), pb + max(need)), dtype=np.int32)
        cursor = pb
        for i, n in enumerate(need):
            tables[i, :pb] = perm[:pb]
            tables[i, pb : pb + n] = perm[cursor : cursor + n]
            cursor += n
    else:
        pb = 0
        tables, pool = _tables_from_lengths(lengths, rng)
    qlens = None
    if workload.query_lens is not None:
        qlens = np.minimum(workload.query_lens[: len(lengths)], lengths).astype(np.int32)
    return DecodeWorkload(workload.name + "_scaled", workload.num_q_heads, workload.num_kv_heads,
                          workload.head_dim, lengths, tables, pool, workload.q_dtype,
                          workload.seed, workload.scale, workload.k_outlier_fraction, pb,
                          query_lens=qlens)


# ---- device materialisation ---------------------------------------------------------


def token_slots(workload, row):
    """int64 slots of every committed token of ``row`` (slot = page*16 + offset,
    state.py:339-344)."""
    ctx = int(workload.context_lens[row])
    pos = np.arange(ctx)
    return workload.block_tables[row][pos // BLOCK].astype(np.int64) * BLOCK + pos % BLOCK


def kv_source(workload, row, generator, device, dtype=None):
    """Seeded N(0,1) K/V source rows ``[ctx, Hkv, D]`` of one sequence (fp32 for
    fp32-query workloads, else bf16), with the K outlier rows scaled by 8."""
    dtype = dtype or (torch.float32 if workload.q_dtype == torch.float32 else torch.bfloat16)
    ctx = int(workload.context_lens[row])
    shape = (ctx, workload.num_kv_heads, workload.head_dim)
    k = torch.randn(shape, generator=generator, device=device, dtype=torch.float32)
    v = torch.randn(shape, generator=generator, device=device, dtype=torch.float32)
    if workload.k_outlier_fraction:
        rows = torch.rand(shape[:2], generator=generator, device=device) < workload.k_outlier_fraction
        k = torch.where(rows[..., None], k * 8, k)
    return k.to(dtype), v.to(dtype)


def device_tables(workload, device):
    return (torch.from_numpy(workload.block_tables).to(device),
            torch.from_numpy(workload.context_lens).to(device))


def device_query_start(workload, device):
    return torch.from_numpy(workload.query_start_loc()).to(device)


def materialize(workload, cache, layer=0, device="cuda", keep_sources=False, hold_last=False):
    """Fill ``cache`` layer ``layer`` with every committed token of every row via the
    HIP quantize-and-append kernel. With ``hold_last`` the step's own tokens (the
    last ``q_lens[row]`` of each row) are left out and returned as the step's append
    batch ``(k [T,Hkv,D], v, slots)`` packed like the queries.
    Returns ``(sources, step)``: per-row fp32/bf16 K/V sources when
    ``keep_sources`` (else None) and the held-back batch (or None)."""
    gen = torch.Generator(device=device)
    gen.manual_seed(workload.seed)
    sources = [] if keep_sources else None
    last_k, last_v, last_slots = [], [], []
    qlens = workload.q_lens
    for row in range(workload.num_seqs):
        k, v = kv_source(workload, row, gen, device)
        slots = torch.from_numpy(token_slots(workload, row)).to(device)
        if hold_last:
            n = int(min(qlens[row], k.shape[0]))
            cut = k.shape[0] - n
            last_k.append(k[cut:]), last_v.append(v[cut:]), last_slots.append(slots[cut:])
            k, v, slots = k[:cut], v[:cut], slots[:cut]
        if k.shape[0]:
            cache.append(layer, k, v, slots)
        if keep_sources:
            sources.append((k, v) if not hold_last else (torch.cat([k, last_k[-1]]),
                                                         torch.cat([v, last_v[-1]])))
    cache.raise_errors()
    step = None
    if hold_last:
        step = (torch.cat(last_k), torch.cat(last_v), torch.cat(last_slots))
    return sources, step


def queries(workload, device="cuda", seed_offset=1000):
    gen = torch.Generator(device=device)
    gen.manual_seed(workload.seed + seed_offset)
    q = torch.randn((workload.num_query_tokens, workload.num_q_heads, workload.head_dim),
                    generator=gen, device=device, dtype=torch.float32)
    return q.to(workload.q_dtype)
