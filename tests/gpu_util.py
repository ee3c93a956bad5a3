"""Helpers shared by the GPU parity tests: move a PagedKVCache layer to numpy in the
oracle's arena layout and run the oracle on it."""

import numpy as np
import torch

from oracle import reference_cpu as ref

# north_star tolerance for attention outputs vs the reference's dequantize-then-attend path
ATOL, RTOL = 2e-3, 1e-2


def arena_numpy(cache, layer=0):
    """(k_codes, k_scales, v_codes, v_scales) as numpy [blocks, Hkv, bs, D] / [blocks, Hkv, bs]."""
    codes = cache.codes[:, layer].cpu().numpy()
    scales = cache.scales[:, layer].cpu().numpy()
    return codes[:, 0], scales[:, 0], codes[:, 1], scales[:, 1]


def oracle_decode(workload_or_tables, cache, query, layer=0, context_lens=None, scale=None,
                  window=None, query_lens=None, causal=True, fp64=False):
    """The oracle's row-by-row paged attention (paged_attention.py:168-215) over this
    cache layer; a workload supplies tables, lengths, scale and query counts. ``fp64``
    runs it in float64, as the reference does for float64 queries (online_attention.py:
    158-159): the exact result over the same codes and scales."""
    if context_lens is None:
        w = workload_or_tables
        tables, lens = w.block_tables, w.context_lens
        scale = w.scale if scale is None else scale
        if query_lens is None and w.query_lens is not None:
            query_lens = w.query_lens
    else:
        tables, lens = workload_or_tables, context_lens
    q = query.double().cpu().numpy() if fp64 else query.float().cpu().numpy()
    padding = cache.key_valid.cpu().numpy().astype(bool) if cache.has_padding else None
    return ref.paged_attention(q, *arena_numpy(cache, layer), tables, lens, block_size=16,
                               scale=scale, window=window, query_lens=query_lens, causal=causal,
                               padding=padding, fmt=cache.quantization.format)


def mark_padding(cache, tables, lens, fraction, seed, *, whole_rows=(), whole_blocks=0):
    """Mark a seeded ``fraction`` of the committed keys of every row as padding keys
    through ``write_key_valid`` (every row's slots in one launch), plus every key of
    the rows in ``whole_rows`` and ``whole_blocks`` whole pages; returns the host
    ``valid`` array [num_blocks, 16]."""
    rng = np.random.default_rng(seed)
    slots, valid = [], []
    picked = set()
    for b, ctx in enumerate(np.asarray(lens).tolist()):
        pages = [int(x) for x in np.asarray(tables[b])[: (ctx + 15) // 16]]
        for i in range(ctx):
            slots.append(pages[i // 16] * 16 + i % 16)
            valid.append(b not in whole_rows and rng.random() >= fraction)
        if len(picked) < whole_blocks and len(pages) > 2:
            picked.add(pages[1])
    valid = np.array(valid)
    for j, slot in enumerate(slots):
        if slot // 16 in picked:
            valid[j] = False
    dev = cache.device
    cache.write_key_valid(torch.tensor(slots, dtype=torch.int64, device=dev),
                          torch.tensor(valid, dtype=torch.bool, device=dev))
    torch.cuda.synchronize(dev)
    cache.raise_errors()
    return cache.key_valid.cpu().numpy()


def assert_attention_close(actual, expected, atol=ATOL, rtol=RTOL):
    """|a - b| <= atol + rtol * |b| elementwise (torch.testing.assert_close semantics)."""
    def host(x):
        return x.float().cpu().numpy() if isinstance(x, torch.Tensor) else x
    np.testing.assert_allclose(host(actual), host(expected), atol=atol, rtol=rtol)
