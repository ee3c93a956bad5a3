"""A decode step (quantize-and-append, then paged attention) captured in a HIP graph
replays exactly what the eager calls produce: the path issues no memset and needs no
host synchronisation inside a step. Replays are interleaved with eager work and
synchronisations, and every replay is checked."""

import numpy as np
import pytest
import torch

from aster_amd import PagedKVCache
from aster_amd import workloads as wl

pytestmark = pytest.mark.gpu


def test_decode_step_replays_in_a_graph(device):
    w = wl.scaled(wl.config2(), num_seqs=12, max_len=600)
    layers = 2
    cache = PagedKVCache(num_blocks=w.num_blocks, num_layers=layers, num_kv_heads=w.num_kv_heads,
                         head_dim=w.head_dim, device=device)
    _, (k_new, v_new, slots) = wl.materialize(w, cache, layer=0, device=device, hold_last=True)
    for layer in range(1, layers):
        cache.codes[:, layer].copy_(cache.codes[:, 0])
        cache.scales[:, layer].copy_(cache.scales[:, 0])
    tables, lens = wl.device_tables(w, device)
    q = wl.queries(w, device)
    outs = [torch.empty_like(q) for _ in range(layers)]
    ws_bytes = cache.workspace_bytes(w.num_seqs, w.num_q_heads, w.max_context_len, 0)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=device)

    def step(layer, out):
        cache.append(layer, k_new, v_new, slots)
        cache.paged_attention(layer, q, tables, lens, max_context_len=w.max_context_len,
                              scale=w.scale, out=out, workspace=ws)

    for layer in range(layers):
        step(layer, outs[layer])
    torch.cuda.synchronize()
    cache.raise_errors()
    ref = [o.clone() for o in outs]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for layer in range(layers):
            step(layer, outs[layer])
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for layer in range(layers):
            step(layer, outs[layer])

    scratch = torch.empty_like(q)
    for _ in range(3):
        for o in outs:
            o.fill_(float("nan"))
        step(1, scratch)  # eager work between the replays, same workspace
        torch.cuda.synchronize()
        assert torch.equal(scratch, ref[1])
        graph.replay()
        torch.cuda.synchronize()
        for o, r in zip(outs, ref):
            assert torch.equal(o, r)
    cache.raise_errors()


def test_mixed_step_replays_in_a_graph(device):
    """A mixed step (chunk rows and decode rows in one varlen call: the decode kernels,
    then the prefill kernel) captured in a graph: replays equal the eager outputs bit
    for bit, interleaved with eager calls, and work the caller enqueues after an eager
    call sees its outputs."""
    rng = np.random.default_rng(5)
    q_lens = np.array([40, 1, 1, 17, 1, 64, 1, 0, 3], np.int32)
    ctx = q_lens + rng.integers(0, 700, q_lens.size).astype(np.int32)
    ctx[7] = 20
    tables_h, pool = wl._tables_from_lengths(ctx, rng, spare_blocks=3)
    w = wl.DecodeWorkload("mixed", 32, 8, 128, ctx, tables_h, pool, torch.bfloat16, 5,
                          128 ** -0.5, query_lens=q_lens)
    cache = PagedKVCache(num_blocks=w.num_blocks, num_layers=1, num_kv_heads=w.num_kv_heads,
                         head_dim=w.head_dim, device=device)
    wl.materialize(w, cache, device=device)
    tables, lens = wl.device_tables(w, device)
    qsl = wl.device_query_start(w, device)
    q = wl.queries(w, device)
    ws_bytes = cache.workspace_bytes(w.num_seqs, w.num_q_heads, w.max_context_len, 0)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=device)
    out = torch.empty_like(q)

    def call():
        cache.paged_attention(0, q, tables, lens, max_context_len=w.max_context_len,
                              scale=w.scale, query_start_loc=qsl, max_query_len=w.max_query_len,
                              out=out, workspace=ws)

    call()
    copy = out.clone()  # enqueued after the call on the caller's stream
    torch.cuda.synchronize()
    cache.raise_errors()
    ref = out.clone()
    assert torch.equal(copy, ref)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for _ in range(3):
        out.fill_(float("nan"))
        call()  # eager, between the replays
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
    cache.raise_errors()
