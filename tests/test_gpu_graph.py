"""A decode step (quantize-and-append, then paged attention) captured in a HIP graph
replays exactly what the eager calls produce: the path issues no memset and needs no
host synchronisation inside a step. Replays are interleaved with eager work and
synchronisations, and every replay is checked."""

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
