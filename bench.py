"""INT8 paged decode benchmark (BASELINE config 2 on one MI355X).

A step is one decode-attention layer invocation of the hot path over the batch:
quantize-and-append of the 64 new bf16 K/V tokens (one per sequence) via
slot_mapping, then ragged paged attention of the 64 bf16 query rows (32 q heads,
8 kv heads, D=128) over their INT8 pages (context U[128,4096]). Steps cycle over
``--layers`` distinct layer arenas (default 4, ~1.1 GB) so each step reads its
K/V from HBM, not from the 256 MB MALL, as a real multi-layer decode does.

value = attended KV-tokens/s = sum(context_lens) / step time. The ``roofline``
object is for the attention call (decode_mfma_kernel plus the split-K
merge_kernel), timed with HIP events on the launch stream; ``cpu_baseline`` times the numpy restatement of the
reference's CPU path (oracle/) on a bounded sample on this host.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense fp16/bf16 MFMA, MI355X


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--config", default="config2",
                   choices=["config2", "config3", "config4", "config5"],
                   help="config2 is the headline workload; the others are extra measurements")
    p.add_argument("--layers", type=int, default=4)
    p.add_argument("--partition", type=int, default=0,
                   help="0 = automatic (stream-K); >0 = fixed split-K partition tokens")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "decode_traffic.json"),
                   help="rocprof-derived HBM bytes per attention launch (optional)")
    return p.parse_args()


def cpu_baseline(w, cache, step_batch, q, budget_s):
    """Time the oracle (numpy restatement of PagedAttentionRunner's row/page/tile
    loop + quantize_kv/copy_kv) on the whole workload, repeated for ~budget_s."""
    import numpy as np

    from oracle import reference_cpu as ref

    codes = cache.codes[:, 0].cpu().numpy()
    scales = cache.scales[:, 0].cpu().numpy()
    arena = [codes[:, 0].copy(), scales[:, 0].copy(), codes[:, 1].copy(), scales[:, 1].copy()]
    k, v, slots = (t.float().cpu().numpy() for t in step_batch)
    qn = q.float().cpu().numpy()
    reps, tokens, start = 0, 0, time.perf_counter()
    while True:
        ref.quantize_append(k, v, slots, arena[0], arena[1], arena[2], arena[3], 16)
        ref.paged_attention(qn, *arena, w.block_tables, w.context_lens, block_size=16,
                            scale=w.scale)
        reps += 1
        tokens += w.attended_tokens
        elapsed = time.perf_counter() - start
        if elapsed >= budget_s or reps >= 20:
            break
    return {"value": tokens / elapsed, "unit": "attended KV-tokens/s", "cores": 1,
            "kind": "port",
            "sample": f"{reps} full {w.name} steps (append 64 tokens + attend "
                      f"{w.attended_tokens} KV-tokens) in {elapsed:.1f}s, numpy oracle, 1 thread"}


def prefill_measurement(w, cache, q, L, args, device):
    """The rows with more than one query token alone (one varlen call over them):
    MFMA flops of the causal chunks / call time. The call also launches the decode
    kernels, which find no decode row, so the rate is a lower bound for the prefill
    kernel itself (rocprofv3 gives the kernel's own time)."""
    import numpy as np
    import torch

    from aster_amd import workloads as wl

    rows = np.nonzero(w.q_lens > 1)[0]
    sub = wl.DecodeWorkload(w.name + "_prefill_rows", w.num_q_heads, w.num_kv_heads,
                            w.head_dim, w.context_lens[rows], w.block_tables[rows],
                            w.num_blocks, w.q_dtype, w.seed, w.scale, query_lens=w.q_lens[rows])
    qsl_h = w.query_start_loc()
    take = torch.as_tensor(np.concatenate([np.arange(qsl_h[r], qsl_h[r + 1]) for r in rows]),
                           device=device).long()
    qp = q[take].contiguous()
    tables, lens = wl.device_tables(sub, device)
    qsl = wl.device_query_start(sub, device)
    out = torch.empty_like(qp)
    ws = cache.workspace(sub.num_seqs, sub.num_q_heads, sub.max_context_len, args.partition)

    def call(layer):
        cache.paged_attention(layer, qp, tables, lens, max_context_len=sub.max_context_len,
                              scale=sub.scale, partition_tokens=args.partition, out=out,
                              workspace=ws, query_start_loc=qsl, max_query_len=sub.max_query_len)

    for i in range(5):
        call(i % L)
    n = max(args.steps // 4, 20)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(n)]
    torch.cuda.synchronize()
    for i in range(n):
        evs[i][0].record()
        call(i % L)
        evs[i][1].record()
    torch.cuda.synchronize()
    cache.raise_errors()
    avg_ms = sum(a.elapsed_time(b) for a, b in evs) / n
    flops = sub.prefill_flops()
    tflops = flops / (avg_ms * 1e-3) / 1e12
    return {"rows": int(len(rows)), "query_tokens": sub.num_query_tokens, "flops": flops,
            "call_us": avg_ms * 1e3, "achieved_tflops": tflops, "bound": "mfma",
            "peak_tflops": MFMA_F16_PEAK_TFLOPS, "frac": tflops / MFMA_F16_PEAK_TFLOPS}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); "
              f"got --gpus {args.gpus}", file=sys.stderr)
        sys.exit(2)
    import torch

    from aster_amd import PagedKVCache
    from aster_amd import workloads as wl

    device = torch.device("cuda:0")
    w = getattr(wl, args.config)()
    L = args.layers
    cache = PagedKVCache(num_blocks=w.num_blocks, num_layers=L, num_kv_heads=w.num_kv_heads,
                         head_dim=w.head_dim, device=device)
    _, step_batch = wl.materialize(w, cache, layer=0, device=device, hold_last=True)
    for layer in range(1, L):
        cache.codes[:, layer].copy_(cache.codes[:, 0])
        cache.scales[:, layer].copy_(cache.scales[:, 0])
    tables, lens = wl.device_tables(w, device)
    varlen = w.query_lens is not None
    qsl = wl.device_query_start(w, device) if varlen else None
    q = wl.queries(w, device)
    out = torch.empty_like(q)
    k_new, v_new, slots = step_batch
    ws_bytes = cache.workspace_bytes(w.num_seqs, w.num_q_heads, w.max_context_len, args.partition)
    workspace = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=device)

    def attend(layer):
        cache.paged_attention(layer, q, tables, lens, max_context_len=w.max_context_len,
                              scale=w.scale, partition_tokens=args.partition, out=out,
                              workspace=workspace, query_start_loc=qsl,
                              max_query_len=w.max_query_len if varlen else None)

    def step(i):
        layer = i % L
        cache.append(layer, k_new, v_new, slots)
        attend(layer)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    cache.raise_errors()

    # ---- timed region: exactly K steps
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(args.steps):
        step(i)
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = start.elapsed_time(end) / args.steps
    cache.raise_errors()

    # ---- roofline: attention call alone, per-launch HIP events on the launch stream
    n = max(args.steps, 50)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(n)]
    torch.cuda.synchronize()
    for i in range(n):
        evs[i][0].record()
        attend(i % L)
        evs[i][1].record()
    torch.cuda.synchronize()
    attn_ms = sorted(a.elapsed_time(b) for a, b in evs)
    attn_avg_ms = sum(attn_ms) / n
    alg_bytes = w.algorithmic_bytes()
    achieved = alg_bytes / (attn_avg_ms * 1e-3) / 1e9
    # HBM bytes per call measured by rocprofv3 (FETCH_SIZE/WRITE_SIZE, calibrated
    # against a copy of known size) for this workload and split mode
    traffic = None
    if os.path.exists(args.traffic):
        mode = "streamk" if args.partition == 0 else f"partition_{args.partition}"
        with open(args.traffic) as f:
            traffic = json.load(f).get(w.name, {}).get(mode, {}).get("bytes_per_launch")

    result = {
        "metric": "attended KV-tokens/s and % of HBM peak, INT8 paged decode, 1xMI355X",
        "value": w.attended_tokens / (ms_per_step * 1e-3),
        "unit": "attended KV-tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,1) K/V quantized in-kernel, N(0,1) bf16 queries)",
        "config": {
            "workload": w.name, "num_seqs": w.num_seqs, "num_q_heads": w.num_q_heads,
            "num_kv_heads": w.num_kv_heads, "head_dim": w.head_dim, "block_size": 16,
            "attended_kv_tokens": w.attended_tokens, "max_context_len": w.max_context_len,
            "append_tokens": int(k_new.shape[0]), "partition_tokens": args.partition,
            "layer_arenas": L,
            "step": f"quantize_append({int(k_new.shape[0])} tok) + paged_attention",
        },
        "hbm_fraction_of_step": alg_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "roofline": {
            "kernel": ("decode_streamk_kernel + merge_streamk_kernel" if args.partition == 0 else
                       "decode_mfma_kernel + merge_kernel")
                      + (" + prefill_mfma_kernel" if varlen else "") + " (one paged_attention call)",
            "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
            "algorithmic_bytes_per_launch": alg_bytes,
            "avg_launch_us": attn_avg_ms * 1e3, "median_launch_us": attn_ms[n // 2] * 1e3,
        },
        "wall_s_timed_region": wall,
    }
    if varlen:
        result["config"]["query_tokens"] = w.num_query_tokens
        result["config"]["max_query_len"] = w.max_query_len
        result["prefill"] = prefill_measurement(w, cache, q, L, args, device)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(w, cache, step_batch, q, args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
