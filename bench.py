"""INT8 paged decode benchmark (the config2 workload on one MI355X).

A step is one decode-attention layer invocation of the hot path over the batch:
quantize-and-append of the 64 new bf16 K/V tokens (one per sequence) via
slot_mapping into their reserved slots, and ragged paged attention of the 64 bf16 query
rows (32 q heads, 8 kv heads, D=128) over their INT8 pages (context U[128,4096]) on the
step's host plan, in one launch as the runner's decode step runs them (the decode
quantizes each new token in the wave that streams its block). Steps
cycle over ``--layers`` distinct layer arenas (default 4, ~1.1 GB) so each step reads
its K/V from HBM, not from the 256 MB MALL, as a real multi-layer decode does.

value = attended KV-tokens/s = sum(context_lens) / step time. The ``roofline``
object is for the attention call (decode_planned_kernel, or without a plan the
stream-K kernel and its merge), timed with HIP events on the launch stream. ``extra`` measures
configs 3, 4 and 5 in the same run the same way (their calls alone).
``cpu_baseline`` times the numpy restatement of the reference's CPU path (oracle/)
on the whole config-2 step with one BLAS thread and with the host's CPU share.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
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
    p.add_argument("--cpu-runs", type=int, default=5, help="timed CPU steps per thread setting")
    p.add_argument("--no-extra", action="store_true", help="skip the config 3/4/5 measurements")
    p.add_argument("--no-plan", action="store_true",
                   help="decode on the unplanned stream-K kernel instead of a host plan")
    p.add_argument("--tail", type=int, default=None,
                   help="planned decode: blocks at the end of each wave's range loaded two "
                        "at a time (default: the library's)")
    p.add_argument("--extra-calls", type=int, default=50)
    p.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "decode_traffic.json"),
                   help="rocprof-derived HBM bytes per attention launch (optional)")
    return p.parse_args()


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_share():
    """Threads for the all-cores leg: the host's CPU share (OMP_NUM_THREADS where the
    environment sets it, else the CPUs this process may run on)."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    return int(env) if env.isdigit() and int(env) > 0 else len(os.sched_getaffinity(0))


def cpu_baseline(w, cache, step_batch, q, runs):
    """The oracle (numpy restatement of PagedAttentionRunner's row/page/tile loop and
    quantize_kv/copy_kv) on the whole config-2 step: one warmup, then the median of
    ``runs`` steps, with one BLAS/torch thread and with the host's CPU share."""
    import torch
    from threadpoolctl import threadpool_limits

    from oracle import reference_cpu as ref

    codes = cache.codes[:, 0].cpu().numpy()
    scales = cache.scales[:, 0].cpu().numpy()
    k, v, slots = (t.float().cpu().numpy() for t in step_batch)
    qn = q.float().cpu().numpy()

    # appending the step's tokens again rewrites the same slots with the same codes
    arena = [codes[:, 0].copy(), scales[:, 0].copy(), codes[:, 1].copy(), scales[:, 1].copy()]

    def step():
        t0 = time.perf_counter()
        ref.quantize_append(k, v, slots, arena[0], arena[1], arena[2], arena[3], 16)
        ref.paged_attention(qn, *arena, w.block_tables, w.context_lens, block_size=16,
                            scale=w.scale)
        return time.perf_counter() - t0

    legs = []
    saved = torch.get_num_threads()
    for threads in sorted({1, cpu_share()}):
        with threadpool_limits(limits=threads), torch.inference_mode():
            torch.set_num_threads(threads)
            step()
            times = [step() for _ in range(runs)]
        med = statistics.median(times)
        legs.append({"threads": threads, "median_s": med, "runs": runs,
                     "value": w.attended_tokens / med})
    torch.set_num_threads(saved)
    best = max(legs, key=lambda leg: leg["value"])
    return {"value": best["value"], "unit": "attended KV-tokens/s", "cores": best["threads"],
            "kind": "port", "cpu_model": cpu_model(), "cpu_count": os.cpu_count(),
            "legs": legs,
            "sample": f"the whole {w.name} step (append {int(step_batch[0].shape[0])} tokens + "
                      f"attend {w.attended_tokens} KV-tokens), numpy oracle, median of {runs} "
                      f"after one warmup, per thread setting (BLAS/torch threads via "
                      f"threadpoolctl)"}


def time_calls(call, n, layers):
    """Average and median ms of ``call(layer)`` from per-launch HIP events on the
    current (launch) stream, after 5 warmup calls, cycling over ``layers`` arenas."""
    import torch

    for i in range(5):
        call(i % layers)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(n)]
    torch.cuda.synchronize()
    for i in range(n):
        evs[i][0].record()
        call(i % layers)
        evs[i][1].record()
    torch.cuda.synchronize()
    ms = sorted(a.elapsed_time(b) for a, b in evs)
    return sum(ms) / n, ms[n // 2]


def build_arena(w, layers, device, hold_last=False):
    import torch

    from aster_amd import PagedKVCache
    from aster_amd import workloads as wl

    cache = PagedKVCache(num_blocks=w.num_blocks, num_layers=layers, num_kv_heads=w.num_kv_heads,
                         head_dim=w.head_dim, device=device)
    _, step_batch = wl.materialize(w, cache, layer=0, device=device, hold_last=hold_last)
    for layer in range(1, layers):
        cache.codes[:, layer].copy_(cache.codes[:, 0])
        cache.scales[:, layer].copy_(cache.scales[:, 0])
    torch.cuda.synchronize()
    return cache, step_batch


def attention_caller(w, cache, q, device, partition, rows=None, packs=False, planned=False,
                     tail=None):
    """``call(layer)`` running one attention call over the workload (or over its rows
    ``rows``, a sub-workload of the same arena) and the workload it covers. With
    ``packs`` a decode batch gets the prefix-pack plan of its block tables, and with
    ``planned`` the host schedule of the planned decode kernel, each built once on the
    host as the runner builds them once per step for every layer (outside the timed
    calls; ``call.plan_us`` is the host time of building the schedule)."""
    import numpy as np
    import torch

    from aster_amd import workloads as wl

    if rows is not None:
        qsl_h = w.query_start_loc()
        take = torch.as_tensor(np.concatenate([np.arange(qsl_h[r], qsl_h[r + 1]) for r in rows]),
                               device=device).long()
        q = q[take].contiguous()
        w = wl.DecodeWorkload(w.name + "_rows", w.num_q_heads, w.num_kv_heads, w.head_dim,
                              w.context_lens[rows], w.block_tables[rows], w.num_blocks, w.q_dtype,
                              w.seed, w.scale, query_lens=w.q_lens[rows])
    tables, lens = wl.device_tables(w, device)
    varlen = w.query_lens is not None
    qsl = wl.device_query_start(w, device) if varlen else None
    out = torch.empty_like(q)
    plan = None
    if packs and not varlen and partition == 0:
        from aster_amd import plan_prefix_packs

        plan = plan_prefix_packs(w.block_tables, w.context_lens, w.num_q_heads, w.num_kv_heads,
                                 device=device)
    decode_plan, plan_us = None, None
    if planned and not varlen and partition == 0:
        from aster_amd.decode_plan import DEFAULT_TAIL_BLOCKS, plan_decode

        kw = dict(num_q_heads=w.num_q_heads, num_kv_heads=w.num_kv_heads, head_dim=w.head_dim,
                  q_dtype=w.q_dtype, device=device,
                  tail_blocks=DEFAULT_TAIL_BLOCKS if tail is None else tail)
        plan_decode(w.block_tables, w.context_lens, **kw)  # warm the occupancy query
        t0 = time.perf_counter()
        for _ in range(20):
            decode_plan = plan_decode(w.block_tables, w.context_lens, **kw)
        plan_us = (time.perf_counter() - t0) / 20 * 1e6
        plan = None
    ws_bytes = (decode_plan.workspace_bytes() if decode_plan is not None else
                cache.workspace_bytes(w.num_seqs, w.num_q_heads, w.max_context_len, partition,
                                      prefix_packs=plan))
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=device)

    def call(layer, append=None):
        cache.paged_attention(layer, q, tables, lens, max_context_len=w.max_context_len,
                              scale=w.scale, partition_tokens=partition, out=out, workspace=ws,
                              query_start_loc=qsl,
                              max_query_len=w.max_query_len if varlen else None,
                              prefix_packs=plan, decode_plan=decode_plan, append=append)

    call.plan_us = plan_us
    call.planned = decode_plan is not None
    call.chunked = decode_plan is not None and decode_plan.info.num_chunked > 0
    return call, w


def hbm_entry(w, avg_ms, med_ms, nbytes=None):
    nbytes = w.algorithmic_bytes() if nbytes is None else nbytes
    gbs = nbytes / (avg_ms * 1e-3) / 1e9
    return {"call_us": avg_ms * 1e3, "median_call_us": med_ms * 1e3, "algorithmic_bytes": nbytes,
            "achieved_gbs": gbs, "frac": gbs / HBM_PEAK_GBS,
            "attended_kv_tokens_per_s": w.attended_tokens / (avg_ms * 1e-3)}


def extra_measurements(device, partition, calls, planned=True, tail=None):
    """Configs 3, 4 and 5: one attention call each (two layer arenas, alternated, so
    the calls do not reuse each other's K/V from the MALL), HIP events per launch."""
    import numpy as np
    import torch

    from aster_amd import workloads as wl

    out = {}
    # config 3: the mixed call, its decode rows alone, its chunk rows alone (the chunk
    # call also launches the decode kernels, which find no decode row: its MFMA rate is
    # a lower bound for the prefill kernel)
    w = wl.config3()
    cache, _ = build_arena(w, 2, device)
    q = wl.queries(w, device)
    call, _ = attention_caller(w, cache, q, device, partition)
    entry = hbm_entry(w, *time_calls(call, calls, 2))
    dec_rows = np.nonzero(w.q_lens == 1)[0]
    pre_rows = np.nonzero(w.q_lens > 1)[0]
    call, wd = attention_caller(w, cache, q, device, partition, rows=dec_rows)
    entry["decode_rows"] = hbm_entry(wd, *time_calls(call, calls, 2))
    call, wp = attention_caller(w, cache, q, device, partition, rows=pre_rows)
    avg, med = time_calls(call, calls, 2)
    flops = wp.prefill_flops()
    tflops = flops / (avg * 1e-3) / 1e12
    entry["prefill_rows"] = {"call_us": avg * 1e3, "median_call_us": med * 1e3, "flops": flops,
                             "achieved_tflops": tflops, "bound": "mfma",
                             "peak_tflops": MFMA_F16_PEAK_TFLOPS,
                             "frac": tflops / MFMA_F16_PEAK_TFLOPS}
    out[w.name] = entry
    del cache
    torch.cuda.empty_cache()
    # config 4: HBM fraction on the distinct K/V bytes, effective rate on the logical;
    # on the host schedule with prefix tiles (as the runner plans decode steps), with
    # the stream-K kernel's prefix packs, and with neither
    w = wl.config4()
    cache, _ = build_arena(w, 2, device)
    q = wl.queries(w, device)
    call, _ = attention_caller(w, cache, q, device, partition)
    unplanned = time_calls(call, calls, 2)
    call, _ = attention_caller(w, cache, q, device, partition, packs=True)
    packs = time_calls(call, calls, 2)
    if planned:
        call, _ = attention_caller(w, cache, q, device, partition, planned=True, tail=tail)
        avg, med = time_calls(call, calls, 2)
    else:
        avg, med = packs
    entry = hbm_entry(w, avg, med)
    entry["mode"] = "planned, prefix tiles" if planned else "stream-K, prefix packs"
    entry["packs_call_us"] = packs[0] * 1e3
    entry["without_plan_call_us"] = unplanned[0] * 1e3
    entry["logical_effective_gbs"] = entry.pop("achieved_gbs")
    entry["logical_frac"] = entry.pop("frac")
    unique = w.unique_kv_bytes() + (w.algorithmic_bytes() - w.attended_tokens * w.num_kv_heads
                                    * (2 * w.head_dim + 8))
    entry["unique_bytes"] = unique
    entry["unique_gbs"] = unique / (avg * 1e-3) / 1e9
    entry["unique_frac"] = entry["unique_gbs"] / HBM_PEAK_GBS
    out[w.name] = entry
    del cache
    torch.cuda.empty_cache()
    # config 2 with fp32 queries: the planned MFMA path over int8 codes, against the exact
    # fp32 VALU kernel the unplanned call takes
    if planned:
        w = wl.config2()
        cache, _ = build_arena(w, 2, device)
        q32 = wl.queries(w, device).float()
        w32 = wl.DecodeWorkload(w.name + "_fp32_queries", w.num_q_heads, w.num_kv_heads,
                                w.head_dim, w.context_lens, w.block_tables, w.num_blocks,
                                torch.float32, w.seed, w.scale)
        call, _ = attention_caller(w32, cache, q32, device, partition, planned=True, tail=tail)
        entry = hbm_entry(w32, *time_calls(call, calls, 2))
        call, _ = attention_caller(w32, cache, q32, device, partition)
        entry["exact_fp32_kernel"] = hbm_entry(w32, *time_calls(call, calls, 2))
        out[w32.name] = entry
        del cache
        torch.cuda.empty_cache()
    # config 5: the planned call (rows cut into chunks across workgroups), the unplanned
    # stream-K call, and the 512-token split-K partitions the configuration names
    w = wl.config5()
    cache, _ = build_arena(w, 2, device)
    q = wl.queries(w, device)
    call, _ = attention_caller(w, cache, q, device, partition, planned=planned, tail=tail)
    entry = hbm_entry(w, *time_calls(call, calls, 2))
    entry["planned"] = call.planned
    call, _ = attention_caller(w, cache, q, device, partition)
    entry["streamk"] = hbm_entry(w, *time_calls(call, calls, 2))
    call, _ = attention_caller(w, cache, q, device, 512)
    entry["partition_512"] = hbm_entry(w, *time_calls(call, calls, 2))
    out[w.name] = entry
    del cache
    torch.cuda.empty_cache()
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); "
              f"got --gpus {args.gpus}", file=sys.stderr)
        sys.exit(2)
    import torch

    from aster_amd import workloads as wl

    device = torch.device("cuda:0")
    w = getattr(wl, args.config)()
    L = args.layers
    cache, step_batch = build_arena(w, L, device, hold_last=True)
    q = wl.queries(w, device)
    planned = not args.no_plan
    call, _ = attention_caller(w, cache, q, device, args.partition, packs=True, planned=planned,
                               tail=args.tail)
    k_new, v_new, slots = step_batch
    varlen = w.query_lens is not None

    # the runner's step: a planned bf16/fp16 decode appends the new tokens inside the
    # attention launch; otherwise one append launch into the reserved slots, then the call
    fused = call.planned and k_new.dtype == q.dtype and cache.decode_appends(q.dtype)

    def step(i):
        layer = i % L
        if fused:
            call(layer, append=(k_new, v_new, slots))
        else:
            cache.append(layer, k_new, v_new, slots, reserved=True)
            call(layer)

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

    # ---- roofline: the attention call alone, per-launch HIP events on the launch stream
    attn_avg_ms, attn_med_ms = time_calls(call, max(args.steps, 50), L)
    alg_bytes = w.algorithmic_bytes()
    achieved = alg_bytes / (attn_avg_ms * 1e-3) / 1e9
    # HBM bytes per call measured by rocprofv3 (FETCH_SIZE/WRITE_SIZE, calibrated
    # against a copy of known size) for this workload and split mode
    # for this workload, split mode and library build: a figure measured on another build
    # of the library is not reported (traffic then stays null)
    traffic = None
    if os.path.exists(args.traffic):
        import hashlib

        from aster_amd import _native

        mode = ("planned" if call.planned else "streamk") if args.partition == 0 else \
            f"partition_{args.partition}"
        with open(args.traffic) as f:
            rec = json.load(f).get(w.name, {}).get(mode, {})
        with open(_native.LIB_PATH, "rb") as f:
            built = hashlib.sha256(f.read()).hexdigest()
        if rec.get("library_sha256") == built:
            traffic = rec.get("bytes_per_launch")

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
            "step": (f"paged_attention with the append of {int(k_new.shape[0])} tokens (one launch)"
                     if fused else
                     f"quantize_append_reserved({int(k_new.shape[0])} tok) + paged_attention"),
        },
        "hbm_fraction_of_step": alg_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "roofline": {
            "kernel": ("decode_planned_kernel" + (" + merge_chunks_kernel" if call.chunked else "")
                       if call.planned else
                       "decode_streamk_kernel + merge_streamk_kernel" if args.partition == 0 else
                       "decode_mfma_kernel + merge_kernel")
                      + (" + prefill_mfma_kernel" if varlen else "") + " (one paged_attention call)",
            "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
            "algorithmic_bytes_per_launch": alg_bytes,
            "avg_launch_us": attn_avg_ms * 1e3, "median_launch_us": attn_med_ms * 1e3,
        },
        "wall_s_timed_region": wall,
    }
    if call.planned:
        # the schedule is built once per decode step on the host and serves every layer
        result["roofline"]["plan_host_us"] = call.plan_us
        result["config"]["decode_plan"] = "host schedule (astr_decode_plan), built once per step"
        plain, _ = attention_caller(w, cache, q, device, args.partition, packs=True)
        result["roofline"]["unplanned_call_us"] = time_calls(plain, max(args.steps, 50), L)[0] * 1e3
    if varlen:
        result["config"]["query_tokens"] = w.num_query_tokens
        result["config"]["max_query_len"] = w.max_query_len
    if not args.no_extra and args.config == "config2":
        del cache
        torch.cuda.empty_cache()
        result["extra"] = extra_measurements(device, args.partition, args.extra_calls,
                                               planned=planned, tail=args.tail)
        cache, step_batch = build_arena(w, 1, device, hold_last=True)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(w, cache, step_batch, q, args.cpu_runs)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
