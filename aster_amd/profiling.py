"""Measurement helpers for the INT8 paged-decode kernels.

  python -m aster_amd.profiling copy [--gib N]
      Copy N GiB (default 1) device-to-device three times. Run under
      ``rocprofv3 --pmc FETCH_SIZE`` / ``--pmc WRITE_SIZE`` to calibrate what those
      counters report for a transfer of known size (bytes per launch = counter
      KiB * 1024 * known_bytes / counted_bytes).
  python -m aster_amd.profiling summarize <rocprof_dir> [kernel_substring]
      Mean, median and maximum of every collected counter per kernel, from the
      ``*_counter_collection.csv`` files rocprofv3 writes with --output-format csv
      (the median is the typical dispatch where a run mixes full and near-empty
      launches of one kernel, e.g. bench.py's prefill-only calls in a mixed step).
  python -m aster_amd.profiling durations <rocprof_dir> [kernel_substring]
      The same statistics of kernel durations (us) from ``*_kernel_trace.csv``.
  python -m aster_amd.profiling timeline [config2|config4|config5] [--packs | --planned [--tail N] [--tile-ranges R]]
      Per-wave timeline of the stream-K (or, --planned, the planned) decode kernel on a
      BASELINE workload, from
      the trace build (``python -m aster_amd.build --trace``, which records wall-clock
      marks per wave): when waves start, have their block ids and first block, and
      end, per XCC and by the number of pieces (rows) a wave streams, and what a row
      start inside a wave costs; with --planned on a plan with prefix tiles (config4),
      also the prefix-tile kernel's waves: members checked, queries quantized, first
      and later key steps, partials stored. Runs a few calls and reads the last one.
  python -m aster_amd.profiling traffic <fetch_dir> <write_dir> <cal_fetch_dir> <cal_write_dir> [kernel_substring]
      HBM bytes per launch per kernel (median dispatch) from a FETCH_SIZE and a
      WRITE_SIZE run, each scaled by what the counter reads for ``copy`` (the
      ``cal_*`` runs): the figures of profiles/decode_traffic.json.
  python -m aster_amd.profiling calls [config] [--packs] [--q-dtype T] [--calls N] [--planned]
      N paged_attention calls of a BASELINE decode workload (four layer arenas,
      cycled), with the workload's queries cast to T: the program to run under
      rocprofv3 for a kernel bench.py does not time (float32 queries run the exact
      fp32 decode kernel).
"""

from __future__ import annotations

import argparse
import collections
import csv
import glob
import re


def copy(gib=1.0):
    import torch

    n = int(gib * (1 << 30))
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"copied {n} bytes x3", flush=True)


def _short(name):
    return re.sub(r"\(anonymous namespace\)::", "", name).replace("void ", "").split("(")[0]


def _stats(values):
    out = {}
    for key, v in sorted(values.items()):
        v = sorted(v)
        out[key] = (len(v), sum(v) / len(v), v[len(v) // 2], v[-1])
    return out


def summarize(root, pattern=""):
    """{(kernel, counter): (dispatches, mean, median, max)}"""
    values = collections.defaultdict(list)
    for path in glob.glob(f"{root}/**/*counter_collection.csv", recursive=True):
        with open(path) as f:
            for row in csv.DictReader(f):
                name = row.get("Kernel_Name", "")
                if pattern not in name:
                    continue
                values[(_short(name), row["Counter_Name"])].append(float(row["Counter_Value"]))
    return _stats(values)


def durations(root, pattern=""):
    """{(kernel, "us"): (dispatches, mean, median, max)}"""
    values = collections.defaultdict(list)
    for path in glob.glob(f"{root}/**/*kernel_trace.csv", recursive=True):
        with open(path) as f:
            for row in csv.DictReader(f):
                name = row.get("Kernel_Name", "")
                if pattern not in name:
                    continue
                us = (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3
                values[(_short(name), "us")].append(us)
    return _stats(values)


def traffic(fetch_dir, write_dir, cal_fetch_dir, cal_write_dir, pattern="astr", gib=1.0):
    """HBM bytes per launch of each kernel matching ``pattern`` (median dispatch) from
    a FETCH_SIZE run and a WRITE_SIZE run, each counter scaled by what it reads for
    ``copy(gib)``: {"bytes_per_launch", "kernels", "calibration"}."""
    known = gib * (1 << 30)

    def per_kernel(root, counter, pat):
        return {k: med for (k, c), (_, _, med, _) in summarize(root, pat).items() if c == counter}

    cal_f = max(per_kernel(cal_fetch_dir, "FETCH_SIZE", "").values())
    cal_w = max(per_kernel(cal_write_dir, "WRITE_SIZE", "").values())
    fs, ws = known / (cal_f * 1024), known / (cal_w * 1024)
    fetch = per_kernel(fetch_dir, "FETCH_SIZE", pattern)
    write = per_kernel(write_dir, "WRITE_SIZE", pattern)
    kernels = {k.split("<")[0]: round(fetch[k] * 1024 * fs + write.get(k, 0.0) * 1024 * ws)
               for k in fetch}
    return {"bytes_per_launch": sum(kernels.values()), "kernels": kernels,
            "calibration": {"fetch_scale": round(fs, 7), "write_scale": round(ws, 7)}}


def _decode_calls(config, packs, q_dtype, calls, planned=False, tail=None, tile_ranges=0):
    """Run ``calls`` paged_attention calls of a BASELINE decode workload over four layer
    arenas, cycled, so that a call does not find the previous call's K/V in the
    memory-side cache (as bench.py does). ``q_dtype`` overrides the workload's query
    type ("float32" routes to the exact fp32 kernel). Returns the decode plan of
    ``planned`` calls (else None)."""
    import torch

    from . import workloads as wl
    from .paged_kv import PagedKVCache
    from .prefix_plan import plan_prefix_packs

    w = getattr(wl, config)()
    dev = torch.device("cuda:0")
    layers = 4
    cache = PagedKVCache(num_blocks=w.num_blocks, num_layers=layers,
                         num_kv_heads=w.num_kv_heads, head_dim=w.head_dim, device=dev)
    wl.materialize(w, cache, device=dev)
    for layer in range(1, layers):
        cache.codes[:, layer].copy_(cache.codes[:, 0])
        cache.scales[:, layer].copy_(cache.scales[:, 0])
    tables, lens = wl.device_tables(w, dev)
    q = wl.queries(w, dev)
    if q_dtype:
        q = q.to(getattr(torch, q_dtype))
    plan = (plan_prefix_packs(w.block_tables, w.context_lens, w.num_q_heads, w.num_kv_heads,
                              device=dev) if packs else None)
    schedule = None
    if planned:
        from .decode_plan import DEFAULT_TAIL_BLOCKS, plan_decode

        schedule = plan_decode(w.block_tables, w.context_lens, num_q_heads=w.num_q_heads,
                               num_kv_heads=w.num_kv_heads, head_dim=w.head_dim,
                               q_dtype=q.dtype, device=dev,
                               tail_blocks=DEFAULT_TAIL_BLOCKS if tail is None else tail,
                               tile_ranges=tile_ranges)
        plan = None
    for i in range(calls):
        cache.paged_attention(i % layers, q, tables, lens, max_context_len=w.max_context_len,
                              scale=w.scale, prefix_packs=plan, decode_plan=schedule)
    torch.cuda.synchronize()
    print(f"{calls} calls of {config} (packs={bool(packs)}, planned={bool(planned)}, "
          f"queries {q.dtype})", flush=True)
    return schedule


def _trace_marks(lib, reader, n):
    """(marks, info) of the first ``n`` waves from a trace build's reader entry."""
    import ctypes

    import numpy as np

    fn = getattr(lib, reader)
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
    marks = np.zeros((n, 8), np.int64)
    info = np.zeros((n, 4), np.int32)
    rc = fn(marks.ctypes.data, info.ctypes.data, n)
    if rc != 0:
        raise RuntimeError(f"{reader} failed ({rc})")
    return marks, info


def _tiles_report(marks, info, decode_start):
    """Timeline of the prefix-tile kernel's waves (us from the first tile wave's start)
    and the gap to the planned decode kernel's first wave (``decode_start``, raw clock)."""
    import numpy as np

    live = marks[:, 0] != 0
    marks, info = marks[live], info[live]
    origin = marks[:, 0].min()
    t = (marks - origin) / 100.0
    steps, xcc = info[:, 0], info[:, 1]
    pct = lambda x, p: [round(float(v), 2) for v in np.percentile(x, p)]
    multi = steps > 1
    return {"waves": int(live.sum()), "steps_per_unit": pct(steps, [0, 50, 100]),
            "start_us": pct(t[:, 0], [0, 50, 100]),
            "checked_us": pct(t[:, 1] - t[:, 0], [50, 90]),
            "queries_us": pct(t[:, 2] - t[:, 1], [50, 90]),
            "first_step_us": pct(t[:, 3] - t[:, 2], [50, 90]),
            "later_step_us": (round(float(((t[multi, 4] - t[multi, 3]) /
                                           (steps[multi] - 1)).mean()), 3)
                              if multi.any() else None),
            "store_us": pct(t[:, 5] - t[:, 4], [50, 90]),
            "exit_pct_50_90_100_us": pct(t[:, 5], [50, 90, 100]),
            "per_xcc_max_exit": {int(x): round(float(t[xcc == x, 5].max()), 2)
                                 for x in np.unique(xcc)},
            "decode_first_wave_after_last_tile_us": round(
                float((decode_start - marks[:, 5].max()) / 100.0), 2)}


def planned_timeline(config="config2", calls=7, tail=None, tile_ranges=0):
    """The trace build's per-wave marks of the planned decode kernel (the last of
    ``calls`` planned calls over ``config``), as a report dict (us from the first wave's
    start): startup to items checked, block ids, first block; streaming end; the
    workgroup barrier; exit after the workgroup's merges. Where the plan has prefix
    tiles, ``tiles`` gives the tile kernel's timeline in the same call."""
    import contextlib
    import io

    import numpy as np

    from . import _native, build

    _native.LIB_PATH = build.TRACE_OUT
    _native._lib = None
    lib = _native.lib()
    with contextlib.redirect_stdout(io.StringIO()):
        plan = _decode_calls(config, False, None, calls, planned=True, tail=tail,
                             tile_ranges=tile_ranges)
    marks, info = _trace_marks(lib, "astr_trace_read_planned", 16384)
    tiles = None
    if plan is not None and plan.info.num_tiles > 0:
        tm, ti = _trace_marks(lib, "astr_trace_read_tiles", 8192)
        tiles = _tiles_report(tm, ti, marks[marks[:, 0] != 0, 0].min())
    live = marks[:, 0] != 0
    wave_ids = np.nonzero(live)[0]
    marks, info = marks[live], info[live]
    t = (marks - marks[:, 0].min()) / 100.0
    nblk, pieces, items, xcc = info.T
    pct = lambda x, p: [round(float(v), 2) for v in np.percentile(x, p)]
    streaming = nblk > 0
    wg = wave_ids // 8
    wg_end = np.array([t[wg == g, 4].max() for g in np.unique(wg)])
    rep = {"config": config, "waves": int(live.sum()), "span_us": round(float(t[:, 6].max()), 2),
           "start_us": pct(t[:, 0], [0, 50, 100]),
           "items_checked_us": pct(t[:, 1] - t[:, 0], [50, 90]),
           "ids_us": pct(t[:, 2] - t[:, 0], [50, 90]),
           "first_block_us": pct(t[streaming, 3] - t[streaming, 0], [50, 90]),
           "stream_end_pct_10_50_90_99_100_us": pct(t[:, 4], [10, 50, 90, 99, 100]),
           "workgroup_stream_end_pct_10_50_90_100_us": pct(wg_end, [10, 50, 90, 100]),
           "barrier_wait_us": pct(t[:, 5] - t[:, 4], [50, 90]),
           "merge_us": pct(t[:, 6] - t[:, 5], [50, 90, 100]),
           "exit_pct_50_90_100_us": pct(t[:, 6], [50, 90, 100]),
           "blocks_per_wave": pct(nblk, [0, 50, 100]),
           "items_per_workgroup": pct(items, [0, 50, 100]),
           "us_per_block": round(float(((t[streaming, 4] - t[streaming, 3]) /
                                        np.maximum(nblk[streaming], 1)).mean()), 3)}
    # spread of the streaming ends: all waves, waves within their workgroup, and the
    # workgroups' mean ends (what balancing inside a workgroup could and could not remove)
    ends = t[:, 4]
    groups = np.unique(wg)
    rep["stream_end_sd_us"] = {
        "waves": round(float(ends.std()), 2),
        "within_workgroups": round(float(np.sqrt(np.mean([ends[wg == g].var()
                                                          for g in groups]))), 2),
        "workgroup_means": round(float(np.std([ends[wg == g].mean() for g in groups])), 2)}
    rep["per_xcc"] = {int(x): {"waves": int((xcc == x).sum()),
                               "mean_end": round(float(t[xcc == x, 4].mean()), 2),
                               "max_end": round(float(t[xcc == x, 4].max()), 2)}
                      for x in np.unique(xcc)}
    if tiles is not None:
        rep["tiles"] = tiles
    # per number of pieces (rows the wave starts): end time and streaming time per block
    rep["by_pieces"] = {}
    for k in sorted(np.unique(np.minimum(pieces[streaming], 4))):
        m = streaming & (np.minimum(pieces, 4) == k)
        rep["by_pieces"][f"{k}{'+' if k == 4 else ''}"] = {
            "waves": int(m.sum()), "mean_end": round(float(t[m, 4].mean()), 2),
            "mean_blocks": round(float(nblk[m].mean()), 1),
            "us_per_block": round(float(((t[m, 4] - t[m, 3]) / np.maximum(nblk[m], 1)).mean()), 3)}
    return rep


def timeline(config="config2", packs=False, calls=7):
    """The trace build's per-wave marks of the last of ``calls`` attention calls over
    ``config`` (four layer arenas, cycled), as a report dict (times in us from the
    first wave's start)."""
    import ctypes
    import contextlib
    import io

    import numpy as np

    from . import _native, build

    _native.LIB_PATH = build.TRACE_OUT
    _native._lib = None
    lib = _native.lib()
    lib.astr_trace_read.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
    with contextlib.redirect_stdout(io.StringIO()):
        _decode_calls(config, packs, None, calls)
    n = 16384
    marks = np.zeros((n, 8), np.int64)
    info = np.zeros((n, 4), np.int32)
    rc = lib.astr_trace_read(marks.ctypes.data, info.ctypes.data, n)
    if rc != 0:
        raise RuntimeError(f"astr_trace_read failed ({rc})")
    live = marks[:, 0] != 0
    marks, info = marks[live], info[live]
    t = (marks - marks[:, 0].min()) / 100.0  # s_memrealtime ticks at 100 MHz
    nblk, pieces, packblk, xcc = info.T
    pct = lambda x, p: [round(float(v), 2) for v in np.percentile(x, p)]
    rep = {"config": config, "packs": bool(packs), "waves": int(live.sum()),
           "span_us": round(float(t[:, 4].max()), 2),
           "start_us": pct(t[:, 0], [0, 50, 100]),
           "prefix_done_us": pct(t[:, 1] - t[:, 0], [50, 90]),
           "ids_us": pct(t[:, 2] - t[:, 0], [50, 90]),
           "first_block_us": pct(t[:, 3] - t[:, 0], [50, 90]),
           "end_pct_10_50_90_99_100_us": pct(t[:, 4], [10, 50, 90, 99, 100]),
           "blocks_per_wave": pct(nblk, [0, 50, 100])}
    rep["per_xcc"] = {int(x): {"waves": int((xcc == x).sum()),
                               "mean_start": round(float(t[xcc == x, 0].mean()), 2),
                               "mean_end": round(float(t[xcc == x, 4].mean()), 2),
                               "max_end": round(float(t[xcc == x, 4].max()), 2)}
                      for x in np.unique(xcc)}
    groups = {}
    for k in sorted(np.unique(np.minimum(pieces, 3))):
        m = np.minimum(pieces, 3) == k
        groups[f"{k}{'+' if k == 3 else ''} pieces"] = {
            "waves": int(m.sum()), "mean_end": round(float(t[m, 4].mean()), 2),
            "p90_end": round(float(np.percentile(t[m, 4], 90)), 2),
            "us_per_block": round(float(((t[m, 4] - t[m, 3]) / np.maximum(nblk[m], 1)).mean()), 3)}
    rep["by_pieces"] = groups
    two = pieces >= 2
    if two.any():
        rep["row_start_us"] = {
            "end_of_first_piece_to_query_ready": pct(t[two, 6] - t[two, 5], [50, 90]),
            "query_ready_to_first_block": pct(t[two, 7] - t[two, 6], [50, 90])}
    if packs:
        kind = np.where(packblk == nblk, "pack", np.where(packblk == 0, "sequence", "mixed"))
        rep["by_kind"] = {k: {"waves": int((kind == k).sum()),
                              "mean_end": round(float(t[kind == k, 4].mean()), 2),
                              "us_per_block": round(float(((t[kind == k, 4] - t[kind == k, 3]) /
                                                          np.maximum(nblk[kind == k], 1)).mean()), 3)}
                          for k in np.unique(kind)}
    return rep


def main():
    p = argparse.ArgumentParser()
    sub = p.add_subparsers(dest="cmd", required=True)
    c = sub.add_parser("copy")
    c.add_argument("--gib", type=float, default=1.0)
    for cmd in ("summarize", "durations"):
        s = sub.add_parser(cmd)
        s.add_argument("root")
        s.add_argument("pattern", nargs="?", default="")
    t = sub.add_parser("timeline")
    t.add_argument("config", nargs="?", default="config2")
    t.add_argument("--packs", action="store_true")
    t.add_argument("--planned", action="store_true")
    t.add_argument("--tail", type=int, default=None)
    t.add_argument("--tile-ranges", type=int, default=0)
    d = sub.add_parser("calls")
    d.add_argument("config", nargs="?", default="config2")
    d.add_argument("--packs", action="store_true")
    d.add_argument("--q-dtype", default=None, choices=["float32", "float16", "bfloat16"])
    d.add_argument("--calls", type=int, default=50)
    d.add_argument("--planned", action="store_true")
    d.add_argument("--tail", type=int, default=None)
    h = sub.add_parser("traffic")
    for name in ("fetch_dir", "write_dir", "cal_fetch_dir", "cal_write_dir"):
        h.add_argument(name)
    h.add_argument("pattern", nargs="?", default="astr")
    args = p.parse_args()
    if args.cmd == "copy":
        copy(args.gib)
        return
    if args.cmd == "traffic":
        import json

        print(json.dumps(traffic(args.fetch_dir, args.write_dir, args.cal_fetch_dir,
                                 args.cal_write_dir, args.pattern), indent=1))
        return
    if args.cmd == "calls":
        _decode_calls(args.config, args.packs, args.q_dtype, args.calls, args.planned, args.tail)
        return
    if args.cmd == "timeline":
        import json

        rep = (planned_timeline(args.config, tail=args.tail, tile_ranges=args.tile_ranges)
               if args.planned else
               timeline(args.config, args.packs))
        print(json.dumps(rep, indent=1))
        return
    table = (summarize if args.cmd == "summarize" else durations)(args.root, args.pattern)
    for (kernel, counter), (n, mean, median, top) in table.items():
        print(f"{kernel:70s} {counter:24s} n={n:4d} mean={mean:.6g} median={median:.6g} "
              f"max={top:.6g}")


if __name__ == "__main__":
    main()
