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


def main():
    p = argparse.ArgumentParser()
    sub = p.add_subparsers(dest="cmd", required=True)
    c = sub.add_parser("copy")
    c.add_argument("--gib", type=float, default=1.0)
    for cmd in ("summarize", "durations"):
        s = sub.add_parser(cmd)
        s.add_argument("root")
        s.add_argument("pattern", nargs="?", default="")
    args = p.parse_args()
    if args.cmd == "copy":
        copy(args.gib)
        return
    table = (summarize if args.cmd == "summarize" else durations)(args.root, args.pattern)
    for (kernel, counter), (n, mean, median, top) in table.items():
        print(f"{kernel:70s} {counter:24s} n={n:4d} mean={mean:.6g} median={median:.6g} "
              f"max={top:.6g}")


if __name__ == "__main__":
    main()
