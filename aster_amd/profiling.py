"""Measurement helpers for the INT8 paged-decode kernels.

  python -m aster_amd.profiling copy [--gib N]
      Copy N GiB (default 1) device-to-device three times. Run under
      ``rocprofv3 --pmc FETCH_SIZE`` / ``--pmc WRITE_SIZE`` to calibrate what those
      counters report for a transfer of known size (bytes per launch = counter
      KiB * 1024 * known_bytes / counted_bytes).
  python -m aster_amd.profiling summarize <rocprof_dir> [kernel_substring]
      Mean value of every collected counter per kernel, from the
      ``*_counter_collection.csv`` files rocprofv3 writes with --output-format csv.
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


def summarize(root, pattern=""):
    values = collections.defaultdict(list)
    for path in glob.glob(f"{root}/**/*counter_collection.csv", recursive=True):
        with open(path) as f:
            for row in csv.DictReader(f):
                name = row.get("Kernel_Name", "")
                if pattern not in name:
                    continue
                short = re.sub(r"\(anonymous namespace\)::", "", name).replace("void ", "")
                values[(short.split("(")[0], row["Counter_Name"])].append(
                    float(row["Counter_Value"]))
    return {key: (len(v), sum(v) / len(v)) for key, v in sorted(values.items())}


def main():
    p = argparse.ArgumentParser()
    sub = p.add_subparsers(dest="cmd", required=True)
    c = sub.add_parser("copy")
    c.add_argument("--gib", type=float, default=1.0)
    s = sub.add_parser("summarize")
    s.add_argument("root")
    s.add_argument("pattern", nargs="?", default="")
    args = p.parse_args()
    if args.cmd == "copy":
        copy(args.gib)
    else:
        for (kernel, counter), (n, mean) in summarize(args.root, args.pattern).items():
            print(f"{kernel:70s} {counter:24s} n={n:4d} mean={mean:.6g}")


if __name__ == "__main__":
    main()
