"""Build ``aster_amd/_lib/libaster_kv.so`` for gfx950 with hipcc (in-tree).

Flags: IEEE-correct fp32 division/sqrt and no denormal flushing (the quantizer is
bit-exact with torch-CPU fp32 arithmetic); packed-FP32 instructions disabled.
Usage: ``python -m aster_amd.build [--verbose]``.
"""

from __future__ import annotations

import concurrent.futures
import os
import re
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_lib")
OUT = os.path.join(OUT_DIR, "libaster_kv.so")
SOURCES = ("errors.hip", "kv_quantize.hip", "paged_attention.hip", "decode_partition.hip",
           "decode_streamk.hip", "decode_planned.hip", "prefill.hip", "kv_copy.hip",
           "softmax_merge.hip", "decode_plan.cpp")
# attention kernels built once per KV code format (int8, FP8 E4M3FN, FP8 E5M2):
# -DASTR_KF=k selects the format of that object's instantiations
PER_FORMAT = ("decode_partition.hip", "decode_streamk.hip", "decode_planned.hip", "prefill.hip")
FORMATS = (0, 1, 2)


# The stream-K source builds as two units per format (decode_streamk.hip, ASTR_SK_PART):
# the launches with prefix packs and the entry point, and the launches without packs
# under the max-ilp scheduler (measured: config 2 69.8 -> 69.4 us, config 4 without a
# plan 154.6 -> 151.8 us; the pack launches, 74.9 -> 76.9 us under it, and the head-dim
# 256 launches, which spill to scratch under it, keep the default scheduler). Trace
# builds keep it as one unit.
STREAMK_PLAIN_FLAGS = ["-mllvm", "-amdgpu-sched-strategy=max-ilp"]


def units(trace=False):
    """(source, object stem, extra flags) of every translation unit."""
    out = []
    for s in SOURCES:
        stem = os.path.splitext(s)[0]
        if s == "decode_streamk.hip" and not trace:
            for k in FORMATS:
                out.append((s, f"{stem}_kf{k}", [f"-DASTR_KF={k}", "-DASTR_SK_PART=1"]))
                out.append((s, f"{stem}_plain_kf{k}",
                            [f"-DASTR_KF={k}", "-DASTR_SK_PART=2", *STREAMK_PLAIN_FLAGS]))
        elif s in PER_FORMAT:
            out += [(s, f"{stem}_kf{k}", [f"-DASTR_KF={k}"]) for k in FORMATS]
        else:
            out.append((s, stem, []))
    return out
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-gpu-flush-denormals-to-zero",
    # keep MFMA accumulators in VGPRs (no AGPR copies): 3 waves/SIMD for D=128
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Wno-unused-command-line-argument",
]
NOISE = "is not a recognized feature for this target"
# Every kernel must run without scratch memory: a lambda or array the compiler
# cannot keep in registers lands in per-lane scratch and costs several times the
# kernel's HBM time, so the build rejects it.
RESOURCE_REMARKS = "-Rpass-analysis=kernel-resource-usage"


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the HIP library cannot be built")
    return path


# MFMA accumulators live in VGPRs (-amdgpu-mfma-vgpr-form), so AGPRs only appear as
# spill space beyond 256 VGPRs, and they cost occupancy (a kernel that needed 217
# registers ran at 313 and one wave per SIMD after a change that went unnoticed).
# The exact fp32 VALU decode kernels (fp32 queries) are known to spill this way.
AGPR_SPILL_ALLOWED = ("decode_valu_kernel",)


def _scratch_kernels(remarks):
    """Kernels whose resource-usage remark reports a non-zero scratch size, or AGPRs
    (spilled VGPRs) outside AGPR_SPILL_ALLOWED."""
    bad, name = [], None
    for line in remarks.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            continue
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and int(m.group(1)) > 0:
            bad.append(f"{name} ({m.group(1)} bytes/lane of scratch)")
        m = re.search(r"AGPRs: (\d+)", line)
        if m and int(m.group(1)) > 0 and not any(k in (name or "") for k in AGPR_SPILL_ALLOWED):
            bad.append(f"{name} ({m.group(1)} AGPRs: VGPRs spilled)")
    return bad


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    lines = [l for l in proc.stderr.splitlines() if NOISE not in l]
    err = "\n".join(l for l in lines if "kernel-resource-usage" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    bad = _scratch_kernels("\n".join(lines))
    if bad:
        raise RuntimeError("kernels spilling registers:\n  " + "\n  ".join(bad))
    if verbose and err.strip():
        print(err, file=sys.stderr)


TRACE_OUT = os.path.join(OUT_DIR, "trace", "libaster_kv.so")
# roctx ranges of the C-ABI calls (rocprofiler-sdk's roctx, part of the ROCm image and
# found at run time through the system library path, like the HIP runtime)
ROCM_LIB = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib")
LINK = [f"-L{ROCM_LIB}", "-lrocprofiler-sdk-roctx"]


def build(verbose=False, jobs=None, trace=False):
    """Compile every translation unit (in parallel) and link the shared library. With
    ``trace`` the stream-K kernel records per-wave wall-clock marks (-DASTR_TRACE=1)
    into a separate library, TRACE_OUT, for ``aster_amd.profiling timeline``."""
    out = TRACE_OUT if trace else OUT
    obj_dir = os.path.join(os.path.dirname(out), "obj")
    os.makedirs(obj_dir, exist_ok=True)
    plan = units(trace)
    objs = [os.path.join(obj_dir, stem + ".o") for _, stem, _ in plan]
    defs = ["-DASTR_TRACE=1"] if trace else []
    compiles = [[hipcc(), *FLAGS, *extra, *defs, RESOURCE_REMARKS, "-I",
                 os.path.join(ROOT, "include"), "-c", os.path.join(CSRC, s), "-o", o]
                for (s, _, extra), o in zip(plan, objs)]
    jobs = jobs or min(len(compiles), os.cpu_count() or 1, 8)
    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        for f in [pool.submit(_run, c, verbose) for c in compiles]:
            f.result()
    tmp = out + ".tmp"
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, *LINK, "-o", tmp], verbose)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose="--verbose" in sys.argv, trace="--trace" in sys.argv))
