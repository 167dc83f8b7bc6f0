"""Build libuttt_hip.so in-tree for gfx950 with hipcc.

    python -m uttt_amd.build

Every csrc/*.hip file is compiled to an object under uttt_amd/_build/ (in
parallel), then linked into uttt_amd/libuttt_hip.so.  All device code is
built with packed-FP32 instructions disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import re
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libuttt_hip.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


# Sources whose kernels must not use scratch memory: the grouped GEMMs and the
# staged uTTT-Dense stage 1 issue their LDS fragment reads as inline asm with
# explicit waits, so a register spill between a read and its wait would save
# the value from before the read;
# the one-launch Newton-Schulz holds its accumulators and the products it
# writes back across barriers, where a spill would cost more than the work.
NO_SCRATCH = {"grouped_gemm.hip", "ns_small.hip", "dense_update.hip"}


def _scratch_kernels(remarks: str) -> list:
    """Kernels with a nonzero ScratchSize in hipcc's resource-usage remarks."""
    bad, name = [], None
    for line in remarks.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            continue
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and name and int(m.group(1)) > 0:
            bad.append(f"{name} ({m.group(1)} bytes/lane)")
    return bad


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src).replace(".hip", ".o"))
    cmd = [HIPCC, *COMMON_FLAGS, "-c", src, "-o", obj]
    guard = os.path.basename(src) in NO_SCRATCH
    if guard:
        cmd.append("-Rpass-analysis=kernel-resource-usage")
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{out}")
    if guard:
        bad = _scratch_kernels(proc.stdout)
        if bad:
            raise RuntimeError(f"{src}: kernels spill to scratch memory: {', '.join(bad)}")
    return obj


def build(verbose: bool = False) -> str:
    """Compile every kernel source and link the shared library; returns its path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
