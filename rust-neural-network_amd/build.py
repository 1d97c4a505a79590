"""Build librnn_hip.so (the C-ABI library of include/rnn_hip.h) for gfx950.

Every .hip file under csrc/ is compiled by hipcc to an object in _build/ and
linked into rust-neural-network_amd/librnn_hip.so, next to this file, so the
library travels with the source tree. The files under csrc/probe/ (the
benchmark's read-floor helper, not part of the C ABI) are linked into
librnn_probe.so beside it. Run `python build.py` or call build().
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
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "librnn_hip.so")
PROBE_LIB = os.path.join(HERE, "librnn_probe.so")

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -ffp-contract=off and correctly rounded division keep every float result
# equal to the Rust reference's (which never fuses a*b+c); packed fp32 ops are
# disabled for all HIP code.
HIPFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def _scratch_kernels(remarks: str) -> list[str]:
    """Kernels whose resource-usage remark reports private (scratch) memory."""
    bad, name = [], None
    for line in remarks.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and int(m.group(1)) > 0:
            bad.append(f"{name} ({m.group(1)} B/lane)")
    return bad


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.relpath(src, CSRC).replace(os.sep, "_") + ".o")
    cmd = [HIPCC, *HIPFLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    # Every kernel here keeps its accumulators and fragments in registers; a
    # kernel the compiler demoted to scratch memory still computes the right
    # values but runs one to two orders of magnitude slower, so it is a build
    # error rather than a silent regression.
    bad = _scratch_kernels(r.stderr)
    if bad:
        raise RuntimeError(f"{src}: kernels use scratch memory: {', '.join(bad)}")
    return obj


def build(verbose: bool = False) -> str:
    """Compile all kernels and link librnn_hip.so; returns the library path."""
    if not os.path.exists(HIPCC) and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found; librnn_hip.so cannot be built")
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    probe_srcs = sorted(glob.glob(os.path.join(CSRC, "probe", "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs) + len(probe_srcs))) as ex:
        objs = list(ex.map(_compile, srcs + probe_srcs))
    for lib, lib_objs in ((LIB, objs[:len(srcs)]), (PROBE_LIB, objs[len(srcs):])):
        tmp = lib + ".tmp"
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *lib_objs]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
        os.replace(tmp, lib)
        if verbose:
            print(f"built {lib}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
