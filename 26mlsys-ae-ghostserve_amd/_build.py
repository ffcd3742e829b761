"""Builds libkvec.so (every csrc/*.hip, gfx950) in-tree with hipcc.

The library has no torch dependency: it is a plain C-ABI shared object that
links only the HIP runtime.  Objects go to ``_build/`` next to this file.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import re
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OBJDIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libkvec.so")

ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    # keep the compiler from forming packed-FP32 VALU ops
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-I", CSRC,
    "-I", INCLUDE,
]


def hipcc() -> str:
    cand = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(cand):
        raise RuntimeError("hipcc not found; libkvec.so cannot be built")
    return cand


def register_spills(remarks: str) -> list:
    """(kernel, kind, count) for every kernel the resource-usage remarks report
    with spilled SGPRs or VGPRs.  Kernels here that spilled SGPRs to VGPR lanes
    produced run-to-run different bytes on gfx950, and a build variant that
    spilled VGPRs to scratch produced wrong bytes, so the build rejects both.
    (Scratch that holds a small array indexed at run time is not a spill.)"""
    out, name = [], None
    for line in remarks.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            continue
        m = re.search(r"([SV]GPRs) Spill: (\d+)", line)
        if m and int(m.group(2)) > 0:
            out.append((name, m.group(1), int(m.group(2))))
    return out


def _compile(src: str) -> str:
    obj = os.path.join(OBJDIR, os.path.basename(src)[:-4] + ".o")
    cmd = [hipcc(), *FLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", src, "-o", obj]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{r.stdout}")
    spills = register_spills(r.stdout)
    if spills:
        names = "\n  ".join(f"{n}: {c} {kind}" for n, kind, c in spills)
        raise RuntimeError(f"{os.path.basename(src)}: kernels spill registers:\n  {names}")
    return obj


def build(jobs: int | None = None) -> str:
    """Compile every csrc/*.hip and link libkvec.so; returns its path."""
    os.makedirs(OBJDIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
           "-Wl,-rpath,/opt/rocm/lib"]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link of libkvec.so failed:\n{r.stdout}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
