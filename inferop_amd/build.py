"""Build libinferop.so in-tree for gfx950.

hipcc compiles the HIP translation units (kernels + thin C launch layer);
g++ compiles the C++ front end (ops.h / inferop_c.h), which includes no HIP
header; hipcc links both into inferop_amd/libinferop.so.  Objects go to
_build/ (git-ignored).  Usage: python -m inferop_amd.build [-v]
"""
from __future__ import annotations

import os
import subprocess
import sys
import time

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(ROOT, "_build")
LIB = os.path.join(PKG, "libinferop.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")

HIP_SOURCES = ["quant.hip", "gemm.hip", "device.hip", "moe.hip"]
CXX_SOURCES = ["ops.cpp"]

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-I" + INCLUDE, "-I" + CSRC,
    # no packed-fp32 instructions anywhere in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]
# per-source extra flags: MFMA results in VGPRs (not AGPRs), so the fp32
# scale promotion reads them directly and independent MFMAs get distinct
# destination registers
EXTRA_FLAGS = {"gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
               "device.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}
# sources whose per-kernel resource usage (registers, scratch, occupancy) the
# compiler reports into _build/<source>.resources.txt rather than the console;
# tests/test_kernel_resources.py reads it
RESOURCE_REPORT = ("gemm.hip", "quant.hip")
RESOURCE_FLAG = "-Rpass-analysis=kernel-resource-usage"
CXX_FLAGS = ["-O2", "-fPIC", "-std=c++17", "-I" + INCLUDE, "-I" + CSRC, "-Wall", "-Wextra"]


def _run(cmds, verbose, reports=None):
    """Run the commands in parallel; reports maps a command's index to a file
    that receives its compiler output instead of the console."""
    reports = reports or {}
    procs = []
    for cmd in cmds:
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                                            text=True)))
    failed = []
    for i, (cmd, p) in enumerate(procs):
        out, _ = p.communicate()
        out = "\n".join(l for l in out.splitlines()
                        if "packed-fp32-ops' is not a recognized feature" not in l)
        if i in reports:
            with open(reports[i], "w") as f:
                f.write(out + "\n")
            if p.returncode == 0:
                continue
        if p.returncode != 0:
            failed.append((cmd, out))
        elif verbose and out.strip():
            print(out)
    if failed:
        for cmd, out in failed:
            sys.stderr.write("FAILED: " + " ".join(cmd) + "\n" + out + "\n")
        raise RuntimeError("libinferop build failed")


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    t0 = time.time()
    objs, cmds, reports = [], [], {}
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, src + ".o")
        objs.append(obj)
        extra = list(EXTRA_FLAGS.get(src, []))
        if src in RESOURCE_REPORT:
            extra.append(RESOURCE_FLAG)
            reports[len(cmds)] = os.path.join(BUILD, src + ".resources.txt")
        cmds.append([HIPCC, *HIP_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj])
    for src in CXX_SOURCES:
        obj = os.path.join(BUILD, src + ".o")
        objs.append(obj)
        cmds.append([CXX, *CXX_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    _run(cmds, verbose, reports)
    tmp = LIB + ".tmp"
    _run([[HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]], verbose)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} in {time.time() - t0:.1f}s")
    return LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
