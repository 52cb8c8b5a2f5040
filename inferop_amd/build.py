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
CXX_FLAGS = ["-O2", "-fPIC", "-std=c++17", "-I" + INCLUDE, "-I" + CSRC, "-Wall", "-Wextra"]


def _run(cmds, verbose):
    procs = []
    for cmd in cmds:
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                                            text=True)))
    failed = []
    for cmd, p in procs:
        out, _ = p.communicate()
        out = "\n".join(l for l in out.splitlines()
                        if "packed-fp32-ops' is not a recognized feature" not in l)
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
    objs, cmds = [], []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, src + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, *EXTRA_FLAGS.get(src, []), "-c", os.path.join(CSRC, src),
                     "-o", obj])
    for src in CXX_SOURCES:
        obj = os.path.join(BUILD, src + ".o")
        objs.append(obj)
        cmds.append([CXX, *CXX_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    _run(cmds, verbose)
    tmp = LIB + ".tmp"
    _run([[HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]], verbose)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} in {time.time() - t0:.1f}s")
    return LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
