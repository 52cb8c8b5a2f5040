"""Register and scratch budget of the HIP kernels, from the compiler's own
per-kernel resource report (-Rpass-analysis=kernel-resource-usage), which the
build writes to _build/<source>.resources.txt.  No GPU needed.

Scratch memory in a streaming kernel is a private per-lane spill area in HBM:
every access to it is a load or store the algorithm does not need.  The
split-K fixup's partial batch, for one, must stay in registers.  Only the
persistent prefill kernels, which hold a 256x256 tile's fp32 accumulators in
two waves per SIMD, are allowed spills; their bound is pinned here too so it
cannot grow unnoticed."""
import os
import re
import subprocess

import pytest

from inferop_amd import build as B


def _report(src):
    """The resource report of src, compiled again (device code only) when the
    build's copy is missing or older than the sources."""
    path = os.path.join(B.BUILD, src + ".resources.txt")
    deps = [os.path.join(B.CSRC, f) for f in os.listdir(B.CSRC)
            if f.endswith((".hip", ".h"))]
    if os.path.exists(path) and os.path.getmtime(path) >= max(os.path.getmtime(d) for d in deps):
        return open(path).read()
    os.makedirs(B.BUILD, exist_ok=True)
    cmd = [B.HIPCC, *B.HIP_FLAGS, *B.EXTRA_FLAGS.get(src, []), B.RESOURCE_FLAG,
           "--cuda-device-only", "-c", os.path.join(B.CSRC, src), "-o",
           os.path.join(B.BUILD, src + ".dev.o")]
    out = subprocess.run(cmd, capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    with open(path, "w") as f:
        f.write(out.stdout + out.stderr)
    return out.stdout + out.stderr


def _kernels(text):
    """{mangled kernel name: {field: int}} from the report."""
    rows, cur = {}, None
    for line in text.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            cur = rows.setdefault(m.group(1), {})
            continue
        m = re.search(r"remark:\s+([A-Za-z ]+?)(?: \[[^\]]*\])?: (\d+)\b", line)
        if m and cur is not None:
            cur[m.group(1).strip()] = int(m.group(2))
    return rows


@pytest.mark.parametrize("src", ["gemm.hip", "quant.hip"])
def test_no_unrolling_failures(src):
    text = _report(src)
    bad = [l for l in text.splitlines() if "loop not unrolled" in l]
    assert not bad, "\n".join(bad[:5])


@pytest.mark.parametrize("src", ["gemm.hip", "quant.hip"])
def test_streaming_kernels_use_no_scratch(src):
    ks = _kernels(_report(src))
    assert len(ks) > (100 if src == "gemm.hip" else 10)
    spill = {k: v["ScratchSize"] for k, v in ks.items()
             if v.get("ScratchSize", 0) and "gemm_persist_kernel" not in k}
    assert not spill, spill


def test_persistent_kernel_spills_stay_bounded():
    # the plain persistent kernels (the M=4096 prefill tiles) spill at most
    # 80 bytes per lane; the grouped ones (MoE experts) at most 224
    ks = _kernels(_report("gemm.hip"))
    per = {k: v for k, v in ks.items() if "gemm_persist_kernel" in k}
    assert per
    for k, v in per.items():
        grouped = k.endswith("ELb1EEEvNS0_8GemmArgsE")
        assert v.get("ScratchSize", 0) <= (224 if grouped else 80), (k, v)
        assert v.get("VGPRs", 0) <= 256, (k, v)
