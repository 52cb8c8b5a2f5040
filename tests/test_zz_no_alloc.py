"""The allocation-free GEMM entry point (inferop_w8a8_block_fp8_gemm_noalloc,
no counterpart in the reference) against the ordinary one
(inferop_w8a8_block_fp8_gemm, ops.h:81-84): same kernel choice, so the
outputs must be identical bit for bit -- on two calls in a row, the second
smaller, so the second runs on the scratch the first left behind -- and
within the GEMM tolerance of the oracle."""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

import datagen
import inferop_amd
import oracle
from gpu_util import assert_gemm_close, device, to_dev

DT = inferop_amd.dtype


def _c_abi(name):
    return getattr(inferop_amd.lib(), name)


@pytest.mark.gpu
def test_noalloc_gemm_matches_allocating_entry_point():
    device()
    # (64, 2112, 7168) and (33, 1024, 7168) split K over 128x32 tiles (the
    # second with fewer tiles and a different split), (1, 512, 57344) over
    # decode stripes, (16, 4096, 7168) splits nothing
    cases = [(64, 2112, 7168), (33, 1024, 7168), (1, 512, 57344), (16, 4096, 7168)]
    noalloc = _c_abi("inferop_w8a8_block_fp8_gemm_noalloc")
    plain = _c_abi("inferop_w8a8_block_fp8_gemm")
    st = torch.cuda.current_stream().cuda_stream
    splits = []
    for (m, n, k) in cases:
        print(f"noalloc {m}x{n}x{k}", flush=True)
        _, a_f32, bq, bs = datagen.gemm_case(m, n, k, seed=m + n)
        aq, as_ = oracle.quant(a_f32)
        args = [to_dev(v) for v in (aq, as_, bq, bs)]
        ptrs = [ctypes.c_void_p(t.data_ptr()) for t in args]
        splits.append(inferop_amd.gemm_select(m, n, k)[1])
        for out in (DT.bf16, DT.fp32):
            tdt = torch.bfloat16 if out == DT.bf16 else torch.float32
            want = torch.full((m, n), float("nan"), dtype=tdt, device="cuda:0")
            got = torch.full((m, n), float("nan"), dtype=tdt, device="cuda:0")
            assert plain(ctypes.c_void_p(want.data_ptr()), *ptrs, m, n, k, 128, 128, int(out),
                         ctypes.c_void_p(st)) == 0
            assert noalloc(ctypes.c_void_p(got.data_ptr()), *ptrs, m, n, k, 128, 128, int(out),
                           ctypes.c_void_p(st)) == 0
            torch.cuda.synchronize()
            assert torch.equal(got, want), f"{m}x{n}x{k} {out.name}"
        assert_gemm_close(got.cpu().numpy(), oracle.gemm(aq, as_, bq, bs), f"{m}x{n}x{k}")
    assert splits[0] > 1 and splits[1] > 1 and splits[2] > 1 and splits[3] == 1, splits


@pytest.mark.gpu
def test_noalloc_gemm_guards_match():
    device()
    noalloc = _c_abi("inferop_w8a8_block_fp8_gemm_noalloc")
    c = torch.full((4, 8), 5.0, dtype=torch.float32, device="cuda:0")
    z = torch.zeros(1024, dtype=torch.uint8, device="cuda:0")
    p = [ctypes.c_void_p(t.data_ptr()) for t in (c, z, z, z, z)]
    S = inferop_amd.Status
    assert noalloc(*p, 4, 8, 100, 128, 128, int(DT.fp32), None) == S.ERR_SHAPE
    assert noalloc(*p, 4, 8, 128, 128, 128, int(DT.fp8_e4m3), None) == S.ERR_DTYPE
    torch.cuda.synchronize()
    assert (c == 5.0).all()


@pytest.mark.gpu
def test_noalloc_split_k_graph_replays_match_eager():
    # a captured split-K no-alloc call (64 x 2112 x 7168: 128x32 tiles, K in
    # 3) replays bit-identically to the eager call, with eager no-alloc calls
    # of another shape between the replays (they leave the counters at zero)
    device()
    m, n, k = 64, 2112, 7168
    assert inferop_amd.gemm_select(m, n, k)[1] > 1
    _, a_f32, bq, bs = datagen.gemm_case(m, n, k, seed=77)
    aq, as_ = oracle.quant(a_f32)
    args = [to_dev(v) for v in (aq, as_, bq, bs)]
    o_m, o_n, o_k = 33, 1024, 7168
    _, o_f32, obq, obs = datagen.gemm_case(o_m, o_n, o_k, seed=78)
    oaq, oas = oracle.quant(o_f32)
    oargs = [to_dev(v) for v in (oaq, oas, obq, obs)]
    st = torch.cuda.Stream()
    want = torch.empty((m, n), dtype=torch.bfloat16, device="cuda:0")
    got = torch.empty_like(want)
    other = torch.empty((o_m, o_n), dtype=torch.bfloat16, device="cuda:0")
    with torch.cuda.stream(st):
        assert inferop_amd.w8a8_block_fp8_gemm_noalloc(want, *args, m, n, k,
                                                       stream=st.cuda_stream) == 0
    st.synchronize()
    assert_gemm_close(want.float().cpu().numpy(), oracle.gemm(aq, as_, bq, bs), "eager")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        assert inferop_amd.w8a8_block_fp8_gemm_noalloc(got, *args, m, n, k,
                                                       stream=st.cuda_stream) == 0
    for rep in range(3):
        got.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {rep}"
        with torch.cuda.stream(st):
            assert inferop_amd.w8a8_block_fp8_gemm_noalloc(other, *oargs, o_m, o_n, o_k,
                                                           stream=st.cuda_stream) == 0
        st.synchronize()


_NOALLOC_FIRST_CALL_CAPTURED = r"""
import sys
import torch
import inferop_amd
m, n, k = 64, 2112, 7168
g = torch.Generator(device="cuda:0").manual_seed(11)
a = torch.randn((m, k), generator=g, device="cuda:0").to(torch.bfloat16)
aq, as_ = inferop_amd.quantize(a)
bq = (torch.randn((n, k), generator=g, device="cuda:0") * 0.3).to(torch.float8_e4m3fn)
bq = bq.view(torch.uint8)
bs = torch.rand(((n + 127) // 128, k // 128), generator=g, device="cuda:0") * 0.01 + 1e-3
assert inferop_amd.gemm_select(m, n, k)[1] > 1
torch.cuda.synchronize()
st = torch.cuda.Stream()
got = torch.empty((m, n), dtype=torch.bfloat16, device="cuda:0")
graph = torch.cuda.CUDAGraph()
# the process's first no-alloc call, inside the capture: the scratch address
# is looked up and its counters zeroed outside the graph
with torch.cuda.graph(graph, stream=st):
    assert inferop_amd.w8a8_block_fp8_gemm_noalloc(got, aq, as_, bq, bs, m, n, k,
                                                   stream=st.cuda_stream) == 0
# an eager no-alloc call before any replay finds the counters at zero
want = torch.empty_like(got)
with torch.cuda.stream(st):
    assert inferop_amd.w8a8_block_fp8_gemm_noalloc(want, aq, as_, bq, bs, m, n, k,
                                                   stream=st.cuda_stream) == 0
st.synchronize()
plain = torch.empty_like(got)
assert inferop_amd.w8a8_block_fp8_gemm(plain, aq, as_, bq, bs, m, n, k) == 0
torch.cuda.synchronize()
if not torch.equal(want, plain):
    print("eager no-alloc call differs from the allocating entry point", flush=True)
    sys.exit(1)
for rep in range(3):
    got.zero_(); torch.cuda.synchronize()
    graph.replay(); torch.cuda.synchronize()
    if not torch.equal(got, want):
        print("replay", rep, "differs from eager", flush=True)
        sys.exit(1)
print("ok", flush=True)
"""


@pytest.mark.gpu
def test_noalloc_first_call_captured_in_fresh_process():
    # a child process, so that the captured call is its first no-alloc call
    device()
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, PYTHONPATH=root + os.pathsep + os.environ.get("PYTHONPATH", ""))
    r = subprocess.run([sys.executable, "-c", _NOALLOC_FIRST_CALL_CAPTURED], env=env,
                       capture_output=True, text=True, timeout=240)
    assert r.returncode == 0 and "ok" in r.stdout, (r.stdout[-2000:], r.stderr[-2000:])
