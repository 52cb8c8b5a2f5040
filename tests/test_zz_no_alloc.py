"""The allocation-free GEMM entry point (inferop_w8a8_block_fp8_gemm_noalloc,
no counterpart in the reference) against the ordinary one
(inferop_w8a8_block_fp8_gemm, ops.h:81-84): same kernel choice, so the
outputs must be identical bit for bit -- on two calls in a row, the second
smaller, so the second runs on the scratch the first left behind -- and
within the GEMM tolerance of the oracle."""
import ctypes

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
