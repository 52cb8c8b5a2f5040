"""The FP8 path inside a captured HIP graph: every replay must reproduce the
eager result bit for bit (split-K counters reset themselves inside the
kernel; nothing in the path records a memset node)."""
import numpy as np
import pytest
import torch

import datagen
import inferop_amd
import oracle
from gpu_util import assert_gemm_close, bf16_dev, device, to_dev, to_np

DT = inferop_amd.dtype


@pytest.mark.gpu
@pytest.mark.parametrize("m,n,k", [(16, 2112, 7168), (64, 4096, 2048), (300, 1024, 1024)])
def test_graph_replays_match_eager(m, n, k):
    device()
    a_bits, a_f32, bq, bs = datagen.gemm_case(m, n, k, seed=m)
    a = bf16_dev(a_bits)
    bqd, bsd = to_dev(bq), to_dev(bs)
    st = torch.cuda.Stream()
    q = torch.empty((m, k), dtype=torch.uint8, device="cuda:0")
    s = torch.empty((m, k // 128), dtype=torch.float32, device="cuda:0")
    c = torch.empty((m, n), dtype=torch.bfloat16, device="cuda:0")

    def run():
        assert inferop_amd.quant_fp8_per_token_group(q, s, a, DT.bf16, m, k, 128,
                                                     st.cuda_stream) == 0
        assert inferop_amd.w8a8_block_fp8_gemm(c, q, s, bqd, bsd, m, n, k, 128, 128, DT.bf16,
                                               st.cuda_stream) == 0

    with torch.cuda.stream(st):
        run()
    st.synchronize()
    eager_q, eager_c = to_np(q), to_np(c)
    aq, as_ = oracle.quant(a_f32)
    assert np.array_equal(eager_q, aq)
    assert_gemm_close(c.float().cpu().numpy(), oracle.gemm(aq, as_, bq, bs), "eager")

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        run()
    for rep in range(4):
        c.zero_()
        q.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(to_np(q), eager_q), f"replay {rep}: quant bytes"
        assert np.array_equal(to_np(c), eager_c), f"replay {rep}: GEMM output"
        # eager work on the same stream between replays
        with torch.cuda.stream(st):
            run()
        st.synchronize()
