"""The FP8 path inside a captured HIP graph: every replay must reproduce the
eager result bit for bit (split-K counters reset themselves inside the
kernel; nothing in the path records a memset node)."""
import os
import subprocess
import sys

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


@pytest.mark.gpu
def test_graph_grouped_masked_routing_changes_between_replays():
    # the masked grouped GEMM is what a captured MoE decode step calls: the
    # shapes are fixed and only the per-expert counts on the device change.
    # Capture once, write new counts before each replay, and every replay must
    # equal an eager call with those counts (valid rows) and leave the other
    # rows alone.
    device()
    experts, max_m, n, k = 8, 16, 384, 1024
    g_ = np.random.default_rng(4)
    a = bf16_dev(datagen.f32_to_bf16_bits(
        g_.standard_normal((experts * max_m, k)).astype(np.float32)))
    aq, as_ = inferop_amd.quantize(a)
    bq, bs = zip(*[oracle.weight_block_quant(datagen.weights(n, k, 90 + e))
                   for e in range(experts)])
    bqd, bsd = to_dev(np.stack(bq)), to_dev(np.stack(bs))
    counts = torch.zeros(experts, dtype=torch.int32, device="cuda:0")
    c = torch.empty((experts, max_m, n), dtype=torch.float32, device="cuda:0")
    st = torch.cuda.Stream()

    def run(out):
        assert inferop_amd.w8a8_block_fp8_grouped_gemm_masked(
            out, aq, as_, bqd, bsd, counts, max_m, n, k, experts, 4, out_dt=DT.fp32,
            stream=st.cuda_stream) == 0

    counts.copy_(torch.full((experts,), max_m, dtype=torch.int32))
    with torch.cuda.stream(st):
        run(c)  # eager first: nothing to allocate inside the capture
    st.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        run(c)
    for rep in range(4):
        cnt = g_.integers(0, max_m + 1, experts).astype(np.int32)
        counts.copy_(torch.from_numpy(cnt))
        c.fill_(-7.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = torch.full_like(c, -7.0)
        with torch.cuda.stream(st):
            run(want)
        st.synchronize()
        assert torch.equal(c, want), f"replay {rep}"
        for e in range(experts):
            assert (c[e, cnt[e]:] == -7.0).all(), f"replay {rep} expert {e}"


def _cfg(name):
    return next(i for i in range(inferop_amd.gemm_num_configs())
                if inferop_amd.gemm_config_name(i) == name)


@pytest.mark.gpu
def test_graph_split_k_workspace_survives_larger_eager_calls():
    # The split-K workspace of a stream has a fixed size and is never freed or
    # replaced: a graph captured with a small split-K shape -- here the first
    # split-K call on its stream, so the workspace is created during the
    # capture -- must replay correctly after larger split-K shapes ran eagerly
    # on the same stream.
    device()
    cfg = _cfg("pre_n128_m32_w8_s4")
    small, large = (64, 256, 2048, 4), (64, 2112, 7168, 14)
    cases = {}
    for (m, n, k, split) in (small, large):
        _, a_f32, bq, bs = datagen.gemm_case(m, n, k, seed=n)
        aq, as_ = oracle.quant(a_f32)
        cases[(m, n, k)] = ([to_dev(v) for v in (aq, as_, bq, bs)],
                            oracle.gemm(aq, as_, bq, bs))
    st = torch.cuda.Stream()
    other = torch.cuda.Stream()

    def call(shape, split, out, stream):
        m, n, k = shape
        args, _ = cases[shape]
        assert inferop_amd.w8a8_block_fp8_gemm_config(out, *args, m, n, k, DT.fp32, cfg, split,
                                                      stream.cuda_stream) == 0

    s_shape, l_shape = small[:3], large[:3]
    c_small = torch.empty(small[:2], dtype=torch.float32, device="cuda:0")
    c_large = torch.empty(large[:2], dtype=torch.float32, device="cuda:0")
    want_small = torch.empty_like(c_small)
    with torch.cuda.stream(other):
        call(s_shape, small[3], want_small, other)
    other.synchronize()
    assert_gemm_close(want_small.cpu().numpy(), cases[s_shape][1], "small eager")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        call(s_shape, small[3], c_small, st)
    for rep in range(3):
        c_large.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(st):
            call(l_shape, large[3], c_large, st)
        st.synchronize()
        assert_gemm_close(c_large.cpu().numpy(), cases[l_shape][1], f"large eager {rep}")
        c_small.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(st):
            g.replay()
        st.synchronize()
        assert torch.equal(c_small, want_small), f"replay {rep}"


_SILU_FIRST_CALL_CAPTURED = r"""
import sys
import torch
import inferop_amd
DT = inferop_amd.dtype
tokens, d = 64, 2048
g = torch.Generator(device="cuda:0").manual_seed(5)
gu = (torch.randn((tokens, 2 * d), generator=g, device="cuda:0") * 3).to(torch.bfloat16)
q = torch.empty((tokens, d), dtype=torch.uint8, device="cuda:0")
s = torch.empty((tokens, d // 128), dtype=torch.float32, device="cuda:0")
st = torch.cuda.Stream()
graph = torch.cuda.CUDAGraph()
# the process's first bf16 SiLU call, inside the capture: the library builds
# its SiLU table on its own stream in relaxed capture mode
with torch.cuda.graph(graph, stream=st):
    assert inferop_amd.silu_and_mul_quant_fp8(q, s, gu, DT.bf16, tokens, d,
                                              stream=st.cuda_stream) == 0
q2, s2 = torch.empty_like(q), torch.empty_like(s)
with torch.cuda.stream(st):
    assert inferop_amd.silu_and_mul_quant_fp8(q2, s2, gu, DT.bf16, tokens, d,
                                              stream=st.cuda_stream) == 0
st.synchronize()
for rep in range(3):
    q.zero_(); s.zero_(); torch.cuda.synchronize()
    graph.replay(); torch.cuda.synchronize()
    if not (torch.equal(q, q2) and torch.equal(s, s2)):
        print("replay", rep, "differs from eager", flush=True)
        sys.exit(1)
print("ok", flush=True)
"""


@pytest.mark.gpu
def test_graph_silu_first_call_captured_in_fresh_process():
    # a child process, so that the captured call is its first bf16 SiLU call
    device()
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, PYTHONPATH=root + os.pathsep + os.environ.get("PYTHONPATH", ""))
    r = subprocess.run([sys.executable, "-c", _SILU_FIRST_CALL_CAPTURED], env=env,
                       capture_output=True, text=True, timeout=240)
    assert r.returncode == 0 and "ok" in r.stdout, (r.stdout[-2000:], r.stderr[-2000:])


@pytest.mark.gpu
def test_graph_fused_producers_replay_match_eager():
    device()
    tokens, d, rows, cols = 48, 4096, 40, 2048
    g = torch.Generator(device="cuda:0").manual_seed(9)
    gu = (torch.randn((tokens, 2 * d), generator=g, device="cuda:0") * 3).to(torch.bfloat16)
    x = torch.randn((rows, cols), generator=g, device="cuda:0").to(torch.bfloat16)
    w = torch.randn((cols,), generator=g, device="cuda:0").to(torch.bfloat16)
    res0 = torch.randn((rows, cols), generator=g, device="cuda:0").to(torch.bfloat16)
    st = torch.cuda.Stream()
    outs = {}

    def run(tag):
        q = torch.empty((tokens, d), dtype=torch.uint8, device="cuda:0")
        s = torch.empty((tokens, d // 128), dtype=torch.float32, device="cuda:0")
        res = res0.clone()
        rq = torch.empty((rows, cols), dtype=torch.uint8, device="cuda:0")
        rs = torch.empty((rows, cols // 128), dtype=torch.float32, device="cuda:0")
        outs[tag] = (q, s, res, rq, rs)

    run("eager")
    run("graph")

    def call(tag):
        q, s, res, rq, rs = outs[tag]
        assert inferop_amd.silu_and_mul_quant_fp8(q, s, gu, DT.bf16, tokens, d,
                                                  stream=st.cuda_stream) == 0
        assert inferop_amd.fused_add_rmsnorm_quant_fp8(res, rq, rs, x, w, DT.bf16, rows, cols,
                                                       stream=st.cuda_stream) == 0

    with torch.cuda.stream(st):
        call("eager")
    st.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        call("graph")
    for rep in range(3):
        q, s, res, rq, rs = outs["graph"]
        q.zero_()
        s.zero_()
        rq.zero_()
        res.copy_(res0)  # the residual is updated in place
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(outs["graph"], outs["eager"]):
            assert torch.equal(a, b), f"replay {rep}"


@pytest.mark.gpu
def test_graph_silu_fp16_lds_kernel_replay_match_eager():
    # 256 tokens x 8192 outputs = 16384 groups: the fp16 kernel that copies
    # a slice of the device's fp16 SiLU table into LDS; replays equal eager
    device()
    tokens, d = 256, 8192
    g = torch.Generator(device="cuda:0").manual_seed(12)
    gu = (torch.randn((tokens, 2 * d), generator=g, device="cuda:0") * 3).to(torch.float16)
    st = torch.cuda.Stream()
    q0 = torch.empty((tokens, d), dtype=torch.uint8, device="cuda:0")
    s0 = torch.empty((tokens, d // 128), dtype=torch.float32, device="cuda:0")
    q = torch.empty_like(q0)
    s = torch.empty_like(s0)
    with torch.cuda.stream(st):
        assert inferop_amd.silu_and_mul_quant_fp8(q0, s0, gu, DT.fp16, tokens, d,
                                                  stream=st.cuda_stream) == 0
    st.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        assert inferop_amd.silu_and_mul_quant_fp8(q, s, gu, DT.fp16, tokens, d,
                                                  stream=st.cuda_stream) == 0
    for rep in range(3):
        q.zero_()
        s.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(q, q0) and torch.equal(s, s0), f"replay {rep}"
