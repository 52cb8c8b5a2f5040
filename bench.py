"""Benchmark of the blockwise-FP8 W8A8 path on one MI355X.

Headline workload (decode-shaped): one step runs,
for each M in {1, 16, 64} and (N, K) in {(7168, 2048), (4096, 7168),
(2112, 7168)}, the quantizer on bf16 activations [M, K] followed by the
blockwise-FP8 GEMM into bf16 [M, N] -- 18 kernel launches, enqueued on one
stream step after step as a serving loop does (the host runs ahead of the
GPU); weights rotate over more than 1 GiB of copies so the 256 MB Infinity
Cache cannot serve them.  `value` is the step's algorithmic HBM bytes divided
by its wall time (GB/s).  The same step replayed as a HIP graph is reported
beside it (slower on this ROCm: each kernel node starts later).

Also reported: the prefill GEMM (configs[2], M = 4096) in TFLOPS against the
5.0 PFLOPS dense-FP8 peak (with the platform's row-wise FP8 GEMM on the same
bytes as a reference point), the quantizer, weight quantizer and fused
producers on large inputs in GB/s, MoE routing, the grouped GEMM over MoE
experts (decode- and prefill-sized routings), and a CPU baseline (the
reference's own CPU golden code, or the oracle restatement, timed
single-threaded on this host over the same decode workload, and the oracle's
GEMM spread over the host cores beside it).
Per-kernel durations come from HIP events on the launch stream around graph
replays of back-to-back launches of one kernel.

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
       python bench.py --traffic-pass   (decode kernels once each, for FETCH_SIZE/WRITE_SIZE)
       python bench.py --mfma-pass      (prefill GEMMs, for the MFMA and LDS counters)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "FP8 GEMM TFLOPS (% MFMA peak) at M=4096; GB/s (% HBM) at M<=64 + quant"
HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
DECODE_M = (1, 16, 64)
DECODE_NK = ((7168, 2048), (4096, 7168), (2112, 7168))
PREFILL_NK = ((24576, 1536), (32768, 512), (7168, 16384), (4608, 7168))
QUANT_SHAPES = ((4096, 7168), (4096, 16384), (8192, 18432))
# BASELINE configs[3] (M sweep on DeepSeek-V3-like dense shapes), configs[4]
# (ragged M, N = 4608 + 64) and the reference's own bench shape 4096^3
# (bench/bench_kernels.cpp:63-80): timed shape by shape, bf16 output
SWEEP_M = (128, 512, 1024, 2048, 8192)
SWEEP_NK = ((7168, 18432), (36864, 7168), (7168, 2048), (4096, 512))
RAGGED = ((1000, 4672, 7168), (77, 4672, 7168))
REF_BENCH = ((4096, 4096, 4096),)
# workgroups per CU tried for the plain-read ceiling of a decode weight stream
READ_BLOCKS_PER_CU = (1, 2, 4, 8)
PER_KERNEL_LAUNCHES = 20
# prefill GEMMs per captured graph: back-to-back launches in steady state (with
# a handful per graph the replay boundaries add tens of microseconds a launch)
PREFILL_LAUNCHES = 20
# HBM bytes per decode-GEMM launch, mean over the 9 decode shapes: FETCH_SIZE +
# WRITE_SIZE from rocprofv3 runs of `bench.py --traffic-pass`, each scaled by
# what the counter reads for a 256 MiB streaming kernel in the same process
# (per-launch table and commands: profiles/decode_step_hbm_traffic.md).
DECODE_GEMM_TRAFFIC_BYTES = 22147667


def quant_bytes(m, k, in_bytes=2):
    return m * k * in_bytes + m * k + 4 * m * (k // 128)


def gemm_bytes(m, n, k, out_bytes=2):
    return (m * k + 4 * m * (k // 128) + n * k + 4 * ((n + 127) // 128) * (k // 128)
            + m * n * out_bytes)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--traffic-pass", action="store_true",
                   help="launch a 256 MiB streaming kernel and every decode-step kernel once "
                        "each (cold weights) for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs; "
                        "prints the launches in order with their algorithmic bytes")
    p.add_argument("--mfma-pass", action="store_true",
                   help="launch the GEMM of every prefill shape (M=4096) three times, "
                        "synchronizing after each, for rocprofv3 --pmc runs of the MFMA "
                        "counters; prints the launches in order with their flops")
    return p.parse_args()


def traffic_pass():
    """Counter-collection workload.  The first launch is a plain streaming
    kernel (fp32 y = x * 1 over 256 MiB: 256 MiB read + 256 MiB written) whose
    FETCH_SIZE / WRITE_SIZE readings calibrate the counters; then, for every
    decode case, one quantizer and one GEMM launch, each GEMM on a weight copy
    no earlier launch touched, so the counters see HBM reads, not cache hits."""
    import torch

    import inferop_amd as ia

    ia.lib()
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    launches = []
    n_el = 64 << 20
    x = torch.randn(n_el, generator=gen, device=dev)
    y = torch.empty_like(x)
    cases = [(m, n, k) for m in DECODE_M for (n, k) in DECODE_NK]
    ws = [(torch.randint(0, 0x7E, (n, k), generator=gen, device=dev, dtype=torch.int32)
           .to(torch.uint8),
           torch.rand(((n + 127) // 128, k // 128), generator=gen, device=dev) * 1e-3 + 1e-4)
          for (_, n, k) in cases]
    acts = [torch.randn((m, k), generator=gen, device=dev).to(torch.bfloat16)
            for (m, _, k) in cases]
    torch.cuda.synchronize()
    torch.mul(x, 1.0, out=y)
    torch.cuda.synchronize()
    launches.append({"launch": "calibration fp32 y = x * 1", "read": 4 * n_el, "write": 4 * n_el})
    for (m, n, k), (bq, bs), a in zip(cases, ws, acts):
        q, s = ia.quantize(a)
        torch.cuda.synchronize()
        launches.append({"launch": f"quant m={m} k={k}", "read": 2 * m * k,
                         "write": m * k + 4 * m * (k // 128)})
        ia.gemm(q, s, bq, bs)
        torch.cuda.synchronize()
        cfg, split = ia.gemm_select(m, n, k)
        launches.append({"launch": f"gemm m={m} n={n} k={k} {ia.gemm_config_name(cfg)}/s{split}",
                         "read": gemm_bytes(m, n, k) - 2 * m * n, "write": 2 * m * n})
    # the quantizer fused with the GEMM, where it is one launch (M <= 8), on
    # weight copies no earlier launch touched
    for (m, n, k), a in zip(cases, acts):
        if ia.quant_gemm_launches(m, n, k) != 1:
            continue
        bq = torch.randint(0, 0x7E, (n, k), generator=gen, device=dev,
                           dtype=torch.int32).to(torch.uint8)
        bs = torch.rand(((n + 127) // 128, k // 128), generator=gen, device=dev) * 1e-3 + 1e-4
        q = torch.empty((m, k), dtype=torch.uint8, device=dev)
        s = torch.empty((m, k // 128), dtype=torch.float32, device=dev)
        c = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        torch.cuda.synchronize()
        assert ia.quant_w8a8_block_fp8_gemm(c, q, s, a, ia.dtype.bf16, bq, bs, m, n, k) == 0
        torch.cuda.synchronize()
        launches.append({"launch": f"quant+gemm m={m} n={n} k={k} (one launch)",
                         "read": 2 * m * k + n * k + 4 * ((n + 127) // 128) * (k // 128),
                         "write": m * k + 4 * m * (k // 128) + 2 * m * n})
    print(json.dumps({"traffic_pass": launches}), flush=True)


def mfma_pass():
    """Counter-collection workload for the prefill GEMM: per configs[2] shape,
    the activations are quantized on the GPU, then the GEMM runs three times
    (bf16 out), each launch on its own, so per-dispatch counters (MFMA busy
    cycles, active cycles) belong to one GEMM."""
    import torch

    import inferop_amd as ia

    ia.lib()
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    launches = []
    m = 4096
    for (n, k) in PREFILL_NK:
        v = torch.randint(0, 0x7E, (n, k), generator=gen, device=dev, dtype=torch.int32)
        sgn = torch.randint(0, 2, (n, k), generator=gen, device=dev, dtype=torch.int32) << 7
        bq = (v | sgn).to(torch.uint8)
        bs = torch.rand(((n + 127) // 128, k // 128), generator=gen, device=dev) * 1e-3 + 1e-4
        q, s = ia.quantize(torch.randn((m, k), generator=gen, device=dev).to(torch.bfloat16))
        torch.cuda.synchronize()
        launches.append({"launch": f"quant m={m} k={k}"})
        cfg, split = ia.gemm_select(m, n, k)
        for _ in range(3):
            ia.gemm(q, s, bq, bs)
            torch.cuda.synchronize()
            launches.append({"launch": f"gemm m={m} n={n} k={k} {ia.gemm_config_name(cfg)}/s{split}",
                             "flops": 2 * m * n * k})
        del bq, bs, q, s
    print(json.dumps({"mfma_pass": launches}), flush=True)


def main():
    args = parse()
    if args.traffic_pass:
        traffic_pass()
        return
    if args.mfma_pass:
        mfma_pass()
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on exactly one GPU: the FP8 path has no "
                                   "multi-GPU component here (each GPU would run its own shard "
                                   "of M, N or K with these kernels); run with --gpus 1"}))
        sys.exit(2)
    import numpy as np
    import torch

    import inferop_amd as ia

    ia.lib()
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)  # default priority
    sp = stream.cuda_stream
    gen = torch.Generator(device=dev).manual_seed(0)
    DT = ia.dtype

    def rand_fp8(shape):
        v = torch.randint(0, 0x7E, shape, generator=gen, device=dev, dtype=torch.int32)
        s = torch.randint(0, 2, shape, generator=gen, device=dev, dtype=torch.int32) << 7
        return (v | s).to(torch.uint8)

    def rand_scales(shape):
        return (torch.rand(shape, generator=gen, device=dev) * 1e-3 + 1e-4).float()

    def ev():
        return torch.cuda.Event(enable_timing=True)

    def capture(fn):
        """HIP graph of fn's launches on `stream` (warm-up runs first, eagerly,
        so every workspace the library needs already exists)."""
        fn()
        stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            fn()
        return g

    def time_graphs(graphs, reps):
        e0, e1 = ev(), ev()
        e0.record(stream)
        for i in range(reps):
            graphs[i % len(graphs)].replay()
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) / reps  # ms per replay

    result = {"metric": METRIC, "n_gpus": 1, "higher_is_better": True, "scaling": "weak",
              "vs_baseline": None, "dtype": "fp8e4m3", "data": "synthetic"}

    with torch.cuda.stream(stream):
        # ---------------- decode workload (the headline value) ----------------
        cases = [(m, n, k) for m in DECODE_M for (n, k) in DECODE_NK]
        wbytes = sum(n * k for n, k in DECODE_NK)
        R = max(2, -(-(1 << 30) // wbytes))  # weight copies: > 1 GiB in rotation
        W = {(n, k): [(rand_fp8((n, k)), rand_scales(((n + 127) // 128, k // 128)))
                      for _ in range(R)] for (n, k) in DECODE_NK}
        A = {(m, k): torch.randn((m, k), generator=gen, device=dev).to(torch.bfloat16)
             for m in DECODE_M for (_, k) in DECODE_NK}
        AQ = {(m, k): (torch.empty((m, k), dtype=torch.uint8, device=dev),
                       torch.empty((m, k // 128), dtype=torch.float32, device=dev))
              for (m, k) in A}
        C = {(m, n): torch.empty((m, n), dtype=torch.bfloat16, device=dev) for (m, n, _) in cases}
        step_bytes = sum(quant_bytes(m, k) + gemm_bytes(m, n, k) for (m, n, k) in cases)

        def quant_call(m, k):
            q, s = AQ[(m, k)]
            st = ia.quant_fp8_per_token_group(q, s, A[(m, k)], DT.bf16, m, k, 128, sp)
            assert st == 0, st

        def gemm_call(m, n, k, r):
            q, s = AQ[(m, k)]
            bq, bs = W[(n, k)][r % R]
            st = ia.w8a8_block_fp8_gemm(C[(m, n)], q, s, bq, bs, m, n, k, 128, 128, DT.bf16, sp)
            assert st == 0, st

        def step(r):
            for (m, n, k) in cases:
                quant_call(m, k)
                gemm_call(m, n, k, r)

        # The headline: K steps launched on the stream as a serving loop
        # enqueues them (host launch calls included; the host runs ahead of
        # the GPU, about 4 us of host time per launch against 5 us of GPU
        # time), after W untimed steps.
        for i in range(args.warmup):
            step(i)
        torch.cuda.synchronize()
        e0, e1 = ev(), ev()
        e0.record(stream)
        for i in range(args.steps):
            step(i)
        e1.record(stream)
        e1.synchronize()
        torch.cuda.synchronize()
        ms_step = e0.elapsed_time(e1) / args.steps
        value = step_bytes / (ms_step * 1e-3) / 1e9
        # the same step captured once per weight copy and replayed as a HIP
        # graph: no host work per step, but on this ROCm each kernel node of
        # the 18-kernel graph starts about 0.3 us later than the same kernel
        # enqueued on the stream, so the replay is the slower of the two
        step_graphs = [capture(lambda r=r: step(r)) for r in range(R)]
        time_graphs(step_graphs, args.warmup)
        ms_step_graph = time_graphs(step_graphs, args.steps)

        # Beside the headline (not the headline): the same nine (quant, GEMM)
        # pairs through the one-call extension quant_w8a8_block_fp8_gemm,
        # which quantizes inside the GEMM where the GEMM runs on the 8-row
        # decode tiles (M = 1 here: 3 of the 9 pairs become one launch) and
        # makes the two launches otherwise; same bytes written, same timing.
        def fused_step(r):
            for (m, n, k) in cases:
                q, s = AQ[(m, k)]
                bq, bs = W[(n, k)][r % R]
                st = ia.quant_w8a8_block_fp8_gemm(C[(m, n)], q, s, A[(m, k)], DT.bf16, bq, bs,
                                                  m, n, k, 128, 128, DT.bf16, sp)
                assert st == 0, st

        for i in range(args.warmup):
            fused_step(i)
        torch.cuda.synchronize()
        e0, e1 = ev(), ev()
        e0.record(stream)
        for i in range(args.steps):
            fused_step(i)
        e1.record(stream)
        e1.synchronize()
        ms_fused = e0.elapsed_time(e1) / args.steps
        fused_launches = sum(ia.quant_gemm_launches(m, n, k) for (m, n, k) in cases)

        # The read ceiling of each decode weight stream: the library's plain
        # read kernel over the same weight copies, launched as the GEMM is (a
        # graph of PER_KERNEL_LAUNCHES back-to-back launches), at the best of
        # a few grid sizes; and the launch floor (a 16-byte read).
        cus = torch.cuda.get_device_properties(dev).multi_processor_count
        sink = torch.zeros(4, dtype=torch.int32, device=dev)

        def read_call(src, nbytes, blocks):
            st = ia.diag_read_stream(src, nbytes, blocks, sink, sp)
            assert st == 0, st

        ceiling = {}
        for (n, k) in DECODE_NK:
            best = None
            for bpc in READ_BLOCKS_PER_CU:
                gr = capture(lambda: [read_call(W[(n, k)][r % R][0], n * k, bpc * cus)
                                      for r in range(PER_KERNEL_LAUNCHES)])
                time_graphs([gr], 4)
                t = time_graphs([gr], 10) / PER_KERNEL_LAUNCHES
                if best is None or t < best[0]:
                    best = (t, bpc)
                del gr
            ceiling[(n, k)] = best
        gl = capture(lambda: [read_call(sink, 16, 1) for _ in range(PER_KERNEL_LAUNCHES)])
        time_graphs([gl], 4)
        launch_floor_us = time_graphs([gl], 10) / PER_KERNEL_LAUNCHES * 1e3
        del gl

        # The decode kernels' unit of work measured without the GEMM: one
        # 8-wave workgroup per 16-row weight stripe, every load of a workgroup
        # in flight at once, in four access patterns, from HBM (the rotating
        # weight copies) and L2-resident (workgroup i reads stripe i % 16):
        # what the load path itself allows per compute unit.
        patterns = ("rows8_regs", "contig_regs", "mfma_layout_regs", "rows8_lds_dma",
                    "rows8_regs_to_lds")
        stripe_reads = []
        for (n, k) in DECODE_NK:
            for src, stripes in (("hbm", 0), ("l2", 16)):
                for pat, pname in enumerate(patterns):
                    gr = capture(lambda: [ia.diag_stripe_read(W[(n, k)][r % R][0], n, k, pat,
                                                              stripes, sink, sp)
                                          for r in range(PER_KERNEL_LAUNCHES)])
                    time_graphs([gr], 4)
                    t = time_graphs([gr], 10) / PER_KERNEL_LAUNCHES
                    del gr
                    stripe_reads.append({
                        "n": n, "k": k, "source": src, "pattern": pname,
                        "us": round(t * 1e3, 2),
                        "tbs": round(n * k / (t * 1e-3) / 1e12, 2),
                        "per_workgroup_gbs_above_floor": round(
                            16 * k / max(t * 1e3 - launch_floor_us, 1e-3) / 1e3, 1)})

        # per-kernel: a graph of PER_KERNEL_LAUNCHES back-to-back launches
        detail = []
        g_bytes = g_ms = q_bytes = q_ms = 0.0
        for (m, n, k) in cases:
            gq = capture(lambda: [quant_call(m, k) for _ in range(PER_KERNEL_LAUNCHES)])
            gg = capture(lambda: [gemm_call(m, n, k, r) for r in range(PER_KERNEL_LAUNCHES)])
            time_graphs([gq, gg], 4)
            qms = time_graphs([gq], 10) / PER_KERNEL_LAUNCHES
            gms = time_graphs([gg], 10) / PER_KERNEL_LAUNCHES
            gb, qb = gemm_bytes(m, n, k), quant_bytes(m, k)
            g_bytes += gb
            g_ms += gms
            q_bytes += qb
            q_ms += qms
            cfg, split = ia.gemm_select(m, n, k)
            rms, rbpc = ceiling[(n, k)]
            detail.append({"m": m, "n": n, "k": k, "gemm_us": round(gms * 1e3, 2),
                           "gemm_gbs": round(gb / (gms * 1e-3) / 1e9, 1),
                           "quant_us": round(qms * 1e3, 2),
                           "kernel": ia.gemm_config_name(cfg), "split_k": split,
                           "stream_read_us": round(rms * 1e3, 2),
                           "stream_ceiling_gbs": round(n * k / (rms * 1e-3) / 1e9, 1),
                           "stream_read_blocks_per_cu": rbpc,
                           "gemm_frac_of_stream_ceiling": round(rms / gms, 4)})
            del gq, gg
        gemm_gbs = g_bytes / (g_ms * 1e-3) / 1e9
        result.update({
            "value": round(value, 1), "unit": "GB/s", "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
            "config": {"workload": "BASELINE configs[1] decode step: per-token-group quant of "
                                   "bf16 A[M,K] + W8A8 block-FP8 GEMM -> bf16 C[M,N], "
                                   "M in {1,16,64} x (N,K) in {(7168,2048),(4096,7168),"
                                   "(2112,7168)}; 18 launches per step enqueued on one "
                                   "stream",
                       "step_bytes": step_bytes, "weight_copies_rotated": R,
                       "hbm_frac_step": round(value / HBM_PEAK_GBS, 4),
                       "ms_per_step_graph_replay": round(ms_step_graph, 5),
                       "gbs_graph_replay": round(step_bytes / (ms_step_graph * 1e-3) / 1e9, 1)},
            "roofline": {"bound": "hbm", "kernel": "w8a8 block-FP8 GEMM, decode tiles",
                         "achieved": round(gemm_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gemm_gbs / HBM_PEAK_GBS, 4),
                         "traffic": DECODE_GEMM_TRAFFIC_BYTES,
                         "algorithmic_bytes_per_launch": int(g_bytes / len(cases)),
                         "algorithmic_bytes_per_step": int(g_bytes),
                         "avg_launch_us": round(g_ms / len(cases) * 1e3, 3)},
            "fused_step": {
                "what": "the same step through quant_w8a8_block_fp8_gemm (one call per pair; "
                        "one launch where M <= 8 runs on the 8-row decode tiles), enqueued "
                        "like the headline; reported beside it, not as value",
                "launches_per_step": fused_launches, "ms_per_step": round(ms_fused, 5),
                "gbs": round(step_bytes / (ms_fused * 1e-3) / 1e9, 1)},
            "decode_detail": detail,
            "decode_ceiling": {
                "what": "stream_read_us: one plain read of the shape's N*K weight bytes "
                        "(inferop_diag_read_stream, best of 1/2/4/8 workgroups per CU) over the "
                        "same rotating weight copies, timed like the GEMM (graph of 20 "
                        "launches); gemm_frac_of_stream_ceiling = stream_read_us / gemm_us",
                "launch_floor_us": round(launch_floor_us, 2),
                "stripe_reads": stripe_reads,
                "stripe_reads_what": "inferop_diag_stripe_read: one 8-wave workgroup per 16-row "
                                     "stripe (workgroup bytes 16*K), all loads in flight; "
                                     "per_workgroup_gbs_above_floor = 16*K / (us - "
                                     "launch_floor_us)",
                "gemm_frac_of_stream_ceiling_mean": round(
                    sum(d["gemm_frac_of_stream_ceiling"] for d in detail) / len(detail), 4)},
            "quant_decode_gbs": round(q_bytes / (q_ms * 1e-3) / 1e9, 1),
            "gpu_clocks": gpu_clocks(),
        })
        del step_graphs, W, A, AQ, C
        torch.cuda.empty_cache()

        # ---------------- prefill GEMM (configs[2], M = 4096) ----------------
        def vendor_rowwise_tflops(q, ws, m, n, k):
            """The platform's FP8 GEMM on the same E4M3 bytes, for reference:
            torch._scaled_mm (hipBLASLt) with one scale per row of A and of B --
            a simpler operation than the blockwise one (no per-group
            promotion), so an upper reference for its throughput, not a
            competitor computing the same result.  None where unavailable."""
            try:
                a8 = q.view(torch.float8_e4m3fn)
                bs8 = [bq.view(torch.float8_e4m3fn) for bq, _ in ws]
                sa = torch.rand((m, 1), generator=gen, device=dev) + 0.5
                sb = torch.rand((1, n), generator=gen, device=dev) + 0.5

                def v(i):
                    torch._scaled_mm(a8, bs8[i % len(bs8)].t(), scale_a=sa, scale_b=sb,
                                     out_dtype=torch.bfloat16)

                gv = capture(lambda: [v(i) for i in range(PREFILL_LAUNCHES)])
                time_graphs([gv], 2)
                vus = time_graphs([gv], 5) / PREFILL_LAUNCHES * 1e3
                del gv
                return round(2.0 * m * n * k / (vus * 1e-6) / 1e12, 1)
            except (RuntimeError, AttributeError, TypeError):
                return None

        pre = []
        m = 4096
        for (n, k) in PREFILL_NK:
            a = torch.randn((m, k), generator=gen, device=dev).to(torch.bfloat16)
            q, s = ia.quantize(a, stream=sp)
            # weight copies: more than 1 GiB in rotation (at most one per launch)
            nw = min(PREFILL_LAUNCHES, max(2, -(-(1 << 30) // (n * k))))
            ws = [(rand_fp8((n, k)), rand_scales(((n + 127) // 128, k // 128))) for _ in range(nw)]
            c = torch.empty((m, n), dtype=torch.bfloat16, device=dev)

            def g(i, n=n, k=k, q=q, s=s, ws=ws, c=c):
                bq, bs = ws[i % len(ws)]
                st = ia.w8a8_block_fp8_gemm(c, q, s, bq, bs, m, n, k, 128, 128, DT.bf16, sp)
                assert st == 0, st

            gg = capture(lambda: [g(i) for i in range(PREFILL_LAUNCHES)])
            time_graphs([gg], 2)
            us = time_graphs([gg], 5) / PREFILL_LAUNCHES * 1e3
            tflops = 2.0 * m * n * k / (us * 1e-6) / 1e12
            ai = 2.0 * m * n * k / gemm_bytes(m, n, k)
            bound = min(FP8_PEAK_TFLOPS, ai * HBM_PEAK_GBS / 1e3)
            cfg, split = ia.gemm_select(m, n, k)
            pre.append({"m": m, "n": n, "k": k, "us": round(us, 2), "tflops": round(tflops, 1),
                        "frac_of_peak": round(tflops / FP8_PEAK_TFLOPS, 4),
                        "frac_of_roofline": round(tflops / bound, 4),
                        "kernel": ia.gemm_config_name(cfg), "split_k": split,
                        "weight_copies": nw,
                        "vendor_rowwise_tflops": vendor_rowwise_tflops(q, ws, m, n, k)})
            del a, q, s, ws, c, gg
        tot_flops = sum(2.0 * p["m"] * p["n"] * p["k"] for p in pre)
        tot_s = sum(p["us"] for p in pre) * 1e-6
        vend = [p["vendor_rowwise_tflops"] for p in pre]
        vend_tflops = (round(tot_flops / sum(2.0 * p["m"] * p["n"] * p["k"] / (t * 1e12)
                                             for p, t in zip(pre, vend)) / 1e12, 1)
                       if all(vend) else None)
        result["prefill"] = {
            "tflops": round(tot_flops / tot_s / 1e12, 1),
            "vendor_rowwise_tflops": vend_tflops,
            "frac_of_peak": round(tot_flops / tot_s / 1e12 / FP8_PEAK_TFLOPS, 4),
            "peak_tflops": FP8_PEAK_TFLOPS, "shapes": pre,
            "roofline": {"bound": "mfma", "kernel": "w8a8 block-FP8 GEMM, prefill tiles",
                         "achieved": round(tot_flops / tot_s / 1e12, 1),
                         "peak": FP8_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tot_flops / tot_s / 1e12 / FP8_PEAK_TFLOPS, 4)}}
        torch.cuda.empty_cache()

        # ---------------- matrix-core ceiling without memory ----------------
        # 2 workgroups of 4 waves per CU (the persistent kernel's 8 waves per
        # CU), the MFMA inner loop from registers, with and without the four
        # promotion FMAs per MFMA; the clock the chip holds under this load
        # sets what any GEMM can reach
        mres = {}
        for promote in (False, True):
            iters = 1024
            flops = 2 * cus * 4 * iters * 32 * 65536

            def fm(promote=promote, iters=iters):
                st = ia.diag_mfma_loop(iters, 2 * cus, promote, sink, sp)
                assert st == 0, st

            gm_ = capture(lambda: [fm() for _ in range(4)])
            time_graphs([gm_], 2)
            us = time_graphs([gm_], 5) / 4 * 1e3
            mres["with_promotion" if promote else "mfma_only"] = {
                "us": round(us, 2), "tflops": round(flops / (us * 1e-6) / 1e12, 1),
                "frac_of_peak": round(flops / (us * 1e-6) / 1e12 / FP8_PEAK_TFLOPS, 4)}
            del gm_
        result["prefill"]["mfma_loop_ceiling"] = mres

        # ---------------- configs[3], configs[4] and 4096^3, shape by shape ----------------
        sweep = []
        for (m, n, k, tag) in ([(m, n, k, "config3") for m in SWEEP_M for (n, k) in SWEEP_NK]
                               + [(m, n, k, "config4") for (m, n, k) in RAGGED]
                               + [(m, n, k, "ref_bench") for (m, n, k) in REF_BENCH]):
            gb = gemm_bytes(m, n, k)
            flops = 2.0 * m * n * k
            bound_tflops = min(FP8_PEAK_TFLOPS, flops / gb * HBM_PEAK_GBS / 1e3)
            hbm_bound = bound_tflops < FP8_PEAK_TFLOPS
            # operand copies: more than 1 GiB in rotation (at most one per
            # launch of the graph), so the Infinity Cache cannot serve the
            # weights of an MFMA-bound shape either -- as in a model, where
            # each layer's weights arrive from HBM
            ncopy = min(PREFILL_LAUNCHES, max(2, -(-(1 << 30) // gb)))
            ops_ = []
            for _ in range(ncopy):
                q_ = rand_fp8((m, k))
                s_ = rand_scales((m, k // 128)) * 1e3
                ops_.append((q_, s_, rand_fp8((n, k)), rand_scales(((n + 127) // 128, k // 128)),
                             torch.empty((m, n), dtype=torch.bfloat16, device=dev)))

            def gs(i, m=m, n=n, k=k, ops_=ops_):
                q_, s_, bq_, bs_, c_ = ops_[i % len(ops_)]
                st = ia.w8a8_block_fp8_gemm(c_, q_, s_, bq_, bs_, m, n, k, 128, 128, DT.bf16, sp)
                assert st == 0, st

            gsw = capture(lambda: [gs(i) for i in range(PREFILL_LAUNCHES)])
            time_graphs([gsw], 2)
            us = time_graphs([gsw], 5) / PREFILL_LAUNCHES * 1e3
            tflops = flops / (us * 1e-6) / 1e12
            gbs = gb / (us * 1e-6) / 1e9
            cfg, split = ia.gemm_select(m, n, k)
            sweep.append({"set": tag, "m": m, "n": n, "k": k, "us": round(us, 2),
                          "tflops": round(tflops, 1), "gbs": round(gbs, 1),
                          "bound": "hbm" if hbm_bound else "mfma",
                          "frac_of_roofline": round(tflops / bound_tflops, 4),
                          "kernel": ia.gemm_config_name(cfg), "split_k": split,
                          "operand_copies": ncopy})
            del ops_, gsw
            torch.cuda.empty_cache()
        result["gemm_shapes"] = {
            "what": "BASELINE configs[3] (M sweep), configs[4] (ragged M) and the reference "
                    "bench's 4096^3, bf16 output, graph of 20 launches per shape; "
                    "frac_of_roofline against min(5 PF, AI x 8 TB/s)",
            "shapes": sweep}

        # ---------------- quantizer on large inputs ----------------
        qres = []
        for (mq, kq) in QUANT_SHAPES:
            nbuf = max(2, -(-(1 << 30) // (mq * kq * 2)))
            xs = [torch.randn((mq, kq), generator=gen, device=dev).to(torch.bfloat16)
                  for _ in range(nbuf)]
            q = torch.empty((mq, kq), dtype=torch.uint8, device=dev)
            s = torch.empty((mq, kq // 128), dtype=torch.float32, device=dev)

            def f(i, xs=xs, q=q, s=s, mq=mq, kq=kq):
                st = ia.quant_fp8_per_token_group(q, s, xs[i % len(xs)], DT.bf16, mq, kq, 128, sp)
                assert st == 0, st

            gq = capture(lambda: [f(i) for i in range(nbuf)])
            time_graphs([gq], 2)
            us = time_graphs([gq], 5) / nbuf * 1e3
            gbs = quant_bytes(mq, kq) / (us * 1e-6) / 1e9
            # the same bytes over the time above the launch floor (an empty
            # launch in the same kind of graph): the streaming rate itself
            gbs_stream = quant_bytes(mq, kq) / (max(us - launch_floor_us, 1e-3) * 1e-6) / 1e9
            qres.append({"m": mq, "k": kq, "us": round(us, 2), "gbs": round(gbs, 1),
                         "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "gbs_above_launch_floor": round(gbs_stream, 1)})
            del xs, q, s, gq
        # ---------------- dequantizer (E4M3 + group scales -> dt) ----------------
        dres = []
        for (md, kd, odt) in ((4096, 7168, torch.bfloat16), (8192, 18432, torch.bfloat16),
                              (4096, 7168, torch.float32)):
            ob = 4 if odt == torch.float32 else 2
            nbuf = max(2, -(-(1 << 30) // (md * kd * (1 + ob))))
            dq = [rand_fp8((md, kd)) for _ in range(nbuf)]
            ds_ = [rand_scales((md, kd // 128)) for _ in range(nbuf)]
            dx = [torch.empty((md, kd), dtype=odt, device=dev) for _ in range(nbuf)]
            dcode = DT.fp32 if odt == torch.float32 else DT.bf16

            def fdq(i, md=md, kd=kd, dq=dq, ds_=ds_, dx=dx, dcode=dcode, nbuf=nbuf):
                st = ia.dequant_fp8_per_token_group(dx[i % nbuf], dcode, dq[i % nbuf],
                                                    ds_[i % nbuf], md, kd, 128, sp)
                assert st == 0, st

            gd = capture(lambda: [fdq(i) for i in range(nbuf)])
            time_graphs([gd], 2)
            us = time_graphs([gd], 5) / nbuf * 1e3
            db = md * kd * (1 + ob) + 4 * md * (kd // 128)
            dres.append({"m": md, "k": kd, "dtype": str(odt).replace("torch.", ""),
                         "us": round(us, 2), "gbs": round(db / (us * 1e-6) / 1e9, 1),
                         "frac": round(db / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
            del dq, ds_, dx, gd
        result["dequant"] = {"shapes": dres, "peak_gbs": HBM_PEAK_GBS}
        # ---------------- weight block quantizer (weight-load time) ----------------
        wres = []
        for (nw, kw, wdt) in ((7168, 16384, torch.float32), (36864, 7168, torch.bfloat16)):
            ebytes = 4 if wdt == torch.float32 else 2
            nbuf = max(2, -(-(1 << 30) // (nw * kw * ebytes)))
            ws_ = [torch.randn((nw, kw), generator=gen, device=dev).to(wdt) * 0.02
                   for _ in range(nbuf)]
            wq = torch.empty((nw, kw), dtype=torch.uint8, device=dev)
            wsc = torch.empty(((nw + 127) // 128, kw // 128), dtype=torch.float32, device=dev)
            code = DT.fp32 if wdt == torch.float32 else DT.bf16

            def fw(i, ws_=ws_, wq=wq, wsc=wsc, nw=nw, kw=kw, code=code):
                st = ia.quant_fp8_weight_block(wq, wsc, ws_[i % len(ws_)], code, nw, kw, 128, 128,
                                               sp)
                assert st == 0, st

            gw = capture(lambda: [fw(i) for i in range(nbuf)])
            time_graphs([gw], 2)
            us = time_graphs([gw], 5) / nbuf * 1e3
            wb = nw * kw * (ebytes + 1) + 4 * ((nw + 127) // 128) * (kw // 128)
            wres.append({"n": nw, "k": kw, "dtype": str(wdt).replace("torch.", ""),
                         "us": round(us, 2), "gbs": round(wb / (us * 1e-6) / 1e9, 1),
                         "frac": round(wb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
            del ws_, wq, wsc, gw
        result["weight_quant"] = {"shapes": wres, "peak_gbs": HBM_PEAK_GBS}

        # ---------------- producers fused with the quantizer ----------------
        fres = []
        # SiLU(gate) * up -> E4M3: DeepSeek-V3 MLP, 4096 tokens x d 18432,
        # bf16 and fp16 gates
        tok, dd = 4096, 18432
        # inputs rotated over more than 1 GiB, so the 256 MB Infinity Cache
        # cannot serve them
        nsilu = max(2, -(-(1 << 30) // (tok * 2 * dd * 2)))
        fq = torch.empty((tok, dd), dtype=torch.uint8, device=dev)
        fs = torch.empty((tok, dd // 128), dtype=torch.float32, device=dev)
        for tdt, sdt, dname in ((torch.bfloat16, DT.bf16, "bfloat16"),
                                (torch.float16, DT.fp16, "float16")):
            gus = [torch.randn((tok, 2 * dd), generator=gen, device=dev).to(tdt)
                   for _ in range(nsilu)]

            def fsilu(i):
                st = ia.silu_and_mul_quant_fp8(fq, fs, gus[i % nsilu], sdt, tok, dd, 128, sp)
                assert st == 0, st

            gf = capture(lambda: [fsilu(i) for i in range(nsilu)])
            time_graphs([gf], 2)
            us = time_graphs([gf], 5) / nsilu * 1e3
            fb = tok * dd * (2 * 2 + 1) + 4 * tok * (dd // 128)
            fres.append({"op": "silu_and_mul_quant_fp8", "tokens": tok, "d": dd, "dtype": dname,
                         "us": round(us, 2), "gbs": round(fb / (us * 1e-6) / 1e9, 1),
                         "frac": round(fb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
            del gus, gf
        del fq, fs
        # residual += x; RMSNorm -> E4M3: 4096 rows x 7168 (the hidden size), bf16
        rows, cols = 4096, 7168
        # (residual, x) pairs rotated over more than 1 GiB
        nrms = max(2, -(-(1 << 30) // (rows * cols * 2 * 2)))
        res_ = [torch.randn((rows, cols), generator=gen, device=dev).to(torch.bfloat16)
                for _ in range(nrms)]
        xs_ = [torch.randn((rows, cols), generator=gen, device=dev).to(torch.bfloat16) * 0.01
               for _ in range(nrms)]
        wn = torch.ones((cols,), dtype=torch.bfloat16, device=dev)
        fq = torch.empty((rows, cols), dtype=torch.uint8, device=dev)
        fs = torch.empty((rows, cols // 128), dtype=torch.float32, device=dev)

        def frms(i):
            st = ia.fused_add_rmsnorm_quant_fp8(res_[i % nrms], fq, fs, xs_[i % nrms], wn, DT.bf16,
                                                rows, cols, 1e-6, 128, sp)
            assert st == 0, st

        gf = capture(lambda: [frms(i) for i in range(nrms)])
        time_graphs([gf], 2)
        us = time_graphs([gf], 5) / nrms * 1e3
        fb = rows * cols * (3 * 2 + 1) + 2 * cols + 4 * rows * (cols // 128)
        fres.append({"op": "fused_add_rmsnorm_quant_fp8", "rows": rows, "cols": cols,
                     "dtype": "bfloat16", "us": round(us, 2),
                     "gbs": round(fb / (us * 1e-6) / 1e9, 1),
                     "frac": round(fb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
        del res_, xs_, wn, fq, fs, gf
        result["fused_producers"] = {"shapes": fres, "peak_gbs": HBM_PEAK_GBS}

        # ---------------- MoE routing: DeepSeek-V3 shape, 256 experts, top-8 ----------------
        tres = []
        for tok in (64, 4096):
            lg = torch.randn((tok, 256), generator=gen, device=dev) * 2.0
            tid = torch.empty((tok, 8), dtype=torch.int32, device=dev)
            twt = torch.empty((tok, 8), dtype=torch.float32, device=dev)

            def ftk(i, lg=lg, tid=tid, twt=twt, tok=tok):
                st = ia.topk_softmax(tid, twt, lg, tok, 256, 8, True, sp)
                assert st == 0, st

            gt = capture(lambda: [ftk(i) for i in range(8)])
            time_graphs([gt], 2)
            us = time_graphs([gt], 5) / 8 * 1e3
            tres.append({"tokens": tok, "experts": 256, "topk": 8, "us": round(us, 2)})
            del lg, tid, twt, gt
        result["topk_softmax"] = {"shapes": tres}

        # ---------------- grouped GEMM over MoE experts ----------------
        # One GPU's share of a DeepSeek-V3-like MoE layer with 8-way expert
        # parallelism: 32 local experts, gate/up projection (N = 2 x 2048,
        # K = 7168), contiguous layout, rows per expert drawn from a uniform
        # multinomial routing.  Decode: 64 token-expert rows (GB/s; the call
        # streams the weights of every expert that has rows, and only those
        # count: 7 of the 32 experts get none with this seed); prefill: 4096
        # rows (TFLOP/s).  Two weight copies (1.9 GB) so neither cache holds
        # them.
        gres = []
        ge_, gn, gk = 32, 4096, 7168
        wsets = [(rand_fp8((ge_, gn, gk)), rand_scales((ge_, gn // 128, gk // 128)))
                 for _ in range(2)]
        for gm in (64, 4096):
            sizes = np.random.default_rng(gm).multinomial(gm, np.ones(ge_) / ge_)
            off = torch.tensor(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32),
                               device=dev)
            gaq = rand_fp8((gm, gk))
            gas = rand_scales((gm, gk // 128))
            gc = torch.empty((gm, gn), dtype=torch.bfloat16, device=dev)

            def fg(i, gm=gm, off=off, gaq=gaq, gas=gas, gc=gc):
                bq, bs = wsets[i % 2]
                st = ia.w8a8_block_fp8_grouped_gemm(gc, gaq, gas, bq, bs, off, gm, gn, gk, ge_,
                                                    128, 128, DT.bf16, sp)
                assert st == 0, st

            gg = capture(lambda: [fg(i) for i in range(10)])
            time_graphs([gg], 2)
            us = time_graphs([gg], 5) / 10 * 1e3
            used = int((sizes > 0).sum())  # experts whose weights the call reads
            wbytes = used * (gn * gk + 4 * (gn // 128) * (gk // 128))
            gbytes = wbytes + gm * gk + 4 * gm * (gk // 128) + 2 * gm * gn
            gres.append({"rows": gm, "experts": ge_, "experts_with_rows": used, "n": gn,
                         "k": gk, "us": round(us, 2),
                         "gbs": round(gbytes / (us * 1e-6) / 1e9, 1),
                         "hbm_frac": round(gbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                         "tflops": round(2.0 * gm * gn * gk / (us * 1e-6) / 1e12, 1),
                         "kernel": ia.gemm_config_name(ia.grouped_gemm_select(gm, gn, gk, ge_))})
            del off, gaq, gas, gc, gg
        del wsets
        result["moe_grouped_gemm"] = {"shapes": gres, "peak_gbs": HBM_PEAK_GBS,
                                      "peak_tflops": FP8_PEAK_TFLOPS}

        # the roofline line carries the worst of the shapes (the reference
        # bench's 4096x7168, bench/bench_kernels.cpp:82-94, is the smallest)
        qworst = min(qres, key=lambda r: r["frac"])
        result["quant"] = {"shapes": qres, "peak_gbs": HBM_PEAK_GBS,
                           "launch_floor_us": round(launch_floor_us, 2),
                           "roofline": {"bound": "hbm", "kernel": "per-token-group quantizer",
                                        "shape": [qworst["m"], qworst["k"]],
                                        "achieved": qworst["gbs"], "peak": HBM_PEAK_GBS,
                                        "unit": "GB/s", "frac": qworst["frac"]}}

    torch.cuda.synchronize()
    if not args.no_cpu:
        result["cpu_baseline"], result["cpu_baseline_parallel"] = cpu_baseline()
        result["cpu_baseline_prefill"] = cpu_baseline_prefill()
    print(json.dumps(result), flush=True)


def gpu_clocks():
    """The clock lines `rocm-smi --showclocks` prints right after the decode
    timing (a child process with its own time limit), or None where the tool
    is missing or fails: context for the measured rates, not a measurement."""
    import shutil
    import subprocess
    exe = shutil.which("rocm-smi")
    if exe is None:
        return None
    try:
        out = subprocess.run([exe, "--showclocks"], capture_output=True, text=True,
                             timeout=20).stdout
    except (OSError, subprocess.SubprocessError):
        return None
    lines = [ln.strip() for ln in out.splitlines() if "clk" in ln.lower() and ":" in ln]
    return lines or None


def host_cpu():
    """The host CPU model string (/proc/cpuinfo, else lscpu) and the core
    count the OS reports."""
    import shutil
    import subprocess
    model = ""
    extra = {}
    try:
        for line in open("/proc/cpuinfo"):
            key = line.split(":", 1)[0].strip().lower()
            if key in ("model name", "cpu model", "processor model") and not model:
                model = line.split(":", 1)[1].strip()
            elif key in ("vendor_id", "cpu family", "model", "stepping", "cache size") \
                    and key not in extra:
                extra[key] = line.split(":", 1)[1].strip()
            elif not line.strip() and model:
                break
    except OSError:
        pass
    if extra:
        # the model string alone can be generic under virtualisation
        model = (model or "unknown model") + " (" + ", ".join(
            f"{k} {v}" for k, v in extra.items()) + ")"
    if not model and shutil.which("lscpu"):
        try:
            out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
            for line in out.splitlines():
                if line.lower().startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
        except (OSError, subprocess.SubprocessError):
            pass
    return f"{model or 'unknown model'}; nproc {os.cpu_count()}"


def cpu_baseline_prefill():
    """The reference's CPU GEMM (reference.cpp:93-110 from oracle/_ref, else the
    oracle's restatement), single-threaded, on two deterministic rows (0 and
    M/2) of each configs[2] shape (M = 4096), extrapolated linearly to all M
    rows: the naive loop's cost per row does not depend on the row."""
    import numpy as np

    import oracle

    use_ref = oracle.ref_available()
    g = np.random.default_rng(1)
    m = 4096
    rows = np.array([0, m // 2])
    shapes = []
    tot_flops = tot_s = 0.0
    for (n, k) in PREFILL_NK:
        aq = g.integers(0, 0x7E, (len(rows), k), dtype=np.uint8)
        as_ = (g.random((len(rows), k // 128), dtype=np.float32) + 0.5)
        bq = g.integers(0, 0x7E, (n, k), dtype=np.uint8)
        bs = (g.random(((n + 127) // 128, k // 128), dtype=np.float32) * 1e-3 + 1e-4)
        t0 = time.perf_counter()
        if use_ref:
            oracle.ref_gemm(aq, as_, bq, bs)
        else:
            oracle.gemm(aq, as_, bq, bs, threads=1)
        dt = time.perf_counter() - t0
        full_s = dt * m / len(rows)
        flops = 2.0 * m * n * k
        tot_flops += flops
        tot_s += full_s
        shapes.append({"n": n, "k": k, "rows_timed": len(rows), "seconds_timed": round(dt, 3),
                       "seconds_extrapolated": round(full_s, 1),
                       "tflops": round(flops / full_s / 1e12, 6)})
    return {"value": round(tot_flops / tot_s / 1e12, 6), "unit": "TFLOP/s", "cores": 1,
            "kind": "reference" if use_ref else "port",
            "sample": f"rows 0 and 2048 of each configs[2] shape (M=4096), single thread, "
                      f"compiled -O2, extrapolated linearly to M=4096; host CPU: {host_cpu()}",
            "shapes": shapes}


def cpu_baseline():
    """The reference's CPU golden code (oracle/_ref when it was built, else the
    oracle's C restatement) over the full decode workload, single-threaded as
    the reference runs it: quant of every A + GEMM of every (M, N, K)."""
    import numpy as np

    import oracle

    use_ref = oracle.ref_available()
    g = np.random.default_rng(0)
    total_bytes = 0
    t_total = 0.0
    for m in DECODE_M:
        for (n, k) in DECODE_NK:
            a = g.standard_normal((m, k), dtype=np.float32)
            bq = g.integers(0, 0x7E, (n, k), dtype=np.uint8)
            bs = (g.random(((n + 127) // 128, k // 128), dtype=np.float32) * 1e-3 + 1e-4)
            t0 = time.perf_counter()
            if use_ref:
                aq, as_ = oracle.ref_quant(a)
                oracle.ref_gemm(aq, as_, bq, bs)
            else:
                aq, as_ = oracle.quant(a)
                oracle.gemm(aq, as_, bq, bs, threads=1)
            t_total += time.perf_counter() - t0
            total_bytes += quant_bytes(m, k) + gemm_bytes(m, n, k)
    cpu = host_cpu()
    single = {"value": round(total_bytes / t_total / 1e9, 4), "unit": "GB/s", "cores": 1,
              "kind": "reference" if use_ref else "port",
              "sample": "the full decode workload once (9 quant + 9 GEMM, the GPU step's "
                        f"shapes), single thread, {t_total:.1f} s, compiled -O2; host CPU: {cpu}",
              "seconds": round(t_total, 2)}
    # The same workload on the oracle's C restatement with its GEMM spread over
    # (row, 64-column block) items on the host cores (at most 16, the GPU
    # box's CPU share; the quantizer stays single-threaded); per-element
    # arithmetic is the reference's.
    cores = max(1, min(os.cpu_count() or 1, 16))
    g = np.random.default_rng(0)
    t_par = 0.0
    for m in DECODE_M:
        for (n, k) in DECODE_NK:
            a = g.standard_normal((m, k), dtype=np.float32)
            bq = g.integers(0, 0x7E, (n, k), dtype=np.uint8)
            bs = (g.random(((n + 127) // 128, k // 128), dtype=np.float32) * 1e-3 + 1e-4)
            t0 = time.perf_counter()
            aq, as_ = oracle.quant(a)
            oracle.gemm(aq, as_, bq, bs, threads=cores)
            t_par += time.perf_counter() - t0
    parallel = {"value": round(total_bytes / t_par / 1e9, 4), "unit": "GB/s", "cores": cores,
                "kind": "port",
                "sample": f"the same workload, GEMM on {cores} OpenMP threads, {t_par:.2f} s",
                "seconds": round(t_par, 3)}
    return single, parallel


if __name__ == "__main__":
    main()
