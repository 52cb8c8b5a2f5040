"""The split-K workspace is a fixed pool of slots per device: streams that are
created and destroyed by the dozen hold no more device memory than the pool,
and every GEMM still meets the tolerance -- bit-identical to the null-stream
result while its stream has a slot, unsplit (so within tolerance of the
oracle, other bits) once the slots are all held.  Runs in a child process so
that the pool starts empty and the exhausted pool does not reach other tests."""
import os
import subprocess
import sys

import pytest

from gpu_util import device

_CHILD = r"""
import ctypes
import sys
import numpy as np
import torch
import datagen
import inferop_amd
import oracle
from gpu_util import assert_gemm_close, to_dev

# the HIP runtime already in the process (torch loaded it; same soname)
hip = ctypes.CDLL("libamdhip64.so.7")
hip.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
hip.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
hip.hipStreamDestroy.argtypes = [ctypes.c_void_p]

m, n, k = 64, 2112, 7168
cfg, split = inferop_amd.gemm_select(m, n, k)
assert split > 1, (cfg, split)
_, a_f32, bq, bs = datagen.gemm_case(m, n, k, seed=5)
aq, as_ = oracle.quant(a_f32)
ref = oracle.gemm(aq, as_, bq, bs)
args = [to_dev(v) for v in (aq, as_, bq, bs)]
used0, total, slot_bytes = inferop_amd.splitk_workspace_info()
assert used0 == 0 and total == 8 and slot_bytes == (64 << 20) + 4 * 16384, (used0, total, slot_bytes)

outs = [torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda:0")
        for _ in range(66)]
extra = torch.empty((m, n), dtype=torch.bfloat16, device="cuda:0")

# the null stream first: its slot, its split result (this first launch also
# loads the library's code objects, so device memory is measured after it)
want = outs[0]
assert inferop_amd.w8a8_block_fp8_gemm(want, *args, m, n, k, stream=0) == 0
torch.cuda.synchronize()
assert_gemm_close(want.float().cpu().numpy(), ref, "null stream")
free0, _ = torch.cuda.mem_get_info()

def new_stream():
    s = ctypes.c_void_p()
    assert hip.hipStreamCreate(ctypes.byref(s)) == 0
    return s

def run(c, s):
    assert inferop_amd.w8a8_block_fp8_gemm(c, *args, m, n, k, stream=s.value) == 0
    assert hip.hipStreamSynchronize(s) == 0

# ten streams alive at once: seven take the remaining slots, three run unsplit;
# a forced split is refused on a stream without a slot and accepted on one with
live = [new_stream() for _ in range(10)]
for i, s in enumerate(live):
    run(outs[1 + i], s)
refused = inferop_amd.w8a8_block_fp8_gemm_config(extra, *args, m, n, k, inferop_amd.dtype.bf16,
                                                 cfg, split, live[9].value)
accepted = inferop_amd.w8a8_block_fp8_gemm_config(extra, *args, m, n, k, inferop_amd.dtype.bf16,
                                                  cfg, split, live[0].value)
assert refused == inferop_amd.Status.ERR_ARGUMENT and accepted == 0, (refused, accepted)
assert hip.hipStreamSynchronize(live[0]) == 0
for s in live:
    assert hip.hipStreamDestroy(s) == 0
# then 55 streams created and destroyed one after another
for i in range(55):
    s = new_stream()
    run(outs[11 + i], s)
    assert hip.hipStreamDestroy(s) == 0
torch.cuda.synchronize()

used, total, _ = inferop_amd.splitk_workspace_info()
free1, _ = torch.cuda.mem_get_info()
grown = free0 - free1
print(f"slots {used}/{total}, device memory grown by {grown / 2**20:.1f} MiB", flush=True)
assert used == total, used
# the seven further slots, each rounded up to 2 MiB pages, plus 64 MiB for
# the runtime's own per-stream state (one 64 MiB workspace per stream, as a
# pool without a bound would take, is 3.9 GiB here)
slot_pages = -(-slot_bytes // (2 << 20)) * (2 << 20)
assert grown <= (total - 1) * slot_pages + (64 << 20), grown
same = 0
for i, c in enumerate(outs[1:]):
    assert_gemm_close(c.float().cpu().numpy(), ref, f"stream {i}")
    same += int(torch.equal(c, want))
# the seven streams that took a slot reproduce the null stream's bits
assert torch.equal(outs[1], want) and same >= 7, same
print("ok", flush=True)
"""


@pytest.mark.gpu
def test_workspace_pool_bounds_memory_over_64_streams():
    device()
    tests = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(tests)
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([root, tests,
                                                       os.environ.get("PYTHONPATH", "")]))
    r = subprocess.run([sys.executable, "-c", _CHILD], env=env, capture_output=True, text=True,
                       timeout=300)
    print(r.stdout[-1000:])
    assert r.returncode == 0 and "ok" in r.stdout, (r.stdout[-2000:], r.stderr[-2000:])
