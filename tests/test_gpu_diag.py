"""The bench's measurement kernels run to completion on the device, and their
host guards reject shapes the kernels do not handle (the numbers they time
are the bench's ceilings, so a kernel that silently failed to launch would
report an impossible ceiling)."""
import pytest
import torch

import inferop_amd
from gpu_util import device


@pytest.mark.gpu
def test_stripe_read_patterns_launch():
    dev = device()
    S = inferop_amd.Status
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    for (n, k) in ((4096, 7168), (2112, 7168), (7168, 2048)):
        b = torch.randint(0, 255, (n, k), dtype=torch.uint8, device=dev)
        for pattern in range(5):
            for stripes in (0, 16):
                print(f"stripe read n={n} k={k} pattern={pattern} stripes={stripes}", flush=True)
                assert inferop_amd.diag_stripe_read(b, n, k, pattern, stripes, sink) == S.OK
        torch.cuda.synchronize()
    b = torch.zeros((64, 2048), dtype=torch.uint8, device=dev)
    assert inferop_amd.diag_stripe_read(b, 64, 3072, 0, 0, sink) == S.ERR_ARGUMENT
    assert inferop_amd.diag_stripe_read(b, 60, 2048, 0, 0, sink) == S.ERR_ARGUMENT
    assert inferop_amd.diag_stripe_read(b, 64, 2048, 5, 0, sink) == S.ERR_ARGUMENT
    assert inferop_amd.diag_stripe_read(b, 64, 2048, 0, 5, sink) == S.ERR_ARGUMENT
    torch.cuda.synchronize()
    assert int(sink[0]) == 0 or int(sink[0]) == int(0x9E3779B9 - (1 << 32))


@pytest.mark.gpu
def test_read_stream_and_mfma_loop_launch():
    dev = device()
    S = inferop_amd.Status
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    src = torch.zeros(1 << 20, dtype=torch.uint8, device=dev)
    assert inferop_amd.diag_read_stream(src, 1 << 20, 256, sink) == S.OK
    assert inferop_amd.diag_mfma_loop(4, 256, True, sink) == S.OK
    assert inferop_amd.diag_mfma_loop(4, 256, False, sink) == S.OK
    assert inferop_amd.diag_read_stream(src, 8, 1, sink) == S.ERR_ARGUMENT
    torch.cuda.synchronize()
