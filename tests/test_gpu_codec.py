"""On-device proof that the hardware E4M3 conversions used by the fast paths
agree with the reference's software codec (all 2^32 fp32 inputs)."""
import json
import os

import numpy as np
import pytest
import torch

import inferop_amd
from gpu_util import device

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.gpu
def test_hw_codec_matches_reference_exhaustive():
    device()
    counts = torch.zeros(4, dtype=torch.int64, device="cuda:0")
    st = inferop_amd.ops.selftest_fp8_codec(counts, 0, 1 << 32)
    assert st == 0
    torch.cuda.synchronize()
    c = counts.cpu().numpy().view(np.uint64)
    print("codec selftest counts:", [int(v) for v in c], flush=True)
    golden = json.load(open(os.path.join(GOLDEN, "codec.json")))
    assert int(c[0]) == 0, "hardware encode differs inside the quantizer fast-path domain"
    assert int(c[2]) == golden["encode_checksum"], "device software encoder != reference"
    assert int(c[3]) == 0, "hardware decode differs from the software decode"
