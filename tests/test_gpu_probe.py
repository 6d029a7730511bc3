"""The matrix-core ceiling probe that bench.py --mfma-ceiling runs
(probe/mfma_ceiling.hip, its own library): every mode launches, finishes and
gives a rate inside what the hardware allows -- products below the 2.5
PFLOP/s the chip is quoted at, LDS reads below one 16-byte read per lane and
clock on every CU.  A short run per mode; the figures themselves are
measurements, not tested."""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent

pytestmark = pytest.mark.gpu


def test_every_probe_mode_runs():
    import torch
    sys.path.insert(0, str(ROOT))
    import bench
    assert torch.cuda.is_available()
    res = bench.mfma_ceiling(torch.device("cuda:0"), seconds=0.05, settle=0.0)
    modes = res["modes"]
    assert [m["mode"] for m in modes] == list(range(len(bench.MFMA_CEILING_MODES)))
    for m in modes:
        if m["mode"] in bench.MFMA_CEILING_LDS_ONLY:
            # 64 lanes x 16 B per clock on 256 CUs at 2.4 GHz: 629 TB/s
            assert 1.0 < m["lds_tbytes_per_s"] < 629.0, m
        else:
            assert 50.0 < m["tflops"] <= bench.PEAK_BF16_TFLOPS, m
