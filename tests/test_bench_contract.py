"""bench.py's contract checked on the CPU: the algorithmic byte and FLOP counts it divides by
(pinned to the figures of the benchmark configurations) and the single-GPU exit."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


@pytest.mark.parametrize("M,want", [(1, 31_232_000), (16, 31_784_960), (2048, 106_692_608)])
def test_w4a16_algorithmic_bytes(M, want):
    # K*N/2 + 2*(K/G)*N*2 + 2*M*K + 2*M*N at K=14336, N=4096, G=128
    assert bench.w4a16_bytes(M) == want
    assert bench.w4a16_bytes(16, 29568, 8192, 64) == 29568 * 8192 // 2 + 2 * (29568 // 64) * 8192 * 2 \
        + 2 * 16 * 29568 + 2 * 16 * 8192


def test_other_config_figures():
    assert bench.gemm_flops(16) == 1_879_048_192
    assert bench.w8a8_bytes(16) == 59_088_928 and bench.w8a8_bytes(512) == 70_263_808
    assert bench.mxfp8_bytes(128) == 63_496_192 and bench.mxfp8_bytes(2048) == 107_610_112
    assert bench.fp8w_bytes(16) == 60_227_584
    assert bench.ffn_bytes() == 757_088_256 and bench.ffn_flops() == 2 * 512 * 6 * 4096 * 14336
    assert bench.qmoe_bytes() == 486_543_360 and bench.qmoe_flops() == 2 * 256 * 2 * 4096 * 14336


def test_roofline_picks_the_binding_term():
    bound, frac = bench.roofline(1e-3, bench.HBM_PEAK * 1e-3, 1.0, bench.PEAK["f16"])
    assert bound == "hbm" and abs(frac - 1.0) < 1e-9
    bound, frac = bench.roofline(2e-3, 1.0, bench.PEAK["f16"] * 1e-3, bench.PEAK["f16"])
    assert bound == "mfma" and abs(frac - 0.5) < 1e-9


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr
