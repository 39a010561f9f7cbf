"""The reference forwards that `bench.py --vs-torch` times (bench.ref_*) agree with the oracle's
torch restatements of the same reference.py lines (oracle/torch_ref.py) on small CPU inputs."""
import torch

import bench
from kernelbench_harbor_amd import inputs
from oracle import torch_ref as tr


def _close(a, b, tol=2e-3):
    a, b = a.float(), b.float()
    return float((a - b).abs().max()) <= tol * max(float(b.abs().max()), 1e-6)


def test_ref_w4a16():
    args = inputs.w4a16(4, 256, 128, seed=1)
    assert _close(bench.ref_w4a16(*args), tr.w4a16(*args))


def test_ref_w8a8():
    args = inputs.w8a8(4, 256, 128, seed=2)
    assert torch.equal(bench.ref_w8a8(*args), tr.w8a8(*args))


def test_ref_fp8w():
    args = inputs.fp8w(4, 256, 128, 128, torch.float16, 3)
    assert _close(bench.ref_fp8w(*args), tr.fp8w(*args))


def test_ref_qmoe():
    args = inputs.qmoe(T=8, D=256, E=4, N=128, seed=4)
    assert _close(bench.ref_qmoe(*args), tr.qmoe(*args))
