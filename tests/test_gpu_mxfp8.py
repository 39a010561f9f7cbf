"""GPU parity of the MXFP8 scaled-MFMA GEMM against the CPU oracle (oracle/mxfp8.py)."""
import numpy as np
import pytest
import torch

from kernelbench_harbor_amd import MXFP8Model, inputs, ops
from kernelbench_harbor_amd.harness import compare
from oracle import mxfp8 as om

pytestmark = pytest.mark.gpu


def _gt(a, sa, b, sb, acc=np.float64):
    return om.forward(a.numpy(), sa.numpy(), b.numpy(), sb.numpy(), accumulate=acc)


# (1024, 1024, 256), (1100, 2048, 512), (2000, 512, 4096) and (1024, 256, 512) take the 256 x 256
# LDS-DMA tiles (the second and third with a partial last row block, the last two without a K
# split, the last one with the minimum K: one pair of slabs); the others the 128-row tiles.
CASES = [(1, 256, 64), (16, 1024, 256), (100, 2048, 320), (128, 4096, 512), (300, 1024, 1024),
         (513, 512, 256), (1024, 1024, 256), (1100, 2048, 512), (2000, 512, 4096),
         (1024, 256, 512)]


@pytest.mark.parametrize("M,K,N", CASES)
@pytest.mark.parametrize("out", [torch.float16, torch.bfloat16])
def test_mxfp8_parity(dev, M, K, N, out):
    print(f"[mxfp8] M={M} K={K} N={N} {out}", flush=True)
    a, sa, b, sb = inputs.mxfp8(M, K, N, seed=M + N)
    y = ops.mxfp8_gemm(a.to(dev), sa.to(dev), b.to(dev), sb.to(dev), out_dtype=out)
    assert y.dtype == out and y.shape == (M, N)
    cmp = compare(y, _gt(a, sa, b, sb))
    assert cmp.ok, cmp


@pytest.mark.parametrize("M,N", [(64, 128), (1024, 256)])
def test_mxfp8_e8m0_decode_bit_exact(dev, M, N):
    """All elements 1.0 with per-block exponents in [124, 128]: every partial sum is exact in
    fp32, so y must equal the oracle's exactly (tests the e8m0 decode and its block mapping, on
    the 128-row and the 256 x 256 tiles)."""
    K = 2048
    g = torch.Generator().manual_seed(9)
    a = torch.full((M, K), 0x38, dtype=torch.uint8)
    b = torch.full((N, K), 0x38, dtype=torch.uint8)
    sa = torch.randint(124, 129, (M, K // 32), generator=g).to(torch.uint8)
    sb = torch.randint(124, 129, (N, K // 32), generator=g).to(torch.uint8)
    y = ops.mxfp8_gemm(a.to(dev), sa.to(dev), b.to(dev), sb.to(dev)).float().cpu().numpy()
    want = _gt(a, sa, b, sb).astype(np.float16).astype(np.float32)
    assert np.array_equal(y, want)


@pytest.mark.parametrize("M", [128, 2048])
def test_mxfp8_full_size(dev, M):
    """The benchmark's MXFP8 configuration: M in {128, 2048}, K=14336, N=4096."""
    print(f"[mxfp8 full] M={M}", flush=True)
    a, sa, b, sb = inputs.mxfp8(M, 14336, 4096, seed=M)
    y = MXFP8Model()(a.to(dev), sa.to(dev), b.to(dev), sb.to(dev))
    cmp = compare(y, _gt(a, sa, b, sb, acc=np.float32))
    assert cmp.ok, cmp
