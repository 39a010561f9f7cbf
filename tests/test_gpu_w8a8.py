"""GPU parity of the W8A8 HIP path against the CPU oracle (oracle/w8a8.py).

The int32 accumulation is exact and the epilogue follows the reference's operation order, so
outputs are compared bit for bit."""
import numpy as np
import pytest
import torch

from kernelbench_harbor_amd import W8A8Model, inputs, ops
from kernelbench_harbor_amd.harness import compare
from oracle import w8a8 as o8

pytestmark = pytest.mark.gpu

CASES = [
    # M, K, N, dist
    (1, 1024, 128, "reference"),
    (3, 2048, 384, "baseline"),
    (16, 4096, 512, "reference"),
    (17, 1024, 256, "baseline"),
    (64, 2048, 1024, "baseline"),
    (128, 1024, 256, "reference"),
    (300, 2048, 384, "baseline"),
    (100, 1088, 256, "reference"),   # K % 128 != 0: split-K path at large M
    # wide-tile int8 kernel (M > 32, N % 256 == 0, K % 128 == 0): with and without split-K,
    # ragged M, 1-3 row blocks
    (33, 2048, 256, "baseline"),
    (257, 1024, 768, "reference"),
    (512, 4096, 512, "baseline"),
    (600, 8192, 256, "reference"),
]


@pytest.mark.parametrize("M,K,N,dist", CASES)
def test_w8a8_bit_exact(dev, M, K, N, dist):
    print(f"[w8a8] M={M} K={K} N={N} {dist}", flush=True)
    x, w, xs, ws = inputs.w8a8(M, K, N, seed=M + K, dist=dist)
    y = ops.w8a8_gemm(x.to(dev), w.to(dev), xs.to(dev), ws.to(dev))
    assert y.dtype == torch.float16 and y.shape == (M, N)
    want = o8.forward(x.numpy(), w.numpy(), xs.float().numpy(), ws.float().numpy())
    got = y.float().cpu().numpy()
    assert np.array_equal(got, want), np.abs(got - want).max()
    acc = ops.w8a8_gemm_i32(x.to(dev), w.to(dev)).cpu().numpy()
    assert np.array_equal(acc, o8.acc_int32(x.numpy(), w.numpy()))


@pytest.mark.parametrize("M", [16, 512])
def test_w8a8_full_size(dev, M):
    """The benchmark's W8A8 configuration: SmoothQuant inputs at M in {16, 512}, K=14336, N=4096."""
    print(f"[w8a8 full] M={M}", flush=True)
    x, w, xs, ws = inputs.w8a8(M, 14336, 4096, seed=M)
    y = W8A8Model()(x.to(dev), w.to(dev), xs.to(dev), ws.to(dev))
    want = o8.forward(x.numpy(), w.numpy(), xs.float().numpy(), ws.float().numpy())
    got = y.float().cpu().numpy()
    assert np.array_equal(got, want)
    assert compare(y, want).ok


@pytest.mark.parametrize("M", [16, 100, 256])
def test_w8a8_int32_extremes(dev, M):
    """|acc| reaches K*127^2 = 231,225,344 (all +127) and K*128*127 (-128 against +127)."""
    K, N = 14336, 256
    x = torch.full((M, K), 127, dtype=torch.int8)
    x[1::2] = -128
    w = torch.full((K, N), 127, dtype=torch.int8)
    w[:, 1::2] = -127
    acc = ops.w8a8_gemm_i32(x.to(dev), w.to(dev)).cpu().numpy()
    assert acc[0, 0] == 231225344 and acc[0, 1] == -231225344
    assert acc[1, 0] == -128 * 127 * K and acc[1, 1] == 128 * 127 * K
    assert np.array_equal(acc, o8.acc_int32(x.numpy(), w.numpy()))
