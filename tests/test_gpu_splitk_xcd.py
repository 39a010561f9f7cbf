"""Split-K slice sums placed on the XCDs that wrote the slices (splitk_sum_kernel, splitk.h).

A decode launch of ntiles x splits workgroups runs the splits of a contiguous range of column
tiles on each XCD; the sum kernel recomputes those ranges. The shapes below take each of its
three geometries, with the whole output checked (the task-grid test only checks the first and
last 256 columns):

* "xcd": every tile's splits on one XCD (grid % 8 == 0, splits divide the per-XCD share),
* "straddle": tiles whose splits span two XCDs (the share is not a multiple of splits),
* "plain": grid % 8 != 0, the sum falls back to linear indexing.

W8A8's raw int32 accumulators are compared bit for bit with an int64 matmul; the fp16/bf16
GEMMs within the benchmark's tolerance of the oracle, and repeated calls must agree bit for bit."""
import numpy as np
import pytest
import torch

from kernelbench_harbor_amd import inputs, ops
from kernelbench_harbor_amd.harness import compare
from oracle import fp8w as of
from oracle import w4a16 as ow

pytestmark = pytest.mark.gpu

# (K, N): geometry at M <= 16 for W4A16 (256-column tiles when N % 256 == 0, else 128)
W4_SHAPES = [(1024, 2048, "xcd"), (1024, 640, "straddle"), (1536, 896, "plain"),
             (1024, 768, "straddle")]
# (K, N): geometry at M <= 16 for the 128-column FP8-weight and W8A8 decode kernels
W8_SHAPES = [(1024, 1024, "xcd"), (1024, 640, "straddle"), (1536, 896, "plain")]


@pytest.mark.parametrize("K,N,geom", W4_SHAPES)
@pytest.mark.parametrize("M", [1, 16, 29])
def test_w4a16_xcd_sum(dev, M, K, N, geom):
    print(f"[xcd-sum w4a16] {geom} M={M} K={K} N={N}", flush=True)
    x, qw, s, z = inputs.w4a16(M, K, N, 128, torch.float16, seed=M + N)
    args = [t.to(dev) for t in (x, qw, s, z)]
    y1 = ops.w4a16_gemm(*args)
    y2 = ops.w4a16_gemm(*args)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    cmp = compare(y1, ow.forward(x.float().numpy(), qw.numpy(), s.float().numpy(),
                                 z.float().numpy()))
    assert cmp.ok, cmp


@pytest.mark.parametrize("K,N,geom", W8_SHAPES)
@pytest.mark.parametrize("M", [1, 16])
def test_w8a8_xcd_sum(dev, M, K, N, geom):
    print(f"[xcd-sum w8a8] {geom} M={M} K={K} N={N}", flush=True)
    x, w, xs, ws = inputs.w8a8(M, K, N, seed=M + N, dist="reference")
    acc = ops.w8a8_gemm_i32(x.to(dev), w.to(dev)).cpu().numpy()
    exact = x.numpy().astype(np.int64) @ w.numpy().astype(np.int64)
    assert np.array_equal(acc.astype(np.int64), exact)
    y1 = ops.w8a8_gemm(x.to(dev), w.to(dev), xs.to(dev), ws.to(dev))
    y2 = ops.w8a8_gemm(x.to(dev), w.to(dev), xs.to(dev), ws.to(dev))
    assert torch.equal(y1, y2)


@pytest.mark.parametrize("K,N,geom", W8_SHAPES)
@pytest.mark.parametrize("M", [1, 16])
def test_fp8w_xcd_sum(dev, M, K, N, geom):
    print(f"[xcd-sum fp8w] {geom} M={M} K={K} N={N}", flush=True)
    x, w, s = inputs.fp8w(M, K, N, 128, torch.bfloat16, seed=M + N)
    y = ops.fp8w_gemm(x.to(dev), w.to(dev), s.to(dev))
    torch.cuda.synchronize()
    cmp = compare(y, of.forward(x.float().numpy(), w.view(torch.uint8).numpy(),
                                s.float().numpy()))
    assert cmp.ok, cmp
