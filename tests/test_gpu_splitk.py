"""Split-K contract of the small-M kernels (W8A8, FP8 weight and MXFP8 GEMMs; W4A16 has its own
test in test_gpu_w4a16.py): each K split stores its partial tile into its own workspace slice and
a second kernel adds the slices in split order, so

* the workspace needs no particular content (a buffer of 0xFF bytes, NaN patterns as fp32,
  changes nothing), and
* repeated calls give identical bits.

Parity of the results themselves is covered by the per-op test modules; W8A8 is also checked
bit-exactly here against the int64 matmul of its integer stage."""
import numpy as np
import pytest
import torch

from kernelbench_harbor_amd import _lib, inputs, ops

pytestmark = pytest.mark.gpu


def _twice_with_garbage(fn, args, dev):
    y1 = fn(*args)
    ops.workspaces.get(0, dev).fill_(255)
    y2 = fn(*args)
    torch.cuda.synchronize()
    return y1, y2


@pytest.mark.parametrize("M", [1, 16, 32])
def test_w8a8_split_k(dev, M):
    K, N = 14336, 4096
    assert _lib.load().kbh_w8a8_workspace_bytes(M, N, K) > 0
    print(f"[split-k w8a8] M={M}", flush=True)
    args = [t.to(dev) for t in inputs.w8a8(M, K, N, seed=M)]
    a1, a2 = _twice_with_garbage(ops.w8a8_gemm_i32, args[:2], dev)
    assert torch.equal(a1, a2)
    exact = args[0].cpu().numpy().astype(np.int64) @ args[1].cpu().numpy().astype(np.int64)
    assert np.array_equal(a1.cpu().numpy().astype(np.int64), exact)
    y1, y2 = _twice_with_garbage(ops.w8a8_gemm, args, dev)
    assert torch.equal(y1, y2)


@pytest.mark.parametrize("M", [1, 16])
def test_fp8w_split_k(dev, M):
    K, N = 14336, 4096
    assert _lib.load().kbh_fp8w_workspace_bytes(M, N, K, 128) > 0
    print(f"[split-k fp8w] M={M}", flush=True)
    args = [t.to(dev) for t in inputs.fp8w(M, K, N, 128, seed=M)]
    y1, y2 = _twice_with_garbage(ops.fp8w_gemm, args, dev)
    assert torch.equal(y1, y2)
    assert torch.isfinite(y1.float()).all()


def test_mxfp8_split_k(dev):
    M, K, N = 128, 14336, 4096
    assert _lib.load().kbh_mxfp8_workspace_bytes(M, N, K) > 0
    print(f"[split-k mxfp8] M={M}", flush=True)
    args = [t.to(dev) for t in inputs.mxfp8(M, K, N, seed=1)]
    y1, y2 = _twice_with_garbage(ops.mxfp8_gemm, args, dev)
    assert torch.equal(y1, y2)
    assert torch.isfinite(y1.float()).all()
