"""GPU parity of the W4A16 HIP path against the CPU oracle (oracle/w4a16.py)."""
import numpy as np
import pytest
import torch

from kernelbench_harbor_amd import W4A16Model, _lib, inputs, ops
from kernelbench_harbor_amd.harness import compare
from oracle import w4a16 as ow

pytestmark = pytest.mark.gpu


def _np(t):
    return t.float().numpy()


def _gt(x, qw, s, z):
    return ow.forward(_np(x), qw.numpy(), _np(s), _np(z))


CASES = [
    # M, K, N, group, dtype, dist
    (1, 1024, 256, 128, torch.float16, "baseline"),
    (3, 2048, 384, 128, torch.float16, "baseline"),
    (16, 4096, 512, 128, torch.float16, "baseline"),
    (17, 1024, 256, 64, torch.float16, "reference"),
    (33, 1024, 128, 128, torch.float16, "baseline"),
    (64, 2048, 1024, 128, torch.float16, "baseline"),
    (100, 512, 256, 32, torch.float16, "baseline"),
    (16, 2048, 512, 256, torch.float16, "baseline"),
    (16, 2048, 512, 128, torch.bfloat16, "baseline"),
    (5, 1024, 384, 64, torch.bfloat16, "reference"),
    (40, 1024, 256, 128, torch.bfloat16, "baseline"),
    # tiled (large-M) path
    (128, 1024, 128, 32, torch.float16, "baseline"),
    (256, 2048, 512, 128, torch.float16, "baseline"),
    (300, 1024, 384, 64, torch.bfloat16, "reference"),
    (513, 4096, 256, 128, torch.float16, "reference"),
    # K not a multiple of 64 -> split-K path even for large M
    (96, 1056, 256, 32, torch.float16, "baseline"),
    # wide-tile kernel: 128x128 tiles (33 <= M <= 128, N % 256 != 0), 128x256 tiles
    # (64 < M <= 256), 256x256 tiles (M > 256), every group size, split-K and not, ragged M
    (33, 2048, 256, 64, torch.float16, "baseline"),
    (128, 4096, 384, 256, torch.bfloat16, "reference"),
    (129, 2048, 512, 32, torch.float16, "reference"),
    (200, 1024, 768, 128, torch.bfloat16, "baseline"),
    (384, 4096, 512, 64, torch.float16, "baseline"),
    (257, 8192, 256, 128, torch.float16, "baseline"),
    # 64 x 256 tiles (M <= 64, N % 256 == 0; two producer sets): every group size, split-K and not
    (48, 2048, 512, 32, torch.float16, "baseline"),
    (64, 1024, 768, 256, torch.bfloat16, "reference"),
    (56, 2048, 512, 128, torch.float16, "baseline"),
    (40, 4096, 256, 128, torch.bfloat16, "reference"),
    # N % 256 != 0 above 128 rows: the 256 x 128 LDS-staged kernel
    (160, 2048, 384, 128, torch.float16, "baseline"),
    # warp-specialised 128-row tiles (64 < M <= 256, N % 256 == 0) and 256-row tiles above, with
    # 256- and 32-row groups
    # (the producers' group schedules SPG = 8 and SPG = 1), fp16 and bf16, ragged M
    (160, 4096, 512, 256, torch.float16, "reference"),
    (72, 2048, 512, 32, torch.bfloat16, "baseline"),
    (350, 2048, 256, 256, torch.bfloat16, "reference"),
    (480, 4096, 512, 128, torch.float16, "baseline"),
    (600, 2048, 512, 32, torch.bfloat16, "baseline"),
    (777, 2048, 256, 256, torch.float16, "reference"),
]


@pytest.mark.parametrize("M,K,N,group,dtype,dist", CASES)
def test_w4a16_parity(dev, M, K, N, group, dtype, dist):
    print(f"[w4a16 parity] M={M} K={K} N={N} g={group} {dtype} {dist}", flush=True)
    x, qw, s, z = inputs.w4a16(M, K, N, group, dtype, seed=M + N, dist=dist)
    y = ops.w4a16_gemm(x.to(dev), qw.to(dev), s.to(dev), z.to(dev))
    assert y.dtype == dtype and y.shape == (M, N)
    cmp = compare(y, _gt(x, qw, s, z))
    assert cmp.ok, cmp


@pytest.mark.parametrize("M", [1, 4, 16])
def test_w4a16_full_size_decode(dev, M):
    """The benchmark's W4A16 shape: K=14336, N=4096, g128, fp16."""
    print(f"[w4a16 full] M={M}", flush=True)
    x, qw, s, z = inputs.w4a16(M, 14336, 4096, 128, torch.float16, seed=M)
    y = W4A16Model()(x.to(dev), qw.to(dev), s.to(dev), z.to(dev))
    cmp = compare(y, _gt(x, qw, s, z))
    assert cmp.ok, cmp


@pytest.mark.parametrize("M,N,zeros", [(16, 512, "uint4"), (64, 512, "uint4"), (64, 512, "frac"),
                                       (64, 512, "partial"),
                                       (200, 512, "uint4"), (200, 512, "frac"),
                                       (200, 512, "partial"), (200, 512, "wide"),
                                       (200, 512, "bound"), (160, 384, "uint4")])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_w4a16_dequant_bit_exact(dev, dtype, M, N, zeros):
    """One-hot activations select single weight rows, so y[m, :] is the dequantized row
    k_m rounded once to the output dtype: it must equal the reference's own dequantization
    (unpack, subtract zero with one rounding, multiply by scale with one rounding) bit for bit.
    M=16 exercises the split-K decode kernel, M=64 and M=200 the wide-tile kernel (64- and
    128-row tiles), N=384 at M=160 the 256 x 128 LDS-staged kernel. Zero points with a
    fractional part make the subtraction round, which the wide kernel reproduces exactly.
    The 64- and 128-row fp16 tiles take a shorter dequantisation when every zero point of a
    workgroup's K range and columns is an integer below 960 in magnitude: "uint4" and "wide"
    (integers in [-900, 900]) take it everywhere, "frac" and "bound" (+-960) nowhere, and
    "partial" (fractional zeros in 4 groups x 100 columns) in some workgroups only."""
    K, G = 4096, 128
    g = torch.Generator().manual_seed(7 + M)
    qw = inputs.random_packed_int4(K, N, g)
    ks = torch.randperm(K, generator=g)[:M]
    x = torch.zeros(M, K, dtype=dtype)
    x[torch.arange(M), ks] = 1.0
    s = (torch.randn(K // G, N, generator=g) * 0.01).to(dtype)
    z = torch.randint(0, 16, (K // G, N), generator=g).to(torch.float32)
    if zeros == "frac":
        z = z + torch.rand(K // G, N, generator=g) * 0.999
    elif zeros == "partial":
        z[8:12, 300:400] += torch.rand(4, 100, generator=g) * 0.999
    elif zeros == "wide":
        z = torch.randint(-900, 901, (K // G, N), generator=g).to(torch.float32)
    elif zeros == "bound":
        z = torch.where(torch.rand(K // G, N, generator=g) < 0.5, 960.0, -960.0)
    z = z.to(dtype)
    y = ops.w4a16_gemm(x.to(dev), qw.to(dev), s.to(dev), z.to(dev)).float().cpu().numpy()
    dt = "f16" if dtype == torch.float16 else "bf16"
    W = ow.dequant(qw.numpy(), s.float().numpy(), z.float().numpy(), dt)
    want = W[ks.numpy()]
    assert np.array_equal(y, want), np.abs(y - want).max()


@pytest.mark.parametrize("M", [64, 256, 1024])
def test_w4a16_full_size_sweep_points(dev, M):
    """The remaining points of the benchmark's W4A16 sweep at K=14336, N=4096, g128 (64-row tiles with
    many K splits, 256-row tiles, split-K 256-row tiles), checked against the oracle on the first
    and last 256 output columns (every K split and group crosses both)."""
    print(f"[w4a16 full] M={M}", flush=True)
    x, qw, s, z = inputs.w4a16(M, 14336, 4096, 128, torch.float16, seed=M)
    y = W4A16Model()(x.to(dev), qw.to(dev), s.to(dev), z.to(dev)).cpu()
    for c in (slice(0, 256), slice(4096 - 256, 4096)):
        gt = ow.forward(_np(x), qw[:, c.start // 8:c.stop // 8].numpy(), _np(s[:, c]), _np(z[:, c]))
        cmp = compare(y[:, c], gt)
        assert cmp.ok, (c, cmp)


def test_w4a16_full_size_prefill(dev):
    """The largest point of the benchmark's W4A16 sweep: M=2048, K=14336, N=4096."""
    print("[w4a16 full] M=2048", flush=True)
    x, qw, s, z = inputs.w4a16(2048, 14336, 4096, 128, torch.float16, seed=5)
    y = W4A16Model()(x.to(dev), qw.to(dev), s.to(dev), z.to(dev))
    cmp = compare(y, _gt(x, qw, s, z))
    assert cmp.ok, cmp


def test_w4a16_split_k_deterministic_with_garbage_workspace(dev):
    """The split-K decode sums its partial slices in a fixed order and reads nothing it did not
    write: a workspace full of 0xFF bytes (NaN patterns) gives the same bits as before."""
    M, K, N = 16, 14336, 4096
    assert _lib.load().kbh_w4a16_workspace_bytes(M, N, K, 128) > 0   # the split-K path
    x, qw, s, z = [t.to(dev) for t in inputs.w4a16(M, K, N, seed=3)]
    y1 = ops.w4a16_gemm(x, qw, s, z)
    ops.workspaces.get(0, x.device).fill_(255)
    y2 = ops.w4a16_gemm(x, qw, s, z)
    assert torch.equal(y1, y2)
    assert compare(y1, _gt(x.cpu(), qw.cpu(), s.cpu(), z.cpu())).ok


def test_w4a16_batched_leading_dims(dev):
    x, qw, s, z = inputs.w4a16(6, 1024, 256, seed=11)
    y = ops.w4a16_gemm(x.reshape(2, 3, 1024).to(dev), qw.to(dev), s.to(dev), z.to(dev))
    assert y.shape == (2, 3, 256)
    assert compare(y.reshape(6, 256), _gt(x, qw, s, z)).ok
