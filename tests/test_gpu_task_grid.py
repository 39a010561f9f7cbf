"""Every task of the reference's four quantized-GEMM families at its real shape, through the
drop-in modules exactly as the grader calls them (``ModelNew()(*get_inputs())``).

The grid is the reference generator's: W4A16 over its layer list x {g64, g128} in fp16 plus g128
in bf16 (generate_tasks.py:481-490, 535-544; M=16), W8A8 over its linear shapes x M in
{16, 64, 256} (generate_tasks.py:268-275, 561-569), FP8 weight-only over the same shapes x
{b32, b128} in fp16 plus b32 in bf16 (generate_tasks.py:572-580; M=16) and the fused qMoE over
its three configurations in fp16 and bf16 (generate_tasks.py:390-394, 617-626; T=256).

The GEMMs are checked against the oracle on the first and last 256 output columns (the oracle's
dense fp32 dequantisation of a 70B-model layer would dominate the suite's time; both slices
cross every K split and group); W8A8 bit-exactly, the others to the benchmark's tolerances and to
the reference grader's own allclose(atol = rtol = 2e-2) on every task, bf16 included (the
reference's own bf16 intermediates fail that allclose on the bf16 W4A16 and qMoE tasks; these
kernels scale after the MFMA and combine in fp32, so they stay inside it). The qMoE output is
checked whole.
"""
import functools

import numpy as np
import pytest
import torch

from kernelbench_harbor_amd import FP8WModel, QMoEModel, W4A16Model, W8A8Model, inputs
from kernelbench_harbor_amd.harness import compare
from oracle import fp8w as of
from oracle import qmoe as oq
from oracle import w4a16 as ow
from oracle import w8a8 as o8

pytestmark = pytest.mark.gpu

LAYERS = [  # (name, K, N), generate_tasks.py:481-490
    ("llama3_8b_gate", 4096, 14336),
    ("llama3_8b_down", 14336, 4096),
    ("llama3_70b_gate", 8192, 28672),
    ("llama3_70b_down", 28672, 8192),
    ("qwen2_7b_gate", 3584, 18944),
    ("qwen2_7b_down", 18944, 3584),
    ("qwen2_72b_gate", 8192, 29568),
    ("qwen2_72b_down", 29568, 8192),
]
LINEAR_SHAPES = [  # (name, K, N), generate_tasks.py:268-275
    ("llama3_8b_qkv", 4096, 6144),
    ("llama3_8b_o", 4096, 4096),
    ("llama3_8b_gate", 4096, 14336),
    ("llama3_8b_down", 14336, 4096),
    ("qwen2_7b_gate", 3584, 18944),
    ("qwen2_72b_down", 29568, 8192),
]
FUSED_QMOE_CFG = [  # (name, D, E, N), generate_tasks.py:390-394
    ("deepseek_moe", 2048, 64, 1408),
    ("mixtral", 4096, 8, 14336),
    ("qwen_moe", 2048, 60, 1408),
]
SL = 256  # columns per checked slice


def _slices(N):
    return [slice(0, SL), slice(N - SL, N)]


def _f(t):
    return t.float().numpy()


def _dt(dtype):
    return "f16" if dtype == torch.float16 else "bf16"


@functools.lru_cache(maxsize=2)
def _w4_inputs(K, N, group, dtype):
    return inputs.w4a16(16, K, N, group, dtype, seed=K + N + group)


W4_GRID = [(n, K, N, g, torch.float16) for (n, K, N) in LAYERS for g in (64, 128)]
W4_GRID += [(n, K, N, 128, torch.bfloat16) for (n, K, N) in LAYERS]


@pytest.mark.parametrize("name,K,N,group,dtype", W4_GRID)
def test_w4a16_task(dev, name, K, N, group, dtype):
    print(f"[grid w4a16] {name} K={K} N={N} g{group} {dtype}", flush=True)
    x, qw, s, z = _w4_inputs(K, N, group, dtype)
    y = W4A16Model()(x.to(dev), qw.to(dev), s.to(dev), z.to(dev)).cpu()
    assert y.shape == (16, N) and y.dtype == dtype
    for c in _slices(N):
        args = (_f(x), qw[:, c.start // 8:c.stop // 8].numpy(), _f(s[:, c]), _f(z[:, c]))
        gt = ow.forward(*args)
        cmp = compare(y[:, c], gt)
        assert cmp.ok, (c, cmp)
        assert cmp.task_ok("quant_w4a16_pa"), (c, cmp)


W8_GRID = [(n, K, N, M) for (n, K, N) in LINEAR_SHAPES for M in (16, 64, 256)]


@pytest.mark.parametrize("name,K,N,M", W8_GRID)
def test_w8a8_task(dev, name, K, N, M):
    print(f"[grid w8a8] {name} K={K} N={N} M={M}", flush=True)
    xi, wi, xs, ws = inputs.w8a8(M, K, N, seed=K + N + M, dist="reference")
    y = W8A8Model()(xi.to(dev), wi.to(dev), xs.to(dev), ws.to(dev)).cpu()
    assert y.shape == (M, N) and y.dtype == torch.float16
    for c in _slices(N):
        want = o8.forward(xi.numpy(), wi[:, c].numpy(), xs.float().numpy(), ws[:, c].float().numpy())
        assert np.array_equal(y[:, c].float().numpy(), want), c


FP8_GRID = [(n, K, N, b, torch.float16) for (n, K, N) in LINEAR_SHAPES for b in (32, 128)]
FP8_GRID += [(n, K, N, 32, torch.bfloat16) for (n, K, N) in LINEAR_SHAPES]


@pytest.mark.parametrize("name,K,N,block,dtype", FP8_GRID)
def test_fp8w_task(dev, name, K, N, block, dtype):
    print(f"[grid fp8w] {name} K={K} N={N} b{block} {dtype}", flush=True)
    x, w, s = inputs.fp8w(16, K, N, block, dtype, seed=K + N + block)
    y = FP8WModel()(x.to(dev), w.to(dev), s.to(dev)).cpu()
    assert y.shape == (16, N) and y.dtype == dtype
    for c in _slices(N):
        args = (_f(x), w[:, c].contiguous().view(torch.uint8).numpy(), _f(s[:, c]))
        gt = of.forward(*args)
        cmp = compare(y[:, c], gt)
        assert cmp.ok, (c, cmp)
        assert cmp.task_ok("fp8_microscale"), (c, cmp)


QMOE_GRID = [(n, D, E, N, dt) for (n, D, E, N) in FUSED_QMOE_CFG
             for dt in (torch.float16, torch.bfloat16)]


@pytest.mark.parametrize("name,D,E,N,dtype", QMOE_GRID)
def test_qmoe_task(dev, name, D, E, N, dtype):
    print(f"[grid qmoe] {name} D={D} E={E} N={N} {dtype}", flush=True)
    ins = inputs.qmoe(256, D, E, N, dtype, seed=D + E + N)
    y = QMoEModel()(*[t.to(dev) for t in ins]).cpu()
    assert y.shape == (256, N) and y.dtype == dtype
    x, q, s, lg = ins
    args = (_f(x), q.numpy(), _f(s), _f(lg))
    gt = oq.qmoe_forward(*args)
    cmp = compare(y, gt)
    assert cmp.ok, cmp
    assert cmp.task_ok("fused_qmoe"), cmp
