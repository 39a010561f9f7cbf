"""Seeded synthetic inputs for the quantized-GEMM ops (CPU tensors; move them to the GPU).

Two distributions per op:
  "reference": the reference task's own get_inputs() distributions (e.g.
               tasks/quant_w4a16_pa/*/environment/reference.py:19-29), seeded;
  "baseline":  the benchmark configurations (scales U[0.002, 0.02], SmoothQuant synthesis,
               MX block quantization, ...).
Every generator draws from one torch.Generator seeded with `seed`, on the CPU, so the CPU
oracle and the GPU kernels see identical tensors.
"""
from __future__ import annotations

import torch


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(int(seed))


def random_packed_int4(K: int, N: int, g: torch.Generator) -> torch.Tensor:
    """qweight [K, N/8] int32 whose 8 nibbles per word are i.i.d. uniform on 0..15.

    Packing i.i.d. uniform nibbles (reference.py:21-25) yields a word that is uniform over all
    2^32 bit patterns, so the words are drawn directly."""
    return torch.randint(-2 ** 31, 2 ** 31, (K, N // 8), generator=g, dtype=torch.int64).to(torch.int32)


def w4a16(M: int, K: int = 14336, N: int = 4096, group: int = 128,
          dtype: torch.dtype = torch.float16, seed: int = 0, dist: str = "baseline"):
    """[x, qweight, scales, zeros] in the layout of reference.py:10 (`forward(x, qweight,
    scales, zeros)`)."""
    g = _gen(seed)
    x = torch.randn(M, K, generator=g).to(dtype)
    qweight = random_packed_int4(K, N, g)
    if dist == "baseline":
        scales = (torch.rand(K // group, N, generator=g) * 0.018 + 0.002).to(dtype)
    elif dist == "reference":
        scales = (torch.randn(K // group, N, generator=g) * 0.01).to(dtype)
    else:
        raise ValueError(dist)
    zeros = torch.randint(0, 16, (K // group, N), generator=g).to(dtype)
    return [x, qweight, scales, zeros]
