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


def w8a8(M: int, K: int = 14336, N: int = 4096, seed: int = 0, dist: str = "baseline"):
    """[x_int8, w_int8, x_scale, w_scale] in the layout of reference.py:7 (W8A8 task).

    "reference": uniform int8 in [-127, 127] and scales U[0.001, 0.011] (reference.py:11-17).
    "baseline":  SmoothQuant synthesis — x ~ N(0,1) fp16 with a fixed 1% of input channels
                 scaled x20, W ~ N(0,1)*0.02 fp16; smoothing s_k = max|x_k|^0.5 / max|W_k|^0.5,
                 x' = x/s, W' = W*s; symmetric absmax int8 per token (x) and per output
                 channel (W) with fp16 scales."""
    g = _gen(seed)
    if dist == "reference":
        x_int8 = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
        w_int8 = torch.randint(-127, 128, (K, N), generator=g, dtype=torch.int8)
        x_scale = (torch.rand(M, 1, generator=g) * 0.01 + 0.001).to(torch.float16)
        w_scale = (torch.rand(1, N, generator=g) * 0.01 + 0.001).to(torch.float16)
        return [x_int8, w_int8, x_scale, w_scale]
    if dist != "baseline":
        raise ValueError(dist)
    x = torch.randn(M, K, generator=g).to(torch.float16).float()
    outliers = torch.randperm(K, generator=torch.Generator().manual_seed(1234))[: max(1, K // 100)]
    x[:, outliers] *= 20.0
    W = (torch.randn(K, N, generator=g) * 0.02).to(torch.float16).float()
    s = (x.abs().amax(dim=0).clamp(min=1e-5) ** 0.5) / (W.abs().amax(dim=1).clamp(min=1e-5) ** 0.5)
    xs_ = x / s
    Ws_ = W * s[:, None]
    x_scale = (xs_.abs().amax(dim=1, keepdim=True) / 127.0).to(torch.float16)
    w_scale = (Ws_.abs().amax(dim=0, keepdim=True) / 127.0).to(torch.float16)
    x_int8 = torch.round(xs_ / x_scale.float()).clamp(-127, 127).to(torch.int8)
    w_int8 = torch.round(Ws_ / w_scale.float()).clamp(-127, 127).to(torch.int8)
    return [x_int8, w_int8, x_scale, w_scale]


def fp8w(M: int, K: int = 14336, N: int = 4096, block: int = 128,
         dtype: torch.dtype = torch.float16, seed: int = 0):
    """[x, w_fp8, scales] with the distributions of reference.py:14-19 (FP8 task): x ~ N(0,1),
    w = (N(0,1) * 0.3) cast to float8_e4m3fn, scales U[0.05, 0.10] fp16 [K/block, N]."""
    g = _gen(seed)
    x = torch.randn(M, K, generator=g).to(dtype)
    w_fp8 = (torch.randn(K, N, generator=g) * 0.3).to(torch.float8_e4m3fn)
    scales = (torch.rand(K // block, N, generator=g) * 0.05 + 0.05).to(torch.float16)
    return [x, w_fp8, scales]


def mx_quantize(src: torch.Tensor):
    """OCP MX block quantisation of float32 rows along the last dim in 1x32 blocks: scale =
    2^ceil(log2(amax/448)) (e8m0 code = exponent + 127; amax = 0 gives code 0 and zero
    elements), elements = e4m3fn(x / scale) rounded to nearest even. Returns (codes uint8,
    scales uint8)."""
    R, K = src.shape
    blk = src.float().reshape(R, K // 32, 32)
    amax = blk.abs().amax(dim=-1)
    mant, expo = torch.frexp(amax / 448.0)
    ceil_log2 = expo - (mant == 0.5).to(expo.dtype)      # exact ceil(log2(v)) for v > 0
    code = (ceil_log2 + 127).clamp(0, 254)
    code = torch.where(amax > 0, code, torch.zeros_like(code))
    scale = torch.ldexp(torch.ones_like(amax), code - 127)
    q = (blk / scale[..., None]).to(torch.float8_e4m3fn)
    return q.reshape(R, K).view(torch.uint8), code.to(torch.uint8)


def mxfp8(M: int, K: int = 14336, N: int = 4096, seed: int = 0):
    """[a, a_scale, b, b_scale] for the benchmark's MXFP8 configuration: fp32 sources ~ N(0,1), [M, K] and
    [N, K], MX-quantised along K."""
    g = _gen(seed)
    a_src = torch.randn(M, K, generator=g)
    b_src = torch.randn(N, K, generator=g)
    a, a_s = mx_quantize(a_src)
    b, b_s = mx_quantize(b_src)
    return [a, a_s, b, b_s]


def _distinct_logits(T: int, E: int, g: torch.Generator, dtype: torch.dtype) -> torch.Tensor:
    """N(0,1) router logits in `dtype` whose top-2 per row has no ties (re-drawn otherwise)."""
    while True:
        lg = torch.randn(T, E, generator=g).to(dtype)
        top = lg.float().topk(3, dim=-1).values
        if bool((top[:, 0] > top[:, 1]).all() and (top[:, 1] > top[:, 2]).all()):
            return lg


def qmoe(T: int = 256, D: int = 4096, E: int = 8, N: int = 14336,
         dtype: torch.dtype = torch.float16, seed: int = 0, group: int = 128):
    """[x, qweight, scales, router_logits] with the distributions of the reference qMoE task
    (reference.py:23-29): qweight int8 in [-8, 7], scales N(0,1)*0.01 [E, D/group, N] (the
    reference's GROUP is 128), logits N(0,1) in x.dtype, drawn as the reference draws them
    (ties included: the routing follows torch.topk's GPU order on ties)."""
    g = _gen(seed)
    x = torch.randn(T, D, generator=g).to(dtype)
    qweight = torch.randint(-8, 8, (E, D, N), generator=g, dtype=torch.int8)
    scales = (torch.randn(E, D // group, N, generator=g) * 0.01).to(dtype)
    logits = torch.randn(T, E, generator=g).to(dtype)
    return [x, qweight, scales, logits]


def qmoe_ffn(T: int = 512, D: int = 4096, F: int = 14336, E: int = 8, group: int = 128,
             dtype: torch.dtype = torch.float16, seed: int = 0):
    """[x, router_logits, gate_q, gate_s, gate_z, up_q, up_s, up_z, down_q, down_s, down_z] for
    the benchmark's SiLU FFN configuration: fp32 logits N(0,1) without top-2 ties, x N(0,1), W4A16 experts
    with scales U[0.002, 0.02] and zero points U{0..15}."""
    g = _gen(seed)
    x = torch.randn(T, D, generator=g).to(dtype)
    logits = _distinct_logits(T, E, g, torch.float32)

    def w4(K, Nc):
        q = torch.stack([random_packed_int4(K, Nc, g) for _ in range(E)])
        s = (torch.rand(E, K // group, Nc, generator=g) * 0.018 + 0.002).to(dtype)
        z = torch.randint(0, 16, (E, K // group, Nc), generator=g).to(dtype)
        return [q, s, z]
    return [x, logits] + w4(D, F) + w4(D, F) + w4(F, D)


def silu_fp8(T: int = 512, H: int = 14336, dtype: torch.dtype = torch.float16, seed: int = 0):
    """[y]: y [T, 2H] ~ N(0, 1) in dtype, as tasks/fused_silu_fp8/*/environment/reference.py:25-28."""
    g = _gen(seed)
    return [torch.randn(T, 2 * H, generator=g).to(dtype)]


def moe(T: int = 16, D: int = 4096, E: int = 8, H: int = 14336, topk: int = 2,
        dtype: torch.dtype = torch.float16, seed: int = 0):
    """[x, w, router_logits] with the distributions of the reference moe task
    (tasks/moe/*/environment/reference.py:19-24): x N(0,1), w N(0,1)*0.02, logits N(0,1), all in
    dtype, drawn as the reference draws them (ties included). `topk` does not change the draw."""
    g = _gen(seed)
    x = torch.randn(T, D, generator=g).to(dtype)
    w = (torch.randn(E, D, H, generator=g) * 0.02).to(dtype)
    logits = torch.randn(T, E, generator=g).to(dtype)
    return [x, w, logits]


def lora_qgemm(T: int = 64, D: int = 4096, N: int = 4096, r: int = 16, L: int = 8,
               dtype: torch.dtype = torch.float16, seed: int = 0):
    """[x, qweight, scales, A, B, lora_ids] with the distributions of the reference task
    (tasks/multi_lora_qgemm/*/environment/reference.py:19-27)."""
    g = _gen(seed)
    x = torch.randn(T, D, generator=g).to(dtype)
    qweight = torch.randint(-8, 8, (D, N), generator=g, dtype=torch.int8)
    scales = (torch.randn(D // 128, N, generator=g) * 0.01).to(dtype)
    A = (torch.randn(L, D, r, generator=g) * 0.02).to(dtype)
    B = (torch.randn(L, r, N, generator=g) * 0.02).to(dtype)
    lora_ids = torch.randint(0, L, (T,), generator=g)
    return [x, qweight, scales, A, B, lora_ids]
