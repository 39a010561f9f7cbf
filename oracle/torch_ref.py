"""The reference modules' forward op sequences as torch code — TEST AND MEASUREMENT
INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg times them on the host; the grader-protocol GPU
test computes its ground truth with them on the device, as the reference grader does; nothing in
the product imports this module).

Each function repeats the torch op sequence of one reference ``Model.forward`` (cited per
function) on tensors of any device, in the dtype of its inputs: called on the task's fp16/bf16 inputs it
is the reference's native path, called on fp32-upcast floating inputs (integer tensors left
alone, common/kb_verifier.py:195-196) it is the grader's fp32 ground truth. The two
Benchmark-only configurations without a reference module (MXFP8, the SiLU FFN) are written in
the same style from the math their sources define.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def upcast(ts):
    """kb_verifier.py:195-196: floating tensors to fp32, integer tensors untouched."""
    return [t.float() if t.is_floating_point() else t for t in ts]


def w4a16(x, qweight, scales, zeros):
    """tasks/quant_w4a16_pa/<task>/environment/reference.py:10-17 (GROUP = K / scales rows)."""
    K = qweight.shape[0]
    N = qweight.shape[1] * 8
    G = K // scales.shape[0]
    shifts = torch.arange(0, 32, 4, device=x.device, dtype=torch.int32)
    w = ((qweight.unsqueeze(-1) >> shifts) & 0xF).reshape(K, N).to(x.dtype)
    g = K // G
    se = scales.reshape(g, 1, N).expand(g, G, N).reshape(K, N).to(x.dtype)
    ze = zeros.reshape(g, 1, N).expand(g, G, N).reshape(K, N).to(x.dtype)
    return torch.matmul(x, (w - ze) * se)


def w8a8(x_int8, w_int8, x_scale, w_scale):
    """tasks/w8a8_smoothquant/<task>/environment/reference.py:7-9."""
    acc = torch.matmul(x_int8.float(), w_int8.float())
    return (acc * x_scale.float() * w_scale.float()).to(torch.float16)


def fp8w(x, w_fp8, scales):
    """tasks/fp8_microscale/<task>/environment/reference.py:9-12 (BLOCK = K / scales rows)."""
    K, N = w_fp8.shape
    B = K // scales.shape[0]
    w = w_fp8.float().reshape(K // B, B, N) * scales[:, None, :].float()
    return torch.matmul(x, w.reshape(K, N).to(x.dtype))


def mxfp8(a, a_scale, b, b_scale, out_dtype=torch.float16):
    """MXFP8 GEMM (no reference module): e4m3 codes decoded as generate_tasks.py:342 decodes its
    float8_e4m3fn tensor, times the e8m0 block scale 2^(e - 127) per 1x32 block along K, then an
    fp32 matmul of the dequantised operands, rounded to the output dtype."""
    def deq(codes, e):
        R, K = codes.shape
        v = codes.view(torch.float8_e4m3fn).float().reshape(R, K // 32, 32)
        return (v * torch.exp2(e.float() - 127.0)[:, :, None]).reshape(R, K)
    return torch.matmul(deq(a, a_scale), deq(b, b_scale).t()).to(out_dtype)


def _route(router_logits, dtype, k=2):
    """tasks/fused_qmoe/<task>/environment/reference.py:14-16."""
    probs = torch.softmax(router_logits.float(), dim=-1)
    topv, topi = probs.topk(k, dim=-1)
    return (topv / topv.sum(dim=-1, keepdim=True)).to(dtype), topi


def qmoe(x, qweight, scales, router_logits):
    """tasks/fused_qmoe/fused_qmoe__mixtral__fp16/environment/reference.py:11-21 (dense over
    all experts, then the top-2 gather, as the reference computes it)."""
    T, D = x.shape
    E, _, N = qweight.shape
    topv, topi = _route(router_logits, x.dtype)
    G = D // scales.shape[1]
    g = D // G
    w = (qweight.reshape(E, g, G, N).to(x.dtype) * scales[:, :, None, :].to(x.dtype)).reshape(E, D, N)
    all_out = torch.einsum("td,edn->ten", x, w)
    sel = torch.gather(all_out, 1, topi.unsqueeze(-1).expand(-1, -1, N))
    return (sel * topv.unsqueeze(-1)).sum(dim=1)


def _w4_experts(q, s, z, dtype):
    """Per-expert W4A16 dequantisation, reference.py:12-16 of the W4A16 task with an expert
    dimension in front."""
    E, K, NP = q.shape
    N = NP * 8
    G = K // s.shape[1]
    shifts = torch.arange(0, 32, 4, dtype=torch.int32)
    w = ((q.unsqueeze(-1) >> shifts) & 0xF).reshape(E, K, N).to(dtype)
    se = s.repeat_interleave(G, dim=1).to(dtype)
    ze = z.repeat_interleave(G, dim=1).to(dtype)
    return (w - ze) * se


def qmoe_ffn(x, router_logits, gq, gs, gz, uq, us, uz, dq, ds, dz):
    """Top-2 SiLU FFN with W4A16 experts (no reference module), written in the reference qMoE's
    dense style (every expert, then the top-2 gather, reference.py:17-21 of fused_qmoe):
    gate/up = x @ W in x.dtype, h = (F.silu(gate.float()) * up.float()).to(x.dtype)
    (generate_tasks.py:337, validate/measure_pass1.py:432-437), o = h @ Wd per expert."""
    T, D = x.shape
    topv, topi = _route(router_logits, x.dtype)
    Wg = _w4_experts(gq, gs, gz, x.dtype)
    Wu = _w4_experts(uq, us, uz, x.dtype)
    gate = torch.einsum("td,edf->tef", x, Wg)
    up = torch.einsum("td,edf->tef", x, Wu)
    del Wg, Wu
    h = (F.silu(gate.float()) * up.float()).to(x.dtype)
    del gate, up
    Wd = _w4_experts(dq, ds, dz, x.dtype)
    all_out = torch.einsum("tef,efd->ted", h, Wd)
    sel = torch.gather(all_out, 1, topi.unsqueeze(-1).expand(-1, -1, D))
    return (sel * topv.unsqueeze(-1)).sum(dim=1)


def silu_fp8(y, group=128):
    """tasks/fused_silu_fp8/fused_silu_fp8__mixtral__T512__fp16/environment/reference.py:13-23."""
    T, H2 = y.shape
    H = H2 // 2
    gate, up = y[:, :H], y[:, H:]
    act = F.silu(gate.float()) * up.float()
    a = act.reshape(T, H // group, group)
    scale = (a.abs().amax(dim=-1, keepdim=True) / 448.0).clamp(min=1e-12)
    q = (a / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).float()
    return (q * scale).reshape(T, H)
