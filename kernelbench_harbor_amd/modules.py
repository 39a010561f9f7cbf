"""Drop-in ``nn.Module`` replacements for the reference task modules.

Each class has the reference ``Model``'s no-argument constructor and ``forward`` signature
(the grader constructs ``ModelNew()`` and calls ``forward(*get_inputs())``,
common/kb_verifier.py:185-197) and returns the reference output dtype. The compute is a call
into the HIP library; a task file only needs ``ModelNew = W4A16Model`` (etc.).
"""
from __future__ import annotations

import torch.nn as nn

from . import ops


class W4A16Model(nn.Module):
    """Packed-asymmetric W4A16 (GPTQ-style) linear.

    Reference: tasks/quant_w4a16_pa/*/environment/reference.py:10-17,
    forward(x [M,K], qweight [K,N/8] int32, scales [K/G,N], zeros [K/G,N]) -> [M,N] x.dtype.
    """

    def forward(self, x, qweight, scales, zeros):
        return ops.w4a16_gemm(x, qweight, scales, zeros)


class W8A8Model(nn.Module):
    """W8A8 SmoothQuant linear.

    Reference: tasks/w8a8_smoothquant/*/environment/reference.py:7-9,
    forward(x_int8 [M,K], w_int8 [K,N], x_scale [M,1] fp16, w_scale [1,N] fp16) -> [M,N] fp16.
    """

    def forward(self, x_int8, w_int8, x_scale, w_scale):
        return ops.w8a8_gemm(x_int8, w_int8, x_scale, w_scale)


class FP8WModel(nn.Module):
    """FP8 (e4m3) block-microscaled weight GEMM.

    Reference: tasks/fp8_microscale/*/environment/reference.py:9-12,
    forward(x [M,K], w_fp8 [K,N] float8_e4m3fn, scales [K/B,N] fp16) -> [M,N] x.dtype.
    """

    def forward(self, x, w_fp8, scales):
        return ops.fp8w_gemm(x, w_fp8, scales)


class MXFP8Model(nn.Module):
    """MXFP8 block-scaled GEMM (both operands e4m3, e8m0 1x32 scales), fp16 output.

    No reference module: written in the reference's Model idiom for the benchmark's MXFP8
    configuration. forward(a [M,K], a_scale [M,K/32], b [N,K], b_scale [N,K/32]) -> [M,N] fp16.
    """

    def forward(self, a, a_scale, b, b_scale):
        return ops.mxfp8_gemm(a, a_scale, b, b_scale)


class QMoEModel(nn.Module):
    """Quantized top-2 MoE (one projection per expert).

    Reference: tasks/fused_qmoe/*/environment/reference.py:11-21,
    forward(x [T,D], qweight [E,D,N] int8, scales [E,D/128,N], router_logits [T,E]) -> [T,N].
    """

    def forward(self, x, qweight, scales, router_logits):
        return ops.qmoe(x, qweight, scales, router_logits)


class QMoEFFNModel(nn.Module):
    """Top-2 MoE SiLU FFN with W4A16 g128 experts (the benchmark's SiLU FFN configuration).

    No reference module; written in the reference's Model idiom with its routing and combine:
    forward(x, router_logits, gate_qweight, gate_scales, gate_zeros, up_qweight, up_scales,
    up_zeros, down_qweight, down_scales, down_zeros) -> [T, D] x.dtype.
    """

    def forward(self, x, router_logits, gate_qweight, gate_scales, gate_zeros, up_qweight,
                up_scales, up_zeros, down_qweight, down_scales, down_zeros):
        return ops.qmoe_ffn(x, router_logits, gate_qweight, gate_scales, gate_zeros, up_qweight,
                            up_scales, up_zeros, down_qweight, down_scales, down_zeros)


class FusedSiluFP8Model(nn.Module):
    """Fused SiLU x up + per-group (128) dynamic FP8 quantisation, returned dequantised.

    Reference: tasks/fused_silu_fp8/*/environment/reference.py:13-23,
    forward(y [T, 2H] fp16/bf16) -> [T, H] float32.
    """

    def forward(self, y):
        return ops.silu_fp8_quant(y, 128)


class MoEModel(nn.Module):
    """Top-k mixture of experts with fp16/bf16 expert weights (sparse dispatch).

    Reference: tasks/moe/*/environment/reference.py:10-17, whose TOPK is a module constant
    (generate_tasks.py:189-195: 2, 6 or 8): forward(x [T,D], w [E,D,H], router_logits [T,E])
    -> [T, H] x.dtype. Subclasses fix TOPK for the top-6 and top-8 tasks.
    """

    TOPK = 2

    def forward(self, x, w, router_logits):
        return ops.moe(x, w, router_logits, self.TOPK)


class MoETop6Model(MoEModel):
    TOPK = 6


class MoETop8Model(MoEModel):
    TOPK = 8


class MultiLoRAQGemmModel(nn.Module):
    """Multi-LoRA quantized linear (int4 base stored int8, GROUP 128 scales, batched adapters).

    Reference: tasks/multi_lora_qgemm/*/environment/reference.py:10-17,
    forward(x [T,D], qweight [D,N] int8, scales [D/128,N], A [L,D,r], B [L,r,N], lora_ids [T])
    -> [T, N] x.dtype.
    """

    def forward(self, x, qweight, scales, A, B, lora_ids):
        return ops.lora_qgemm(x, qweight, scales, A, B, lora_ids)
