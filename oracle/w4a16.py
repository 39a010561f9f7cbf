"""Oracle for the packed-asymmetric W4A16 group-quantized GEMM (test infrastructure only).

Reference: tasks/quant_w4a16_pa/quant_w4a16_pa__llama3_8b_down__g128__fp16/environment/
reference.py (template generate_tasks.py:45-74); ground-truth construction common/kb_verifier.py
:195-196 (floating inputs upcast to fp32, integer inputs untouched).
"""
from __future__ import annotations

import numpy as np

from .numerics import F32, round_to


def pack_int4_along_n(nib: np.ndarray) -> np.ndarray:
    """nib [K, N] values 0..15 -> qweight [K, N/8] int32 with nibble i of word j = column 8j+i.

    reference.py:21-25 (`packed |= nib[:, i::8] << 4*i`, then `.to(torch.int32)`, which keeps
    the low 32 bits two's-complement)."""
    nib = np.asarray(nib, dtype=np.int64)
    K, N = nib.shape
    assert N % 8 == 0
    packed = np.zeros((K, N // 8), dtype=np.int64)
    for i in range(8):
        packed |= nib[:, i::8] << (4 * i)
    return packed.astype(np.uint32).view(np.int32)


def unpack_int4_along_n(qweight: np.ndarray) -> np.ndarray:
    """qweight [K, N/8] int32 -> [K, N] uint8 nibbles.

    reference.py:12-13: `(qweight.unsqueeze(-1) >> arange(0,32,4)) & 0xF` on int32 (arithmetic
    shift; the mask removes the sign fill), reshaped so word j nibble i -> column 8j+i."""
    q = np.asarray(qweight, dtype=np.int32)
    K, NP = q.shape
    shifts = np.arange(0, 32, 4, dtype=np.int32)
    w = (q[:, :, None] >> shifts[None, None, :]) & 0xF
    return w.reshape(K, NP * 8).astype(np.uint8)


def dequant(qweight, scales, zeros, dtype: str) -> np.ndarray:
    """W = (unpack(qweight) - zeros[k//G]) * scales[k//G] in `dtype` (float32 values).

    reference.py:14-17: the nibbles are cast to x.dtype, scales/zeros are expanded per group of
    G = K / scales.shape[0] rows, `(w - ze)` rounds to x.dtype (exact when the zero points are
    integers, as the reference generates them) and `* se` rounds once more to x.dtype. dtype
    'f32' is the ground-truth mode (all floating inputs upcast; both steps exact in fp32 for
    fp16/bf16 inputs)."""
    w = unpack_int4_along_n(qweight).astype(np.float32)
    s = np.asarray(scales, dtype=np.float32)
    z = np.asarray(zeros, dtype=np.float32)
    K = w.shape[0]
    G = K // s.shape[0]
    se = np.repeat(s, G, axis=0)
    ze = np.repeat(z, G, axis=0)
    d = round_to(w - ze, dtype)
    return round_to(d * se, dtype)


def forward(x, qweight, scales, zeros, dtype: str = F32) -> np.ndarray:
    """y = x @ dequant(...), reference.py:17 (`torch.matmul(x, (w - ze) * se)`).

    dtype F32: ground truth (fp32 operands and accumulation, fp32 result).
    dtype 'f16'/'bf16': the reference's native-dtype path — W rounded to dtype, fp32
    accumulation, result rounded to dtype. Returned as float32 values."""
    W = dequant(qweight, scales, zeros, dtype)
    xf = round_to(np.asarray(x, dtype=np.float32), dtype)
    y = xf @ W
    return round_to(y, dtype)
