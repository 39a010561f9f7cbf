"""Oracle for the MXFP8 block-scaled GEMM (test infrastructure only).

No reference module exists for this configuration; the math follows the OCP MX definition used
by the benchmark's MXFP8 configuration and the reference's FP8 pieces: absmax / 448 and the e4m3fn cast
(generate_tasks.py:337-342), fp8 decode times scale (tasks/fp8_microscale/*/environment/
reference.py:11).
"""
from __future__ import annotations

import numpy as np

from .numerics import e4m3fn_decode, e4m3fn_encode_rne, e8m0_decode


def ceil_log2(v) -> np.ndarray:
    """Exact ceil(log2(v)) for positive finite v (frexp: v = m 2^e, m in [0.5, 1))."""
    m, e = np.frexp(np.asarray(v, dtype=np.float64))
    return np.where(m == 0.5, e - 1, e).astype(np.int64)


def quantize(src):
    """Rows of src along K in 1x32 blocks: e8m0 code = ceil(log2(amax/448)) + 127 (0 when the
    block is all zero), element code = e4m3fn_rne(x / 2^(code-127))."""
    x = np.asarray(src, dtype=np.float64)
    R, K = x.shape
    blk = x.reshape(R, K // 32, 32)
    amax = np.abs(blk).max(axis=-1)
    code = np.zeros(amax.shape, np.int64)
    nz = amax > 0
    code[nz] = np.clip(ceil_log2(amax[nz] / 448.0) + 127, 0, 254)
    scale = np.ldexp(1.0, code - 127)
    q = e4m3fn_encode_rne(blk / scale[..., None])
    return q.reshape(R, K), code.astype(np.uint8)


def dequant(codes, scales) -> np.ndarray:
    """Exact float64 values: e4m3fn(code) * 2^(e8m0 - 127) per 1x32 block."""
    v = e4m3fn_decode(codes).astype(np.float64)
    R, K = v.shape
    s = e8m0_decode(scales)
    return (v.reshape(R, K // 32, 32) * s[..., None]).reshape(R, K)


def forward(a, a_scale, b, b_scale, accumulate=np.float64) -> np.ndarray:
    """Ground truth: GEMM of the dequantised operands, y = A @ B^T, returned as float32."""
    A = dequant(a, a_scale).astype(accumulate)
    B = dequant(b, b_scale).astype(accumulate)
    return (A @ B.T).astype(np.float32)
