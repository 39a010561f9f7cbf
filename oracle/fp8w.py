"""Oracle for the FP8 (e4m3fn) block-scaled weight GEMM (test infrastructure only).

Reference: tasks/fp8_microscale/fp8_microscale__llama3_8b_down__b128__fp16/environment/
reference.py:9-12 (template generate_tasks.py:218-237).
"""
from __future__ import annotations

import numpy as np

from .numerics import F32, e4m3fn_decode, round_to


def dequant(w_codes, scales, dtype: str) -> np.ndarray:
    """reference.py:11: fp32(w_fp8).reshape(K/B, B, N) * fp32(scales)[:, None, :], then
    .to(x.dtype) (one rounding; none in the fp32 ground truth)."""
    w = e4m3fn_decode(w_codes).astype(np.float32)
    s = np.asarray(scales, dtype=np.float32)
    K, N = w.shape
    B = K // s.shape[0]
    W = (w.reshape(K // B, B, N) * s[:, None, :]).reshape(K, N)
    return round_to(W, dtype)


def forward(x, w_codes, scales, dtype: str = F32) -> np.ndarray:
    """reference.py:12: x @ W. dtype F32 = ground truth; 'f16'/'bf16' = native path with an
    fp32-accumulated product rounded to dtype."""
    W = dequant(w_codes, scales, dtype)
    xf = round_to(np.asarray(x, dtype=np.float32), dtype)
    return round_to(xf @ W, dtype)
