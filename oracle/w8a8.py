"""Oracle for the W8A8 SmoothQuant GEMM (test infrastructure only).

Reference: tasks/w8a8_smoothquant/w8a8_smoothquant__llama3_8b_down__M16/environment/
reference.py:7-9 (template generate_tasks.py:198-215).
"""
from __future__ import annotations

import numpy as np


def acc_int32(x_int8, w_int8) -> np.ndarray:
    """Exact x_int8 @ w_int8 as int64 (reference.py:8 computes it as an fp32 matmul).

    Every partial sum is an integer of magnitude <= K * 128^2, far below 2^53, so a float64
    matmul is exact regardless of summation order."""
    a = np.asarray(x_int8, dtype=np.float64)
    b = np.asarray(w_int8, dtype=np.float64)
    return np.rint(a @ b).astype(np.int64)


def epilogue(acc, x_scale, w_scale) -> np.ndarray:
    """reference.py:9: (acc * x_scale.float() * w_scale.float()).to(float16), evaluated left to
    right in fp32. Returns float32 values of the fp16 result."""
    a = np.asarray(acc).astype(np.float32)
    xs = np.asarray(x_scale, dtype=np.float32).reshape(-1, 1)
    ws = np.asarray(w_scale, dtype=np.float32).reshape(1, -1)
    t = (a * xs).astype(np.float32)
    return (t * ws).astype(np.float32).astype(np.float16).astype(np.float32)


def forward(x_int8, w_int8, x_scale, w_scale) -> np.ndarray:
    return epilogue(acc_int32(x_int8, w_int8), x_scale, w_scale)
