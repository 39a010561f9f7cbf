"""Oracle for the fused SiLU x up + per-group dynamic FP8 quantisation (test infrastructure only).

Restates tasks/fused_silu_fp8/fused_silu_fp8__mixtral__T512__fp16/environment/reference.py:13-23
(template generate_tasks.py:321-348) in numpy float32, step for step:
  gate, up = y[:, :H], y[:, H:]                       (:15-16)
  act   = silu(fp32(gate)) * fp32(up)                  (:17; silu(x) = x / (1 + exp(-x)))
  scale = max(amax(|act|) over GROUP columns / 448, 1e-12)     (:18-20)
  q     = fp32(e4m3fn_rne(clamp(act / scale, -448, 448)))      (:21)
  out   = q * scale                                    (:22)
Every step after `act` is an exactly rounded fp32 operation (division, clamp, RNE cast, product),
so given the same `act` the result is bit-determined; `act` itself depends on the exp routine
(numpy's here) to a few ulp.
"""
from __future__ import annotations

import numpy as np

from .numerics import e4m3fn_decode, e4m3fn_encode_rne

FP8_MAX = np.float32(448.0)


def silu_mul(gate, up) -> np.ndarray:
    """fp32 silu(gate) * up, both given as float32 arrays of the input dtype's values."""
    g = np.asarray(gate, dtype=np.float32)
    u = np.asarray(up, dtype=np.float32)
    with np.errstate(over="ignore"):
        s = g / (np.float32(1.0) + np.exp(-g))
    return (s * u).astype(np.float32)


def quantize(act, group: int = 128):
    """Per-row, per-`group`-columns dynamic e4m3fn quantisation of fp32 `act` [T, H].
    Returns (dequantised fp32 [T, H], e4m3fn codes uint8 [T, H], scales fp32 [T, H/group])."""
    a = np.asarray(act, dtype=np.float32)
    T, H = a.shape
    ag = a.reshape(T, H // group, group)
    with np.errstate(invalid="ignore"):
        amax = np.abs(ag).max(axis=-1, keepdims=True)
        scale = np.maximum(amax / FP8_MAX, np.float32(1e-12)).astype(np.float32)
        scale = np.where(np.isnan(amax), np.float32(np.nan), scale)   # torch.clamp keeps NaN
        v = (ag / scale).astype(np.float32)
        v = np.where(np.isnan(v), v, np.clip(v, -FP8_MAX, FP8_MAX))
    codes = e4m3fn_encode_rne(v)
    q = e4m3fn_decode(codes)
    out = (q * scale).astype(np.float32)
    return out.reshape(T, H), codes.reshape(T, H), scale.reshape(T, H // group)


def forward(y, group: int = 128):
    """y [T, 2H] (float32 array holding fp16/bf16 values) -> (out, codes, scales)."""
    y = np.asarray(y, dtype=np.float32)
    H = y.shape[1] // 2
    return quantize(silu_mul(y[:, :H], y[:, H:]), group)
