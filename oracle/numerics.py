"""Bit-level number formats used by the quantized-GEMM oracle (numpy, CPU only).

fp16 is numpy's float16. bfloat16 has no numpy dtype: it is carried as float32 arrays holding
bf16-representable values, or as uint16 bit patterns. e4m3fn follows the OCP FP8 E4M3
definition used by torch.float8_e4m3fn (bias 7, no infinities, S.1111.111 = NaN, max 448).
e8m0 is the OCP MX shared-scale format: value 2^(e-127), e = 255 is NaN.
"""
from __future__ import annotations

import numpy as np

F16, BF16, F32 = "f16", "bf16", "f32"


def f32_to_bf16_bits(a) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even; NaN stays NaN."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_to(a, dtype: str) -> np.ndarray:
    """Rounds float values to `dtype` ('f16', 'bf16', 'f32'); returns float32 values."""
    a = np.asarray(a, dtype=np.float32)
    if dtype == F32:
        return a
    if dtype == F16:
        return a.astype(np.float16).astype(np.float32)
    if dtype == BF16:
        return bf16_bits_to_f32(f32_to_bf16_bits(a))
    raise ValueError(dtype)


# ---- e4m3fn -------------------------------------------------------------------------------

def e4m3fn_decode_table() -> np.ndarray:
    """float32[256]: value of each e4m3fn code (NaN for 0x7F and 0xFF)."""
    codes = np.arange(256, dtype=np.int64)
    s = np.where(codes >> 7, -1.0, 1.0)
    e = (codes >> 3) & 0xF
    m = codes & 0x7
    v = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * 2.0 ** (e - 7))
    v = s * v
    v[(codes & 0x7F) == 0x7F] = np.nan
    return v.astype(np.float32)


_E4M3_TABLE = e4m3fn_decode_table()


def e4m3fn_decode(codes) -> np.ndarray:
    return _E4M3_TABLE[np.asarray(codes, dtype=np.uint8)]


def e4m3fn_encode_rne(a) -> np.ndarray:
    """float -> e4m3fn code, round to nearest even. |a| beyond the rounding range of 448
    (> 464) and NaN map to NaN (0x7F / 0xFF), matching torch's float8_e4m3fn cast."""
    a = np.asarray(a, dtype=np.float64)
    sign = np.signbit(a)
    x = np.abs(a)
    pos = _E4M3_TABLE[:127].astype(np.float64)          # codes 0..126 ascending, all finite
    hi = np.clip(np.searchsorted(pos, x, side="left"), 1, 126)   # pos[hi-1] < x <= pos[hi]
    lo = hi - 1
    d_lo = x - pos[lo]
    d_hi = pos[hi] - x
    code = np.where(d_lo < d_hi, lo, hi)
    code = np.where(d_lo == d_hi, np.where(lo % 2 == 0, lo, hi), code)   # ties to even code
    code = np.where(x <= 0.0, 0, code)
    code = np.where(x > 448.0, 126, code)               # (448, 464] rounds to 448 (464: tie, even)
    code = np.where((x > 464.0) | np.isnan(x), 0x7F, code)    # 464 = midpoint of 448 and 480
    code = code | np.where(sign, 0x80, 0)
    return code.astype(np.uint8)


# ---- e8m0 ---------------------------------------------------------------------------------

def e8m0_decode(e) -> np.ndarray:
    """float64 value 2^(e-127) of each e8m0 code; code 255 is NaN."""
    e = np.asarray(e, dtype=np.int64)
    v = np.ldexp(1.0, e - 127)
    return np.where(e == 255, np.nan, v)
