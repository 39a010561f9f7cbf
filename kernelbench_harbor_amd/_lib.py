"""ctypes binding of the C-ABI library ``lib/libkbh_qgemm.so`` (declared in include/kbh_qgemm.h).

The library is loaded lazily, once per process, after ``torch`` so that it binds to the HIP
runtime torch already loaded (both carry the SONAME ``libamdhip64.so.7``). There is no
fallback: if the library is missing or fails to load, every op raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

from .build import LIB_PATH

_lock = threading.Lock()
_lib = None

# Status codes of include/kbh_qgemm.h (enum kbh_status).
KBH_OK = 0
KBH_ERR_NULL = 1
KBH_ERR_SHAPE = 2
KBH_ERR_DTYPE = 3
KBH_ERR_WORKSPACE = 4
KBH_ERR_ALIGN = 5
KBH_ERR_LAUNCH = 6
KBH_ERR_SCRATCH_LIMIT = 7

# KBH_W4A16_NOALLOC_SCRATCH_BYTES of include/kbh_qgemm.h: the fixed per-GPU scratch of
# kbh_w4a16_gemm_noalloc.
W4A16_NOALLOC_SCRATCH_BYTES = 64 << 20

KBH_F16 = 0
KBH_BF16 = 1
KBH_F32 = 2   # routing weights only

_vp = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t

# name -> (restype, argtypes); one entry per function declared in include/kbh_qgemm.h.
SIGNATURES = {
    "kbh_abi_version": (_i, []),
    "kbh_status_string": (ctypes.c_char_p, [_i]),
    "kbh_last_hip_error": (_i, []),
    "kbh_w4a16_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "kbh_w4a16_scratch_bytes": (_sz, [_i, _i, _i, _i]),
    "kbh_w4a16_gemm": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp, _sz, _i, _i, _i, _i, _i, _vp]),
    "kbh_w4a16_gemm_noalloc": (_i, [_vp] * 5 + [_i] * 5 + [_vp]),
    "kbh_w8a8_workspace_bytes": (_sz, [_i, _i, _i]),
    "kbh_w8a8_scratch_bytes": (_sz, [_i, _i, _i]),
    "kbh_w8a8_gemm": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp, _sz, _i, _i, _i, _vp]),
    "kbh_w8a8_gemm_i32": (_i, [_vp, _vp, _vp, _vp, _sz, _vp, _sz, _i, _i, _i, _vp]),
    "kbh_fp8w_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "kbh_fp8w_gemm": (_i, [_vp, _vp, _vp, _vp, _vp, _sz, _i, _i, _i, _i, _i, _vp]),
    "kbh_mxfp8_workspace_bytes": (_sz, [_i, _i, _i]),
    "kbh_mxfp8_gemm": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _i, _i, _i, _i, _vp]),
    "kbh_qmoe_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "kbh_moe_route_top2": (_i, [_vp, _i, _vp, _vp, _vp, _sz, _i, _i, _i, _vp]),
    "kbh_qmoe": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _vp, _sz, _i, _i, _i, _i, _i, _i, _vp]),
    "kbh_qmoe_ffn_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "kbh_qmoe_ffn": (_i, [_vp, _vp, _i] + [_vp] * 9 + [_vp, _vp, _sz, _i, _i, _i, _i, _i, _i, _vp]),
    "kbh_silu_fp8_quant": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "kbh_moe_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "kbh_moe_route_topk": (_i, [_vp, _i, _vp, _vp, _vp, _sz, _i, _i, _i, _i, _vp]),
    "kbh_moe": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _sz, _i, _i, _i, _i, _i, _i, _vp]),
    "kbh_lora_qgemm_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "kbh_lora_qgemm": (_i, [_vp] * 7 + [_vp, _sz] + [_i] * 7 + [_vp]),
}


class KbhError(RuntimeError):
    """A nonzero kbh_status returned by a library entry point."""


def load(path: str | None = None):
    """Loads (once) and returns the ctypes library handle with typed entry points."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            raise KbhError(
                f"HIP library not built: {p} is missing (run kernelbench_harbor_amd.build.build())")
        try:
            import torch  # noqa: F401  (bind the library to torch's HIP runtime)
        except ImportError:
            pass
        lib = ctypes.CDLL(p)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if path is None:
            _lib = lib
        return lib


def check(status: int, op: str) -> None:
    """Raises KbhError for a nonzero status from entry point `op`."""
    if status != KBH_OK:
        lib = load()
        msg = lib.kbh_status_string(status).decode()
        extra = ""
        if status == KBH_ERR_LAUNCH:
            extra = f" (hipError {lib.kbh_last_hip_error()})"
        raise KbhError(f"{op}: status {status}: {msg}{extra}")
