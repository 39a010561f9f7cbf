"""CPU checks of the C ABI: the library builds, loads and exports every declared entry point;
argument checks in the library reject bad shapes/pointers before any launch."""
import ctypes
import os
import re

import pytest

from kernelbench_harbor_amd import _lib
from kernelbench_harbor_amd.build import LIB_PATH

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "kbh_qgemm.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(kbh_[a-z0-9_]+)\s*\(", src)))


def test_library_exists():
    assert os.path.exists(LIB_PATH), "run kernelbench_harbor_amd.build.build() first"


def test_every_declared_symbol_is_exported_and_bound():
    lib = ctypes.CDLL(LIB_PATH)
    names = declared_functions()
    assert len(names) >= 5
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/kbh_qgemm.h but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature in _lib.py"


def test_version_and_status_strings():
    lib = _lib.load()
    assert lib.kbh_abi_version() == 1
    assert lib.kbh_status_string(0) == b"ok"
    assert b"shape" in lib.kbh_status_string(_lib.KBH_ERR_SHAPE)
    assert lib.kbh_status_string(999) == b"unknown status"


def test_host_checks_run_without_gpu():
    """Bad arguments are rejected by the library before it touches the device."""
    lib = _lib.load()
    p = ctypes.c_void_p(16)  # aligned fake address; never dereferenced on these paths
    assert lib.kbh_w4a16_gemm(None, p, p, p, p, p, 1 << 20, p, 1 << 20, 16, 4096, 4096, 128, 0, None) == _lib.KBH_ERR_NULL
    assert lib.kbh_w4a16_gemm(p, p, p, p, p, p, 1 << 20, p, 1 << 20, 16, 4100, 4096, 128, 0, None) == _lib.KBH_ERR_SHAPE
    assert lib.kbh_w4a16_gemm(p, p, p, p, p, p, 1 << 20, p, 1 << 20, 16, 4096, 4096, 100, 0, None) == _lib.KBH_ERR_SHAPE
    assert lib.kbh_w4a16_gemm(p, p, p, p, p, p, 1 << 20, p, 1 << 20, 16, 4096, 4096, 128, 7, None) == _lib.KBH_ERR_DTYPE
    assert lib.kbh_w4a16_gemm(p, ctypes.c_void_p(18), p, p, p, p, 1 << 20, p, 1 << 20, 16, 4096, 4096, 128, 0, None) == _lib.KBH_ERR_ALIGN
    assert lib.kbh_w4a16_gemm(p, p, p, p, p, p, 8, p, 1 << 20, 16, 4096, 4096, 128, 0, None) == _lib.KBH_ERR_WORKSPACE
    # large M runs the wide-tile kernel, whose split-K partials need the scratch buffer
    need = lib.kbh_w4a16_scratch_bytes(2048, 4096, 14336, 128)
    assert lib.kbh_w4a16_gemm(p, p, p, p, p, p, 1 << 20, p, need - 1, 2048, 4096, 14336, 128, 0, None) == _lib.KBH_ERR_WORKSPACE
    assert lib.kbh_w4a16_gemm(p, p, p, p, p, p, 1 << 20, None, 0, 2048, 4096, 14336, 128, 0, None) == _lib.KBH_ERR_WORKSPACE
    # the no-alloc W4A16 entry point checks its arguments and the size of its fixed scratch
    # before any HIP call
    assert lib.kbh_w4a16_gemm_noalloc(None, p, p, p, p, 16, 4096, 4096, 128, 0, None) == _lib.KBH_ERR_NULL
    assert lib.kbh_w4a16_gemm_noalloc(p, p, p, p, p, 16, 4096, 4100, 128, 0, None) == _lib.KBH_ERR_SHAPE
    assert lib.kbh_w4a16_gemm_noalloc(p, p, p, p, p, 24, 12288, 65536, 64, 0, None) == _lib.KBH_ERR_SCRATCH_LIMIT
    assert b"fixed scratch" in lib.kbh_status_string(_lib.KBH_ERR_SCRATCH_LIMIT)
    assert lib.kbh_w4a16_scratch_bytes(2048, 4096, 14336, 128) <= _lib.W4A16_NOALLOC_SCRATCH_BYTES
    # the wide-tile planner keeps its K-split partial sums within the fixed scratch for any M
    for M in (33, 64, 257, 300, 385, 1025, 2048, 2305, 8192):
        for N, K in ((4096, 14336), (12288, 14336), (28672, 4096), (256, 4096)):
            assert lib.kbh_w4a16_scratch_bytes(M, N, K, 128) <= _lib.W4A16_NOALLOC_SCRATCH_BYTES
    assert lib.kbh_w8a8_gemm(p, p, p, p, p, p, 1 << 20, p, 1 << 20, 16, 4096, 100, None) == _lib.KBH_ERR_SHAPE
    assert lib.kbh_w8a8_gemm(p, p, p, p, p, None, 0, p, 1 << 20, 16, 4096, 4096, None) == _lib.KBH_ERR_WORKSPACE
    need = lib.kbh_w8a8_scratch_bytes(512, 4096, 14336)
    assert need >= 512 * 4096 * 4 * 2
    assert lib.kbh_w8a8_gemm(p, p, p, p, p, p, 1 << 20, p, need - 1, 512, 4096, 14336, None) == _lib.KBH_ERR_WORKSPACE
    # MXFP8: K % 256, N % 64, and the 32-bit operand offsets (M*K, N*K < 2^31)
    assert lib.kbh_mxfp8_gemm(p, p, p, p, p, p, 1 << 20, 128, 4096, 14300, 0, None) == _lib.KBH_ERR_SHAPE
    assert lib.kbh_mxfp8_gemm(p, p, p, p, p, p, 1 << 20, 128, 4000, 14336, 0, None) == _lib.KBH_ERR_SHAPE
    assert lib.kbh_mxfp8_gemm(p, p, p, p, p, p, 1 << 20, 1 << 18, 4096, 8192, 0, None) == _lib.KBH_ERR_SHAPE
    assert lib.kbh_mxfp8_gemm(p, p, p, p, p, p, 1 << 20, 128, 1 << 18, 8192, 0, None) == _lib.KBH_ERR_SHAPE

    # fused SiLU + FP8 quantisation: group, divisibility, dtype, alignment; T = 0 is a no-op
    assert lib.kbh_silu_fp8_quant(None, p, None, None, 4, 256, 128, 0, None) == _lib.KBH_ERR_NULL
    assert lib.kbh_silu_fp8_quant(p, p, None, None, 4, 256, 100, 0, None) == _lib.KBH_ERR_SHAPE
    assert lib.kbh_silu_fp8_quant(p, p, None, None, 4, 320, 128, 0, None) == _lib.KBH_ERR_SHAPE
    assert lib.kbh_silu_fp8_quant(p, p, None, None, 4, 256, 128, 5, None) == _lib.KBH_ERR_DTYPE
    assert lib.kbh_silu_fp8_quant(p, ctypes.c_void_p(20), None, None, 4, 256, 128, 0, None) == _lib.KBH_ERR_ALIGN
    assert lib.kbh_silu_fp8_quant(p, p, ctypes.c_void_p(20), None, 4, 256, 128, 0, None) == _lib.KBH_ERR_ALIGN
    assert lib.kbh_silu_fp8_quant(p, p, None, None, 0, 256, 128, 0, None) == _lib.KBH_OK
    # top-k MoE: k range, D / H divisibility, workspace size
    need = lib.kbh_moe_workspace_bytes(16, 4096, 14336, 8, 2)
    assert need >= 2 * 16 * 14336 * 2 and lib.kbh_moe_workspace_bytes(16, 4096, 14336, 8, 9) == 0
    assert lib.kbh_moe(p, p, p, 0, p, p, need, 16, 4096, 14336, 8, 9, 0, None) == _lib.KBH_ERR_SHAPE
    assert lib.kbh_moe(p, p, p, 0, p, p, need, 16, 4096, 14336, 8, 0, 0, None) == _lib.KBH_ERR_SHAPE
    assert lib.kbh_moe(p, p, p, 0, p, p, need, 16, 4000, 14336, 8, 2, 0, None) == _lib.KBH_ERR_SHAPE
    assert lib.kbh_moe(p, p, p, 0, p, p, need, 16, 4096, 14300, 8, 2, 0, None) == _lib.KBH_ERR_SHAPE
    assert lib.kbh_moe(p, p, p, 0, p, p, need - 1, 16, 4096, 14336, 8, 2, 0, None) == _lib.KBH_ERR_WORKSPACE
    assert lib.kbh_moe(p, p, p, 3, p, p, need, 16, 4096, 14336, 8, 2, 0, None) == _lib.KBH_ERR_DTYPE
    assert lib.kbh_moe(None, p, p, 0, p, p, need, 16, 4096, 14336, 8, 2, 0, None) == _lib.KBH_ERR_NULL
    assert lib.kbh_moe_route_topk(p, 0, p, p, p, need, 16, 4, 6, 0, None) == _lib.KBH_ERR_SHAPE
    # multi-LoRA: rank, group, N divisibility, workspace
    need = lib.kbh_lora_qgemm_workspace_bytes(64, 4096, 4096, 16)
    assert need >= 64 * 16 * 2
    args = lambda T=64, D=4096, N=4096, r=16, g=128, dt=0, ws=need: (
        p, p, p, p, p, p, p, p, ws, T, D, N, r, 8, g, dt, None)
    assert lib.kbh_lora_qgemm(*args(r=12)) == _lib.KBH_ERR_SHAPE
    assert lib.kbh_lora_qgemm(*args(g=100)) == _lib.KBH_ERR_SHAPE
    assert lib.kbh_lora_qgemm(*args(N=4000)) == _lib.KBH_ERR_SHAPE
    assert lib.kbh_lora_qgemm(*args(dt=2)) == _lib.KBH_ERR_DTYPE
    assert lib.kbh_lora_qgemm(*args(ws=need - 1)) == _lib.KBH_ERR_WORKSPACE


def test_workspace_sizes():
    lib = _lib.load()
    assert lib.kbh_w4a16_workspace_bytes(16, 4096, 14336, 128) >= 16 * 4096 * 4
    assert lib.kbh_w8a8_workspace_bytes(16, 4096, 14336) >= 16 * 4096 * 4
    assert lib.kbh_w4a16_workspace_bytes(0, 4096, 14336, 128) == 0
    assert lib.kbh_w4a16_scratch_bytes(16, 4096, 14336, 128) == 0       # decode kernel
    assert lib.kbh_w4a16_scratch_bytes(2048, 4096, 14336, 128) >= 2048 * 4096 * 4 * 2  # split-K


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(_lib.KbhError, match="not built"):
        _lib.load(str(tmp_path / "missing.so"))
