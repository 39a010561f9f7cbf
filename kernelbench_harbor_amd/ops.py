"""Host side of the quantized-GEMM ops: argument validation, workspace management and the call
into the C ABI on torch's current HIP stream.

Each function mirrors the math of one reference ``Model.forward`` (cited per function); the
arithmetic itself always runs in the HIP library — there is no CPU or torch fallback.
"""
from __future__ import annotations

import threading

import torch

from . import _lib

_DT_CODE = {torch.float16: _lib.KBH_F16, torch.bfloat16: _lib.KBH_BF16}


class _WorkspacePool:
    """Device buffers per (device, stream), grown on demand. The kernels put no requirement on
    their content, so one buffer serves every call ordered on the same stream; the two pools
    below exist because an op may need a workspace and a scratch buffer that do not overlap.

    A buffer is never freed: a HIP graph captured while it was current keeps its address, and
    replays must not write into memory the caching allocator has handed to someone else. When a
    larger call outgrows the current buffer, it is retired (kept alive for the process) and
    replaced by one at least twice its size, so the retired buffers together stay below the
    size of the current one."""

    def __init__(self):
        self._bufs: dict[tuple[int, int], tuple[torch.Tensor, int]] = {}
        self._retired: list[torch.Tensor] = []
        self._lock = threading.Lock()

    def get(self, nbytes: int, device: torch.device, stream: int | None = None) -> torch.Tensor:
        """A buffer of at least `nbytes` for calls on `stream` (default: the current stream of
        `device`)."""
        idx = device.index if device.index is not None else torch.cuda.current_device()
        key = (idx, _stream_ptr(device) if stream is None else stream)
        hit = self._bufs.get(key)            # a dict read is atomic; only growth takes the lock
        if hit is not None and hit[1] >= nbytes:
            return hit[0]
        with self._lock:
            hit = self._bufs.get(key)
            if hit is None or hit[1] < nbytes:
                size = max(nbytes, 256)
                if hit is not None:
                    self._retired.append(hit[0])
                    size = max(size, 2 * hit[1])
                hit = (torch.empty(size, dtype=torch.uint8, device=device), size)
                self._bufs[key] = hit
            return hit[0]


workspaces = _WorkspacePool()
scratches = _WorkspacePool()


def _require(cond: bool, msg) -> None:
    """Raises ValueError(msg) when cond is false; msg may be a callable returning the text, so
    that a formatted message costs nothing on the passing path (~0.4 us per f-string, several
    per call of a decode-sized op)."""
    if not cond:
        raise ValueError(msg() if callable(msg) else msg)


# torch's current-stream handle as a plain integer: the raw accessor costs ~0.1 us where
# torch.cuda.current_stream(...).cuda_stream builds a Stream object (~2 us), a large share of a
# decode-sized call.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_ptr(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if _raw_stream is not None:
        return _raw_stream(idx)
    return torch.cuda.current_stream(idx).cuda_stream


def _check_device(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    _require(dev.type == "cuda", lambda: f"tensors must be on a HIP device, got {dev}")
    for t in tensors[1:]:
        _require(t.device == dev, lambda: f"all tensors must be on {dev}, got {t.device}")
    return dev


# Workspace and scratch sizes per (op, shape): the plans are pure functions of the shape, and
# the two C calls cost ~0.35 us each per op call (a cached lookup ~0.1 us).
_sizes: dict[tuple, tuple[int, int]] = {}


def _w4a16_sizes(lib, M: int, N: int, K: int, group: int) -> tuple[int, int]:
    key = ("w4a16", M, N, K, group)
    hit = _sizes.get(key)
    if hit is None:
        hit = (lib.kbh_w4a16_workspace_bytes(M, N, K, group),
               lib.kbh_w4a16_scratch_bytes(M, N, K, group))
        _sizes[key] = hit
    return hit


def _w8a8_sizes(lib, M: int, N: int, K: int) -> tuple[int, int]:
    key = ("w8a8", M, N, K)
    hit = _sizes.get(key)
    if hit is None:
        hit = (lib.kbh_w8a8_workspace_bytes(M, N, K), lib.kbh_w8a8_scratch_bytes(M, N, K))
        _sizes[key] = hit
    return hit


def w4a16_gemm(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor,
               zeros: torch.Tensor) -> torch.Tensor:
    """y = x @ ((unpack(qweight) - zeros) * scales), the packed-asymmetric W4A16 linear.

    Follows tasks/quant_w4a16_pa/quant_w4a16_pa__llama3_8b_down__g128__fp16/environment/
    reference.py:10-17: qweight [K, N/8] int32 with nibble i of word [k, j] = column 8j+i,
    scales/zeros [K/G, N] in x.dtype; the group size G is K / scales.shape[0].
    """
    # Shapes and dtypes are read once into locals: each tensor attribute access costs ~0.1-0.2 us
    # and a reshape ~1.5 us, a large share of a decode-sized call.
    xd = x.dtype
    code = _DT_CODE.get(xd)
    _require(code is not None, lambda: f"x must be float16 or bfloat16, got {xd}")
    _require(qweight.dtype == torch.int32, lambda: f"qweight must be int32, got {qweight.dtype}")
    xs, qs, ss, zs = x.shape, qweight.shape, scales.shape, zeros.shape
    _require(len(qs) == 2 and len(ss) == 2 and len(zs) == 2,
             "qweight, scales and zeros must be 2-D")
    K, NP = qs
    N = NP * 8
    _require(len(xs) >= 1 and xs[-1] == K,
             lambda: f"x last dim {tuple(xs)[-1:]} != qweight rows {K}")
    _require(ss[1] == N and zs == ss,
             lambda: f"scales/zeros must be [K/G, {N}], got {tuple(ss)} / {tuple(zs)}")
    _require(ss[0] > 0 and K % ss[0] == 0, lambda: f"K={K} not divisible by scales rows {ss[0]}")
    group = K // ss[0]
    _require(scales.dtype == xd and zeros.dtype == xd, "scales and zeros must have x's dtype")
    dev = _check_device(x, qweight, scales, zeros)
    flat = len(xs) == 2
    x2 = x.contiguous() if flat else x.reshape(-1, K).contiguous()
    M = xs[0] if flat else x2.shape[0]
    y = torch.empty((M, N), dtype=xd, device=dev)
    if M > 0:
        qweight = qweight.contiguous()
        scales = scales.contiguous()
        zeros = zeros.contiguous()
        st = _stream_ptr(dev)
        lib = _lib.load()
        ws_bytes, sc_bytes = _w4a16_sizes(lib, M, N, K, group)
        ws = workspaces.get(ws_bytes, dev, st)
        sc = scratches.get(sc_bytes, dev, st)
        _lib.check(lib.kbh_w4a16_gemm(x2.data_ptr(), qweight.data_ptr(), scales.data_ptr(),
                                      zeros.data_ptr(), y.data_ptr(), ws.data_ptr(), ws.numel(),
                                      sc.data_ptr(), sc.numel(), M, N, K, group, code, st),
                   "kbh_w4a16_gemm")
    return y if flat else y.reshape(*xs[:-1], N)


def _w8a8_args(x_int8, w_int8):
    """(x as [M, K], M, N, K, whether x was already 2-D)."""
    _require(x_int8.dtype == torch.int8 and w_int8.dtype == torch.int8,
             lambda: f"x_int8/w_int8 must be int8, got {x_int8.dtype}/{w_int8.dtype}")
    xs, wsh = x_int8.shape, w_int8.shape
    _require(len(wsh) == 2, "w_int8 must be [K, N]")
    K, N = wsh
    _require(len(xs) >= 1 and xs[-1] == K, lambda: f"x_int8 last dim {tuple(xs)[-1:]} != K={K}")
    if len(xs) == 2:
        return x_int8, xs[0], N, K, True
    x2 = x_int8.reshape(-1, K)
    return x2, x2.shape[0], N, K, False


def w8a8_gemm(x_int8: torch.Tensor, w_int8: torch.Tensor, x_scale: torch.Tensor,
              w_scale: torch.Tensor) -> torch.Tensor:
    """out = fp16((fp32(x_int8 @ w_int8) * x_scale) * w_scale), int32-exact accumulation.

    Follows tasks/w8a8_smoothquant/w8a8_smoothquant__llama3_8b_down__M16/environment/
    reference.py:7-9: x_int8 [M, K], w_int8 [K, N], x_scale [M, 1] fp16, w_scale [1, N] fp16."""
    x2, M, N, K, flat = _w8a8_args(x_int8, w_int8)
    _require(x_scale.dtype == torch.float16 and w_scale.dtype == torch.float16,
             "x_scale and w_scale must be float16")
    _require(x_scale.numel() == M and w_scale.numel() == N,
             lambda: f"x_scale must hold {M} values and w_scale {N}")
    dev = _check_device(x_int8, w_int8, x_scale, w_scale)
    y = torch.empty((M, N), dtype=torch.float16, device=dev)
    if M > 0:
        # the scales are read as flat vectors: [M, 1] / [1, N] in place when contiguous
        x2, w = x2.contiguous(), w_int8.contiguous()
        xsc, wsc = x_scale.contiguous(), w_scale.contiguous()
        st = _stream_ptr(dev)
        lib = _lib.load()
        ws_bytes, sc_bytes = _w8a8_sizes(lib, M, N, K)
        ws = workspaces.get(ws_bytes, dev, st)
        sc = scratches.get(sc_bytes, dev, st)
        _lib.check(lib.kbh_w8a8_gemm(x2.data_ptr(), w.data_ptr(), xsc.data_ptr(), wsc.data_ptr(),
                                     y.data_ptr(), ws.data_ptr(), ws.numel(), sc.data_ptr(),
                                     sc.numel(), M, N, K, st), "kbh_w8a8_gemm")
    return y if flat else y.reshape(*x_int8.shape[:-1], N)


def w8a8_gemm_i32(x_int8: torch.Tensor, w_int8: torch.Tensor) -> torch.Tensor:
    """The exact int32 accumulators x_int8 @ w_int8 (reference.py:8 before the scales)."""
    x2, M, N, K, _ = _w8a8_args(x_int8, w_int8)
    dev = _check_device(x_int8, w_int8)
    x2, w = x2.contiguous(), w_int8.contiguous()
    acc = torch.empty((M, N), dtype=torch.int32, device=dev)
    if M == 0:
        return acc
    st = _stream_ptr(dev)
    lib = _lib.load()
    ws_bytes, sc_bytes = _w8a8_sizes(lib, M, N, K)
    ws = workspaces.get(ws_bytes, dev, st)
    sc = scratches.get(sc_bytes, dev, st)
    st = lib.kbh_w8a8_gemm_i32(x2.data_ptr(), w.data_ptr(), acc.data_ptr(), ws.data_ptr(),
                               ws.numel(), sc.data_ptr(), sc.numel(), M, N, K, st)
    _lib.check(st, "kbh_w8a8_gemm_i32")
    return acc


def fp8w_gemm(x: torch.Tensor, w_fp8: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """y = x @ (fp32(w_fp8) * fp32(scales[k // B])).to(x.dtype), the FP8 block-scaled weight GEMM.

    Follows tasks/fp8_microscale/fp8_microscale__llama3_8b_down__b128__fp16/environment/
    reference.py:9-12: w_fp8 [K, N] float8_e4m3fn, scales [K/B, N] fp16; the block size B is
    K / scales.shape[0]."""
    xd = x.dtype
    code = _DT_CODE.get(xd)
    _require(code is not None, lambda: f"x must be float16 or bfloat16, got {xd}")
    _require(w_fp8.dtype in (torch.float8_e4m3fn, torch.uint8),
             lambda: f"w_fp8 must be float8_e4m3fn (or its uint8 bits), got {w_fp8.dtype}")
    xs, wsh, ss = x.shape, w_fp8.shape, scales.shape
    _require(len(wsh) == 2 and len(ss) == 2, "w_fp8 and scales must be 2-D")
    K, N = wsh
    _require(len(xs) >= 1 and xs[-1] == K, lambda: f"x last dim {tuple(xs)[-1:]} != K={K}")
    _require(scales.dtype == torch.float16, lambda: f"scales must be float16, got {scales.dtype}")
    _require(ss[1] == N and ss[0] > 0 and K % ss[0] == 0,
             lambda: f"scales must be [K/B, {N}], got {tuple(ss)}")
    block = K // ss[0]
    dev = _check_device(x, w_fp8, scales)
    flat = len(xs) == 2
    x2 = x.contiguous() if flat else x.reshape(-1, K).contiguous()
    M = xs[0] if flat else x2.shape[0]
    y = torch.empty((M, N), dtype=xd, device=dev)
    if M > 0:
        w8 = w_fp8.contiguous()             # 1-byte elements: the pointer is the same as uint8
        sc = scales.contiguous()
        st = _stream_ptr(dev)
        lib = _lib.load()
        ws = workspaces.get(lib.kbh_fp8w_workspace_bytes(M, N, K, block), dev, st)
        _lib.check(lib.kbh_fp8w_gemm(x2.data_ptr(), w8.data_ptr(), sc.data_ptr(), y.data_ptr(),
                                     ws.data_ptr(), ws.numel(), M, N, K, block, code, st),
                   "kbh_fp8w_gemm")
    return y if flat else y.reshape(*xs[:-1], N)


_BYTE_DTYPES = (torch.uint8, torch.float8_e4m3fn)
_SCALE_DTYPES = (torch.uint8,) + ((torch.float8_e8m0fnu,) if hasattr(torch, "float8_e8m0fnu") else ())


def mxfp8_gemm(a: torch.Tensor, a_scale: torch.Tensor, b: torch.Tensor, b_scale: torch.Tensor,
               out_dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """MXFP8 GEMM: y[m, n] = sum_k dec(a[m, k]) dec(b[n, k]) with per-1x32-block e8m0 scales.

    a [M, K] and b [N, K] are float8_e4m3fn (or their uint8 bits), K-contiguous; a_scale
    [M, K/32] and b_scale [N, K/32] are e8m0 codes (uint8, or float8_e8m0fnu)."""
    _require(out_dtype in _DT_CODE,
             lambda: f"out_dtype must be float16 or bfloat16, got {out_dtype}")
    _require(a.dtype in _BYTE_DTYPES and b.dtype in _BYTE_DTYPES,
             lambda: f"a and b must be float8_e4m3fn or uint8, got {a.dtype}/{b.dtype}")
    _require(a_scale.dtype in _SCALE_DTYPES and b_scale.dtype in _SCALE_DTYPES,
             "scales must be e8m0 codes (uint8)")
    ash, bsh = a.shape, b.shape
    _require(len(ash) == 2 and len(bsh) == 2, "a and b must be 2-D")
    M, K = ash
    N = bsh[0]
    _require(bsh[1] == K, lambda: f"b must be [N, {K}], got {tuple(bsh)}")
    _require(K % 32 == 0 and a_scale.shape == (M, K // 32) and b_scale.shape == (N, K // 32),
             lambda: f"scales must be [M, K/32] and [N, K/32]")
    dev = _check_device(a, a_scale, b, b_scale)
    y = torch.empty((M, N), dtype=out_dtype, device=dev)
    if M == 0:
        return y
    st = _stream_ptr(dev)
    lib = _lib.load()
    ws = workspaces.get(lib.kbh_mxfp8_workspace_bytes(M, N, K), dev, st)
    # 1-byte elements: contiguous tensors of any of the accepted dtypes are the byte arrays
    a8, b8, as8, bs8 = a.contiguous(), b.contiguous(), a_scale.contiguous(), b_scale.contiguous()
    st = lib.kbh_mxfp8_gemm(a8.data_ptr(), as8.data_ptr(), b8.data_ptr(), bs8.data_ptr(),
                            y.data_ptr(), ws.data_ptr(), ws.numel(), M, N, K, _DT_CODE[out_dtype],
                            st)
    _lib.check(st, "kbh_mxfp8_gemm")
    return y


_LOGIT_CODE = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}
# Routing weights may also come back unrounded (fp32): KBH_F32.
_W_CODE = {torch.float16: _lib.KBH_F16, torch.bfloat16: _lib.KBH_BF16, torch.float32: _lib.KBH_F32}


def _check_logits(router_logits, T):
    _require(router_logits.dtype in _LOGIT_CODE,
             lambda: (f"router_logits must be float16, bfloat16 "
                      f"or float32, got {router_logits.dtype}"))
    _require(router_logits.dim() == 2 and router_logits.shape[0] == T,
             lambda: f"router_logits must be [{T}, E], got {tuple(router_logits.shape)}")
    E = router_logits.shape[1]
    _require(2 <= E <= 256, lambda: f"number of experts must be in [2, 256], got {E}")
    return E


def moe_route_top2(router_logits: torch.Tensor, dtype: torch.dtype = torch.float16):
    """(topi [T, 2] int32, topw [T, 2] dtype): softmax(fp32 logits), top-2 in the order
    torch.topk returns on the GPU, renormalised (tasks/fused_qmoe/*/environment/
    reference.py:14-16); dtype float16, bfloat16 or float32 (unrounded weights)."""
    _require(dtype in _W_CODE, lambda: f"dtype must be float16, bfloat16 or float32, got {dtype}")
    T = router_logits.shape[0]
    E = _check_logits(router_logits, T)
    dev = _check_device(router_logits)
    topi = torch.empty((T, 2), dtype=torch.int32, device=dev)
    topw = torch.empty((T, 2), dtype=dtype, device=dev)
    if T == 0:
        return topi, topw
    st = _stream_ptr(dev)
    lib = _lib.load()
    ws = scratches.get(lib.kbh_qmoe_workspace_bytes(T, 0, 0, E), dev, st)
    st = lib.kbh_moe_route_top2(router_logits.contiguous().data_ptr(), _LOGIT_CODE[router_logits.dtype],
                                topi.data_ptr(), topw.data_ptr(), ws.data_ptr(), ws.numel(), T, E,
                                _W_CODE[dtype], st)
    _lib.check(st, "kbh_moe_route_top2")
    return topi, topw


def qmoe(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor,
         router_logits: torch.Tensor) -> torch.Tensor:
    """Top-2 quantized MoE of tasks/fused_qmoe/fused_qmoe__mixtral__fp16/environment/
    reference.py:11-21: x [T, D], qweight [E, D, N] int8 (int4 values), scales [E, D/G, N] in
    x.dtype, router_logits [T, E]; G = D / scales.shape[1]."""
    _require(x.dtype in _DT_CODE, lambda: f"x must be float16 or bfloat16, got {x.dtype}")
    _require(x.dim() == 2, "x must be [T, D]")
    T, D = x.shape
    _require(qweight.dtype == torch.int8 and qweight.dim() == 3 and qweight.shape[1] == D,
             lambda: (f"qweight must be int8 [E, {D}, N], got "
                      f"{qweight.dtype} {tuple(qweight.shape)}"))
    E, _, N = qweight.shape
    _require(scales.dtype == x.dtype and scales.dim() == 3 and scales.shape[0] == E and
             scales.shape[2] == N and D % scales.shape[1] == 0,
             lambda: (f"scales must be x.dtype [E, D/G, N], got "
                      f"{scales.dtype} {tuple(scales.shape)}"))
    group = D // scales.shape[1]
    _require(_check_logits(router_logits, T) == E, "router_logits must have E columns")
    dev = _check_device(x, qweight, scales, router_logits)
    y = torch.empty((T, N), dtype=x.dtype, device=dev)
    if T == 0:
        return y
    st = _stream_ptr(dev)
    lib = _lib.load()
    ws = scratches.get(lib.kbh_qmoe_workspace_bytes(T, D, N, E), dev, st)
    st = lib.kbh_qmoe(x.contiguous().data_ptr(), qweight.contiguous().data_ptr(),
                      scales.contiguous().data_ptr(), router_logits.contiguous().data_ptr(),
                      _LOGIT_CODE[router_logits.dtype], y.data_ptr(), ws.data_ptr(), ws.numel(),
                      T, D, N, E, group, _DT_CODE[x.dtype], st)
    _lib.check(st, "kbh_qmoe")
    return y


def qmoe_ffn(x, router_logits, gate_qweight, gate_scales, gate_zeros, up_qweight, up_scales,
             up_zeros, down_qweight, down_scales, down_zeros) -> torch.Tensor:
    """Top-2 MoE SiLU FFN with W4A16 experts: y[t] = sum_k w_k * down_e(silu(gate_e x) * up_e x).

    gate/up qweight [E, D, F/8] int32 (packed along F), scales/zeros [E, D/G, F]; down
    qweight [E, F, D/8], scales/zeros [E, F/G, D]; all scales/zeros in x.dtype."""
    _require(x.dtype in _DT_CODE and x.dim() == 2, "x must be a float16/bfloat16 [T, D] tensor")
    T, D = x.shape
    E = _check_logits(router_logits, T)
    _require(gate_qweight.dtype == torch.int32 and gate_qweight.dim() == 3 and
             gate_qweight.shape[:2] == (E, D), lambda: f"gate_qweight must be int32 [E, D, F/8]")
    F = gate_qweight.shape[2] * 8
    _require(up_qweight.shape == gate_qweight.shape and up_qweight.dtype == torch.int32,
             "up_qweight must match gate_qweight")
    _require(down_qweight.dtype == torch.int32 and tuple(down_qweight.shape) == (E, F, D // 8),
             lambda: f"down_qweight must be int32 [E, {F}, {D // 8}]")
    group = D // gate_scales.shape[1]
    for name, t_, shape in [("gate_scales", gate_scales, (E, D // group, F)),
                            ("gate_zeros", gate_zeros, (E, D // group, F)),
                            ("up_scales", up_scales, (E, D // group, F)),
                            ("up_zeros", up_zeros, (E, D // group, F)),
                            ("down_scales", down_scales, (E, F // group, D)),
                            ("down_zeros", down_zeros, (E, F // group, D))]:
        _require(t_.dtype == x.dtype and tuple(t_.shape) == shape,
                 lambda: f"{name} must be x.dtype {shape}, got {t_.dtype} {tuple(t_.shape)}")
    ts = [x, gate_qweight, gate_scales, gate_zeros, up_qweight, up_scales, up_zeros,
          down_qweight, down_scales, down_zeros]
    dev = _check_device(router_logits, *ts)
    y = torch.empty((T, D), dtype=x.dtype, device=dev)
    if T == 0:
        return y
    st = _stream_ptr(dev)
    lib = _lib.load()
    ws = scratches.get(lib.kbh_qmoe_ffn_workspace_bytes(T, D, F, E), dev, st)
    ts = [t_.contiguous() for t_ in ts]
    st = lib.kbh_qmoe_ffn(ts[0].data_ptr(), router_logits.contiguous().data_ptr(),
                          _LOGIT_CODE[router_logits.dtype], *[t_.data_ptr() for t_ in ts[1:]],
                          y.data_ptr(), ws.data_ptr(), ws.numel(), T, D, F, E, group,
                          _DT_CODE[x.dtype], st)
    _lib.check(st, "kbh_qmoe_ffn")
    return y


def silu_fp8_quant(y: torch.Tensor, group: int = 128, return_codes: bool = False):
    """Fused SiLU x up with per-group dynamic e4m3fn quantisation, returned dequantised.

    Follows tasks/fused_silu_fp8/fused_silu_fp8__mixtral__T512__fp16/environment/reference.py:13-23:
    y [T, 2H] = concat(gate, up); act = silu(fp32 gate) * fp32 up; per `group` columns
    scale = max(amax|act| / 448, 1e-12), q = e4m3fn(clamp(act / scale, +-448));
    returns fp32(q) * scale as float32 [T, H]. With ``return_codes`` also returns the codes
    (torch.float8_e4m3fn [T, H]) and the scales (float32 [T, H / group]).
    """
    _require(y.dtype in _DT_CODE, lambda: f"y must be float16 or bfloat16, got {y.dtype}")
    _require(y.dim() == 2, lambda: f"y must be 2-D [T, 2H], got {tuple(y.shape)}")
    T, H2 = y.shape
    _require(H2 % 2 == 0, lambda: f"y's last dim {H2} must be even (gate and up halves)")
    H = H2 // 2
    _require(group in (32, 64, 128), lambda: f"group must be 32, 64 or 128, got {group}")
    # the reference's reshape(T, H // GROUP, GROUP) raises for any other H
    _require(H % group == 0, lambda: f"H={H} must be a multiple of the group size {group}")
    dev = _check_device(y)
    out = torch.empty((T, H), dtype=torch.float32, device=dev)
    codes = scales = None
    if return_codes:
        codes = torch.empty((T, H), dtype=torch.uint8, device=dev)
        scales = torch.empty((T, H // group), dtype=torch.float32, device=dev)
    if T > 0 and H > 0:
        st = _stream_ptr(dev)
        lib = _lib.load()
        yc = y.contiguous()
        st = lib.kbh_silu_fp8_quant(yc.data_ptr(), out.data_ptr(),
                                    codes.data_ptr() if return_codes else None,
                                    scales.data_ptr() if return_codes else None,
                                    T, H, group, _DT_CODE[y.dtype], st)
        _lib.check(st, "kbh_silu_fp8_quant")
    if return_codes:
        return out, codes.view(torch.float8_e4m3fn), scales
    return out


def moe_route_topk(router_logits: torch.Tensor, topk: int, dtype: torch.dtype = torch.float16):
    """(topi [T, topk] int32, topw [T, topk] dtype): softmax(fp32 logits), top-k in the order
    torch.topk returns on the GPU (descending; the lower indices win a tie at the boundary),
    weights renormalised and rounded to dtype, or unrounded for float32
    (tasks/moe/*/environment/reference.py:11-13)."""
    _require(dtype in _W_CODE, lambda: f"dtype must be float16, bfloat16 or float32, got {dtype}")
    T = router_logits.shape[0]
    E = _check_logits(router_logits, T)
    _require(1 <= topk <= min(8, E), lambda: f"topk must be in [1, min(8, E={E})], got {topk}")
    dev = _check_device(router_logits)
    topi = torch.empty((T, topk), dtype=torch.int32, device=dev)
    topw = torch.empty((T, topk), dtype=dtype, device=dev)
    if T == 0:
        return topi, topw
    st = _stream_ptr(dev)
    lib = _lib.load()
    ws = scratches.get(lib.kbh_moe_workspace_bytes(T, 0, 0, E, topk), dev, st)
    st = lib.kbh_moe_route_topk(router_logits.contiguous().data_ptr(),
                                _LOGIT_CODE[router_logits.dtype], topi.data_ptr(), topw.data_ptr(),
                                ws.data_ptr(), ws.numel(), T, E, topk, _W_CODE[dtype],
                                st)
    _lib.check(st, "kbh_moe_route_topk")
    return topi, topw


def moe(x: torch.Tensor, w: torch.Tensor, router_logits: torch.Tensor, topk: int) -> torch.Tensor:
    """Top-k MoE with fp16/bf16 experts: y[t] = sum_j w_j * (x[t] @ w[e_j]), sparse dispatch.

    Follows tasks/moe/moe_top2__mixtral_8x7b__T16__fp16/environment/reference.py:10-17: x [T, D],
    w [E, D, H] in x.dtype, router_logits [T, E]; each expert output and each weighted product
    rounded to x.dtype, the k products summed in fp32 and rounded once."""
    _require(x.dtype in _DT_CODE and x.dim() == 2, "x must be a float16/bfloat16 [T, D] tensor")
    T, D = x.shape
    E = _check_logits(router_logits, T)
    _require(w.dtype == x.dtype and w.dim() == 3 and w.shape[:2] == (E, D),
             lambda: f"w must be x.dtype [{E}, {D}, H], got {w.dtype} {tuple(w.shape)}")
    H = w.shape[2]
    _require(1 <= topk <= min(8, E), lambda: f"topk must be in [1, min(8, E={E})], got {topk}")
    _require(D % 128 == 0 and D >= 128, lambda: f"D={D} must be a positive multiple of 128")
    _require(H % 128 == 0 and H >= 128, lambda: f"H={H} must be a positive multiple of 128")
    dev = _check_device(x, w, router_logits)
    y = torch.empty((T, H), dtype=x.dtype, device=dev)
    if T == 0:
        return y
    st = _stream_ptr(dev)
    lib = _lib.load()
    ws = scratches.get(lib.kbh_moe_workspace_bytes(T, D, H, E, topk), dev, st)
    xc, wc = x.contiguous(), w.contiguous()
    st = lib.kbh_moe(xc.data_ptr(), wc.data_ptr(), router_logits.contiguous().data_ptr(),
                     _LOGIT_CODE[router_logits.dtype], y.data_ptr(), ws.data_ptr(), ws.numel(),
                     T, D, H, E, topk, _DT_CODE[x.dtype], st)
    _lib.check(st, "kbh_moe")
    return y


def lora_qgemm(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor, A: torch.Tensor,
               B: torch.Tensor, lora_ids: torch.Tensor) -> torch.Tensor:
    """Multi-LoRA quantized linear: y = x @ dequant(W) + (x @ A[id]) @ B[id] per token.

    Follows tasks/multi_lora_qgemm/multi_lora_qgemm__llama3_8b_r16__fp16/environment/
    reference.py:10-17: qweight [D, N] int8 holding int4 values, scales [D/G, N] (G = D /
    scales.shape[0]), A [L, D, r], B [L, r, N], lora_ids [T] integer; every intermediate
    (dequantised weight, base, shrink, expand) rounded to x.dtype as the reference."""
    _require(x.dtype in _DT_CODE and x.dim() == 2, "x must be a float16/bfloat16 [T, D] tensor")
    T, D = x.shape
    _require(qweight.dtype == torch.int8 and qweight.dim() == 2 and qweight.shape[0] == D,
             lambda: f"qweight must be int8 [{D}, N], got {qweight.dtype} {tuple(qweight.shape)}")
    N = qweight.shape[1]
    _require(scales.dim() == 2 and scales.shape[1] == N and scales.shape[0] > 0 and
             D % scales.shape[0] == 0,
             lambda: f"scales must be [D/G, {N}], got {tuple(scales.shape)}")
    group = D // scales.shape[0]
    _require(A.dim() == 3 and A.shape[1] == D and B.dim() == 3 and B.shape[0] == A.shape[0] and
             B.shape[1] == A.shape[2] and B.shape[2] == N,
             lambda: (f"A must be [L, {D}, r] and B [L, r, {N}], "
                      f"got {tuple(A.shape)} / {tuple(B.shape)}"))
    L, r = A.shape[0], A.shape[2]
    for name, t_ in (("scales", scales), ("A", A), ("B", B)):
        _require(t_.dtype == x.dtype,
                 lambda: f"{name} must have x's dtype {x.dtype}, got {t_.dtype}")
    _require(lora_ids.dim() == 1 and lora_ids.shape[0] == T and not lora_ids.is_floating_point(),
             lambda: f"lora_ids must be an integer [{T}] tensor")
    _require(r in (4, 8, 16, 32, 64), lambda: f"rank r must be 4, 8, 16, 32 or 64, got {r}")
    _require(N % 128 == 0 and D % 32 == 0,
             lambda: f"need N % 128 == 0 and D % 32 == 0 (D={D}, N={N})")
    _require(group in (32, 64, 128, 256), lambda: f"group size {group} not supported")
    dev = _check_device(x, qweight, scales, A, B, lora_ids)
    y = torch.empty((T, N), dtype=x.dtype, device=dev)
    if T == 0:
        return y
    st = _stream_ptr(dev)
    lib = _lib.load()
    ws = workspaces.get(lib.kbh_lora_qgemm_workspace_bytes(T, D, N, r), dev, st)
    ts = [t_.contiguous() for t_ in (x, qweight, scales, A, B)]
    ids = lora_ids.to(torch.int64).contiguous()
    st = lib.kbh_lora_qgemm(*[t_.data_ptr() for t_ in ts], ids.data_ptr(), y.data_ptr(),
                            ws.data_ptr(), ws.numel(), T, D, N, r, L, group, _DT_CODE[x.dtype],
                            st)
    _lib.check(st, "kbh_lora_qgemm")
    return y
