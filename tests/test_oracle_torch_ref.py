"""CPU checks that pin oracle/torch_ref.py (the reference op sequences bench.py times on the host)
against the committed golden vectors and the numpy oracle: the timed CPU baseline computes the
same ops as the reference."""
import os

import numpy as np
import torch

from oracle import mxfp8 as omx
from oracle import qmoe as oq
from oracle import torch_ref as tr

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _g(name):
    with np.load(os.path.join(GOLD, f"{name}.npz"), allow_pickle=False) as z:
        return {k: torch.from_numpy(z[k]) for k in z.files}


def _rel(y, want):
    y, want = y.double(), want.double()
    return float((y - want).abs().max() / want.abs().max())


def test_w4a16_ground_truth_and_native():
    g = _g("w4a16")
    ins = [g["x"], g["qweight"], g["scales"], g["zeros"]]
    assert _rel(tr.w4a16(*tr.upcast(ins)), g["y_gt"]) <= 1e-6
    y16 = tr.w4a16(*ins)
    assert y16.dtype == torch.float16
    assert _rel(y16.float(), g["x"].float() @ g["W_f16"].float()) <= 2e-3


def test_w8a8_bit_exact():
    g = _g("w8a8")
    y = tr.w8a8(g["x_int8"], g["w_int8"], g["x_scale"], g["w_scale"])
    assert torch.equal(y, g["out"])


def test_fp8w_ground_truth():
    g = _g("fp8w")
    w = g["w_codes"].view(torch.float8_e4m3fn)
    assert _rel(tr.fp8w(g["x"].float(), w, g["scales"].float()), g["y_gt"]) <= 1e-6


def test_mxfp8_matches_oracle():
    rng = np.random.default_rng(3)
    a, a_s = omx.quantize(rng.normal(size=(8, 256)))
    b, b_s = omx.quantize(rng.normal(size=(16, 256)))
    want = omx.forward(a, a_s, b, b_s)
    y = tr.mxfp8(*[torch.from_numpy(np.ascontiguousarray(t)) for t in (a, a_s, b, b_s)])
    assert y.dtype == torch.float16
    assert _rel(y.float(), torch.from_numpy(want)) <= 1e-3


def test_qmoe_matches_dense_oracle():
    rng = np.random.default_rng(4)
    T, D, E, N = 6, 256, 4, 32
    x = rng.normal(size=(T, D)).astype(np.float32)
    q = rng.integers(-8, 8, (E, D, N)).astype(np.int8)
    s = (rng.normal(size=(E, D // 128, N)) * 0.01).astype(np.float32)
    lg = rng.normal(size=(T, E)).astype(np.float32)
    y = tr.qmoe(*[torch.from_numpy(t) for t in (x, q, s, lg)])
    assert _rel(y, torch.from_numpy(oq.qmoe_dense_forward(x, q, s, lg))) <= 1e-5


def test_qmoe_ffn_ground_truth():
    g = _g("qmoe_ffn")
    keys = ["x", "logits", "gq", "gs", "gz", "uq", "us", "uz", "dq", "ds", "dz"]
    y = tr.qmoe_ffn(*[g[k] for k in keys])
    assert _rel(y, g["y_gt"]) <= 1e-5


def test_silu_fp8_bit_exact():
    g = _g("silu_fp8")
    y = tr.silu_fp8(g["y_f16"].half())
    assert torch.equal(y, g["out_f16"])
