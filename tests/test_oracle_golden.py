"""CPU checks of the oracle against the committed golden vectors (tests/golden/*.npz, *.json),
which torch's library routines produced from the reference modules' op sequences."""
import json
import os

import numpy as np
import pytest

from oracle import fp8w as of
from oracle import mxfp8 as omx
from oracle import numerics as nm
from oracle import qmoe as oq
from oracle import w4a16 as ow
from oracle import w8a8 as o8

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    with np.load(os.path.join(GOLD, f"{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _close(y, gt, rtol=1e-5):
    err = np.abs(y.astype(np.float64) - gt.astype(np.float64)).max()
    assert err <= rtol * np.abs(gt).max(), err


def test_e4m3fn_table():
    with open(os.path.join(GOLD, "e4m3fn_table.json")) as f:
        vals = json.load(f)["values"]
    got = nm.e4m3fn_decode_table()
    for c, v in enumerate(vals):
        if v == "nan":
            assert np.isnan(got[c]), c
        else:
            assert got[c] == float.fromhex(v), c


def test_w4a16_golden():
    g = _load("w4a16")
    assert np.array_equal(ow.unpack_int4_along_n(g["qweight"]), g["nib"])
    assert np.array_equal(ow.pack_int4_along_n(g["nib"]), g["qweight"])
    W = ow.dequant(g["qweight"], g["scales"], g["zeros"], "f16")
    assert np.array_equal(W, g["W_f16"].astype(np.float32))        # one RNE, bit-exact
    _close(ow.forward(g["x"], g["qweight"], g["scales"], g["zeros"]), g["y_gt"])


def test_w8a8_golden():
    g = _load("w8a8")
    acc = o8.acc_int32(g["x_int8"], g["w_int8"])
    assert np.array_equal(acc, g["acc"])
    assert acc[0, 0] == 512 * 127 * 127
    out = o8.epilogue(acc, g["x_scale"], g["w_scale"])
    assert np.array_equal(out, g["out"].astype(np.float32))         # same fp32 order, one RNE


def test_fp8w_golden():
    g = _load("fp8w")
    W = of.dequant(g["w_codes"], g["scales"], "f16")
    assert np.array_equal(W, g["W_f16"].astype(np.float32))
    _close(of.forward(g["x"], g["w_codes"], g["scales"]), g["y_gt"])


def test_mxfp8_golden():
    g = _load("mxfp8")
    q, s = omx.quantize(g["src"])
    assert np.array_equal(s, g["scales"])
    assert s[5, 1] == 0
    assert np.array_equal(q, g["codes"])
    assert np.array_equal(omx.dequant(q, s).astype(np.float32), g["deq"])


@pytest.mark.parametrize("dtype", ["f16"])
def test_qmoe_route_golden(dtype):
    g = _load("qmoe_route")
    topi, topw = oq.route_top2(g["logits"], dtype)
    assert np.array_equal(topi, g["topi"])
    assert np.array_equal(topw, g["topw"].astype(np.float32))
