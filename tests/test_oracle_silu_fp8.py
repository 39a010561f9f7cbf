"""CPU checks of the fused SiLU + per-group FP8 quantisation oracle (oracle/silu_fp8.py).

Pinned by: golden vectors written by torch's CPU ops running the reference sequence
(tests/golden/silu_fp8.npz), closed forms (silu(x) = x for x >= 17; power-of-two scales make
act / scale exact, so hand-computed RNE codes on and between e4m3 grid points are fixed), and
invariants (the group's absmax element quantises to +-448; the quantisation error is at most half
an e4m3 step)."""
import os

import numpy as np
import pytest

from oracle import silu_fp8 as o
from oracle.numerics import e4m3fn_encode_rne

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "silu_fp8.npz")


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_quantize_matches_torch_golden_bit_for_bit(dt):
    d = np.load(GOLD)
    out, codes, scales = o.quantize(d[f"act_{dt}"])
    assert np.array_equal(codes, d[f"codes_{dt}"])
    assert np.array_equal(scales, d[f"scales_{dt}"])
    assert np.array_equal(out, d[f"out_{dt}"])


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_silu_mul_within_a_few_ulp_of_torch(dt):
    d = np.load(GOLD)
    y = d[f"y_{dt}"]
    H = y.shape[1] // 2
    act = o.silu_mul(y[:, :H], y[:, H:])
    ulp = np.abs(act.view(np.int32).astype(np.int64) - d[f"act_{dt}"].view(np.int32).astype(np.int64))
    assert ulp.max() <= 4
    _, codes, _ = o.forward(y)
    assert (codes == d[f"codes_{dt}"]).mean() >= 0.99


def test_zero_row_scale_clamps():
    out, codes, scales = o.quantize(np.zeros((2, 256), np.float32))
    assert np.all(scales == np.float32(1e-12)) and np.all(codes == 0) and np.all(out == 0)


def test_large_gate_silu_is_identity():
    g = np.float16([17.0, 20.0, 64.0, 1000.0, 65504.0]).astype(np.float32)
    u = np.float16([1.5, -3.0, 0.125, 7.0, -1.0]).astype(np.float32)
    assert np.array_equal(o.silu_mul(g, u), g * u)
    # small and negative gates: the closed form x / (1 + e^-x) in float64
    x = np.linspace(-20, 20, 81).astype(np.float32)
    ref = x.astype(np.float64) / (1 + np.exp(-x.astype(np.float64)))
    assert np.allclose(o.silu_mul(x, np.ones_like(x)), ref, rtol=1e-6, atol=1e-30)


def test_absmax_element_maps_to_448_and_sign():
    rng = np.random.default_rng(3)
    a = rng.standard_normal((8, 512)).astype(np.float32) * np.float32(3.7)
    a[0, 5] = -50.0                           # negative absmax: an absmax without |.| fails
    _, codes, _ = o.quantize(a)
    grp = np.abs(a).reshape(8, 4, 128).argmax(-1)
    for t in range(8):
        for gi in range(4):
            c = codes[t, gi * 128 + grp[t, gi]]
            assert c & 0x7F == 0x7E
    assert codes[0, 5] == 0xFE


def test_power_of_two_scale_ties_round_to_even():
    # amax = 448 -> scale = 1 exactly, so act / scale = act and the codes are the e4m3 RNE of act
    vals = {1.0: 0x38, 1.0625: 0x38, 1.125: 0x39, 1.1875: 0x3A, 1.3125: 0x3A, 2.0 ** -10: 0x00,
            3 * 2.0 ** -10: 0x02, 2.0 ** -9: 0x01, 240.0: 0x77, 248.0: 0x78, 416.0: 0x7D,
            432.0: 0x7E, -1.0625: 0xB8, -3 * 2.0 ** -10: 0x82}
    a = np.zeros((1, 128), np.float32)
    a[0, 0] = 448.0
    for i, v in enumerate(vals):
        a[0, i + 1] = v
    _, codes, scales = o.quantize(a)
    assert scales[0, 0] == 1.0
    got = [int(codes[0, i + 1]) for i in range(len(vals))]
    assert got == list(vals.values())
    assert codes[0, 0] == 0x7E


def test_error_within_half_step_and_nan_group():
    rng = np.random.default_rng(5)
    a = (rng.standard_normal((4, 256)) * np.exp(rng.uniform(-8, 8, (4, 1)))).astype(np.float32)
    out, codes, scales = o.quantize(a)
    s = np.repeat(scales, 128, axis=1)
    bound = np.abs(a) * 2.0 ** -4 + s * 2.0 ** -10
    assert np.all(np.abs(out - a) <= bound * (1 + 1e-6))
    # the RNE encoder is the checked library routine: the codes are its image of act / scale
    assert np.array_equal(codes, e4m3fn_encode_rne((a / s).astype(np.float32)))
    a[2, 130] = np.nan
    out, codes, scales = o.quantize(a)
    assert np.isnan(scales[2, 1]) and np.all(np.isnan(out[2, 128:]))
    assert np.all(codes[2, 128:] & 0x7F == 0x7F)
    assert np.all(np.isfinite(out[2, :128])) and np.all(np.isfinite(out[:2]))
