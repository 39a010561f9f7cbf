"""CPU checks that pin oracle/mxfp8.py (closed forms, bounds, torch cross-check)."""
import numpy as np
import torch

from kernelbench_harbor_amd import inputs
from oracle import mxfp8 as om


def test_ceil_log2_kats():
    assert om.ceil_log2([1.0, 2.0, 3.0, 0.5, 0.75, 448.0 / 448.0, 2.0 ** -130]).tolist() == [0, 1, 2, -1, 0, 0, -130]


def test_scale_choice_bounds_quantized_values():
    rng = np.random.default_rng(0)
    x = rng.normal(size=(8, 256)) * rng.uniform(1e-3, 1e3, (8, 1))
    q, s = om.quantize(x)
    scale = np.ldexp(1.0, s.astype(np.int64) - 127)
    blk = np.abs(x.reshape(8, 8, 32)).max(-1)
    assert (blk / scale <= 448).all() and (blk / scale > 224).all()   # smallest power of two
    err = np.abs(om.dequant(q, s) - x).reshape(8, 8, 32).max(-1)
    assert (err <= scale * 16 + 1e-300).all()                         # half an ulp at 2^8 * scale


def test_zero_block_gives_zero_code():
    x = np.zeros((1, 64))
    x[0, 40] = 3.0
    q, s = om.quantize(x)
    assert s[0, 0] == 0 and (q[0, :32] == 0).all() and s[0, 1] == 127 - 7


def test_quantizer_matches_torch_synthesis():
    g = torch.Generator().manual_seed(1)
    src = torch.randn(16, 512, generator=g)
    q_t, s_t = inputs.mx_quantize(src)
    q_o, s_o = om.quantize(src.numpy().astype(np.float64))
    assert np.array_equal(s_t.numpy(), s_o)
    assert np.array_equal(q_t.numpy(), q_o)


def test_forward_power_of_two_kat():
    """A = B = 1.0 codes with chosen block exponents: y = 32 * sum_b 2^(ea_b+eb_b-254)."""
    K = 128
    a = np.full((1, K), 0x38, np.uint8)
    b = np.full((1, K), 0x38, np.uint8)
    ea = np.array([[127, 128, 126, 130]], np.uint8)
    eb = np.array([[127, 127, 129, 120]], np.uint8)
    want = 32 * sum(2.0 ** (int(x) + int(y) - 254) for x, y in zip(ea[0], eb[0]))
    assert om.forward(a, ea, b, eb)[0, 0] == np.float32(want)
