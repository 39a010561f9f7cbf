"""CPU checks that pin oracle/fp8w.py."""
import numpy as np
import torch

from oracle import fp8w as of


def test_block_index_is_k_div_block():
    """Scale row k // B (the reference), not k // 32: one-hot scale rows expose the index."""
    K, N, B = 256, 8, 128
    codes = np.full((K, N), 0x38, np.uint8)          # all 1.0
    s = np.zeros((K // B, N), np.float32)
    s[1] = 2.0                                       # rows 128..255 scaled by 2
    W = of.dequant(codes, s, "f32")
    assert (W[:128] == 0).all() and (W[128:] == 2).all()


def test_dequant_matches_torch_reference_sequence():
    g = torch.Generator().manual_seed(0)
    K, N, B = 256, 64, 32
    w = (torch.randn(K, N, generator=g) * 0.3).to(torch.float8_e4m3fn)
    s = (torch.rand(K // B, N, generator=g) * 0.05 + 0.05).to(torch.float16)
    ref = (w.float().reshape(K // B, B, N) * s[:, None, :].float()).reshape(K, N).to(torch.float16)
    got = of.dequant(w.view(torch.uint8).numpy(), s.float().numpy(), "f16")
    assert np.array_equal(got, ref.float().numpy())


def test_forward_brute_force():
    rng = np.random.default_rng(1)
    K, N, B = 64, 4, 32
    codes = rng.integers(0, 0x7E, (K, N)).astype(np.uint8)
    s = rng.uniform(0.05, 0.1, (K // B, N)).astype(np.float16).astype(np.float32)
    x = rng.normal(size=(2, K)).astype(np.float32)
    from oracle.numerics import e4m3fn_decode
    want = np.zeros((2, N))
    for m in range(2):
        for n in range(N):
            want[m, n] = sum(float(x[m, k]) * float(e4m3fn_decode(codes[k, n])) * float(s[k // B, n]) for k in range(K))
    assert np.allclose(of.forward(x, codes, s), want, rtol=1e-5, atol=1e-5)
