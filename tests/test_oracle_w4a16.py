"""CPU checks that pin oracle/w4a16.py: unpack KATs, pack/unpack inverse, brute-force dequant,
and agreement with the reference's op sequence executed by torch on the CPU (library routines:
int32 shift/mask, fp16 RNE multiply, matmul)."""
import numpy as np
import torch

from oracle import w4a16 as ow
from oracle.numerics import round_to


def test_unpack_kats():
    q = np.array([[0x76543210, np.int32(-19088744), np.int32(-2**31)]], dtype=np.int32)
    w = ow.unpack_int4_along_n(q)
    assert w[0, :8].tolist() == list(range(8))            # 0x76543210
    assert w[0, 8:16].tolist() == list(range(8, 16))      # 0xFEDCBA98 (negative int32)
    assert w[0, 16:24].tolist() == [0] * 7 + [8]          # 0x80000000: nibble 7 = 8


def test_pack_unpack_inverse():
    rng = np.random.default_rng(0)
    nib = rng.integers(0, 16, (33, 64))
    assert np.array_equal(ow.unpack_int4_along_n(ow.pack_int4_along_n(nib)), nib)


def test_dequant_brute_force():
    rng = np.random.default_rng(1)
    K, N, G = 8, 16, 4
    nib = rng.integers(0, 16, (K, N))
    q = ow.pack_int4_along_n(nib)
    s = rng.normal(0, 0.01, (K // G, N)).astype(np.float16).astype(np.float32)
    z = rng.integers(0, 16, (K // G, N)).astype(np.float32)
    W = ow.dequant(q, s, z, "f16")
    for k in range(K):
        for n in range(N):
            want = np.float16(np.float16(nib[k, n] - z[k // G, n]) * np.float16(s[k // G, n]))
            assert W[k, n] == np.float32(want)


def _torch_reference(x, qweight, scales, zeros, G):
    """The reference module's op sequence (reference.py:11-17) run by torch on the CPU."""
    K = qweight.shape[0]
    N = qweight.shape[1] * 8
    shifts = torch.arange(0, 32, 4, dtype=torch.int32)
    w = ((qweight.unsqueeze(-1) >> shifts) & 0xF).reshape(K, N).to(x.dtype)
    g = K // G
    se = scales.reshape(g, 1, N).expand(g, G, N).reshape(K, N).to(x.dtype)
    ze = zeros.reshape(g, 1, N).expand(g, G, N).reshape(K, N).to(x.dtype)
    return (w - ze) * se, torch.matmul(x.float(), ((w - ze) * se).float())


def test_oracle_matches_torch_op_sequence():
    g = torch.Generator().manual_seed(3)
    M, K, N, G = 3, 256, 64, 64
    x = torch.randn(M, K, generator=g).half()
    q = torch.randint(-2**31, 2**31, (K, N // 8), generator=g, dtype=torch.int64).to(torch.int32)
    s = (torch.randn(K // G, N, generator=g) * 0.01).half()
    z = torch.randint(0, 16, (K // G, N), generator=g).half()
    W_t, _ = _torch_reference(x, q, s, z, G)
    W_o = ow.dequant(q.numpy(), s.float().numpy(), z.float().numpy(), "f16")
    assert np.array_equal(W_t.float().numpy(), W_o)
    y_gt = ow.forward(x.float().numpy(), q.numpy(), s.float().numpy(), z.float().numpy())
    _, y_t = _torch_reference(x.float(), q, s.float(), z.float(), G)
    assert np.allclose(y_gt, y_t.numpy(), rtol=1e-5, atol=1e-5)


def test_one_hot_selects_rows():
    rng = np.random.default_rng(2)
    K, N = 128, 32
    nib = rng.integers(0, 16, (K, N))
    q = ow.pack_int4_along_n(nib)
    s = np.ones((1, N), np.float32)
    z = np.zeros((1, N), np.float32)
    x = np.zeros((2, K), np.float32)
    x[0, 5] = 1
    x[1, 77] = 1
    y = ow.forward(x, q, s, z)
    assert np.array_equal(y, nib[[5, 77]].astype(np.float32))


def test_native_dtype_rounds_once():
    W = ow.dequant(ow.pack_int4_along_n(np.full((4, 8), 15)), np.full((1, 8), 0.1, np.float32),
                   np.zeros((1, 8), np.float32), "bf16")
    assert np.array_equal(W, round_to(np.full((4, 8), 1.5, np.float32), "bf16"))
