"""CPU checks of the multi-LoRA quantized linear oracle (oracle/lora.py).

Pinned by golden vectors (tests/golden/lora.npz: torch's CPU ops running the reference sequence
in fp16 and on fp32-upcast inputs), brute-force per-token loops, and closed forms: with zero
adapters y is the base GEMM alone, with one-hot x every stage selects a row (exact values)."""
import os

import numpy as np

from oracle import lora as ol
from oracle.numerics import round_to

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "lora.npz")


def _args(d):
    return [d[k] for k in ("x", "qweight", "scales", "A", "B", "lora_ids")]


def test_matches_torch_golden():
    d = np.load(GOLD)
    assert np.array_equal(ol.forward(*_args(d), dtype="f16"), d["y_f16"])
    np.testing.assert_allclose(ol.forward(*_args(d)), d["y_gt"], rtol=0, atol=2e-6)


def test_brute_force_loops_and_closed_forms():
    rng = np.random.default_rng(1)
    T, D, N, r, L = 4, 256, 8, 4, 3
    x = rng.standard_normal((T, D)).astype(np.float32)
    q = rng.integers(-8, 8, (D, N)).astype(np.int8)
    s = (rng.standard_normal((D // 128, N)) * 0.01).astype(np.float32)
    A = (rng.standard_normal((L, D, r)) * 0.02).astype(np.float32)
    B = (rng.standard_normal((L, r, N)) * 0.02).astype(np.float32)
    ids = np.array([2, 0, 2, 1])
    y = ol.forward(x, q, s, A, B, ids)
    for t in range(T):
        for n in range(N):
            base = sum(float(x[t, d]) * float(q[d, n]) * float(s[d // 128, n]) for d in range(D))
            lo = [sum(float(x[t, d]) * float(A[ids[t], d, j]) for d in range(D)) for j in range(r)]
            e = sum(lo[j] * float(B[ids[t], j, n]) for j in range(r))
            assert abs(y[t, n] - (base + e)) <= 1e-5 * (1 + abs(base + e))
    # zero adapters: the base GEMM alone
    y0 = ol.forward(x, q, s, A * 0, B, ids)
    np.testing.assert_allclose(y0, x.astype(np.float64) @ (q * np.repeat(s, 128, 0)), rtol=1e-5, atol=1e-6)
    # one-hot x in fp16: base = W row (one rounding of q s), lo = A row, exact
    xo = np.zeros((T, D), np.float32)
    ks = np.array([3, 100, 200, 255])
    xo[np.arange(T), ks] = 1.0
    s16, A16, B16 = round_to(s, "f16"), round_to(A, "f16"), round_to(B, "f16")
    y = ol.forward(xo, q, s16, A16, B16, ids, dtype="f16")
    W = round_to(q * np.repeat(s16, 128, 0), "f16")
    e = round_to(np.einsum("tr,trn->tn", A16[ids, ks].astype(np.float64), B16[ids]).astype(np.float32), "f16")
    assert np.array_equal(y, round_to(W[ks] + e, "f16"))
