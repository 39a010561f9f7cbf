"""CPU checks that pin oracle/qmoe.py."""
import math
import os

import numpy as np
import pytest
import torch

from oracle import qmoe as oq

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_top2_closed_form():
    """Top-2 of softmax = top-2 of logits; w1 = 1 / (1 + exp(l2 - l1))."""
    rng = np.random.default_rng(0)
    l = rng.normal(size=(64, 8)).astype(np.float32)
    topi, w = oq.route_top2(l)
    srt = np.argsort(-l, axis=-1)[:, :2]
    assert np.array_equal(topi, srt)
    l1 = l[np.arange(64), srt[:, 0]]
    l2 = l[np.arange(64), srt[:, 1]]
    assert np.allclose(w[:, 0], 1 / (1 + np.exp(l2 - l1)), rtol=1e-6)
    assert np.allclose(w.sum(axis=1), 1, rtol=1e-6)


def test_routing_matches_torch_reference_sequence():
    g = torch.Generator().manual_seed(1)
    lg = torch.randn(100, 8, generator=g).half()
    probs = torch.softmax(lg.float(), dim=-1)
    topv, topi = probs.topk(2, dim=-1)
    topv = (topv / topv.sum(dim=-1, keepdim=True)).half()
    oi, ow = oq.route_top2(lg.float().numpy(), "f16")
    assert np.array_equal(oi, topi.numpy())
    assert np.array_equal(ow, topv.float().numpy())


def test_sparse_equals_dense_reference_formulation():
    rng = np.random.default_rng(2)
    T, D, E, N = 6, 256, 4, 16
    x = rng.normal(size=(T, D)).astype(np.float32)
    q = rng.integers(-8, 8, (E, D, N)).astype(np.int8)
    s = (rng.normal(size=(E, D // 128, N)) * 0.01).astype(np.float32)
    lg = rng.normal(size=(T, E)).astype(np.float32)
    assert np.allclose(oq.qmoe_forward(x, q, s, lg), oq.qmoe_dense_forward(x, q, s, lg),
                       rtol=1e-5, atol=1e-6)


def test_native_dtype_path_matches_torch_sequence():
    """The fp16 path (dequant, einsum, gather, weighted sum) against torch on the CPU."""
    g = torch.Generator().manual_seed(3)
    T, D, E, N = 5, 256, 4, 32
    x = torch.randn(T, D, generator=g).half()
    q = torch.randint(-8, 8, (E, D, N), generator=g, dtype=torch.int8)
    s = (torch.randn(E, D // 128, N, generator=g) * 0.01).half()
    lg = torch.randn(T, E, generator=g).half()
    probs = torch.softmax(lg.float(), dim=-1)
    topv, topi = probs.topk(2, dim=-1)
    topv = (topv / topv.sum(dim=-1, keepdim=True)).half()
    w = (q.reshape(E, 2, 128, N).half() * s[:, :, None, :].half()).reshape(E, D, N)
    all_out = torch.einsum("td,edn->ten", x.float(), w.float()).half()   # fp32 accumulate
    sel = torch.gather(all_out, 1, topi.unsqueeze(-1).expand(-1, -1, N))
    ref = (sel * topv.unsqueeze(-1)).sum(dim=1)
    got = oq.qmoe_forward(x.float().numpy(), q.numpy(), s.float().numpy(), lg.float().numpy(), "f16")
    assert np.allclose(got, ref.float().numpy(), rtol=2e-3, atol=2e-3)


def test_silu_matches_torch():
    """oracle silu against torch.nn.functional.silu (the library routine generate_tasks.py:337
    calls) over a dense grid, including the saturated ends (silu(v) = v for v >= 17 in fp32,
    silu(v) -> -0 for very negative v)."""
    v = np.concatenate([np.linspace(-40, 40, 20001), [0.0, 17.0, 100.0, -100.0]]).astype(np.float32)
    want = torch.nn.functional.silu(torch.from_numpy(v)).numpy()
    with np.errstate(over="ignore"):
        got = oq.silu(v)
    assert np.allclose(got, want, rtol=2e-6, atol=1e-30)
    assert got[-3] == 17.0 and got[-2] == 100.0 and got[20001] == 0.0


def _gold(name):
    with np.load(os.path.join(GOLD, f"{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


FFN_ARGS = ["x", "logits", "gq", "gs", "gz", "uq", "us", "uz", "dq", "ds", "dz"]


def test_ffn_golden_ground_truth():
    """ffn_forward (fp32 ground truth) against torch's per-token loop (tests/golden)."""
    g = _gold("qmoe_ffn")
    y = oq.ffn_forward(*[g[k] for k in FFN_ARGS])
    assert np.abs(y - g["y_gt"]).max() <= 1e-5 * np.abs(g["y_gt"]).max()


def test_ffn_golden_native_fp16():
    """The fp16 path (h, expert outputs and combine rounded to fp16) against the same torch loop
    in fp16: nearly all elements bit-identical and the rest within a few fp16 ulps (the two
    fp32 accumulation orders may round a near-tie of h differently, which the down projection
    carries on; where the combine cancels to ~0 the bound is relative to the output's scale)."""
    g = _gold("qmoe_ffn")
    y = oq.ffn_forward(*[g[k] for k in FFN_ARGS], dtype="f16")
    want = g["y_f16"]
    ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float32)
    tol = np.maximum(4 * ulp, 2.0 ** -11 * np.abs(want).max())   # near-zero sums cancel
    assert (np.abs(y - want) <= tol).all()
    assert (y == want).mean() >= 0.95


def _nib(q, k, n):
    return ((int(q[k, n // 8]) & 0xFFFFFFFF) >> (4 * (n % 8))) & 0xF


def _w(q, s, z, k, n, G):
    return (_nib(q, k, n) - float(z[k // G, n])) * float(s[k // G, n])


def test_ffn_brute_force_loops():
    """Float64 per-token loops written from the definition (softmax, top-2 by sorting,
    renormalisation, nibble n%8 of word n//8, (q - z[k//G]) * s[k//G], silu(gate) * up, down,
    weighted sum) against the fp32 ground-truth path; 32-row groups so every matrix spans
    several groups."""
    rng = np.random.default_rng(11)
    T, D, F, E, G = 4, 64, 32, 3, 32
    x = rng.normal(size=(T, D)).astype(np.float32)
    lg = rng.normal(size=(T, E)).astype(np.float32)

    def w4(K, N):
        q = rng.integers(-2 ** 31, 2 ** 31, (E, K, N // 8), dtype=np.int64).astype(np.int32)
        s = rng.uniform(0.002, 0.02, (E, K // G, N)).astype(np.float32)
        z = rng.integers(0, 16, (E, K // G, N)).astype(np.float32)
        return q, s, z
    gq, gs, gz = w4(D, F)
    uq, us, uz = w4(D, F)
    dq, ds, dz = w4(F, D)
    got = oq.ffn_forward(x, lg, gq, gs, gz, uq, us, uz, dq, ds, dz)
    want = np.zeros((T, D))
    for t in range(T):
        ex = [math.exp(float(v)) for v in lg[t]]
        p = [v / sum(ex) for v in ex]
        top = sorted(range(E), key=lambda e: -p[e])[:2]
        for e in top:
            wk = p[e] / (p[top[0]] + p[top[1]])
            h = []
            for f in range(F):
                gate = sum(float(x[t, d]) * _w(gq[e], gs[e], gz[e], d, f, G) for d in range(D))
                up = sum(float(x[t, d]) * _w(uq[e], us[e], uz[e], d, f, G) for d in range(D))
                h.append(gate / (1.0 + math.exp(-gate)) * up)
            for c in range(D):
                want[t, c] += wk * sum(h[f] * _w(dq[e], ds[e], dz[e], f, c, G) for f in range(F))
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


def _closed_form_case(rng, T=6, D=128, F=64, E=4, G=64):
    """One-hot x (row t selects input channel d_t); up weights of those channels dequantise to
    exactly 1 and the down matrix is zero except row f0 = 3. Then gate = Wg_e[d_t, :],
    h = silu(gate) and every output column of expert e is 3 * h[f0]."""
    ks = rng.choice(D, T, replace=False)
    x = np.zeros((T, D), np.float32)
    x[np.arange(T), ks] = 1.0
    lg = rng.normal(size=(T, E)).astype(np.float32)
    gq = rng.integers(-2 ** 31, 2 ** 31, (E, D, F // 8), dtype=np.int64).astype(np.int32)
    gs = rng.uniform(0.05, 0.5, (E, D // G, F)).astype(np.float16).astype(np.float32)
    gz = rng.integers(0, 16, (E, D // G, F)).astype(np.float32)
    one = np.int32(0x11111111)                        # every nibble 1
    uq = np.full((E, D, F // 8), one, np.int32)
    us = np.ones((E, D // G, F), np.float32)
    uz = np.zeros((E, D // G, F), np.float32)
    f0 = 5
    dq = np.zeros((E, F, D // 8), np.int32)
    dq[:, f0, :] = np.int32(0x33333333)               # row f0: nibble 3, others 0
    ds = np.ones((E, F // G if F >= G else 1, D), np.float32)
    dz = np.zeros_like(ds)
    return ks, f0, [x, lg, gq, gs, gz, uq, us, uz, dq, ds, dz]


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_ffn_closed_form_gated_product(dtype):
    """With up == 1 the FFN output is the combine of 3 * silu(Wg_e[d_t, f0]) over the two routed
    experts. The expected values come from torch (dequantised gate row, F.silu, fp16 casts of
    h and of the expert output in the fp16 case): bit-exact in fp16, within fp32 rounding of
    the two silu implementations in fp32. Swapping the gate and up operands in the call
    (silu(1) * gate instead of silu(gate) * 1) must break the identity."""
    import torch.nn.functional as Fn
    rng = np.random.default_rng(21)
    ks, f0, args = _closed_form_case(rng)
    x, lg, gq, gs, gz = args[:5]
    topi, w = oq.route_top2(lg, dtype)
    tdt = torch.float32 if dtype == "f32" else torch.float16
    want = []
    for t, k in enumerate(ks):
        outs = []
        for j in range(2):
            e = int(topi[t, j])
            nib = (int(gq[e, k, f0 // 8]) & 0xFFFFFFFF) >> (4 * (f0 % 8)) & 0xF
            gv = torch.tensor((nib - gz[e, k // 64, f0]) * gs[e, k // 64, f0]).to(tdt)
            h = Fn.silu(gv.float()).to(tdt)
            o = (h.float() * 3.0).to(tdt)
            outs.append((o * torch.tensor(w[t, j]).to(tdt)).float())
        want.append(float((outs[0] + outs[1]).to(tdt)))
    y = oq.ffn_forward(*args, dtype=dtype)
    want = np.array(want, np.float32)[:, None]
    if dtype == "f16":
        assert np.array_equal(y, np.broadcast_to(want, y.shape)), np.abs(y - want).max()
    else:
        assert np.abs(y - want).max() <= 4e-7 * np.abs(want).max()
    swapped = oq.ffn_forward(x, lg, *args[5:8], *args[2:5], *args[8:], dtype=dtype)
    assert np.abs(swapped - want).max() > 1e-3 * np.abs(want).max()
