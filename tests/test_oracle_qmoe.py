"""CPU checks that pin oracle/qmoe.py."""
import numpy as np
import torch

from oracle import qmoe as oq


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


def test_silu_closed_form():
    v = np.array([-3.0, 0.0, 1.0, 5.0], np.float32)
    assert np.allclose(oq.silu(v), v / (1 + np.exp(-v)))
    assert oq.silu(np.array([0.0]))[0] == 0.0
