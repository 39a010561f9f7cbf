"""CPU checks of the top-k fp16/bf16 MoE oracle (oracle/moe.py).

Pinned by golden vectors (tests/golden/moe.npz: torch's CPU softmax / topk / einsum / gather /
sum running the reference sequence, top-2 and top-6, native fp16 and fp32 ground truth), the
dense literal restatement against the sparse one, and the closed form of the routing weights
(w_i = e^{l_i} / sum over the selected j of e^{l_j})."""
import os

import numpy as np
import pytest

from oracle import moe as om

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "moe.npz")


@pytest.mark.parametrize("k", [2, 6])
def test_matches_torch_golden(k):
    d = np.load(GOLD)
    ti, tw = om.route_topk(d["logits"], k, "f16")
    assert np.array_equal(ti, d[f"topi_k{k}"])
    assert np.array_equal(tw, d[f"topw_f16_k{k}"])
    y16 = om.forward(d["x"], d["w"], d["logits"], k, "f16")
    assert np.array_equal(y16, d[f"y_f16_k{k}"])          # every rounding as torch's fp16 path
    y = om.forward(d["x"], d["w"], d["logits"], k)
    np.testing.assert_allclose(y, d[f"y_gt_k{k}"], rtol=0, atol=1e-6)


@pytest.mark.parametrize("k", [1, 2, 6, 8])
def test_sparse_equals_dense_and_closed_form_weights(k):
    rng = np.random.default_rng(k)
    T, D, E, H = 9, 32, 12, 8
    x = rng.standard_normal((T, D)).astype(np.float32)
    w = (rng.standard_normal((E, D, H)) * 0.02).astype(np.float32)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    np.testing.assert_allclose(om.forward(x, w, lg, k), om.dense_forward(x, w, lg, k),
                               rtol=1e-5, atol=1e-7)
    ti, tw = om.route_topk(lg, k)
    want_ids = np.argsort(-lg, axis=-1, kind="stable")[:, :k]   # top-k of logits = of probs
    assert np.array_equal(ti, want_ids)
    sel = np.take_along_axis(lg.astype(np.float64), ti, axis=1)
    closed = np.exp(sel - sel[:, :1]) / np.exp(sel - sel[:, :1]).sum(axis=1, keepdims=True)
    np.testing.assert_allclose(tw, closed, rtol=2e-6)
    if k == 1:
        assert np.all(tw == 1.0)


def test_ties_take_the_lower_indices_in_device_order():
    """Ties: the selected set is the lowest indices (torch's gather step), and the order is the
    device's (oracle/topk.py; pinned on GPU-recorded ids in test_oracle_topk.py)."""
    lg = np.array([[0.5, 2.0, 2.0, 1.0, 2.0, 2.0]], np.float32)
    ti, tw = om.route_topk(lg, 3)
    assert sorted(ti[0].tolist()) == [1, 2, 4]
    np.testing.assert_allclose(tw, [[1 / 3, 1 / 3, 1 / 3]], rtol=1e-6)
