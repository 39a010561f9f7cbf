"""The oracle's restatement of torch.topk on the GPU (oracle/topk.py), pinned on ids recorded on
the device: tests/golden/topk_device.npz (make_topk_device_golden.py; tie-heavy integer logits
and unfiltered fp16/bf16 N(0,1) draws for every (experts, k) of the reference's routing tasks)
and crafted rows whose device ids were printed on an MI355X with torch 2.10.0+rocm7.0."""
import re

import numpy as np
import pytest

from oracle import moe as om
from oracle import qmoe as oq
from oracle.qmoe import softmax_fp32
from oracle.topk import device_topk_ids

GOLD = np.load(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden",
                                           "topk_device.npz"))
CASES = sorted(k[:-7] for k in GOLD.files if k.endswith("_logits"))


@pytest.mark.parametrize("case", CASES)
def test_device_ids(case):
    k = int(re.search(r"_k(\d+)_", case).group(1))
    lg = GOLD[case + "_logits"]
    want = GOLD[case + "_ids"].astype(np.int64)
    assert np.array_equal(device_topk_ids(softmax_fp32(lg), k), want)
    if k == 2:
        assert np.array_equal(oq.route_top2(lg)[0], want)
    assert np.array_equal(om.route_topk(lg, k)[0], want)


# Rows of 8 logits and the ids torch.topk(softmax(logits), 2) returned on the device.
CRAFTED = [
    ([1, 1, 0, 0, 0, 0, 0, 0], [1, 0]), ([0, 0, 0, 0, 0, 0, 1, 1], [7, 6]),
    ([2, 1, 1, 0, 0, 0, 0, 0], [0, 1]), ([0, 1, 1, 2, 0, 0, 0, 0], [3, 1]),
    ([0, 0, 0, 0, 0, 0, 0, 1], [7, 0]), ([1, 0, 0, 0, 0, 0, 0, 0], [0, 1]),
    ([0, 0, 0, 0, 0, 0, 0, 0], [1, 0]), ([0, 0, 5, 0, 5, 0, 5, 0], [4, 2]),
    ([3, 0, 0, 0, 0, 0, 0, 3], [7, 0]), ([0, 2, 0, 2, 0, 2, 0, 9], [7, 1]),
]


def test_crafted_device_rows():
    lg = np.array([r for r, _ in CRAFTED], np.float32)
    assert device_topk_ids(softmax_fp32(lg), 2).tolist() == [w for _, w in CRAFTED]


def test_distinct_values_sort_descending():
    """Without ties the device order is the plain descending order."""
    rng = np.random.default_rng(3)
    v = rng.permutation(np.arange(64 * 50, dtype=np.float32)).reshape(50, 64)
    for k in (1, 2, 3, 6, 8, 17, 32):
        assert np.array_equal(device_topk_ids(v, k), np.argsort(-v, axis=1)[:, :k])


def test_boundary_ties_take_lowest_indices():
    """The selected set: every value above the k-th largest, then its ties lowest index first."""
    rng = np.random.default_rng(4)
    v = rng.integers(-2, 3, (400, 16)).astype(np.float32)
    for k in (2, 5, 8):
        ids = device_topk_ids(v, k)
        kth = -np.sort(-v, axis=1)[:, k - 1:k]
        for t in range(len(v)):
            above = set(np.nonzero(v[t] > kth[t])[0])
            ties = list(np.nonzero(v[t] == kth[t])[0])[:k - len(above)]
            assert set(ids[t]) == above | set(ties)
