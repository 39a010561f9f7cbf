"""Top-k selection and ordering of torch.topk on the GPU (test infrastructure only).

The reference routes with `probs.topk(k, dim=-1)` on the device
(tasks/fused_qmoe/fused_qmoe__mixtral__fp16/environment/reference.py:15,
tasks/moe/moe_top2__mixtral_8x7b__T16__fp16/environment/reference.py:12; the grader's ground
truth runs there too, common/kb_verifier.py:195-196). That routine is torch's (torch 2.5.1 in
the reference's task image, generate_tasks.py:109; not part of the reference tree). For short
rows and k <= 32 it runs two published steps (PyTorch aten/src/ATen/native/cuda TensorTopK /
Sort):
  1. selection: the k-th largest value v_k is found; the output slots are filled first with
     the values > v_k in ascending index order, then with values == v_k in ascending index
     order until k are taken (so the lowest indices win a tie at the boundary);
  2. ordering: an unstable bitonic sort of 32 slots (the k selected entries, then invalid
     padding) into descending order, whose compare-exchange keeps or swaps equal keys
     depending on their slot positions.
For distinct values the result is the plain descending order; with ties it is not the stable
order (e.g. probabilities [a, a, b, ...] with a > b give ids [1, 0]). Pinned by device ids
recorded on the GPU (tests/golden/topk_device.npz, written by make_topk_device_golden.py) and
by crafted rows whose device ids were printed there.
"""
from __future__ import annotations

import numpy as np

SORT_SLOTS = 32


def _select(v, k):
    """Step 1: [T, k] ids in selection (slot) order."""
    T, E = v.shape
    kth = -np.sort(-v, axis=1)[:, k - 1:k]
    gt = v > kth
    eq = v == kth
    need = k - gt.sum(axis=1, keepdims=True)
    eq_take = eq & (np.cumsum(eq, axis=1) <= need)
    grp = np.where(gt, 0, np.where(eq_take, 1, 2))
    # slot order: group 0 (above v_k) then group 1 (ties), each in ascending index
    key = grp * (E + 1) + np.arange(E)[None, :]
    return np.argsort(key, axis=1, kind="stable")[:, :k]


def _bitonic_slots(val, ids, k):
    """Step 2: the 32-slot bitonic network, descending, invalid slots sinking to the end. A
    compare-exchange of slots a < b = a ^ stride swaps when
    ((val[a] > val[b] and a valid) or b invalid) == dir, dir = (a & size) != 0 while building
    and False in the final merge."""
    T = val.shape[0]
    V = np.full((T, SORT_SLOTS), -np.inf, dtype=val.dtype)
    I = np.zeros((T, SORT_SLOTS), dtype=np.int64)
    ok = np.zeros((T, SORT_SLOTS), dtype=bool)
    V[:, :k], I[:, :k], ok[:, :k] = val, ids, True

    def stage(size, stride, final):
        a = np.array([p for p in range(SORT_SLOTS) if not p & stride])
        b = a ^ stride
        d = np.zeros(a.shape, bool) if final else (a & size) != 0
        gtv = (V[:, a] > V[:, b]) | (np.isnan(V[:, a]) & ~np.isnan(V[:, b]))
        sw = ((gtv & ok[:, a]) | ~ok[:, b]) == d[None, :]
        for arr in (V, I, ok):
            xa, xb = arr[:, a].copy(), arr[:, b].copy()
            arr[:, a] = np.where(sw, xb, xa)
            arr[:, b] = np.where(sw, xa, xb)

    size = 2
    while size < SORT_SLOTS:
        stride = size // 2
        while stride:
            stage(size, stride, False)
            stride //= 2
        size *= 2
    stride = SORT_SLOTS // 2
    while stride:
        stage(SORT_SLOTS, stride, True)
        stride //= 2
    return I[:, :k]


def device_topk_ids(values, k: int) -> np.ndarray:
    """ids [T, k] that torch.topk(values, k, dim=-1) returns on the GPU, for rows of any length
    and 1 <= k <= 32."""
    v = np.asarray(values)
    assert 1 <= k <= min(SORT_SLOTS, v.shape[1])
    ids = _select(v, k)
    if k == 1:
        return ids.astype(np.int64)
    return _bitonic_slots(np.take_along_axis(v, ids, axis=1), ids, k)
