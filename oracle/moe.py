"""Oracle for the top-k MoE with fp16/bf16 expert weights (test infrastructure only).

Reference: tasks/moe/moe_top2__mixtral_8x7b__T16__fp16/environment/reference.py:10-17 (template
generate_tasks.py:162-186; TOPK 2, 6 or 8 per generate_tasks.py:189-195):
  probs = softmax(fp32 logits)                            (:11)
  topv, topi = probs.topk(TOPK)                           (:12; descending)
  topv = dtype(topv / topv.sum())                         (:13)
  all_out = einsum('td,edh->teh', x, w)  in dtype          (:14; fp32 accumulate, one rounding)
  y = (gather(all_out, topi) * topv).sum(dim=1)  in dtype  (:16-17; products rounded to dtype,
                                                            summed in fp32, rounded once)
With dtype F32 every rounding is the identity: the fp32 ground truth of the grader
(common/kb_verifier.py:195-196).
"""
from __future__ import annotations

import numpy as np

from .numerics import F32, round_to
from .qmoe import softmax_fp32
from .topk import device_topk_ids


def route_topk(logits, k: int, dtype: str = F32):
    """:11-13 — ids [T, k] in the order torch.topk returns them on the GPU (oracle/topk.py:
    descending probability; the lower indices win a tie at the boundary, equal selected values
    in the order of torch's bitonic sort) and weights topv / sum(topv) (summed in that order)
    rounded to dtype."""
    p = softmax_fp32(logits)
    T = p.shape[0]
    order = device_topk_ids(p, k)
    topv = p[np.arange(T)[:, None], order].astype(np.float32)
    s = np.zeros((T, 1), np.float32)
    for j in range(k):
        s = (s + topv[:, j:j + 1]).astype(np.float32)
    return order.astype(np.int64), round_to((topv / s).astype(np.float32), dtype)


def forward(x, w, logits, k: int, dtype: str = F32) -> np.ndarray:
    """Sparse restatement: only the selected experts are evaluated (float64 products, one
    rounding to dtype per expert output, as an fp32-accumulating GEMM rounded once)."""
    topi, tw = route_topk(logits, k, dtype)
    xf = np.asarray(x, dtype=np.float64)
    T = xf.shape[0]
    H = w.shape[2]
    acc = np.zeros((T, H), np.float32)
    for j in range(k):
        oj = np.zeros((T, H), np.float32)
        for e in np.unique(topi[:, j]):
            rows = np.nonzero(topi[:, j] == e)[0]
            oj[rows] = round_to((xf[rows] @ np.asarray(w[e], np.float64)).astype(np.float32), dtype)
        acc = (acc + round_to(oj * tw[:, j:j + 1], dtype)).astype(np.float32)
    return round_to(acc, dtype)


def dense_forward(x, w, logits, k: int) -> np.ndarray:
    """Literal fp32 restatement of :14-17 (every expert, einsum, gather) for tiny shapes."""
    topi, tw = route_topk(logits, k, F32)
    all_out = np.einsum("td,edh->teh", np.asarray(x, np.float64), np.asarray(w, np.float64))
    sel = np.take_along_axis(all_out, topi[:, :, None], axis=1)
    return (sel * tw[:, :, None]).sum(axis=1).astype(np.float32)
