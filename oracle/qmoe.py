"""Oracle for the top-2 quantized MoE ops (test infrastructure only).

Reference: tasks/fused_qmoe/fused_qmoe__mixtral__fp16/environment/reference.py:11-21 (template
generate_tasks.py:358-387). The SiLU FFN follows the same routing and combine with W4A16
experts (oracle/w4a16.py) and SiLU(gate) * up as in generate_tasks.py:337 and
validate/measure_pass1.py:432-437.
"""
from __future__ import annotations

import numpy as np

from . import w4a16
from .numerics import F32, round_to
from .topk import device_topk_ids


def softmax_fp32(logits) -> np.ndarray:
    """reference.py:14: torch.softmax(router_logits.float(), dim=-1)."""
    l = np.asarray(logits, dtype=np.float32)
    e = np.exp(l - l.max(axis=-1, keepdims=True))
    return (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)


def route_top2(logits, dtype: str = F32):
    """reference.py:14-16: probabilities, top-2 in the order torch.topk returns them on the GPU
    (oracle/topk.py: the lower indices win a tie at the boundary; two equal selected values come
    out higher index first), weights topv / sum(topv) rounded to the activation dtype."""
    p = softmax_fp32(logits)
    T = p.shape[0]
    order = device_topk_ids(p, 2)
    topv = p[np.arange(T)[:, None], order]
    w = (topv / topv.sum(axis=-1, keepdims=True)).astype(np.float32)
    return order.astype(np.int64), round_to(w, dtype)


def dequant_expert(q, s, dtype: str) -> np.ndarray:
    """reference.py:18: (qweight.reshape(E,G,GROUP,N).to(dtype) * scales[:,:,None,:].to(dtype))
    for one expert: one rounding of the exact product."""
    q = np.asarray(q, dtype=np.float32)
    s = np.asarray(s, dtype=np.float32)
    G = q.shape[0] // s.shape[0]
    return round_to(q * np.repeat(s, G, axis=0), dtype)


def combine(out_k, w, dtype: str):
    """reference.py:20-21: (sel * topv).sum(dim=1) in the activation dtype: each product
    rounded to dtype, the two summed in fp32 and rounded."""
    p = [round_to(out_k[k] * w[:, k:k + 1], dtype) for k in range(2)]
    return round_to(p[0] + p[1], dtype)


def qmoe_forward(x, qweight, scales, logits, dtype: str = F32) -> np.ndarray:
    """Sparse restatement of reference.py:17-21: only the selected experts are evaluated (the
    reference evaluates all of them and gathers; tests check the two agree)."""
    topi, w = route_top2(logits, dtype)
    xf = round_to(np.asarray(x, dtype=np.float32), dtype)
    T = xf.shape[0]
    N = qweight.shape[2]
    out_k = [np.zeros((T, N), np.float32), np.zeros((T, N), np.float32)]
    for e in np.unique(topi):
        W = dequant_expert(qweight[e], scales[e], dtype)
        for k in range(2):
            rows = np.nonzero(topi[:, k] == e)[0]
            if rows.size:
                out_k[k][rows] = round_to(xf[rows] @ W, dtype)
    return combine(out_k, w, dtype)


def qmoe_dense_forward(x, qweight, scales, logits) -> np.ndarray:
    """Literal fp32 restatement of reference.py:17-21 (all experts, einsum, gather) for tiny
    shapes."""
    topi, w = route_top2(logits, F32)
    E = qweight.shape[0]
    W = np.stack([dequant_expert(qweight[e], scales[e], F32) for e in range(E)])
    all_out = np.einsum("td,edn->ten", np.asarray(x, np.float32), W)
    sel = np.take_along_axis(all_out, topi[:, :, None], axis=1)
    return (sel * w[:, :, None]).sum(axis=1).astype(np.float32)


def silu(v):
    """SiLU in fp32, v / (1 + e^-v) (torch.nn.functional.silu, generate_tasks.py:337)."""
    v = np.asarray(v, dtype=np.float32)
    return (v / (1.0 + np.exp(-v))).astype(np.float32)


def ffn_forward(x, logits, gq, gs, gz, uq, us, uz, dq, ds, dz, dtype: str = F32) -> np.ndarray:
    """y[t] = sum_k w_k * down_e(silu(gate_e x_t) * up_e x_t) with W4A16 experts, e = topi[t, k].

    Routing and combine: reference.py:14-16, 20-21 (fused_qmoe). Expert weights: the W4A16
    dequantisation of tasks/quant_w4a16_pa/<task>/environment/reference.py:12-17 (oracle/w4a16.py).
    The gated product: `F.silu(gate.float()) * up.float()` (generate_tasks.py:337). dtype F32 is the
    ground truth (every floating input upcast, all math in fp32). The FFN has no reference
    module, so its 16-bit path is the fused one the GPU computes: the dequantised weights are
    rounded to dtype, gate and up stay fp32 (accumulators) and h = dtype(silu(gate) * up) is
    rounded once, then each expert output dtype(h @ Wd) and the combine round as
    qmoe_forward's. (validate/measure_pass1.py:432-437 also rounds each x @ W to dtype before the
    SiLU; in bf16 those two extra roundings alone exceed the 5e-3 Frobenius gate.) Down weights
    may be a column slice of D (packed words [:, :, c0/8:c1/8] with the matching scale/zero
    columns); the result then holds those columns."""
    topi, w = route_top2(logits, dtype)
    xf = round_to(np.asarray(x, dtype=np.float32), dtype)
    T = xf.shape[0]
    D = dq.shape[2] * 8
    out_k = [np.zeros((T, D), np.float32), np.zeros((T, D), np.float32)]
    for e in np.unique(topi):
        Wg = w4a16.dequant(gq[e], gs[e], gz[e], dtype)
        Wu = w4a16.dequant(uq[e], us[e], uz[e], dtype)
        Wd = w4a16.dequant(dq[e], ds[e], dz[e], dtype)
        for k in range(2):
            rows = np.nonzero(topi[:, k] == e)[0]
            if rows.size:
                h = round_to(silu(xf[rows] @ Wg) * (xf[rows] @ Wu), dtype)
                out_k[k][rows] = round_to(h @ Wd, dtype)
    return combine(out_k, w, dtype)
