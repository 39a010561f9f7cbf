"""Writes the golden vectors under tests/golden/ (run: python tests/golden/make_golden.py).

The reference repository holds no test vectors, so these are produced here by torch's CPU
library routines executing each reference module's op sequence on small seeded inputs. They
freeze those library semantics (int32 shift/mask, fp16/bf16 RNE, the e4m3fn cast, softmax/topk)
as data, so the numpy oracle is checked against an independent implementation that does not
move with the installed torch. The sequences follow:
  W4A16   tasks/quant_w4a16_pa/<task>/environment/reference.py:11-17 (packing :21-25)
  W8A8    tasks/w8a8_smoothquant/<task>/environment/reference.py:7-9 (int64 accumulate instead
          of the reference's fp32 matmul, which is inexact above 2^24)
  FP8     tasks/fp8_microscale/<task>/environment/reference.py:9-12
  MXFP8   generate_tasks.py:337-342 (amax/448, e4m3fn cast) with a power-of-two block scale
  qMoE    tasks/fused_qmoe/<task>/environment/reference.py:14-21
  SiLU-FP8 tasks/fused_silu_fp8/<task>/environment/reference.py:13-23
  MoE     tasks/moe/<task>/environment/reference.py:10-17 (top-2 and top-6)
  LoRA    tasks/multi_lora_qgemm/<task>/environment/reference.py:10-17
  SiLU FFN routing and combine of tasks/fused_qmoe/<task>/environment/reference.py:14-21, W4A16
          experts as reference.py:11-17 of the W4A16 task, `F.silu(gate.float()) * up.float()`
          (generate_tasks.py:337), h rounded once to the activation dtype

`python tests/golden/make_golden.py [name ...]` rewrites only the named files (default: all);
each file draws from its own seeded generator, so one can be rewritten without the others.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _np(t):
    return t.detach().cpu().numpy()


def w4a16(g):
    M, K, N, G = 3, 256, 16, 128
    x = torch.randn(M, K, generator=g).half()
    nib = torch.randint(0, 16, (K, N), generator=g, dtype=torch.int64)
    packed = torch.zeros(K, N // 8, dtype=torch.int64)
    for i in range(8):
        packed |= nib[:, i::8] << (4 * i)
    qweight = packed.to(torch.int32)  # keeps the low 32 bits (two's complement)
    scales = (torch.rand(K // G, N, generator=g) * 0.018 + 0.002).half()
    zeros = torch.randint(0, 16, (K // G, N), generator=g).half()
    shifts = torch.arange(0, 32, 4, dtype=torch.int32)
    w = ((qweight.unsqueeze(-1) >> shifts) & 0xF).reshape(K, N)
    se = scales.repeat_interleave(G, dim=0)
    ze = zeros.repeat_interleave(G, dim=0)
    W16 = (w.half() - ze) * se
    Wgt = (w.float() - ze.float()) * se.float()
    y_gt = x.float() @ Wgt
    return dict(x=_np(x), qweight=_np(qweight), scales=_np(scales), zeros=_np(zeros),
                nib=_np(nib).astype(np.uint8), W_f16=_np(W16), y_gt=_np(y_gt))


def w8a8(g):
    M, K, N = 4, 512, 16
    x = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (K, N), generator=g, dtype=torch.int8)
    x[0, :] = 127
    w[:, 0] = 127
    x[1, :] = -128
    xs = (torch.rand(M, 1, generator=g) * 0.01 + 0.001).half()
    ws = (torch.rand(1, N, generator=g) * 0.01 + 0.001).half()
    acc = x.long() @ w.long()
    out = (acc.float() * xs.float() * ws.float()).half()
    return dict(x_int8=_np(x), w_int8=_np(w), x_scale=_np(xs), w_scale=_np(ws),
                acc=_np(acc), out=_np(out))


def fp8w(g):
    M, K, N, B = 2, 256, 16, 128
    x = torch.randn(M, K, generator=g).half()
    w = (torch.randn(K, N, generator=g) * 0.3).to(torch.float8_e4m3fn)
    s = (torch.rand(K // B, N, generator=g) * 0.05 + 0.05).half()
    W = (w.float() * s.float().repeat_interleave(B, dim=0)).half()
    y_gt = x.float() @ (w.float() * s.float().repeat_interleave(B, dim=0))
    return dict(x=_np(x), w_codes=_np(w.view(torch.uint8)), scales=_np(s), W_f16=_np(W),
                y_gt=_np(y_gt))


def mxfp8(g):
    R, K = 6, 128
    src = torch.randn(R, K, generator=g) * torch.logspace(-3, 3, R).unsqueeze(1)
    src[5, 32:64] = 0.0  # an all-zero block: code 0
    blk = src.reshape(R, K // 32, 32)
    amax = blk.abs().amax(-1)
    e = torch.where(amax > 0, torch.ceil(torch.log2(amax / 448.0)), torch.full_like(amax, -127.0))
    code = (e + 127).clamp(0, 254).to(torch.uint8)
    scale = torch.exp2(code.float() - 127)
    q = (blk / scale.unsqueeze(-1)).to(torch.float8_e4m3fn).reshape(R, K)
    deq = (q.float().reshape(R, K // 32, 32) * scale.unsqueeze(-1)).reshape(R, K)
    return dict(src=_np(src), codes=_np(q.view(torch.uint8)), scales=_np(code), deq=_np(deq))


def qmoe_route(g):
    T, E = 9, 8
    logits = torch.randn(T, E, generator=g)
    p = torch.softmax(logits.float(), dim=-1)
    topv, topi = torch.topk(p, 2, dim=-1)
    w = (topv / topv.sum(-1, keepdim=True)).half()
    return dict(logits=_np(logits), topi=_np(topi), topw=_np(w))


def silu_fp8(g):
    """Two rows each in fp16 and bf16 (H = 256, group 128) at several magnitudes, one fp16 row of
    zeros (amax 0: scale clamps to 1e-12, codes 0) and one with large gates (silu(x) = x)."""
    import torch.nn.functional as F
    T, H, G = 6, 256, 128
    mag = torch.tensor([1.0, 0.01, 30.0, 1.0, 0.0, 1.0]).unsqueeze(1)
    y = torch.randn(T, 2 * H, generator=g) * mag
    y[5, :H] = torch.rand(H, generator=g) * 64 + 20
    out = {}
    for name, dt in (("f16", torch.float16), ("bf16", torch.bfloat16)):
        yt = y.to(dt)
        gate, up = yt[:, :H], yt[:, H:]
        act = F.silu(gate.float()) * up.float()
        a = act.reshape(T, H // G, G)
        scale = (a.abs().amax(dim=-1, keepdim=True) / 448.0).clamp(min=1e-12)
        q = (a / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
        deq = (q.float() * scale).reshape(T, H)
        out.update({f"y_{name}": _np(yt.float()), f"act_{name}": _np(act),
                    f"codes_{name}": _np(q.view(torch.uint8).reshape(T, H)),
                    f"scales_{name}": _np(scale.reshape(T, H // G)), f"out_{name}": _np(deq)})
    return out


def moe(g):
    """Top-k fp16 MoE at T=6, D=64, E=8, H=16 for k = 2 and 6: the reference's op sequence in
    fp16 (native path) and on fp32-upcast inputs (the grader's ground truth)."""
    T, D, E, H = 6, 64, 8, 16
    x = torch.randn(T, D, generator=g).half()
    w = (torch.randn(E, D, H, generator=g) * 0.02).half()
    lg = torch.randn(T, E, generator=g).half()
    out = {"x": _np(x.float()), "w": _np(w.float()), "logits": _np(lg.float())}
    for k in (2, 6):
        for tag, (xx, ww, ll) in (("f16", (x, w, lg)), ("gt", (x.float(), w.float(), lg.float()))):
            probs = torch.softmax(ll.float(), dim=-1)
            topv, topi = probs.topk(k, dim=-1)
            topv = (topv / topv.sum(dim=-1, keepdim=True)).to(xx.dtype)
            all_out = torch.einsum("td,edh->teh", xx, ww)
            sel = torch.gather(all_out, 1, topi.unsqueeze(-1).expand(-1, -1, H))
            y = (sel * topv.unsqueeze(-1)).sum(dim=1)
            out[f"y_{tag}_k{k}"] = _np(y.float())
            out[f"topi_k{k}"] = _np(topi)
            out[f"topw_{tag}_k{k}"] = _np(topv.float())
    return out


def lora(g):
    """Multi-LoRA quantized linear at T=5, D=256, N=16, r=4, L=3 (GROUP 128): the reference's op
    sequence in fp16 (native path) and on fp32-upcast inputs (the ground truth)."""
    T, D, N, r, L, G = 5, 256, 16, 4, 3, 128
    x = torch.randn(T, D, generator=g).half()
    q = torch.randint(-8, 8, (D, N), generator=g, dtype=torch.int8)
    s = (torch.randn(D // G, N, generator=g) * 0.01).half()
    A = (torch.randn(L, D, r, generator=g) * 0.02).half()
    B = (torch.randn(L, r, N, generator=g) * 0.02).half()
    ids = torch.randint(0, L, (T,), generator=g)
    out = {"x": _np(x.float()), "qweight": _np(q), "scales": _np(s.float()), "A": _np(A.float()),
           "B": _np(B.float()), "lora_ids": _np(ids)}
    for tag, (xx, ss, AA, BB) in (("f16", (x, s, A, B)),
                                  ("gt", (x.float(), s.float(), A.float(), B.float()))):
        w = (q.reshape(D // G, G, N).to(xx.dtype) * ss[:, None, :].to(xx.dtype)).reshape(D, N)
        base = xx @ w
        lo = torch.einsum("td,tdr->tr", xx, AA[ids])
        lo = torch.einsum("tr,trn->tn", lo, BB[ids])
        out[f"y_{tag}"] = _np((base + lo).float())
    return out


def qmoe_ffn(g):
    """Top-2 SiLU FFN with W4A16 experts at T=7, D=256, F=128, E=4 (GROUP 128), fp32 router
    logits: one per-token loop in torch, run once on fp32-upcast inputs (the ground truth) and
    once in fp16 the way the fused GPU path rounds: dequantised weights in fp16, gate and up
    accumulated in fp32, h = fp16(silu(gate) * up), each expert output fp16(h @ Wd), the weighted
    products and their sum in fp16."""
    import torch.nn.functional as F
    T, D, Fd, E, G = 7, 256, 128, 4, 128
    x = torch.randn(T, D, generator=g).half()
    lg = torch.randn(T, E, generator=g)

    def w4(K, N):
        nib = torch.randint(0, 16, (E, K, N), generator=g, dtype=torch.int64)
        packed = torch.zeros(E, K, N // 8, dtype=torch.int64)
        for i in range(8):
            packed |= nib[:, :, i::8] << (4 * i)
        s = (torch.rand(E, K // G, N, generator=g) * 0.018 + 0.002).half()
        z = torch.randint(0, 16, (E, K // G, N), generator=g).half()
        return packed.to(torch.int32), s, z

    gq, gs, gz = w4(D, Fd)
    uq, us, uz = w4(D, Fd)
    dq, ds, dz = w4(Fd, D)
    shifts = torch.arange(0, 32, 4, dtype=torch.int32)

    def deq(q, s, z, dt):
        w = ((q.unsqueeze(-1) >> shifts) & 0xF).reshape(q.shape[0], q.shape[1], -1)
        return (w.to(dt) - z.repeat_interleave(G, dim=1).to(dt)) * s.repeat_interleave(G, dim=1).to(dt)

    out = {"x": _np(x.float()), "logits": _np(lg), "gq": _np(gq), "gs": _np(gs.float()),
           "gz": _np(gz.float()), "uq": _np(uq), "us": _np(us.float()), "uz": _np(uz.float()),
           "dq": _np(dq), "ds": _np(ds.float()), "dz": _np(dz.float())}
    for tag, dt in (("gt", torch.float32), ("f16", torch.float16)):
        probs = torch.softmax(lg.float(), dim=-1)
        topv, topi = probs.topk(2, dim=-1)
        topv = (topv / topv.sum(dim=-1, keepdim=True)).to(dt)
        Wg, Wu, Wd = deq(gq, gs, gz, dt), deq(uq, us, uz, dt), deq(dq, ds, dz, dt)
        xx = x.to(dt)
        o = torch.zeros(T, 2, D, dtype=dt)
        for t in range(T):
            for k in range(2):
                e = int(topi[t, k])
                gate = xx[t].float() @ Wg[e].float()
                up = xx[t].float() @ Wu[e].float()
                h = (F.silu(gate) * up).to(dt)
                o[t, k] = (h.float() @ Wd[e].float()).to(dt)
        y = (o * topv.unsqueeze(-1)).sum(dim=1)
        out[f"y_{tag}"] = _np(y.float())
        out["topi"] = _np(topi)
    return out


def e4m3fn_table():
    v = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    return ["nan" if np.isnan(a) else float(a).hex() for a in v.tolist()]


SEEDS = {"w4a16": 20240611, "silu_fp8": 20240612, "moe": 20240613, "lora": 20240614,
         "qmoe_ffn": 20240615}
SETS = (("w4a16", w4a16), ("w8a8", w8a8), ("fp8w", fp8w), ("mxfp8", mxfp8),
        ("qmoe_route", qmoe_route))


def main(names=()):
    names = set(names) or {n for n, _ in SETS} | {"silu_fp8", "moe", "lora", "qmoe_ffn",
                                                  "e4m3fn_table"}
    # The first five sets share one generator, drawn in this order (as first written).
    if names & {n for n, _ in SETS}:
        g = torch.Generator().manual_seed(SEEDS["w4a16"])
        for name, fn in SETS:
            d = fn(g)
            if name in names:
                np.savez(os.path.join(HERE, f"{name}.npz"), **d)
    if "silu_fp8" in names:
        g = torch.Generator().manual_seed(SEEDS["silu_fp8"])
        np.savez(os.path.join(HERE, "silu_fp8.npz"), **silu_fp8(g))
    if "moe" in names:
        g = torch.Generator().manual_seed(SEEDS["moe"])
        np.savez(os.path.join(HERE, "moe.npz"), **moe(g))
    if "lora" in names:
        g = torch.Generator().manual_seed(SEEDS["lora"])
        np.savez(os.path.join(HERE, "lora.npz"), **lora(g))
    if "qmoe_ffn" in names:
        g = torch.Generator().manual_seed(SEEDS["qmoe_ffn"])
        np.savez(os.path.join(HERE, "qmoe_ffn.npz"), **qmoe_ffn(g))
    if "e4m3fn_table" in names:
        with open(os.path.join(HERE, "e4m3fn_table.json"), "w") as f:
            json.dump({"source": "torch.float8_e4m3fn -> float32, codes 0..255",
                       "values": e4m3fn_table()}, f, indent=0)
            f.write("\n")


if __name__ == "__main__":
    main(sys.argv[1:])
