#!/usr/bin/env python3
"""Benchmark of the quantized-GEMM operator path on one MI355X.

Headline (BASELINE metric, configs[1]): the W4A16 g128 GEMM sweep. One step = one W4A16 call
at every M in {1, 4, 16, 64, 256, 1024, 2048} with K=14336, N=4096, fp16. `value` = total
FLOPs of a step / wall time of a step (TFLOP/s).

Also measured (reported under "configs", not part of `value`): W8A8 at M in {16, 512}, MXFP8 at
M in {128, 2048}, the top-2 W4A16 MoE SiLU FFN (T=512, Mixtral layer), the reference qMoE op
(T=256), the reference FP8 weight-only op (M=16) and the reference fused SiLU + FP8 quantisation
(T=512, H=14336).

Inputs are synthetic (seeded, BASELINE distributions) and resident in HBM before timing. Each
configuration rotates over enough input copies (> 2x the 256 MB Infinity Cache) that every call
streams its weights from HBM. Per configuration two timings are reported: the median of
event-bracketed single calls (the reference grader's protocol, which includes ~4-5 us of event
overhead per call) and the mean of a batch of back-to-back calls between two events
(`us_batched`, close to the kernel duration); roofline fractions use the batched time.

Prints ONE JSON line. The CPU baseline times the numpy oracle on the host cores.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

K_DIM, N_DIM, GROUP = 14336, 4096, 128
SWEEP_M = [1, 4, 16, 64, 256, 1024, 2048]
HBM_PEAK = 8.0e12           # bytes/s, MI355X datasheet
PEAK = {"f16": 2.5e15, "i8": 5.0e15, "f8": 5.0e15}   # dense MFMA, datasheet
ROTATE_BYTES = 640 << 20    # > 2 x 256 MB Infinity Cache
METRIC = "W4A16 GEMM TFLOP/s + HBM GB/s (% roofline), M=1..2048, K=14336 N=4096"


# ---- algorithmic work ------------------------------------------------------------------------
def w4a16_bytes(M, K=K_DIM, N=N_DIM, G=GROUP):
    """Packed weights + fp16 scales and zeros + x + y."""
    return K * N // 2 + 2 * (K // G) * N * 2 + 2 * M * K + 2 * M * N


# HBM bytes per kbh_w4a16_gemm call at the sweep's two regimes, from rocprofv3 PMC runs:
# FETCH_SIZE scaled by 2.0 (a plain 256 MiB device copy reads as 131085.4 KiB) plus WRITE_SIZE
# (exact on the same copy), summed over the call's launches (GEMM + split-K slice sum).
# Keyed by M; other M report null.
W4A16_PMC_TRAFFIC = {16: 43_591_066, 2048: 466_528_461}


def gemm_flops(M, N=N_DIM, K=K_DIM):
    return 2 * M * N * K


def w8a8_bytes(M, K=K_DIM, N=N_DIM):
    return K * N + M * K + 2 * M + 2 * N + 2 * M * N


def mxfp8_bytes(M, K=K_DIM, N=N_DIM):
    return M * K + N * K + (M + N) * K // 32 + 2 * M * N


def fp8w_bytes(M, K=K_DIM, N=N_DIM, B=128):
    return K * N + 2 * (K // B) * N + 2 * M * K + 2 * M * N


def ffn_bytes(T=512, D=4096, F=14336, E=8, G=GROUP):
    per_expert = 3 * D * F // 2 + 3 * 2 * (D * F // G) * 2
    return E * per_expert + 2 * T * D * 2 + 4 * T * E


def ffn_flops(T=512, D=4096, F=14336):
    return 2 * T * 6 * D * F


def qmoe_bytes(T=256, D=4096, N=14336, E=8, G=GROUP):
    return E * D * N + E * (D // G) * N * 2 + 2 * T * D + 2 * T * N + 2 * T * E


def qmoe_flops(T=256, D=4096, N=14336):
    return 2 * T * 2 * D * N


def moe_bytes(T, D, E, H, k):
    """x, y, logits and the weights of the experts the routing selects (expected count for
    uniform routing: E (1 - (1 - k/E)^T))."""
    touched = E * (1.0 - (1.0 - k / E) ** T)
    return int(touched * D * H * 2) + 2 * T * D + 2 * T * H + 2 * T * E


def moe_flops(T, D, H, k):
    return 2 * T * k * D * H


def lora_bytes(T, D, N, r, L):
    """int8 base weight + scales + every adapter (ids drawn uniformly: all touched) + x + y."""
    return D * N + 2 * (D // 128) * N + 2 * L * r * (D + N) + 2 * T * D + 2 * T * N + 8 * T


def lora_flops(T, D, N, r):
    return 2 * T * N * D + 2 * T * r * (D + N)


def silu_fp8_bytes(T=512, H=14336):
    """gate and up (fp16/bf16) read once, the fp32 dequantised output written once."""
    return T * 2 * H * 2 + T * H * 4


def silu_fp8_flops(T=512, H=14336):
    return 0   # elementwise: no MFMA term; the bound is HBM


def roofline(seconds, by, fl, peak):
    t_mem, t_cmp = by / HBM_PEAK, fl / peak
    bound = "hbm" if t_mem >= t_cmp else "mfma"
    return bound, max(t_mem, t_cmp) / seconds


# ---- timing helpers --------------------------------------------------------------------------
def rotation(make, per_set_bytes, limit=32):
    """Clones of one input set, enough to exceed ROTATE_BYTES."""
    base = make()
    R = max(2, min(limit, math.ceil(ROTATE_BYTES / per_set_bytes)))
    return [base] + [[t.clone() for t in base] for _ in range(R - 1)]


def graph_batch(torch, fn, sets, batch, reps=4):
    """Mean device seconds per call of `batch` calls over rotating input sets, captured in one
    HIP graph and replayed `reps` times (no host launch overhead, which otherwise dominates
    kernels of a few microseconds). Every replay's outputs are checked against eager runs of
    the same calls; returns None when capture is not possible or a replay disagrees."""
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        ref = [fn(*sets[i % len(sets)]).float() for i in range(batch)]  # also sizes the pools
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    try:
        with torch.cuda.graph(g, stream=st):
            outs = [fn(*sets[i % len(sets)]) for i in range(batch)]
    except RuntimeError:
        return None
    times = []
    for _ in range(reps):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(st):  # replay() launches on the current stream
            a.record()
            g.replay()
            b.record()
        b.synchronize()
        times.append(a.elapsed_time(b) * 1e-3 / batch)
        for o, r in zip(outs, ref):  # fp32 atomics may reorder sums: tolerance, not bits
            if float((o.float() - r).abs().max()) > 1e-3 * float(r.abs().max()):
                return None
    del g
    return sorted(times)[len(times) // 2]


def time_config(torch, fn, sets, iters, batch):
    """(per-call event times [s], batched mean [s]) over rotating input sets. The batched time
    comes from graph_batch, falling back to back-to-back eager calls."""
    for i in range(3):
        fn(*sets[i % len(sets)])
    torch.cuda.synchronize()
    ts = []
    for i in range(iters):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        fn(*sets[i % len(sets)])
        b.record()
        b.synchronize()
        ts.append(a.elapsed_time(b) * 1e-3)
    gb = graph_batch(torch, fn, sets, batch)
    if gb is not None:
        return sorted(ts), gb
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(batch):
        fn(*sets[i % len(sets)])
    b.record()
    b.synchronize()
    return sorted(ts), a.elapsed_time(b) * 1e-3 / batch


def record(name, ts, batched, by, fl, peak, **extra):
    med = ts[len(ts) // 2]
    bound, frac = roofline(batched, by, fl, peak)
    out = {"name": name, **extra, "us_median": round(med * 1e6, 2),
           "us_batched": round(batched * 1e6, 2), "tflops": round(fl / batched / 1e12, 2),
           "gbps": round(by / batched / 1e9, 1), "bound": bound, "roofline_frac": round(frac, 4),
           "bytes": by, "flops": fl}
    return out


# ---- the reference's task grid ---------------------------------------------------------------
# The task lists of generate_tasks.py:268-275 (linear shapes), 390-394 (qMoE) and 481-490 (W4A16
# layers), with the families' grid axes (generate_tasks.py:535-544, 561-580, 617-626).
GRID_LAYERS = [("llama3_8b_gate", 4096, 14336), ("llama3_8b_down", 14336, 4096),
               ("llama3_70b_gate", 8192, 28672), ("llama3_70b_down", 28672, 8192),
               ("qwen2_7b_gate", 3584, 18944), ("qwen2_7b_down", 18944, 3584),
               ("qwen2_72b_gate", 8192, 29568), ("qwen2_72b_down", 29568, 8192)]
GRID_LINEAR = [("llama3_8b_qkv", 4096, 6144), ("llama3_8b_o", 4096, 4096),
               ("llama3_8b_gate", 4096, 14336), ("llama3_8b_down", 14336, 4096),
               ("qwen2_7b_gate", 3584, 18944), ("qwen2_72b_down", 29568, 8192)]
GRID_QMOE = [("deepseek_moe", 2048, 64, 1408), ("mixtral", 4096, 8, 14336),
             ("qwen_moe", 2048, 60, 1408)]
GRID_MOE = [("mixtral_8x7b", 4096, 8, 14336, 2), ("grok1", 6144, 8, 8192, 2),   # generate_tasks.py:189-195
            ("qwen2_57b", 3584, 64, 2560, 8), ("deepseek_v2_lite", 2048, 64, 1408, 6),
            ("qwen3_30b", 2048, 128, 768, 8)]
GRID_LORA = [("llama3_8b_r16", 4096, 4096, 16, 8), ("qwen_7b_r32", 3584, 3584, 32, 8),  # generate_tasks.py:427-431
             ("llama3_8b_r64", 4096, 4096, 64, 4)]
GRID_SILU = [("deepseek_moe", 1408), ("qwen_moe", 2560), ("mixtral", 14336)]   # generate_tasks.py:351-355


def run_grid(torch, dev, inputs, ops, families=None):
    """Times every task of the grid (M=16 unless the task says otherwise; T=256 for the qMoE)
    on rotated HBM-cold inputs; one record per task. `families` limits it to some of
    w4a16, w8a8, fp8w, qmoe, moe, lora, silu_fp8."""
    recs = []
    fams = set(families or ["w4a16", "w8a8", "fp8w", "qmoe", "moe", "lora", "silu_fp8"])
    f16, bf16 = torch.float16, torch.bfloat16

    def one(name, make, fn, by, fl, peak, n_sets_bytes, **extra):
        sets = rotation(make, n_sets_bytes)
        ts, bm = time_config(torch, fn, sets, 10, 20)
        recs.append(record(name, ts, bm, by, fl, peak, **extra))
        del sets
        torch.cuda.empty_cache()
        print(f"[grid] {name}: {recs[-1]['us_batched']} us, frac {recs[-1]['roofline_frac']}",
              file=sys.stderr, flush=True)

    for (n, K, N) in (GRID_LAYERS if "w4a16" in fams else []):
        for g, dt in ((64, f16), (128, f16), (128, bf16)):
            by = w4a16_bytes(16, K, N, g)
            one(f"w4a16 {n} g{g} {str(dt)[6:]}",
                lambda: [t.to(dev) for t in inputs.w4a16(16, K, N, g, dt, seed=1)],
                ops.w4a16_gemm, by, 2 * 16 * N * K, PEAK["f16"], by, M=16, K=K, N=N)
    for (n, K, N) in (GRID_LINEAR if "w8a8" in fams else []):
        for M in (16, 64, 256):
            by = w8a8_bytes(M, K, N)
            one(f"w8a8 {n} M={M}",
                lambda: [t.to(dev) for t in inputs.w8a8(M, K, N, seed=1, dist="reference")],
                ops.w8a8_gemm, by, 2 * M * N * K, PEAK["i8"], by, M=M, K=K, N=N)
    for (n, K, N) in (GRID_LINEAR if "fp8w" in fams else []):
        for b, dt in ((32, f16), (128, f16), (32, bf16)):
            by = fp8w_bytes(16, K, N, b)
            one(f"fp8w {n} b{b} {str(dt)[6:]}",
                lambda: [t.to(dev) for t in inputs.fp8w(16, K, N, b, dt, seed=1)],
                ops.fp8w_gemm, by, 2 * 16 * N * K, PEAK["f16"], by, M=16, K=K, N=N)
    for (n, D, E, N) in (GRID_QMOE if "qmoe" in fams else []):
        for dt in (f16, bf16):
            by = qmoe_bytes(256, D, N, E)
            one(f"qmoe {n} {str(dt)[6:]}",
                lambda: [t.to(dev) for t in inputs.qmoe(256, D, E, N, dt, seed=1)],
                ops.qmoe, by, qmoe_flops(256, D, N), PEAK["f16"], by, T=256, D=D, E=E, N=N)
    for (n, D, E, H, k) in (GRID_MOE if "moe" in fams else []):
        for T, dt in ((16, f16), (128, f16), (512, f16), (512, bf16)):
            by = moe_bytes(T, D, E, H, k)
            one(f"moe {n} top{k} T={T} {str(dt)[6:]}",
                lambda: [t.to(dev) for t in inputs.moe(T, D, E, H, k, dt, seed=1)],
                lambda x, w, lg, k=k: ops.moe(x, w, lg, k), by, moe_flops(T, D, H, k), PEAK["f16"],
                E * D * H * 2, T=T, D=D, E=E, H=H, topk=k)
    for (n, D, N, r, L) in (GRID_LORA if "lora" in fams else []):
        for dt in (f16, bf16):
            by = lora_bytes(64, D, N, r, L)
            one(f"lora {n} {str(dt)[6:]}",
                lambda: [t.to(dev) for t in inputs.lora_qgemm(64, D, N, r, L, dt, seed=1)],
                ops.lora_qgemm, by, lora_flops(64, D, N, r), PEAK["f16"], by, T=64, D=D, N=N, r=r,
                L=L)
    for (n, H) in (GRID_SILU if "silu_fp8" in fams else []):
        for T, dt in ((256, f16), (512, f16), (512, bf16)):
            by = silu_fp8_bytes(T, H)
            one(f"silu_fp8 {n} T={T} {str(dt)[6:]}",
                lambda: [t.to(dev) for t in inputs.silu_fp8(T, H, dt, seed=1)],
                ops.silu_fp8_quant, by, 0, PEAK["f16"], by, T=T, H=H)
    return recs


# ---- CPU baseline ----------------------------------------------------------------------------
def cpu_baseline(sample_m, seed=0, per_m_seconds=3.0):
    """Times the numpy oracle (oracle/w4a16.py, fp32 ground-truth path) on the host cores: a
    bounded sample of repeated calls, about per_m_seconds at each M (10-30 s in all)."""
    import torch

    from kernelbench_harbor_amd import inputs
    from oracle import w4a16 as ow
    try:
        from threadpoolctl import threadpool_info
        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        threads = os.cpu_count() or 1
    total_flops, total_s, per = 0.0, 0.0, []
    for M in sample_m:
        x, qw, s, z = inputs.w4a16(M, K_DIM, N_DIM, GROUP, torch.float16, seed=seed)
        xn, qn, sn, zn = x.float().numpy(), qw.numpy(), s.float().numpy(), z.float().numpy()
        ts = []
        while not ts or (sum(ts) < per_m_seconds and len(ts) < 50):
            t0 = time.perf_counter()
            ow.forward(xn, qn, sn, zn)
            ts.append(time.perf_counter() - t0)
        total_flops += gemm_flops(M) * len(ts)
        total_s += sum(ts)
        per.append({"M": M, "calls": len(ts), "median_s": round(sorted(ts)[len(ts) // 2], 4)})
    return {"value": total_flops / total_s / 1e12, "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": (f"repeated calls of the numpy oracle forward (unpack, fp32 dequant, fp32 "
                       f"BLAS matmul), about {per_m_seconds:g} s at each M in {sample_m}, "
                       "K=14336 N=4096 g128; value = total FLOPs / total seconds"),
            "seconds": round(total_s, 2), "per_m": per}


# ---- main ------------------------------------------------------------------------------------
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--m", type=str, default=",".join(map(str, SWEEP_M)))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="only the W4A16 sweep")
    ap.add_argument("--grid", action="store_true",
                    help="only time the reference's task grid (all W4A16/W8A8/FP8/qMoE tasks at "
                         "their real shapes) and print one JSON line of per-task records")
    ap.add_argument("--families", type=str, default="",
                    help="with --grid: comma list of task families to time (default: all)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run 5 device copies of MIB MiB (calibrates rocprofv3 FETCH_SIZE/"
                         "WRITE_SIZE against a kernel of known traffic) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no "
              "multi-GPU path: the W4A16 GEMM would shard over N with no exchange.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from kernelbench_harbor_amd import build as kbuild
    from kernelbench_harbor_amd import inputs, ops
    if not os.path.exists(kbuild.LIB_PATH):
        kbuild.build()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_probe:
        n = args.copy_probe << 20
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": n, "copies": 5}))
        return
    if args.grid:
        recs = run_grid(torch, dev, inputs, ops, [f for f in args.families.split(",") if f])
        print(json.dumps({"grid": recs, "n_gpus": 1, "data": "synthetic (seeded; the reference "
                          "task distributions; inputs rotated to stay HBM-cold)"}))
        return
    ms = [int(v) for v in args.m.split(",") if v]

    # ---- headline: W4A16 sweep ----
    sets = {}
    for M in ms:
        sets[M] = rotation(lambda: [t.to(dev) for t in inputs.w4a16(M, K_DIM, N_DIM, GROUP,
                                                                     torch.float16, seed=0)],
                           w4a16_bytes(M))
    torch.cuda.synchronize()
    calls = {M: 0 for M in ms}
    ev = {M: [] for M in ms}

    def step(rec):
        for M in ms:
            i = calls[M] % len(sets[M])
            calls[M] += 1
            if rec:
                a = torch.cuda.Event(enable_timing=True)
                b = torch.cuda.Event(enable_timing=True)
                a.record()
                ops.w4a16_gemm(*sets[M][i])
                b.record()
                ev[M].append((a, b))
            else:
                ops.w4a16_gemm(*sets[M][i])

    for _ in range(args.warmup):
        step(False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(True)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    sweep, step_flops, mean_s = [], 0, {}
    for M in ms:
        ts = sorted(a.elapsed_time(b) * 1e-3 for a, b in ev[M])
        mean_s[M] = sum(ts) / len(ts)
        _, batched = time_config(torch, ops.w4a16_gemm, sets[M], 3, 20)
        sweep.append(record(f"w4a16 M={M}", ts, batched, w4a16_bytes(M), gemm_flops(M),
                            PEAK["f16"], M=M, us_mean=round(mean_s[M] * 1e6, 2)))
        step_flops += gemm_flops(M)
    del sets
    torch.cuda.empty_cache()

    # Dominant launch of a step: the M whose calls take the most time.
    Md = max(ms, key=lambda m: mean_s[m])
    d = next(r for r in sweep if r["M"] == Md)
    if d["bound"] == "hbm":
        ach = d["bytes"] / mean_s[Md] / 1e9
        roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": round(ach / (HBM_PEAK / 1e9), 4)}
    else:
        ach = d["flops"] / mean_s[Md] / 1e12
        roof = {"bound": "mfma", "achieved": round(ach, 1), "peak": PEAK["f16"] / 1e12,
                "unit": "TFLOP/s", "frac": round(ach / (PEAK["f16"] / 1e12), 4)}
    roof.update({"traffic": W4A16_PMC_TRAFFIC.get(Md), "launch": f"kbh_w4a16_gemm M={Md} K=14336 N=4096 g128",
                 "avg_launch_us": round(mean_s[Md] * 1e6, 2),
                 "timing": "mean of the HIP-event-bracketed launches of the timed steps"})

    # ---- the other BASELINE configurations ----
    configs = []
    if not args.no_configs:
        it, bt = 20, 20
        for M in (16, 512):
            s_ = rotation(lambda: [t.to(dev) for t in inputs.w8a8(M, K_DIM, N_DIM, seed=0)],
                          w8a8_bytes(M))
            ts, bm = time_config(torch, ops.w8a8_gemm, s_, it, bt)
            configs.append(record(f"w8a8 M={M}", ts, bm, w8a8_bytes(M), gemm_flops(M), PEAK["i8"], M=M))
            del s_
        for M in (128, 2048):
            s_ = rotation(lambda: [t.to(dev) for t in inputs.mxfp8(M, K_DIM, N_DIM, seed=0)],
                          mxfp8_bytes(M))
            ts, bm = time_config(torch, ops.mxfp8_gemm, s_, it, bt)
            configs.append(record(f"mxfp8 M={M}", ts, bm, mxfp8_bytes(M), gemm_flops(M), PEAK["f8"], M=M))
            del s_
        s_ = rotation(lambda: [t.to(dev) for t in inputs.fp8w(16, K_DIM, N_DIM, 128, torch.float16, 0)],
                      fp8w_bytes(16))
        ts, bm = time_config(torch, ops.fp8w_gemm, s_, it, bt)
        configs.append(record("fp8w (reference op) M=16 b128", ts, bm, fp8w_bytes(16), gemm_flops(16),
                              PEAK["f16"], M=16))
        del s_
        torch.cuda.empty_cache()
        s_ = [[t.to(dev) for t in inputs.qmoe_ffn(seed=0)]]   # 757 MB of weights: no rotation
        ts, bm = time_config(torch, ops.qmoe_ffn, s_, 10, 10)
        configs.append(record("qmoe_ffn T=512 D=4096 F=14336 E=8 top2", ts, bm, ffn_bytes(),
                              ffn_flops(), PEAK["f16"], T=512))
        del s_
        torch.cuda.empty_cache()
        s_ = rotation(lambda: [t.to(dev) for t in inputs.silu_fp8(512, 14336, torch.float16, 0)],
                      silu_fp8_bytes())
        ts, bm = time_config(torch, ops.silu_fp8_quant, s_, it, bt)
        configs.append(record("silu_fp8 (reference op) T=512 H=14336 g128", ts, bm,
                              silu_fp8_bytes(), 0, PEAK["f16"], T=512, H=14336))
        del s_
        torch.cuda.empty_cache()
        s_ = [[t.to(dev) for t in inputs.qmoe(seed=0)]]       # 470 MB of weights
        ts, bm = time_config(torch, ops.qmoe, s_, 10, 10)
        configs.append(record("qmoe (reference op) T=256 D=4096 N=14336 E=8", ts, bm,
                              qmoe_bytes(), qmoe_flops(), PEAK["f16"], T=256))
        del s_
        torch.cuda.empty_cache()

    out = {
        "metric": METRIC,
        "value": round(step_flops / (wall / args.steps) / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded; BASELINE distributions; weights rotated to stay HBM-cold)",
        "config": {"workload": "W4A16 g128 GEMM sweep, one call per M per step",
                   "M": ms, "K": K_DIM, "N": N_DIM, "group": GROUP,
                   "qweight_layout": "int32 [K, N/8], 8 nibbles along N",
                   "parallelism": "none (1 GPU)"},
        "sweep": sweep,
        "roofline": roof,
        "configs": configs,
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline([m for m in ms if m <= 256] or ms[:1])
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
