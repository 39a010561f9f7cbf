"""GPU parity of the top-2 quantized MoE ops against the CPU oracle (oracle/qmoe.py)."""
import numpy as np
import pytest
import torch

from kernelbench_harbor_amd import QMoEFFNModel, QMoEModel, inputs, ops
from kernelbench_harbor_amd.harness import compare
from oracle import qmoe as oq
from oracle.numerics import round_to

pytestmark = pytest.mark.gpu


def _np(ts):
    return [t.float().numpy() if t.is_floating_point() else t.numpy() for t in ts]


@pytest.mark.parametrize("ldt", [torch.float16, torch.bfloat16, torch.float32])
def test_route_top2(dev, ldt):
    g = torch.Generator().manual_seed(4)
    lg = torch.randn(300, 8, generator=g).to(ldt)
    topi, topw = ops.moe_route_top2(lg.to(dev), torch.float16)
    oi, ow = oq.route_top2(lg.float().numpy(), "f16")
    assert np.array_equal(topi.cpu().numpy(), oi)
    assert np.abs(topw.float().cpu().numpy() - ow).max() <= 2 ** -11   # at most one fp16 ulp


CASES = [
    # T, D, E, N, dtype
    (32, 256, 4, 256, torch.float16),
    (64, 1024, 8, 512, torch.float16),
    (100, 512, 8, 384, torch.bfloat16),
    (300, 1024, 16, 256, torch.float16),
]


@pytest.mark.parametrize("T,D,E,N,dtype", CASES)
def test_qmoe_parity(dev, T, D, E, N, dtype):
    print(f"[qmoe] T={T} D={D} E={E} N={N} {dtype}", flush=True)
    ins = inputs.qmoe(T, D, E, N, dtype, seed=T + N)
    y = ops.qmoe(*[t.to(dev) for t in ins])
    assert y.dtype == dtype and y.shape == (T, N)
    gt = oq.qmoe_forward(*_np(ins))
    cmp = compare(y, gt)
    assert cmp.ok, cmp


def _one_hot_want(q, s, ks, gi, gw, dt):
    """One-hot rows of x make expert e's output row q[e][k] * s[e][k / G] exactly (integer B
    operands, one fp32 product per group), so kbh_qmoe's result is the fp32 combine of those
    rows with the GPU's fp32 routing weights, rounded once to dt."""
    W = {e: oq.dequant_expert(q[e].numpy(), s[e].float().numpy(), "f32") for e in np.unique(gi)}
    T = len(ks)
    out_k = [np.stack([W[gi[t, k]][ks[t]] for t in range(T)]) for k in range(2)]
    return round_to(oq.combine(out_k, gw, "f32"), dt)


@pytest.mark.parametrize("group", [32, 64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_qmoe_group_sizes(dev, group, dtype):
    """Every scale group (the fold scales each group's fp32 sums): tolerance against the ground
    truth, and one-hot activations bit-exact against the fp32 combine of exact weight rows."""
    print(f"[qmoe group] g{group} {dtype}", flush=True)
    T, D, E, N = 96, 1024, 8, 256
    x, q, s, lg = inputs.qmoe(T, D, E, N, dtype, seed=group, group=group)
    y = ops.qmoe(*[t.to(dev) for t in (x, q, s, lg)])
    cmp = compare(y, oq.qmoe_forward(*_np([x, q, s, lg])))
    assert cmp.ok and cmp.allclose_ref, cmp
    g = torch.Generator().manual_seed(group + 1)
    ks = torch.randint(0, D, (T,), generator=g)
    xo = torch.zeros(T, D, dtype=dtype)
    xo[torch.arange(T), ks] = 1.0
    yo = ops.qmoe(*[t.to(dev) for t in (xo, q, s, lg)]).float().cpu().numpy()
    dt = "f16" if dtype == torch.float16 else "bf16"
    gi, gw = ops.moe_route_top2(lg.to(dev), torch.float32)
    gi, gw = gi.cpu().numpy(), gw.cpu().numpy()
    assert np.array_equal(gi, oq.route_top2(lg.float().numpy())[0])
    want = _one_hot_want(q, s, ks.numpy(), gi, gw, dt)
    assert np.array_equal(yo, want), np.abs(yo - want).max()


def test_qmoe_one_hot_full_range_int8(dev):
    """Integer weights over the whole int8 range (the producers convert any int8 exactly) with
    signed, subnormal-free scales: one-hot rows bit-exact in fp16 and bf16."""
    T, D, E, N = 64, 512, 4, 256
    for dtype, dt in ((torch.float16, "f16"), (torch.bfloat16, "bf16")):
        x, _, s, lg = inputs.qmoe(T, D, E, N, dtype, seed=5)
        q = torch.randint(-128, 128, (E, D, N), generator=torch.Generator().manual_seed(6),
                          dtype=torch.int8)
        ks = torch.randint(0, D, (T,), generator=torch.Generator().manual_seed(7))
        xo = torch.zeros(T, D, dtype=dtype)
        xo[torch.arange(T), ks] = 1.0
        y = ops.qmoe(xo.to(dev), q.to(dev), s.to(dev), lg.to(dev)).float().cpu().numpy()
        gi, gw = ops.moe_route_top2(lg.to(dev), torch.float32)
        want = _one_hot_want(q, s, ks.numpy(), gi.cpu().numpy(), gw.cpu().numpy(), dt)
        assert np.array_equal(y, want), (dt, np.abs(y - want).max())


def test_qmoe_full_size(dev):
    """Reference subset task (mixtral): T=256, D=4096, E=8, N=14336."""
    print("[qmoe full]", flush=True)
    ins = inputs.qmoe(seed=1)
    y = QMoEModel()(*[t.to(dev) for t in ins])
    assert compare(y, oq.qmoe_forward(*_np(ins))).ok


FFN_CASES = [
    # T, D, F, E, dtype
    (64, 256, 512, 4, torch.float16),
    (128, 512, 1024, 8, torch.float16),
    (96, 512, 384, 8, torch.bfloat16),
    # 64..191 rows per expert: 128-row tiles, experts above 128 rows on one 256-row tile
    (300, 256, 512, 4, torch.float16),
    (160, 512, 256, 4, torch.bfloat16),      # all experts at most 128 rows: big table empty
    # >= 192 routed rows per expert on average: 256-row expert tiles
    (400, 256, 256, 4, torch.float16),
    (512, 512, 512, 4, torch.bfloat16),
]


@pytest.mark.parametrize("T,D,F,E,dtype", FFN_CASES)
def test_qmoe_ffn_parity(dev, T, D, F, E, dtype):
    print(f"[qmoe ffn] T={T} D={D} F={F} E={E} {dtype}", flush=True)
    ins = inputs.qmoe_ffn(T, D, F, E, dtype=dtype, seed=T + F)
    y = ops.qmoe_ffn(*[t.to(dev) for t in ins])
    assert y.dtype == dtype and y.shape == (T, D)
    cmp = compare(y, oq.ffn_forward(*_np(ins)))
    assert cmp.ok, cmp


@pytest.mark.parametrize("group", [32, 64, 256])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_qmoe_ffn_group_sizes(dev, group, dtype):
    """128-row expert tiles (64-191 routed rows per expert) on the warp-specialised kernel with
    every other quantization group (32, 64 and 256 rows: 1, 2 and 8 slabs per group) for both
    GEMMs; the down projection splits K."""
    T, D, F, E = 192, 512, 1024, 4
    print(f"[qmoe ffn group] g{group} {dtype}", flush=True)
    ins = inputs.qmoe_ffn(T, D, F, E, group=group, dtype=dtype, seed=group)
    y = ops.qmoe_ffn(*[t.to(dev) for t in ins])
    cmp = compare(y, oq.ffn_forward(*_np(ins)))
    assert cmp.ok, cmp


@pytest.mark.parametrize("T,D,F,E,dtype", [(64, 256, 512, 4, torch.float16),
                                            (300, 256, 512, 4, torch.float16)])
def test_qmoe_ffn_native_rounding(dev, T, D, F, E, dtype):
    """Against the oracle's fp16 sequence (dequantised weights, h, expert outputs and the
    combine rounded to fp16 where the kernels round them): only the fp32 accumulation order
    differs, so nearly every output is bit-identical and the rest within a few ulps."""
    ins = inputs.qmoe_ffn(T, D, F, E, dtype=dtype, seed=T + F + 1)
    y = ops.qmoe_ffn(*[t.to(dev) for t in ins]).float().cpu().numpy()
    want = oq.ffn_forward(*_np(ins), dtype="f16")
    ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float32)
    tol = np.maximum(4 * ulp, 2.0 ** -11 * np.abs(want).max())
    assert (np.abs(y - want) <= tol).all(), np.abs(y - want).max()
    assert (y == want).mean() >= 0.9, (y == want).mean()


def _routed_logits(counts, seed):
    """fp32 logits whose top-2 experts give each expert exactly counts[e] of the 2T slots:
    token t picks experts L[t] and L[t + T] of the sorted slot list L (distinct, since no count
    reaches T), with random distinct margins."""
    L = np.repeat(np.arange(len(counts)), counts)
    T = len(L) // 2
    rng = np.random.default_rng(seed)
    lg = rng.normal(size=(T, len(counts))).astype(np.float32) - 4.0
    first, second = L[:T], L[T:]
    lg[np.arange(T), first] = 3.0 + rng.uniform(0, 1, T)
    lg[np.arange(T), second] = 1.0 + rng.uniform(0, 1, T)
    return torch.from_numpy(lg)


@pytest.mark.parametrize("F,dtype", [(512, torch.float16), (512, torch.bfloat16),
                                     (256, torch.float16)])
def test_qmoe_ffn_tile_overflow_rows(dev, F, dtype):
    """Experts whose rows overflow a 128-row expert tile by a few (140, 144 and 145 routed
    rows: a second tile of 12, 16 and 17 rows) beside one that fits (123), with the down
    projection split over K (F=512) and unsplit (F=256)."""
    counts = [140, 144, 145, 123]
    T, D, E = sum(counts) // 2, 256, len(counts)
    ins = inputs.qmoe_ffn(T, D, F, E, dtype=dtype, seed=F + 7)
    ins[1] = _routed_logits(counts, F)
    topi, _ = oq.route_top2(ins[1].numpy())
    assert np.bincount(topi.ravel(), minlength=E).tolist() == counts
    y = ops.qmoe_ffn(*[t.to(dev) for t in ins])
    cmp = compare(y, oq.ffn_forward(*_np(ins)))
    assert cmp.ok, cmp


def test_qmoe_ffn_full_size_all_experts(dev):
    """The benchmark's SiLU FFN configuration (T=512, D=4096, F=14336, E=8): the whole layer runs on the GPU;
    the oracle checks every token (so all eight experts' gate, up and down matrices) on two
    256-column slices of the output, the first and the last."""
    print("[qmoe ffn full]", flush=True)
    ins = inputs.qmoe_ffn(seed=2)
    y = QMoEFFNModel()(*[t.to(dev) for t in ins]).float().cpu().numpy()
    topi, _ = oq.route_top2(ins[1].numpy())
    assert set(np.unique(topi)) == set(range(8))
    a = _np(ins)
    D = a[0].shape[1]
    cols = np.r_[0:256, D - 256:D]
    down = [np.concatenate([a[8][:, :, :32], a[8][:, :, -32:]], axis=2), a[9][:, :, cols],
            a[10][:, :, cols]]
    gt = oq.ffn_forward(*a[:8], *down)     # one pass over gate/up for both slices
    for h in (slice(0, 256), slice(256, 512)):
        cmp = compare(y[:, cols[h]], gt[:, h])
        assert cmp.ok, (h, cmp)


def test_moe_then_split_k_gemm_on_one_stream(dev):
    """MoE calls (scratch pool) and a split-K GEMM (workspace pool) interleaved on one stream."""
    args = [t.to(dev) for t in inputs.qmoe(T=64, D=256, N=256, E=4, seed=2)]
    ops.qmoe(*args)
    x, qw, s, z = inputs.w4a16(4, 1024, 256, seed=4)
    y = ops.w4a16_gemm(x.to(dev), qw.to(dev), s.to(dev), z.to(dev))
    from oracle import w4a16 as ow
    gt = ow.forward(x.float().numpy(), qw.numpy(), s.float().numpy(), z.float().numpy())
    assert compare(y, gt).ok
