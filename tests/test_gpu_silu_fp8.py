"""GPU parity of the fused SiLU x up + per-group FP8 quantisation (kbh_silu_fp8_quant) against
the CPU oracle (oracle/silu_fp8.py).

* Exact cases: gates >= 32 make silu(gate) = gate exactly on both sides (e^-x < 2^-24), so act =
  gate * up is exact and every later step is exactly rounded: codes, scales and outputs must be
  bit-identical, including crafted values on and between e4m3 grid points (ties to even).
* The reference's task grid (generate_tasks.py:351-355, 610-614; N(0,1) inputs): the SiLU's
  exp differs from numpy's by a few ulp, so outputs are compared to the benchmark's tolerance and
  the reference's own cosine / relative-L1 gate (common/kb_verifier.py:172-176), and at least
  99.9% of the e4m3 codes must be identical.
"""
import numpy as np
import pytest
import torch

from kernelbench_harbor_amd import FusedSiluFP8Model, inputs, ops
from kernelbench_harbor_amd.harness import compare
from oracle import silu_fp8 as o

pytestmark = pytest.mark.gpu

FUSED_CFG = [("deepseek_moe", 1408), ("qwen_moe", 2560), ("mixtral", 14336)]
GRID = [(n, H, T, torch.float16) for n, H in FUSED_CFG for T in (256, 512)] + \
       [(n, H, 512, torch.bfloat16) for n, H in FUSED_CFG]


def _run(y, group=128):
    out, codes, scales = ops.silu_fp8_quant(y, group, return_codes=True)
    torch.cuda.synchronize()
    return out.cpu().numpy(), codes.view(torch.uint8).cpu().numpy(), scales.cpu().numpy()


def _cosine_rel(out, ref):
    yf, gf = torch.from_numpy(out).flatten(), torch.from_numpy(ref).flatten()
    cos = torch.nn.functional.cosine_similarity(yf, gf, dim=0).item()
    rel = (yf - gf).abs().sum().item() / (gf.abs().sum().item() + 1e-8)
    return cos, rel


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_exact_when_silu_is_identity(dev, dtype, group):
    print(f"[silu_fp8 exact] {dtype} group={group}", flush=True)
    T, H = 7, 4 * 128 + group * 3
    H -= H % group
    g = torch.Generator().manual_seed(group)
    gate = (torch.rand(T, H, generator=g) * 40 + 32).to(dtype)
    up = (torch.randn(T, H, generator=g) * torch.logspace(-4, 2, T).unsqueeze(1)).to(dtype)
    # row 0, first group: amax 448 (scale exactly 1) and values on and between grid points
    gate[0, :group] = 64.0
    vals = torch.tensor([448.0, 1.0625, 1.1875, 1.3125, 2.0 ** -10, 3 * 2.0 ** -10, 248.0, 432.0,
                         -1.0625, -3 * 2.0 ** -10, 0.0, 1.5])
    up[0, :group] = 0
    up[0, :len(vals)] = (vals / 64.0).to(dtype)
    y = torch.cat([gate, up], dim=1)
    act = (gate.float() * up.float()).numpy()
    r_out, r_codes, r_scales = o.quantize(act, group)
    out, codes, scales = _run(y.to(dev), group)
    assert np.array_equal(codes, r_codes)
    assert np.array_equal(scales, r_scales)
    assert np.array_equal(out, r_out)
    assert scales[0, 0] == 1.0 and codes[0, 0] == 0x7E


@pytest.mark.parametrize("name,H,T,dtype", GRID)
def test_reference_task_grid(dev, name, H, T, dtype):
    print(f"[silu_fp8 grid] {name} T={T} H={H} {dtype}", flush=True)
    (y,) = inputs.silu_fp8(T, H, dtype, seed=T + H)
    out = FusedSiluFP8Model()(y.to(dev))
    assert out.dtype == torch.float32 and out.shape == (T, H)
    r_out, r_codes, _ = o.forward(y.float().numpy())
    cmp = compare(out, r_out)
    assert cmp.ok and cmp.task_ok("fused_silu_fp8"), cmp
    cos, rel = _cosine_rel(out.cpu().numpy(), r_out)
    assert cos >= 0.99 and rel <= 0.05, (cos, rel)
    _, codes, _ = _run(y.to(dev))
    assert (codes == r_codes).mean() >= 0.999


def test_small_and_ragged(dev):
    for T, H, group in [(1, 128, 128), (3, 384, 128), (5, 96, 32), (2, 192, 64), (33, 1408, 128)]:
        print(f"[silu_fp8 small] T={T} H={H} g={group}", flush=True)
        (y,) = inputs.silu_fp8(T, H, torch.float16, seed=T * H)
        out, codes, scales = _run(y.to(dev), group)
        r_out, r_codes, r_scales = o.forward(y.float().numpy(), group)
        assert compare(out, r_out).ok
        assert (codes == r_codes).mean() >= 0.99
        np.testing.assert_allclose(scales, r_scales, rtol=1e-5)


def test_empty_and_repeat(dev):
    y = torch.zeros(0, 256, dtype=torch.float16, device=dev)
    assert ops.silu_fp8_quant(y).shape == (0, 128)
    (y,) = inputs.silu_fp8(64, 1408, torch.bfloat16, seed=1)
    y = y.to(dev)
    a = ops.silu_fp8_quant(y)
    b = ops.silu_fp8_quant(y)
    assert torch.equal(a, b)


def test_nan_group_and_zero_row(dev):
    (y,) = inputs.silu_fp8(4, 512, torch.float16, seed=9)
    y[1, 130] = float("nan")       # gate of row 1, group 1
    y[3] = 0
    out, codes, scales = _run(y.to(dev))
    assert np.isnan(scales[1, 1]) and np.all(np.isnan(out[1, 128:256]))
    assert np.all(codes[1, 128:256] & 0x7F == 0x7F)
    assert np.all(np.isfinite(out[1, :128])) and np.all(np.isfinite(out[1, 256:]))
    assert np.all(out[3] == 0) and np.all(codes[3] == 0) and np.all(scales[3] == np.float32(1e-12))
    r_out, _, _ = o.forward(np.nan_to_num(y.float().numpy()[[0, 2]]))
    assert compare(out[[0, 2]], r_out).ok
