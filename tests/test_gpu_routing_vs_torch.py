"""The HIP routing against the reference's own routing on the device: torch.softmax of the
fp32-upcast logits, then torch.topk (tasks/fused_qmoe/<task>/environment/reference.py:14-16,
tasks/moe/<task>/environment/reference.py:11-13; the grader computes its ground truth on the GPU,
common/kb_verifier.py:195-196). Logits are drawn exactly as the tasks' get_inputs draw them (N(0,1)
in x.dtype, no tie filtering: ties at the selection boundary occur in 12-99% of such draws) and,
to stress the tie order, as small integers. The ids must agree with torch in value and order; the
renormalised weights to a few fp32 ulps (the softmax's exp differs in its last bits)."""
import os
import re

import numpy as np
import pytest
import torch

from kernelbench_harbor_amd import ops

pytestmark = pytest.mark.gpu

# (experts, k) of the fused_qmoe tasks (generate_tasks.py:390-394) and the moe tasks
# (generate_tasks.py:189-195).
ROUTES = [(8, 2), (64, 2), (60, 2), (64, 6), (64, 8), (128, 8)]


def _torch_route(lg, k):
    p = torch.softmax(lg.float(), dim=-1)
    v, i = p.topk(k, dim=-1)
    return i.int(), v / v.sum(dim=-1, keepdim=True)


@pytest.mark.parametrize("E,k", ROUTES)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("kind", ["randn", "ints"])
def test_route_matches_torch_topk(dev, E, k, dtype, kind):
    print(f"[route vs torch] E={E} k={k} {dtype} {kind}", flush=True)
    ties = 0
    for seed in range(8):
        g = torch.Generator().manual_seed(100 * E + 10 * k + seed)
        if kind == "randn":
            lg = torch.randn(512, E, generator=g).to(dtype).to(dev)
        else:
            lg = torch.randint(-2, 3, (512, E), generator=g).to(dtype).to(dev)
        ti, tw = _torch_route(lg, k)
        hi, hw = ops.moe_route_topk(lg, k, torch.float32)
        assert torch.equal(hi, ti), (seed, int((hi != ti).any(-1).sum()))
        assert float((hw - tw).abs().max()) <= 4e-7
        if k == 2:
            hi2, hw2 = ops.moe_route_top2(lg, torch.float32)
            assert torch.equal(hi2, ti)
            assert torch.equal(hw2, hw)
        srt = torch.softmax(lg.float(), -1).sort(dim=-1, descending=True).values
        ties += int((srt[:, k - 1] == srt[:, k]).sum()) if k < E else 0
    if kind == "ints":
        assert ties > 0   # the draws did exercise boundary ties


def test_route_reproduces_device_golden(dev):
    """The ids torch.topk gave on an MI355X (tests/golden/topk_device.npz) for every case."""
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "topk_device.npz"))
    for key in gold.files:
        if not key.endswith("_logits"):
            continue
        base = key[:-7]
        k = int(re.search(r"_k(\d+)_", base).group(1))
        if k > 8:
            continue
        lg = torch.from_numpy(gold[key]).to(dev)
        hi, _ = ops.moe_route_topk(lg, k, torch.float32)
        assert np.array_equal(hi.cpu().numpy(), gold[base + "_ids"]), base
