"""Writes tests/golden/topk_device.npz: the routing ids torch.topk returns ON THE GPU (run on a
GPU box: python tests/golden/make_topk_device_golden.py [output path]).

The reference routes with `probs.topk(k)` of `torch.softmax(router_logits.float())` on the
device (tasks/fused_qmoe/<task>/environment/reference.py:14-15, tasks/moe/<task>/environment/
reference.py:11-12; the grader's ground truth runs there too, common/kb_verifier.py:195-196).
torch's CPU topk orders ties differently from its GPU kernels, so the device behaviour is frozen
here as data: for each case, the logits and the device ids. Cases: integer-valued logits in
[-2, 2] (most rows hold ties at the selection boundary and inside the selection) for every
(experts, k) the reference's task families use, and N(0,1) logits drawn in fp16 and bf16 exactly
as the tasks' get_inputs draw them (no tie filtering).
"""
from __future__ import annotations

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

# (experts, k): fused_qmoe (8, 60, 64 experts, top-2; generate_tasks.py:390-394) and moe
# (generate_tasks.py:189-195: top-2 over 8, top-6 over 64, top-8 over 64 and 128), plus edge ks.
CASES = [(8, 1), (8, 2), (8, 3), (8, 8), (16, 8), (60, 2), (60, 4), (64, 2), (64, 6), (64, 8),
         (128, 8), (256, 8)]
T = 256


def main(path=os.path.join(HERE, "topk_device.npz")):
    dev = torch.device("cuda:0")
    out = {}
    for i, (E, k) in enumerate(CASES):
        g = torch.Generator().manual_seed(1000 + i)
        ints = torch.randint(-2, 3, (T, E), generator=g).to(torch.float16)
        for name, lg in (("int", ints),
                         ("f16", torch.randn(T, E, generator=g).to(torch.float16)),
                         ("bf16", torch.randn(T, E, generator=g).to(torch.bfloat16))):
            p = torch.softmax(lg.to(dev).float(), dim=-1)
            ids = p.topk(k, dim=-1).indices.cpu()
            key = f"E{E}_k{k}_{name}"
            out[key + "_logits"] = lg.float().numpy()
            out[key + "_ids"] = ids.numpy().astype(np.int16)
    out["device"] = np.array(torch.cuda.get_device_name(dev))
    out["torch"] = np.array(torch.__version__)
    np.savez_compressed(path, **out)
    print(f"wrote {len(CASES)} x 3 cases to {path} on {out['device']}")


if __name__ == "__main__":
    import sys
    main(*sys.argv[1:2])
