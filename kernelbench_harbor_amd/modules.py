"""Drop-in ``nn.Module`` replacements for the reference task modules.

Each class has the reference ``Model``'s no-argument constructor and ``forward`` signature
(the grader constructs ``ModelNew()`` and calls ``forward(*get_inputs())``,
common/kb_verifier.py:185-197) and returns the reference output dtype. The compute is a call
into the HIP library; a task file only needs ``ModelNew = W4A16Model`` (etc.).
"""
from __future__ import annotations

import torch.nn as nn

from . import ops


class W4A16Model(nn.Module):
    """Packed-asymmetric W4A16 (GPTQ-style) linear.

    Reference: tasks/quant_w4a16_pa/*/environment/reference.py:10-17,
    forward(x [M,K], qweight [K,N/8] int32, scales [K/G,N], zeros [K/G,N]) -> [M,N] x.dtype.
    """

    def forward(self, x, qweight, scales, zeros):
        return ops.w4a16_gemm(x, qweight, scales, zeros)
