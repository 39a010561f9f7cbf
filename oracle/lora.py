"""Oracle for the multi-LoRA quantized linear (test infrastructure only).

Reference: tasks/multi_lora_qgemm/multi_lora_qgemm__llama3_8b_r16__fp16/environment/
reference.py:10-17 (template generate_tasks.py:396-420), in the activation dtype:
  W    = dtype(dtype(qweight) * dtype(scales))   per GROUP rows of qweight   (:12)
  base = dtype(x @ W)                                                      (:13)
  lo   = dtype(x[t] @ A[id_t])                                             (:14-15)
  e    = dtype(lo[t] @ B[id_t])                                            (:16)
  y    = dtype(base + e)                                                   (:17)
Products are accumulated in float64 and rounded once (an fp32-accumulating GEMM rounded once, up
to the fp32 summation error). With dtype F32 every rounding is the identity: the grader's fp32
ground truth (common/kb_verifier.py:195-196).
"""
from __future__ import annotations

import numpy as np

from .numerics import F32, round_to
from .qmoe import dequant_expert


def forward(x, qweight, scales, A, B, lora_ids, dtype: str = F32) -> np.ndarray:
    W = dequant_expert(qweight, scales, dtype).astype(np.float64)
    xf = np.asarray(x, dtype=np.float64)
    ids = np.asarray(lora_ids, dtype=np.int64)
    base = round_to((xf @ W).astype(np.float32), dtype)
    A = np.asarray(A, dtype=np.float64)
    B = np.asarray(B, dtype=np.float64)
    lo = round_to(np.einsum("td,tdr->tr", xf, A[ids]).astype(np.float32), dtype)
    e = round_to(np.einsum("tr,trn->tn", lo.astype(np.float64), B[ids]).astype(np.float32), dtype)
    return round_to(base + e, dtype)
