"""MI355X (gfx950) quantized-GEMM operators behind the kernelbench-harbor task interface.

The compute lives in hand-written HIP kernels compiled into ``lib/libkbh_qgemm.so`` (C ABI in
``include/kbh_qgemm.h``); this package holds the ctypes binding, host-side validation and the
drop-in ``nn.Module`` classes.
"""
from ._lib import KbhError  # noqa: F401
from .modules import (FP8WModel, FusedSiluFP8Model, MoEModel, MoETop6Model,  # noqa: F401
                      MoETop8Model, MultiLoRAQGemmModel, MXFP8Model, QMoEFFNModel, QMoEModel,
                      W4A16Model, W8A8Model)

__all__ = ["KbhError", "W4A16Model", "W8A8Model", "FP8WModel", "MXFP8Model", "QMoEModel", "QMoEFFNModel",
           "FusedSiluFP8Model", "MoEModel", "MoETop6Model", "MoETop8Model",
           "MultiLoRAQGemmModel"]
