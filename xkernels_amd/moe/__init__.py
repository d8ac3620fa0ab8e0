"""Quantized fused-MoE ops on gfx950: router (topk_softmax) -> align -> INT4 / MXFP4
grouped GEMM -> combine.

The HIP backend registers inside ``backend_registration_guard``: if the native
library is missing the failure is recorded (``backend_diagnostics()``) and any
call raises — there is no CPU fallback in this package.
"""
from .._backends import Backend
from .._dispatch import backend_registration_guard
from .align import moe_align_block_size
from .interface import fused_moe_int4_w4a16
from .mxfp4_interface import fused_moe_mxfp4
from .sum_reduce import moe_sum_reduce
from .topk_softmax import topk_softmax
from .weights import make_mxfp4_moe_weights, make_w4a16_weights
from .workspace import MoeAlignWorkspace, MoeInt4Workspace, MoeMxfp4Workspace

_KERNELS = ("moe_align_block_size", "moe_sum_reduce", "moe_int4_w4a16", "moe_mxfp4", "topk_softmax")

with backend_registration_guard(_KERNELS, Backend.HIP, source="xkernels_amd.moe.hip_backend"):
    from . import hip_backend

    hip_backend.register_all()

__all__ = [
    "fused_moe_int4_w4a16",
    "fused_moe_mxfp4",
    "moe_align_block_size",
    "moe_sum_reduce",
    "topk_softmax",
    "make_w4a16_weights",
    "make_mxfp4_moe_weights",
    "MoeAlignWorkspace",
    "MoeInt4Workspace",
    "MoeMxfp4Workspace",
]
