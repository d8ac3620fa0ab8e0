"""xkernels_amd — MI355X (gfx950) native quantized fused-MoE path of xkernels.

Public ops (same names and signatures as ``xkernels``):
``fused_moe_int4_w4a16``, ``fused_moe_mxfp4``, ``moe_align_block_size``,
``moe_sum_reduce``, ``topk_softmax``; harness: ``find_impl``, ``verify``, ``verify_parity``,
``backend_diagnostics``. The ops run hand-written HIP kernels from
``libxk_moe.so``; they raise if the library is missing or the tensors are not on
the GPU.
"""
from . import registry
from ._backends import Backend
from ._dispatch import backend_diagnostics
from .moe import (
    MoeAlignWorkspace,
    MoeInt4Workspace,
    MoeMxfp4Workspace,
    fused_moe_int4_w4a16,
    fused_moe_mxfp4,
    make_mxfp4_moe_weights,
    make_w4a16_weights,
    moe_align_block_size,
    moe_sum_reduce,
    topk_softmax,
)
from .retrieval import find_impl
from .verify import verify, verify_parity

__version__ = "0.1.0"
__all__ = [
    "Backend", "backend_diagnostics", "registry", "fused_moe_int4_w4a16", "fused_moe_mxfp4",
    "moe_align_block_size", "moe_sum_reduce", "topk_softmax", "make_w4a16_weights", "make_mxfp4_moe_weights",
    "MoeAlignWorkspace", "MoeInt4Workspace", "MoeMxfp4Workspace", "find_impl", "verify",
    "verify_parity", "__version__",
]
