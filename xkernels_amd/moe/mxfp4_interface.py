"""Public ``fused_moe_mxfp4`` op (signature of the reference's
src/xkernels/ops/moe/mxfp4_interface.py:22-100)."""
from __future__ import annotations

import torch

from .._backends import Backend
from .._dispatch import dispatch


def fused_moe_mxfp4(
    A: torch.Tensor,
    w13: torch.Tensor,
    w13_scale: torch.Tensor,
    w2: torch.Tensor,
    w2_scale: torch.Tensor,
    topk_ids: torch.Tensor,
    topk_w: torch.Tensor,
    *,
    b13: torch.Tensor | None = None,
    b2: torch.Tensor | None = None,
    swiglu_limit: float | None = 10.0,
    group_size: int = 32,
    mul_routed_weight: bool = True,
    expert_map: torch.Tensor | None = None,
    backend: Backend | str = "auto",
    workspace=None,
) -> torch.Tensor:
    """MXFP4 fused-MoE: gate_up GEMM -> clamped SwiGLU -> down GEMM -> weighted combine.

    Shapes: ``A [M, hidden]``; ``w13 [E, 2*ispp, hidden//2]`` uint8 (rows
    ``[gate; up]``) with ``w13_scale [E, 2*ispp, hidden//32]`` e8m0; ``w2
    [E, hidden, ispp//2]`` with ``w2_scale [E, hidden, ispp//32]``; optional bf16
    biases ``b13 [E, 2*ispp]`` and ``b2 [E, hidden]``; ``topk_ids`` / ``topk_w``
    ``[M, top_k]``. ``swiglu_limit`` None or <= 0 disables the clamp. Returns
    ``[M, hidden]`` in ``A.dtype``.
    """
    return dispatch(
        "moe_mxfp4", A, w13, w13_scale, w2, w2_scale, topk_ids, topk_w,
        b13=b13, b2=b2, swiglu_limit=swiglu_limit, group_size=group_size,
        mul_routed_weight=mul_routed_weight, expert_map=expert_map, workspace=workspace,
        backend=backend,
    )
