"""Public ``fused_moe_int4_w4a16`` op (signature of the reference's
src/xkernels/ops/moe/interface.py:19-83)."""
from __future__ import annotations

import torch

from .._backends import Backend
from .._dispatch import dispatch


def fused_moe_int4_w4a16(
    A: torch.Tensor,
    packed: torch.Tensor,
    scale: torch.Tensor,
    topk_ids: torch.Tensor,
    topk_w: torch.Tensor,
    *,
    group_size: int = 32,
    mul_routed_weight: bool = True,
    fused_combine: bool | None = None,
    expert_map: torch.Tensor | None = None,
    backend: Backend | str = "auto",
    workspace=None,
) -> torch.Tensor:
    """INT4 W4A16 grouped fused-MoE GEMM ``out[m] = sum_j w[m,j] * (A[m] @ W[e_j]^T)``.

    Args:
        A: ``[M, K]`` activations, bf16 (or fp32).
        packed: ``[E, N, K // 8]`` int32, 8 ``uint4b8`` nibbles per word, low nibble
            = lowest k. Rank-local slice under expert parallelism.
        scale: ``[E, N, K // group_size]`` bf16 group scales.
        topk_ids: ``[M, top_k]`` int32 **global** expert ids.
        topk_w: ``[M, top_k]`` fp32 routing weights.
        group_size: quantisation group along K (32 for compressed-tensors).
        mul_routed_weight: fold the routing weights into the sum.
        fused_combine: accepted for API parity; the HIP backend always combines
            through fp32 per-slot rows.
        expert_map: optional ``[num_global_experts]`` global -> local row map
            (``-1`` = not on this rank); the result is then this rank's partial.
        backend: ``"auto"`` or a ``Backend`` / its value.
        workspace: optional :class:`MoeInt4Workspace` for address-stable buffers.

    Returns:
        ``[M, N]`` in ``A.dtype`` (fp32 accumulation).
    """
    return dispatch(
        "moe_int4_w4a16", A, packed, scale, topk_ids, topk_w,
        group_size=group_size, mul_routed_weight=mul_routed_weight,
        fused_combine=fused_combine, expert_map=expert_map, workspace=workspace,
        backend=backend,
    )
