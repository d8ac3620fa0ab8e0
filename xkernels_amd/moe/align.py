"""Public ``moe_align_block_size`` op (signature of the reference's
src/xkernels/ops/moe/align.py:34-70)."""
from __future__ import annotations

import torch

from .._backends import Backend
from .._dispatch import dispatch


def moe_align_block_size(
    topk_ids: torch.Tensor,
    block_size: int,
    num_experts: int,
    *,
    backend: Backend | str = "auto",
    truncate: bool = True,
    workspace=None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Sort/pad routed token-slots into per-expert blocks.

    Returns ``(sorted_token_ids [max_pad], expert_ids, num_tokens_post_padded [1])``
    with ``max_pad = M*top_k + (num_experts+1)*(block_size-1)`` and pad id
    ``M*top_k``. ``truncate=True`` trims ``expert_ids`` to the used blocks (one
    host sync); ``truncate=False`` returns all ``ceil(max_pad/block_size)`` blocks,
    unused ones 0, with no host sync.
    """
    return dispatch(
        "moe_align_block_size", topk_ids, block_size, num_experts,
        backend=backend, truncate=truncate, workspace=workspace,
    )
