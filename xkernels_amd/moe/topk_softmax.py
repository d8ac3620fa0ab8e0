"""Public ``topk_softmax`` op, the MoE router (signature of the reference's
src/xkernels/ops/moe/topk_softmax.py:98-120): fp32 softmax over all experts,
the ``topk`` most probable in descending order (ties to the lower expert id),
optionally renormalised. Returns ``(topk_weights fp32 [M, topk], topk_ids
int32 [M, topk])``, the inputs ``fused_moe_*`` take."""
from __future__ import annotations

import torch

from .._backends import Backend
from .._dispatch import dispatch


def topk_softmax(
    gating_output: torch.Tensor,
    topk: int,
    *,
    renormalize: bool = True,
    backend: Backend | str = "auto",
) -> tuple[torch.Tensor, torch.Tensor]:
    return dispatch("topk_softmax", gating_output, topk, renormalize=renormalize, backend=backend)
