"""Public ``moe_sum_reduce`` op (signature of the reference's
src/xkernels/ops/moe/sum_reduce.py:45-58)."""
from __future__ import annotations

import torch

from .._backends import Backend
from .._dispatch import dispatch


def moe_sum_reduce(
    y: torch.Tensor,
    w: torch.Tensor | None = None,
    *,
    routed_scaling_factor: float = 1.0,
    backend: Backend | str = "auto",
) -> torch.Tensor:
    """``out[m] = routed_scaling_factor * sum_k w[m,k] * y[m,k,:]`` in fp32, cast to ``y.dtype``."""
    return dispatch(
        "moe_sum_reduce", y, w, routed_scaling_factor=routed_scaling_factor, backend=backend
    )
