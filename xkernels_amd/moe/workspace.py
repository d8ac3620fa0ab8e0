"""Address-stable scratch for the MoE ops (the reference's ``workspace=`` kwarg,
src/xkernels/ops/moe/workspace.py:85-289).

Pass a workspace to an op to keep every buffer address fixed across calls, the
precondition for HIP-graph capture. Each class keeps the reference's
``allocate(...)`` / ``matches(...)`` signatures. The HIP pipelines carve their
scratch (align outputs, per-slot GEMM rows, SwiGLU activations) out of ONE byte
buffer whose size the C library reports, so ``scratch`` replaces the Triton
backend's individual intermediate tensors; it is sized lazily on first use when
the expert count is not known at ``allocate`` time, exactly like the
reference's lazily-sized ``align_workspace``.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

__all__ = ["MoeAlignWorkspace", "MoeInt4Workspace", "MoeMxfp4Workspace"]


def _same_device(a: torch.device, b) -> bool:
    b = torch.device(b) if not isinstance(b, torch.device) else b
    if a.type != b.type:
        return False
    if a.type != "cuda":
        return True
    ai = a.index if a.index is not None else torch.cuda.current_device()
    bi = b.index if b.index is not None else torch.cuda.current_device()
    return ai == bi


def align_max_pad(M: int, top_k: int, num_experts: int, block_size: int) -> int:
    """Length of ``sorted_token_ids``: ``M*top_k + (num_experts+1)*(block_size-1)``."""
    return M * top_k + (num_experts + 1) * (block_size - 1)


def _cdiv(a: int, b: int) -> int:
    return (a + b - 1) // b


def _ensure(buf: torch.Tensor | None, nbytes: int, device) -> torch.Tensor:
    if buf is not None and buf.numel() >= nbytes and _same_device(buf.device, device):
        return buf
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)


@dataclass
class MoeAlignWorkspace:
    """Outputs + scratch of ``moe_align_block_size``.

    ``sorted_ids [max_pad]``, ``expert_ids [max_blocks]``, ``num_post [1]`` are
    the op's outputs (every element is rewritten each call); ``scratch`` holds
    the grid path's per-chunk histograms.
    """

    sorted_ids: torch.Tensor
    expert_ids: torch.Tensor
    num_post: torch.Tensor
    scratch: torch.Tensor

    @classmethod
    def allocate(cls, M: int, top_k: int, num_experts: int, block_size: int, *, device):
        from .. import _lib

        max_pad = align_max_pad(M, top_k, num_experts, block_size)
        nbytes = _lib.query("xk_moe_align_workspace_bytes", M * top_k, num_experts)
        return cls(
            sorted_ids=torch.empty(max_pad, dtype=torch.int32, device=device),
            expert_ids=torch.empty(_cdiv(max_pad, block_size), dtype=torch.int32, device=device),
            num_post=torch.empty(1, dtype=torch.int32, device=device),
            scratch=torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device),
        )

    def matches(self, M: int, top_k: int, num_experts: int, block_size: int, *, device) -> bool:
        from .. import _lib

        max_pad = align_max_pad(M, top_k, num_experts, block_size)
        nbytes = _lib.query("xk_moe_align_workspace_bytes", M * top_k, num_experts)
        return (
            self.sorted_ids.numel() >= max_pad
            and self.expert_ids.numel() >= _cdiv(max_pad, block_size)
            and self.num_post.numel() >= 1
            and self.scratch.numel() >= nbytes
            and _same_device(self.sorted_ids.device, device)
        )


@dataclass
class MoeInt4Workspace:
    """Scratch of ``fused_moe_int4_w4a16``: the ``[M, N]`` output plus one byte
    buffer for align outputs and the fp32 per-slot GEMM rows.

    ``out`` is fully overwritten each call (no zeroing needed). ``scratch`` is
    sized on first use for the call's expert count, or up front when
    ``num_experts`` / ``K`` are given.
    """

    out: torch.Tensor
    dtype: torch.dtype
    top_k: int
    scratch: torch.Tensor | None = None
    num_experts: int | None = field(default=None)

    @classmethod
    def allocate(cls, max_M: int, top_k: int, N: int, *, dtype: torch.dtype, device,
                 num_experts: int | None = None, K: int | None = None):
        ws = cls(out=torch.empty((max_M, N), dtype=dtype, device=device), dtype=dtype, top_k=top_k)
        if num_experts is not None:
            ws.scratch_for(max_M, num_experts, N, K or 0)
        return ws

    def scratch_for(self, M: int, E: int, N: int, K: int, num_global_experts: int = 0) -> torch.Tensor:
        """The byte buffer for a call with E local experts (of
        ``num_global_experts`` under an expert map; 0 without one), grown when
        needed, never shrunk."""
        from .. import _lib

        nbytes = _lib.query("xk_moe_int4_w4a16_ep_workspace_bytes", M, self.top_k, E, N, K,
                            num_global_experts)
        self.scratch = _ensure(self.scratch, nbytes, self.out.device)
        self.num_experts = E
        return self.scratch

    def matches(self, M: int, top_k: int, N: int, *, dtype: torch.dtype, device) -> bool:
        return (
            self.out.shape[1] == N
            and self.out.shape[0] >= M
            and top_k == self.top_k
            and self.dtype == dtype
            and _same_device(self.out.device, device)
        )


@dataclass
class MoeMxfp4Workspace:
    """Scratch of ``fused_moe_mxfp4``: the ``[M, hidden]`` output plus one byte
    buffer for align outputs, the SwiGLU activations and the per-slot rows."""

    out: torch.Tensor
    dtype: torch.dtype
    scratch: torch.Tensor
    top_k: int
    num_experts: int
    ispp: int

    @classmethod
    def allocate(cls, max_M: int, top_k: int, num_experts: int, block_size: int, ispp: int,
                 hidden: int, *, dtype: torch.dtype, device):
        from .. import _lib

        del block_size  # the HIP pipeline fixes its own token block
        nbytes = _lib.query("xk_moe_mxfp4_workspace_bytes", max_M, top_k, num_experts, hidden, ispp)
        return cls(
            out=torch.empty((max_M, hidden), dtype=dtype, device=device),
            dtype=dtype,
            scratch=torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device),
            top_k=top_k,
            num_experts=num_experts,
            ispp=ispp,
        )

    def matches(self, M: int, top_k: int, num_experts: int, block_size: int, ispp: int,
                hidden: int, *, dtype: torch.dtype, device) -> bool:
        from .. import _lib

        del block_size
        nbytes = _lib.query("xk_moe_mxfp4_workspace_bytes", M, top_k, num_experts, hidden, ispp)
        return (
            self.out.shape[1] == hidden
            and self.out.shape[0] >= M
            and self.scratch.numel() >= nbytes
            and self.dtype == dtype
            and _same_device(self.out.device, device)
        )
