"""HIP backend of the five MoE ops: thin wrappers over libxk_moe.so.

Each callable has the reference backend's exact signature (the kwargs splatted
by ``verify``; src/xkernels/ops/moe/reference.py:22-33, w4a16.py:53-56,
sum_reduce.py:20-24, mxfp4_reference.py:28-43, topk_softmax.py:33-37), checks device / dtype / shape
on the host, allocates outputs and scratch with torch on the caller's device
and launches on torch's current stream. Errors from the library surface as
``RuntimeError``. CPU tensors are rejected with ``RuntimeError`` (the reference
card convention for GPU-only backends), so nothing here ever computes on the
host.
"""
from __future__ import annotations

import torch

from .. import _lib
from .._backends import Backend
from .._dispatch import register
from .workspace import MoeAlignWorkspace, MoeInt4Workspace, MoeMxfp4Workspace, align_max_pad

_DT = {torch.bfloat16: _lib.XK_DT_BF16, torch.float32: _lib.XK_DT_FP32}
_ROUTER_DT = {**_DT, torch.float16: _lib.XK_DT_FP16}


def _need_gpu(op: str, *tensors: torch.Tensor | None) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(f"{op}: the HIP backend needs device tensors, got {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{op}: tensors on different devices ({dev} vs {t.device})")
    return dev


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _contig(t: torch.Tensor, dtype: torch.dtype | None = None) -> torch.Tensor:
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    return t.contiguous()


def _dtype_code(op: str, t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise RuntimeError(f"{op}: unsupported dtype {t.dtype} (bf16 or fp32)") from None


def _emap(expert_map: torch.Tensor | None, dev) -> tuple[torch.Tensor | None, int]:
    if expert_map is None:
        return None, 0
    m = _contig(expert_map.to(dev), torch.int32)
    return m, m.numel()


# --------------------------------------------------------------------- align ----

def moe_align_block_size_hip(topk_ids: torch.Tensor, block_size: int, num_experts: int,
                             truncate: bool = True, workspace=None):
    """``moe_align_block_size`` on the GPU (contract of w4a16.py:53-101)."""
    dev = _need_gpu("moe_align_block_size", topk_ids)
    if topk_ids.dim() != 2:
        raise RuntimeError(f"moe_align_block_size: topk_ids must be [M, top_k], got {tuple(topk_ids.shape)}")
    if block_size <= 0 or num_experts <= 0:
        raise RuntimeError("moe_align_block_size: block_size and num_experts must be positive")
    M, top_k = topk_ids.shape
    ids = _contig(topk_ids, torch.int32)
    numel = M * top_k
    max_pad = align_max_pad(M, top_k, num_experts, block_size)
    max_blocks = (max_pad + block_size - 1) // block_size
    if workspace is not None and workspace.matches(M, top_k, num_experts, block_size, device=dev):
        sorted_ids, expert_ids = workspace.sorted_ids, workspace.expert_ids
        num_post, scratch = workspace.num_post, workspace.scratch
    else:
        sorted_ids = torch.empty(max_pad, dtype=torch.int32, device=dev)
        expert_ids = torch.empty(max_blocks, dtype=torch.int32, device=dev)
        num_post = torch.empty(1, dtype=torch.int32, device=dev)
        nbytes = _lib.query("xk_moe_align_workspace_bytes", numel, num_experts)
        scratch = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    _lib.call(
        "xk_moe_align_block_size", _ptr(ids), numel, num_experts, block_size, None, 0,
        _ptr(sorted_ids), _ptr(expert_ids), _ptr(num_post), None, _ptr(scratch),
        scratch.numel(), _stream(dev),
    )
    sorted_ids, expert_ids, num_post = sorted_ids[:max_pad], expert_ids[:max_blocks], num_post[:1]
    if truncate:
        # Eager form (w4a16.py:89-90): trim to the used blocks, [0] when none.
        n = int(num_post.item())
        return sorted_ids, expert_ids[: max(n // block_size, 1)], num_post
    return sorted_ids, expert_ids, num_post


# ---------------------------------------------------------------- sum_reduce ----

def moe_sum_reduce_hip(y: torch.Tensor, w: torch.Tensor | None = None,
                       routed_scaling_factor: float = 1.0) -> torch.Tensor:
    """``moe_sum_reduce`` on the GPU (contract of sum_reduce.py:20-39)."""
    dev = _need_gpu("moe_sum_reduce", y, w)
    if y.dim() != 3:
        raise RuntimeError(f"moe_sum_reduce: y must be [M, top_k, H], got {tuple(y.shape)}")
    M, top_k, H = y.shape
    yc = y.contiguous()
    y_dt = _dtype_code("moe_sum_reduce", yc)
    wc, w_dt = None, _lib.XK_DT_NONE
    if w is not None:
        if tuple(w.shape) != (M, top_k):
            raise RuntimeError(f"moe_sum_reduce: w must be [{M}, {top_k}], got {tuple(w.shape)}")
        wc = w if w.dtype in _DT else w.float()
        wc = wc.contiguous()
        w_dt = _DT[wc.dtype]
    out = torch.empty((M, H), dtype=y.dtype, device=dev)
    _lib.call("xk_moe_sum_reduce", _ptr(yc), y_dt, M, top_k, H, _ptr(wc), w_dt,
              float(routed_scaling_factor), _ptr(out), _stream(dev))
    return out


# ---------------------------------------------------------------------- int4 ----

def moe_int4_w4a16_hip(A: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor,
                       topk_ids: torch.Tensor, topk_w: torch.Tensor, group_size: int = 32,
                       mul_routed_weight: bool = True, fused_combine: bool | None = None,
                       expert_map: torch.Tensor | None = None, workspace=None) -> torch.Tensor:
    """``fused_moe_int4_w4a16`` on the GPU (contract of reference.py:22-70).

    ``fused_combine`` is accepted for signature parity; the HIP pipeline always
    combines through fp32 per-slot rows (deterministic, no atomics). Every
    dequantised weight is rounded to bf16 before the contraction, as the
    reference does.
    """
    del fused_combine
    dev = _need_gpu("moe_int4_w4a16", A, packed, scale, topk_ids, topk_w)
    if A.dim() != 2 or packed.dim() != 3 or scale.dim() != 3 or topk_ids.dim() != 2:
        raise RuntimeError("moe_int4_w4a16: expected A [M,K], packed [E,N,K/8], scale [E,N,K/g], topk_ids [M,top_k]")
    M, K = A.shape
    E, N, kp = packed.shape
    top_k = topk_ids.shape[1]
    if kp * 8 != K:
        raise RuntimeError(f"moe_int4_w4a16: packed K/8={kp} does not match A K={K}")
    if group_size <= 0 or K % group_size or tuple(scale.shape) != (E, N, K // group_size):
        raise RuntimeError(f"moe_int4_w4a16: scale shape {tuple(scale.shape)} != {(E, N, K // max(group_size, 1))}")
    if topk_ids.shape[0] != M or tuple(topk_w.shape) != (M, top_k):
        raise RuntimeError("moe_int4_w4a16: topk_ids / topk_w must be [M, top_k]")
    a_dt = _dtype_code("moe_int4_w4a16", A)
    Ac = A.contiguous()
    pk = _contig(packed, torch.int32)
    sc = _contig(scale, torch.bfloat16)
    ids = _contig(topk_ids, torch.int32)
    tw = _contig(topk_w, torch.float32)
    emap, n_global = _emap(expert_map, dev)
    nbytes = _lib.query("xk_moe_int4_w4a16_ep_workspace_bytes", M, top_k, E, N, K, n_global)
    if isinstance(workspace, MoeInt4Workspace) and workspace.matches(M, top_k, N, dtype=A.dtype, device=dev):
        out = workspace.out[:M]
        scratch = workspace.scratch_for(M, E, N, K, num_global_experts=n_global)
    else:
        out = torch.empty((M, N), dtype=A.dtype, device=dev)
        scratch = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    _lib.call(
        "xk_moe_int4_w4a16", _ptr(Ac), a_dt, M, K, _ptr(pk), _ptr(sc), E, N, int(group_size),
        _ptr(ids), _ptr(tw), top_k, _ptr(emap), n_global, int(bool(mul_routed_weight)),
        0, _ptr(out), _ptr(scratch),
        scratch.numel(), _stream(dev),
    )
    return out


# --------------------------------------------------------------------- mxfp4 ----

def moe_mxfp4_hip(A: torch.Tensor, w13: torch.Tensor, w13_scale: torch.Tensor, w2: torch.Tensor,
                  w2_scale: torch.Tensor, topk_ids: torch.Tensor, topk_w: torch.Tensor,
                  b13: torch.Tensor | None = None, b2: torch.Tensor | None = None,
                  swiglu_limit: float | None = 10.0, group_size: int = 32,
                  mul_routed_weight: bool = True, expert_map: torch.Tensor | None = None,
                  workspace=None) -> torch.Tensor:
    """``fused_moe_mxfp4`` on the GPU (contract of mxfp4_reference.py:28-112)."""
    dev = _need_gpu("moe_mxfp4", A, w13, w13_scale, w2, w2_scale, topk_ids, topk_w, b13, b2)
    M, hidden = A.shape
    E, two_ispp, hb = w13.shape
    ispp = two_ispp // 2
    top_k = topk_ids.shape[1]
    if group_size != 32:
        raise RuntimeError(f"moe_mxfp4: group_size={group_size}; MXFP4 blocks are 32 elements")
    checks = {
        "w13": (tuple(w13.shape), (E, 2 * ispp, hidden // 2)),
        "w13_scale": (tuple(w13_scale.shape), (E, 2 * ispp, hidden // 32)),
        "w2": (tuple(w2.shape), (E, hidden, ispp // 2)),
        "w2_scale": (tuple(w2_scale.shape), (E, hidden, ispp // 32)),
        "topk_w": (tuple(topk_w.shape), (M, top_k)),
    }
    if b13 is not None:
        checks["b13"] = (tuple(b13.shape), (E, 2 * ispp))
    if b2 is not None:
        checks["b2"] = (tuple(b2.shape), (E, hidden))
    for name, (got, want) in checks.items():
        if got != want:
            raise RuntimeError(f"moe_mxfp4: {name} shape {got} != {want}")
    if w13.dtype != torch.uint8 or w2.dtype != torch.uint8:
        raise RuntimeError("moe_mxfp4: packed weights must be uint8")
    a_dt = _dtype_code("moe_mxfp4", A)
    limit = float(swiglu_limit) if (swiglu_limit is not None and swiglu_limit > 0) else 0.0
    Ac = A.contiguous()
    t13, s13 = w13.contiguous(), _contig(w13_scale, torch.uint8)
    t2, s2 = w2.contiguous(), _contig(w2_scale, torch.uint8)
    bb13 = None if b13 is None else _contig(b13, torch.bfloat16)
    bb2 = None if b2 is None else _contig(b2, torch.bfloat16)
    ids = _contig(topk_ids, torch.int32)
    tw = _contig(topk_w, torch.float32)
    emap, n_global = _emap(expert_map, dev)
    if isinstance(workspace, MoeMxfp4Workspace) and workspace.matches(
        M, top_k, E, 16, ispp, hidden, dtype=A.dtype, device=dev
    ):
        out, scratch = workspace.out[:M], workspace.scratch
    else:
        nbytes = _lib.query("xk_moe_mxfp4_workspace_bytes", M, top_k, E, hidden, ispp)
        out = torch.empty((M, hidden), dtype=A.dtype, device=dev)
        scratch = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    _lib.call(
        "xk_moe_mxfp4", _ptr(Ac), a_dt, M, hidden, _ptr(t13), _ptr(s13), _ptr(t2), _ptr(s2), E,
        ispp, _ptr(bb13), _ptr(bb2), limit, int(group_size), _ptr(ids), _ptr(tw), top_k,
        _ptr(emap), n_global, int(bool(mul_routed_weight)), _ptr(out), _ptr(scratch),
        scratch.numel(), _stream(dev),
    )
    return out


# ------------------------------------------------------------- topk_softmax ----

def topk_softmax_hip(gating_output: torch.Tensor, topk: int,
                     renormalize: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    """``topk_softmax`` on the GPU (contract of topk_softmax.py:33-95)."""
    dev = _need_gpu("topk_softmax", gating_output)
    if gating_output.dim() != 2:
        raise RuntimeError(f"topk_softmax: gating_output must be [M, E], got {tuple(gating_output.shape)}")
    M, E = gating_output.shape
    if not (1 <= int(topk) <= E):
        raise ValueError(f"topk must satisfy 1 <= topk <= E (got topk={topk}, E={E})")
    try:
        dt = _ROUTER_DT[gating_output.dtype]
    except KeyError:
        raise RuntimeError(f"topk_softmax: unsupported dtype {gating_output.dtype} (bf16, fp16, fp32)") from None
    g = gating_output.contiguous()
    k = int(topk)
    weights = torch.empty((M, k), dtype=torch.float32, device=dev)
    ids = torch.empty((M, k), dtype=torch.int32, device=dev)
    _lib.call("xk_moe_topk_softmax", _ptr(g), dt, M, E, k, int(bool(renormalize)), _ptr(weights),
              _ptr(ids), _stream(dev))
    return weights, ids


def register_all() -> None:
    """Load the library (raises if absent) and register the five HIP callables."""
    lib = _lib.load()
    missing = [n for n in _lib.SIGNATURES if not hasattr(lib, n)]
    if missing:
        raise RuntimeError(f"libxk_moe.so lacks exports {missing}")
    register("moe_align_block_size", Backend.HIP)(moe_align_block_size_hip)
    register("moe_sum_reduce", Backend.HIP)(moe_sum_reduce_hip)
    register("moe_int4_w4a16", Backend.HIP)(moe_int4_w4a16_hip)
    register("moe_mxfp4", Backend.HIP)(moe_mxfp4_hip)
    register("topk_softmax", Backend.HIP)(topk_softmax_hip)


__all__ = [
    "moe_align_block_size_hip",
    "moe_sum_reduce_hip",
    "moe_int4_w4a16_hip",
    "moe_mxfp4_hip",
    "topk_softmax_hip",
    "register_all",
    "MoeAlignWorkspace",
]
