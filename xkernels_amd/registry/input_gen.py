"""Seeded input generators for ``verify`` / ``verify_parity``, one per Op Spec.

Recipes follow the reference's registry/input_gen.py:68-159 (same seeds per
tensor, same distributions) so the same (point, seed, device) gives the same
inputs; ``moe_mxfp4`` has no generator upstream and gets one here. The
``topk_softmax`` logits are N(0, 1) in the point's dtype (:203-215).
"""
from __future__ import annotations

from collections.abc import Callable
from typing import Any

import torch

from .dtypes import to_torch_dtype


def _randn(device: str, dtype: torch.dtype, *shape: int, seed: int) -> torch.Tensor:
    g = torch.Generator(device=device).manual_seed(int(seed))
    return torch.randn(*shape, generator=g, device=device, dtype=dtype)


def _moe_sum_reduce(p: dict[str, Any], seed: int, device: str) -> dict[str, Any]:
    dt = to_torch_dtype(p["dtype"])
    y = _randn(device, dt, p["M"], p["top_k"], p["H"], seed=seed)
    w = _randn(device, torch.float32, p["M"], p["top_k"], seed=seed + 1)
    return {"y": y, "w": w, "routed_scaling_factor": 1.0}


def _moe_align_block_size(p: dict[str, Any], seed: int, device: str) -> dict[str, Any]:
    g = torch.Generator(device=device).manual_seed(int(seed))
    E = int(p["num_experts"])
    ids = torch.randint(0, E, (int(p["M"]), int(p["top_k"])), generator=g, device=device,
                        dtype=torch.int32)
    return {"topk_ids": ids, "block_size": int(p["block_size"]), "num_experts": E,
            "truncate": bool(p.get("truncate", True))}


def _moe_int4_w4a16(p: dict[str, Any], seed: int, device: str) -> dict[str, Any]:
    from ..moe.weights import make_w4a16_weights

    dt = to_torch_dtype(p["dtype"])
    M, K, N, E, k = (int(p[x]) for x in ("M", "K", "N", "E", "top_k"))
    gs = int(p.get("group_size", 32))
    A = _randn(device, dt, M, K, seed=seed)
    packed, scale, _ = make_w4a16_weights(E, N, K, gs, device=device, seed=seed + 1)
    g = torch.Generator(device=device).manual_seed(seed + 2)
    ids = torch.randint(0, E, (M, k), generator=g, device=device, dtype=torch.int32)
    w = torch.rand(M, k, generator=g, device=device, dtype=torch.float32)
    return {"A": A, "packed": packed, "scale": scale, "topk_ids": ids, "topk_w": w,
            "group_size": gs, "mul_routed_weight": True}


def _moe_mxfp4(p: dict[str, Any], seed: int, device: str) -> dict[str, Any]:
    from ..moe.weights import make_mxfp4_moe_weights

    dt = to_torch_dtype(p["dtype"])
    M, E, k = int(p["M"]), int(p["E"]), int(p["top_k"])
    hidden, ispp = int(p["hidden"]), int(p["ispp"])
    bias = bool(p.get("bias", False))
    A = _randn(device, dt, M, hidden, seed=seed)
    if "a_scale" in p:  # optional input scale of a sweep point
        A = (A.float() * float(p["a_scale"])).to(dt)
    sc = {k: int(p[k]) for k in ("scale_lo", "scale_hi") if k in p}  # e8m0 bytes [lo, hi)
    wts = make_mxfp4_moe_weights(E, hidden, ispp, with_bias=bias, device=device, seed=seed + 1, **sc)
    g = torch.Generator(device=device).manual_seed(seed + 2)
    ids = torch.stack([torch.randperm(E, generator=g, device=device)[:k] for _ in range(M)]).to(torch.int32)
    logits = torch.randn(M, k, generator=g, device=device, dtype=torch.float32)
    return {"A": A, "w13": wts["w13"], "w13_scale": wts["w13_scale"], "w2": wts["w2"],
            "w2_scale": wts["w2_scale"], "topk_ids": ids, "topk_w": torch.softmax(logits, -1),
            "b13": wts["b13"], "b2": wts["b2"], "swiglu_limit": float(p.get("swiglu_limit", 10.0))}


def _topk_softmax(p: dict[str, Any], seed: int, device: str) -> dict[str, Any]:
    dt = to_torch_dtype(p["dtype"])
    gating = _randn(device, dt, int(p["M"]), int(p["E"]), seed=seed)
    return {"gating_output": gating, "topk": int(p["topk"]), "renormalize": bool(p["renormalize"])}


_GENERATORS: dict[str, Callable[[dict, int, str], dict[str, Any]]] = {
    "moe_sum_reduce@1.0.0": _moe_sum_reduce,
    "moe_align_block_size@1.0.0": _moe_align_block_size,
    "moe_int4_w4a16@1.0.0": _moe_int4_w4a16,
    "moe_mxfp4@1.0.0": _moe_mxfp4,
    "topk_softmax@1.0.0": _topk_softmax,
}


def has_generator(op_id: str) -> bool:
    return op_id in _GENERATORS


def register_input_gen(op_id: str, fn) -> None:
    _GENERATORS[op_id] = fn


def generate_inputs(op_id: str, point: dict[str, Any], seed: int, device: str) -> dict[str, Any]:
    if op_id not in _GENERATORS:
        raise KeyError(f"no input generator for {op_id!r}; have {sorted(_GENERATORS)}")
    return _GENERATORS[op_id](point, seed, device)


def supported_op_ids() -> list[str]:
    return sorted(_GENERATORS)
