"""ctypes wrapper of oracle/_build/liboracle.so (test infrastructure only).

Accepts torch CPU tensors, returns torch CPU tensors.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "liboracle.so"
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE), "-B"], check=True)
    return LIB


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = ctypes.CDLL(str(LIB))
        _lib.xko_bf16_round.restype = ctypes.c_float
        _lib.xko_bf16_round.argtypes = [ctypes.c_float]
    return _lib


def _p(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _c(t: torch.Tensor | None, dtype=None):
    if t is None:
        return None
    t = t.detach().cpu()
    if dtype is not None:
        t = t.to(dtype)
    return t.contiguous()


def align(topk_ids, block_size: int, num_experts: int, expert_map=None):
    """-> (sorted_ids [max_pad], expert_ids [max_blocks] full form, num_post [1])."""
    ids = _c(topk_ids, torch.int32).reshape(-1)
    numel = ids.numel()
    max_pad = numel + (num_experts + 1) * (block_size - 1)
    max_blocks = (max_pad + block_size - 1) // block_size
    emap = _c(expert_map, torch.int32)
    sorted_ids = torch.empty(max_pad, dtype=torch.int32)
    expert_ids = torch.empty(max_blocks, dtype=torch.int32)
    num_post = torch.empty(1, dtype=torch.int32)
    rc = lib().xko_align(_p(ids), ctypes.c_int64(numel), num_experts, block_size, _p(emap),
                         0 if emap is None else emap.numel(), _p(sorted_ids), _p(expert_ids),
                         ctypes.c_int64(max_blocks), _p(num_post))
    if rc:
        raise MemoryError("xko_align")
    return sorted_ids, expert_ids, num_post


def dequant_int4(packed, scale, group_size: int = 32, round_bf16: bool = True):
    E, N, kp = packed.shape
    K = kp * 8
    pk, sc = _c(packed, torch.int32), _c(scale, torch.bfloat16).view(torch.int16)
    out = torch.empty(E, N, K, dtype=torch.float32)
    lib().xko_dequant_int4(_p(pk), _p(sc), ctypes.c_int64(E * N), ctypes.c_int64(K), group_size,
                           int(round_bf16), _p(out))
    return out


def int4_moe(A, packed, scale, topk_ids, topk_w, group_size=32, mul_routed_weight=True,
             expert_map=None):
    """fp32 [M, N] (cast to A's dtype by the caller if wanted)."""
    M, K = A.shape
    E, N, _ = packed.shape
    top_k = topk_ids.shape[1]
    a = _c(A, torch.float32)
    pk, sc = _c(packed, torch.int32), _c(scale, torch.bfloat16).view(torch.int16)
    ids, w = _c(topk_ids, torch.int32), _c(topk_w, torch.float32)
    emap = _c(expert_map, torch.int32)
    out = torch.empty(M, N, dtype=torch.float32)
    i64 = ctypes.c_int64
    lib().xko_int4_moe(_p(a), int(A.dtype == torch.bfloat16), i64(M), i64(K), _p(pk), _p(sc), i64(E),
                       i64(N), group_size, _p(ids), _p(w), i64(top_k), _p(emap),
                       0 if emap is None else emap.numel(), int(mul_routed_weight), _p(out))
    return out


def sum_reduce(y, w=None, routed_scaling_factor: float = 1.0):
    M, k, H = y.shape
    yy, ww = _c(y, torch.float32), _c(w, torch.float32)
    out = torch.empty(M, H, dtype=torch.float32)
    i64 = ctypes.c_int64
    lib().xko_sum_reduce(_p(yy), i64(M), i64(k), i64(H), _p(ww), ctypes.c_float(routed_scaling_factor), _p(out))
    return out


def dequant_mxfp4(packed, scale):
    *lead, kb = packed.shape
    K = kb * 2
    rows = 1
    for d in lead:
        rows *= d
    pk, sc = _c(packed, torch.uint8), _c(scale, torch.uint8)
    out = torch.empty(*lead, K, dtype=torch.float32)
    lib().xko_dequant_mxfp4(_p(pk), _p(sc), ctypes.c_int64(rows), ctypes.c_int64(K), _p(out))
    return out


def mxfp4_moe(A, w13, w13_scale, w2, w2_scale, topk_ids, topk_w, b13=None, b2=None,
              swiglu_limit=10.0, mul_routed_weight=True, expert_map=None):
    M, hidden = A.shape
    E, two_ispp, _ = w13.shape
    ispp = two_ispp // 2
    top_k = topk_ids.shape[1]
    a = _c(A, torch.float32)
    t13, s13, t2, s2 = (_c(x, torch.uint8) for x in (w13, w13_scale, w2, w2_scale))
    bb13, bb2 = _c(b13, torch.float32), _c(b2, torch.float32)
    ids, w = _c(topk_ids, torch.int32), _c(topk_w, torch.float32)
    emap = _c(expert_map, torch.int32)
    limit = float(swiglu_limit) if (swiglu_limit is not None and swiglu_limit > 0) else 0.0
    out = torch.empty(M, hidden, dtype=torch.float32)
    i64 = ctypes.c_int64
    lib().xko_mxfp4_moe(_p(a), i64(M), i64(hidden), _p(t13), _p(s13), _p(t2), _p(s2), i64(E), i64(ispp),
                        _p(bb13), _p(bb2), ctypes.c_float(limit), _p(ids), _p(w), i64(top_k), _p(emap),
                        0 if emap is None else emap.numel(), int(mul_routed_weight), _p(out))
    return out
