"""CPU oracle of the quantized fused-MoE path — TEST INFRASTRUCTURE ONLY.

A pure-torch restatement of the xkernels reference backend for the five ops on
the path. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU
baseline may import it, and only as the checker / the timed CPU baseline; the
``xkernels_amd`` package never imports it. ``register_reference_backends()``
installs these functions as the REFERENCE backend so ``verify_parity`` has a
second backend to compare with.

Reference behaviour followed (paths in the xkernels checkout):
  dequant_w4a16              src/xkernels/ops/moe/w4a16.py:21-50
  moe_align_block_size_ref   src/xkernels/ops/moe/w4a16.py:53-101
  moe_align_block_size_ep    src/xkernels/ops/moe/w4a16.py:104-155
  moe_w4a16_ref              src/xkernels/ops/moe/reference.py:22-70
  moe_sum_reduce_ref         src/xkernels/ops/moe/sum_reduce.py:20-39
  dequant_mxfp4(_weight)     src/xkernels/ops/gather/mxfp4.py:39-68, ops/moe/mxfp4.py:38-56
  moe_mxfp4_ref              src/xkernels/ops/moe/mxfp4_reference.py:28-112
  topk_softmax_ref           src/xkernels/ops/moe/topk_softmax.py:33-95

Each function is pinned by tests/test_oracle.py against closed forms, brute
force on tiny inputs, invariants and the independent C restatement
(oracle/moe_oracle.c); see that file's header for the list.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

E2M1_MAGNITUDES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)


# ------------------------------------------------------------------ int4 ----

def dequant_w4a16(packed: torch.Tensor, scale: torch.Tensor, group_size: int = 32, *,
                  out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """``W[e,n,k] = (nibble_k(packed[e,n,k//8]) - 8) * scale[e,n,k//g]`` in fp32, then
    one cast to ``out_dtype`` (bf16 by default) — w4a16.py:21-50."""
    E, N, kp = packed.shape
    K = kp * 8
    shifts = torch.arange(8, dtype=torch.int32, device=packed.device) * 4
    nib = (packed.to(torch.int32).unsqueeze(-1) >> shifts) & 0xF
    w = (nib.reshape(E, N, K).float() - 8.0).view(E, N, K // group_size, group_size)
    w = w * scale.float().unsqueeze(-1)
    return w.reshape(E, N, K).to(out_dtype or torch.bfloat16)


def moe_w4a16_ref(A, packed, scale, topk_ids, topk_w, group_size: int = 32,
                  mul_routed_weight: bool = True, fused_combine=None, expert_map=None,
                  workspace=None) -> torch.Tensor:
    """``out[m] = sum_j [w[m,j]] * (A[m] @ W[e_j]^T)`` in fp32, cast to ``A.dtype``.

    Computed per expert over the slots routed to it (the same sum as the
    per-(m, j) loop of reference.py:59-69; only the fp32 summation order of the
    top-k terms differs). Dequant rounds to ``A.dtype`` (w4a16.py:50 as called at
    reference.py:57). Under ``expert_map`` only local experts contribute.
    """
    del fused_combine, workspace
    M, top_k = topk_ids.shape
    E_local = packed.shape[0]
    out = torch.zeros(M, packed.shape[1], dtype=torch.float32, device=A.device)
    ids = topk_ids.to(A.device).long().reshape(-1)
    if expert_map is not None:
        emap = expert_map.to(A.device).long()
        ok = (ids >= 0) & (ids < emap.numel())
        ids = torch.where(ok, emap[ids.clamp(0, emap.numel() - 1)], torch.full_like(ids, -1))
    w = topk_w.to(A.device).float().reshape(-1)
    tok = torch.arange(M, device=A.device).repeat_interleave(top_k)
    for e in torch.unique(ids).tolist():
        if e < 0 or e >= E_local:
            continue
        sel = ids == e
        We = dequant_w4a16(packed[e:e + 1], scale[e:e + 1], group_size, out_dtype=A.dtype)[0]
        contrib = A[tok[sel]].float() @ We.float().T
        if mul_routed_weight:
            contrib = contrib * w[sel].unsqueeze(-1)
        out.index_add_(0, tok[sel], contrib)
    return out.to(A.dtype)


def moe_w4a16_ref_loop(A, packed, scale, topk_ids, topk_w, group_size: int = 32,
                       mul_routed_weight: bool = True, expert_map=None) -> torch.Tensor:
    """The literal per-(token, slot) loop of reference.py:57-70 (full dequant of
    every expert first). Slow; the CPU baseline and tiny cross-checks use it."""
    W = dequant_w4a16(packed, scale, group_size, out_dtype=A.dtype)
    M, top_k = topk_ids.shape
    out = torch.zeros(M, W.shape[1], dtype=torch.float32, device=A.device)
    for m in range(M):
        for j in range(top_k):
            e = int(topk_ids[m, j])
            if expert_map is not None:
                e = int(expert_map[e])
                if e < 0:
                    continue
            c = A[m].float() @ W[e].float().T
            if mul_routed_weight:
                c = topk_w[m, j].float() * c
            out[m] += c
    return out.to(A.dtype)


# ----------------------------------------------------------------- align ----

def moe_align_block_size_ref(topk_ids: torch.Tensor, block_size: int, num_experts: int,
                             truncate: bool = True, workspace=None):
    """Stable group-by-expert of the flattened slots, per-expert padding to
    ``block_size`` with pad id ``numel`` (w4a16.py:53-101).

    Ids outside ``[0, num_experts)`` are never placed (the reference counts them
    in an extra bin it does not iterate). ``truncate=True`` keeps the used blocks
    (``[0]`` if none); ``False`` keeps all ``ceil(max_pad/bs)`` blocks, tail 0.
    """
    del workspace
    dev = topk_ids.device
    flat = topk_ids.reshape(-1).long()
    total = flat.numel()
    max_pad = total + (num_experts + 1) * (block_size - 1)
    max_blocks = (max_pad + block_size - 1) // block_size
    key = torch.where((flat >= 0) & (flat < num_experts), flat, torch.full_like(flat, num_experts))
    order = torch.argsort(key, stable=True)
    counts = torch.bincount(key, minlength=num_experts + 1)[:num_experts]
    padded = (counts + block_size - 1) // block_size * block_size
    off = torch.zeros(num_experts + 1, dtype=torch.long, device=dev)
    off[1:] = torch.cumsum(padded, 0)
    start = torch.zeros(num_experts + 1, dtype=torch.long, device=dev)
    start[1:] = torch.cumsum(counts, 0)
    nvalid = int(start[-1])
    sorted_ids = torch.full((max_pad,), total, dtype=torch.int32, device=dev)
    if nvalid:
        keys = key[order[:nvalid]]
        rank = torch.arange(nvalid, device=dev) - start[keys]
        sorted_ids[off[keys] + rank] = order[:nvalid].to(torch.int32)
    blocks = torch.repeat_interleave(torch.arange(num_experts, device=dev), padded // block_size)
    expert_ids = blocks.to(torch.int32)
    if expert_ids.numel() == 0:
        expert_ids = torch.zeros(1, dtype=torch.int32, device=dev)
    if not truncate:
        tail = torch.zeros(max_blocks - expert_ids.numel(), dtype=torch.int32, device=dev)
        expert_ids = torch.cat([expert_ids, tail]) if blocks.numel() else torch.zeros(max_blocks, dtype=torch.int32, device=dev)
    num_post = torch.tensor([int(off[-1])], dtype=torch.int32, device=dev)
    return sorted_ids, expert_ids, num_post


def moe_align_block_size_ep(topk_ids, block_size: int, num_experts: int, expert_map,
                            truncate: bool = True):
    """EP form (w4a16.py:104-155): global ids -> local rows via ``expert_map``;
    non-local slots are dropped; the align runs over the E_local local experts."""
    emap = expert_map.to(topk_ids.device).long()
    e_local = int((emap >= 0).sum())
    if e_local == 0:
        return moe_align_block_size_ref(torch.zeros_like(topk_ids), block_size, 0, truncate)
    local = torch.where(emap >= 0, emap, torch.full_like(emap, e_local))
    return moe_align_block_size_ref(local[topk_ids.long()].to(torch.int32), block_size, e_local,
                                    truncate)


# ------------------------------------------------------------ sum_reduce ----

def moe_sum_reduce_ref(y: torch.Tensor, w: torch.Tensor | None = None,
                       routed_scaling_factor: float = 1.0) -> torch.Tensor:
    """``s * sum_k w[m,k] * y[m,k,:]`` in fp32, cast to ``y.dtype`` (sum_reduce.py:36-39)."""
    yf = y.float()
    if w is not None:
        yf = yf * w.float().unsqueeze(-1)
    return (yf.sum(dim=1) * routed_scaling_factor).to(y.dtype)


# ----------------------------------------------------------------- mxfp4 ----

def dequant_mxfp4(packed: torch.Tensor, scale: torch.Tensor, group_size: int = 32) -> torch.Tensor:
    """e2m1 pairs (low nibble = even index) times ``2^(byte-127)`` (0xFF -> 0), fp32
    (gather/mxfp4.py:39-68)."""
    mag = torch.tensor(E2M1_MAGNITUDES, dtype=torch.float32, device=packed.device)
    lut = torch.cat([mag, -mag])
    p = packed.to(torch.int64)
    vals = torch.stack((lut[p & 0xF], lut[(p >> 4) & 0xF]), dim=-1).reshape(*packed.shape[:-1], -1)
    s = scale.to(torch.int64)
    mult = torch.where(s == 0xFF, torch.zeros((), device=s.device), torch.exp2((s - 127).float()))
    return vals * mult.repeat_interleave(group_size, dim=-1)


def dequant_mxfp4_weight(packed, scale, group_size: int = 32) -> torch.Tensor:
    """bf16 form used as the GEMM operand (ops/moe/mxfp4.py:38-56)."""
    return dequant_mxfp4(packed, scale, group_size).to(torch.bfloat16)


def moe_mxfp4_ref(A, w13, w13_scale, w2, w2_scale, topk_ids, topk_w, b13=None, b2=None,
                  swiglu_limit: float | None = 10.0, group_size: int = 32,
                  mul_routed_weight: bool = True, expert_map=None, workspace=None) -> torch.Tensor:
    """Per active expert: gate_up (bf16) -> +b13 -> clamped SwiGLU -> bf16 act ->
    down (bf16) -> +b2 -> routed weight -> fp32 scatter-add (mxfp4_reference.py:69-112)."""
    del workspace
    M, top_k = topk_ids.shape
    out = torch.zeros(M, A.shape[1], dtype=torch.float32, device=A.device)
    E_local = w13.shape[0]
    flat = topk_ids.reshape(-1)
    fw = topk_w.reshape(-1).float()
    tok = torch.arange(M, device=A.device).repeat_interleave(top_k)
    emap = None if expert_map is None else expert_map.to(A.device)
    for eg in torch.unique(flat).tolist():
        e = int(eg) if emap is None else int(emap[int(eg)])
        if e < 0 or e >= E_local:
            continue
        sel = flat == eg
        x = A[tok[sel]].to(torch.bfloat16)
        gu = x @ dequant_mxfp4_weight(w13[e], w13_scale[e], group_size).T
        if b13 is not None:
            gu = gu + b13[e].to(gu.dtype)
        g, u = gu.float().chunk(2, dim=-1)
        if swiglu_limit is not None and swiglu_limit > 0:
            g = g.clamp(max=swiglu_limit)
            u = u.clamp(min=-swiglu_limit, max=swiglu_limit)
        act = (F.silu(g) * u).to(torch.bfloat16)
        down = act @ dequant_mxfp4_weight(w2[e], w2_scale[e], group_size).T
        if b2 is not None:
            down = down + b2[e].to(down.dtype)
        c = down.float()
        if mul_routed_weight:
            c = c * fw[sel].unsqueeze(-1)
        out.index_add_(0, tok[sel], c)
    return out.to(A.dtype)


# ----------------------------------------------------------- topk_softmax ----

def topk_softmax_ref(gating_output: torch.Tensor, topk: int, renormalize: bool = True):
    """fp32 softmax over all experts, the ``topk`` largest probabilities in
    descending order with ties to the lower expert id (a stable descending
    sort), then optional division by their sum (topk_softmax.py:33-95).
    Returns ``(weights fp32 [M, topk], ids int32 [M, topk])``."""
    M, E = gating_output.shape
    if not 1 <= int(topk) <= E:
        raise ValueError(f"topk must satisfy 1 <= topk <= E (got topk={topk}, E={E})")
    probs = torch.softmax(gating_output.float(), dim=1)
    ids = torch.sort(probs, dim=1, descending=True, stable=True).indices[:, : int(topk)]
    w = probs.gather(1, ids)
    if renormalize:
        w = w / w.sum(dim=1, keepdim=True)
    return w.contiguous(), ids.to(torch.int32).contiguous()


# ------------------------------------------------------------ registration ----

# The Op Specs name the reference repository's own oracle functions.
SPEC_REFERENCES = {
    "xkernels.ops.moe.reference:moe_w4a16_ref": moe_w4a16_ref,
    "xkernels.ops.moe.w4a16:moe_align_block_size_ref": moe_align_block_size_ref,
    "xkernels.ops.moe.sum_reduce:moe_sum_reduce_ref": moe_sum_reduce_ref,
    "xkernels.ops.moe.mxfp4_reference:moe_mxfp4_ref": moe_mxfp4_ref,
    "xkernels.ops.moe.topk_softmax:topk_softmax_ref": topk_softmax_ref,
}


def register_reference_backends() -> None:
    """Install the oracle as the REFERENCE backend of the five kernels and as the
    resolution of the Op Specs' reference paths (test harness only)."""
    from xkernels_amd._backends import Backend
    from xkernels_amd._dispatch import register
    from xkernels_amd.registry import bind_reference

    register("moe_int4_w4a16", Backend.REFERENCE)(moe_w4a16_ref)
    register("moe_align_block_size", Backend.REFERENCE)(moe_align_block_size_ref)
    register("moe_sum_reduce", Backend.REFERENCE)(moe_sum_reduce_ref)
    register("moe_mxfp4", Backend.REFERENCE)(moe_mxfp4_ref)
    register("topk_softmax", Backend.REFERENCE)(topk_softmax_ref)
    for path, fn in SPEC_REFERENCES.items():
        bind_reference(path, fn)
