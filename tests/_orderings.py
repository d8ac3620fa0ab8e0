"""The oracles' bf16 pipelines restated with float64 contractions.

Each function rounds to bf16 at exactly the points its oracle does
(mxfp4_reference.py:90-110 upstream for MXFP4; the bf16 matmul outputs and the
bf16 SwiGLU activation of the INT4 layer composition), but sums every
contraction in float64 instead of the oracle's fp32 kernels. The two are
equally correct readings of the reference; their difference is the spread
that summation order alone produces, which the tests use to size tolerances
(a kernel is held to a small multiple of it, not to a guess).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from oracle.torch_ref import dequant_mxfp4_weight, dequant_w4a16


def moe_mxfp4_f64(A, w13, w13_scale, w2, w2_scale, topk_ids, topk_w, b13=None, b2=None,
                  swiglu_limit=10.0, group_size=32):
    M, k = topk_ids.shape
    out = torch.zeros(M, A.shape[1], dtype=torch.float64, device=A.device)
    flat = topk_ids.reshape(-1)
    fw = topk_w.reshape(-1).double()
    tok = torch.arange(M, device=A.device).repeat_interleave(k)
    for e in torch.unique(flat).tolist():
        sel = flat == e
        x = A[tok[sel]].to(torch.bfloat16).double()
        gu = (x @ dequant_mxfp4_weight(w13[e], w13_scale[e], group_size).double().T).to(torch.bfloat16)
        if b13 is not None:
            gu = gu + b13[e].to(torch.bfloat16)
        g, u = gu.float().chunk(2, dim=-1)
        if swiglu_limit is not None and swiglu_limit > 0:
            g = g.clamp(max=swiglu_limit)
            u = u.clamp(min=-swiglu_limit, max=swiglu_limit)
        act = (F.silu(g) * u).to(torch.bfloat16)
        down = (act.double() @ dequant_mxfp4_weight(w2[e], w2_scale[e], group_size).double().T)
        down = down.to(torch.bfloat16)
        if b2 is not None:
            down = down + b2[e].to(torch.bfloat16)
        out.index_add_(0, tok[sel], down.double() * fw[sel].unsqueeze(-1))
    return out.to(A.dtype)


def int4_layer_f64(A, w13p, w13s, w2p, w2s, ids, w, limit):
    """gate/up (bf16 out) -> clamped SwiGLU (bf16) -> down (bf16 out) per slot,
    then the fp32-weighted top-k sum (sum_reduce.py:36-39), every contraction
    in float64."""
    M, k = ids.shape
    flat = ids.reshape(-1).long()
    tok = torch.arange(M, device=A.device).repeat_interleave(k)
    y = torch.empty(M * k, w2p.shape[1], dtype=torch.bfloat16, device=A.device)
    for e in flat.unique().tolist():
        sel = (flat == e).nonzero().reshape(-1)
        W13 = dequant_w4a16(w13p[e:e + 1], w13s[e:e + 1], 32, out_dtype=torch.bfloat16)[0].double()
        W2 = dequant_w4a16(w2p[e:e + 1], w2s[e:e + 1], 32, out_dtype=torch.bfloat16)[0].double()
        gu = (A[tok[sel]].double() @ W13.T).to(torch.bfloat16)
        g, u = gu.float().chunk(2, dim=-1)
        act = (F.silu(g.clamp(max=limit)) * u.clamp(min=-limit, max=limit)).to(torch.bfloat16)
        y[sel] = (act.double() @ W2.T).to(torch.bfloat16)
    out = (y.view(M, k, -1).double() * w.double().unsqueeze(-1)).sum(1)
    return out.to(torch.bfloat16)


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm())
