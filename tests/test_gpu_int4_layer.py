"""A whole INT4 MoE layer built from the library's stages, against the
oracle's composition: gate/up projection (N = 2 * 2048, K = 7168) per routed
slot, clamped SwiGLU, down projection (N = 7168, K = 2048) per slot, weighted
top-k sum. This is the layer whose two GEMM shapes the reference tunes for
E = 48 (its tuned tables for N=4096,K=7168 and N=7168,K=2048).

The HIP side: ``xk_moe_int4_w4a16_gemm`` gives the fp32 gate/up row of every
slot (rounded to bf16 as the reference's bf16 matmul output is), the SwiGLU is
plain torch on the device (the path has no activation kernel), the down
projection is ``fused_moe_int4_w4a16`` over the M * top_k activation rows with
top_k = 1 and unit weights, and ``moe_sum_reduce`` combines the slots. The
bound is 4x the spread that summation order alone gives (the oracle against the
same composition with float64 contractions, tests/_orderings.py).
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle.torch_ref import dequant_w4a16, moe_sum_reduce_ref
from tests._helpers import softmax_weights, uniform_topk, zipf_topk
from tests._orderings import int4_layer_f64, rel_l2
from tests.test_gpu_int4_exact import _gemm_rows
from xkernels_amd import Backend, fused_moe_int4_w4a16, make_w4a16_weights, moe_sum_reduce

pytestmark = pytest.mark.gpu
LIMIT = 7.0


def _swiglu(gu: torch.Tensor) -> torch.Tensor:
    g, u = gu.float().chunk(2, dim=-1)
    g = g.clamp(max=LIMIT)
    u = u.clamp(min=-LIMIT, max=LIMIT)
    return (F.silu(g) * u).to(torch.bfloat16)


def _oracle_layer(A, w13p, w13s, w2p, w2s, ids, w):
    M, k = ids.shape
    flat = ids.reshape(-1).long()
    tok = torch.arange(M, device=A.device).repeat_interleave(k)
    y = torch.empty(M * k, w2p.shape[1], dtype=torch.bfloat16, device=A.device)
    for e in flat.unique().tolist():
        sel = (flat == e).nonzero().reshape(-1)
        W13 = dequant_w4a16(w13p[e:e + 1], w13s[e:e + 1], 32, out_dtype=torch.bfloat16)[0]
        W2 = dequant_w4a16(w2p[e:e + 1], w2s[e:e + 1], 32, out_dtype=torch.bfloat16)[0]
        act = _swiglu(A[tok[sel]] @ W13.T)
        y[sel] = (act.float() @ W2.float().T).to(torch.bfloat16)
    return moe_sum_reduce_ref(y.view(M, k, -1), w)


def _hip_layer(A, w13p, w13s, w2p, w2s, ids, w):
    M, k = ids.shape
    act = _swiglu(_gemm_rows(A, w13p, w13s, ids).to(torch.bfloat16))
    flat = ids.reshape(-1, 1).contiguous()
    ones = torch.ones(M * k, 1, dtype=torch.float32, device=A.device)
    y = fused_moe_int4_w4a16(act, w2p, w2s, flat, ones, mul_routed_weight=False, backend=Backend.HIP)
    return moe_sum_reduce(y.view(M, k, -1), w, backend=Backend.HIP)


@pytest.mark.parametrize("M,routing", [(64, "uniform"), (16, "uniform"), (1, "uniform"), (256, "zipf")])
def test_int4_layer_matches_oracle_composition(M, routing, dev):
    E, hidden, inter, k = 48, 7168, 2048, 8
    print(f"int4 layer M={M} {routing}", flush=True)
    w13p, w13s, _ = make_w4a16_weights(E, 2 * inter, hidden, 32, device=dev, seed=31, scale_hi=0.02)
    w2p, w2s, _ = make_w4a16_weights(E, hidden, inter, 32, device=dev, seed=32, scale_hi=0.02)
    g = torch.Generator(device=dev).manual_seed(33)
    A = torch.randn(M, hidden, generator=g, device=dev).to(torch.bfloat16)
    ids = (uniform_topk(M, k, E, 34) if routing == "uniform" else zipf_topk(M, k, E, 1.2, 34)).to(dev)
    w = softmax_weights(M, k, 35).to(dev)
    got = _hip_layer(A, w13p, w13s, w2p, w2s, ids, w)
    want = _oracle_layer(A, w13p, w13s, w2p, w2s, ids, w)
    assert got.shape == (M, hidden) and got.dtype == torch.bfloat16
    # the oracle's bf16 roundings of the gate/up and down outputs make the
    # summation order visible: bound the layer by 4x the spread between the
    # oracle and the same composition with float64 contractions
    alt = int4_layer_f64(A, w13p, w13s, w2p, w2s, ids, w, LIMIT)
    spread = rel_l2(want, alt)
    assert spread < 1e-2, spread
    assert rel_l2(got, want) <= 4 * spread, (rel_l2(got, want), spread)
    worst = float((want.float() - alt.float()).abs().max())
    assert float((got.float() - want.float()).abs().max()) <= 4 * worst
