"""Whole-call HIP-graph capture of the three MoE entry points that take a
workspace (the reference's tests/test_moe_workspace.py:290-315 captures align;
here the fused int4 and mxfp4 calls are captured as well).

Each test warms the call up eagerly, captures it once into a
``torch.cuda.CUDAGraph`` with address-stable workspace buffers, and then
replays it several times: before every replay new inputs are copied into the
captured input tensors, and between replays the same call runs eagerly with
fresh allocations. Every replay must equal that eager result bit for bit (same
kernels, deterministic reductions) and the oracle within the op's tolerance.
None of the captured library calls records a memset node: every buffer the
kernels read is written by an earlier kernel of the same call.
"""
from __future__ import annotations

import pytest
import torch

from oracle.torch_ref import moe_mxfp4_ref, moe_w4a16_ref
from tests._helpers import assert_close, softmax_weights, uniform_topk, zipf_topk
from xkernels_amd import (Backend, MoeAlignWorkspace, MoeInt4Workspace, MoeMxfp4Workspace,
                          fused_moe_int4_w4a16, fused_moe_mxfp4, make_mxfp4_moe_weights,
                          make_w4a16_weights, moe_align_block_size)

pytestmark = pytest.mark.gpu
REPLAYS = 4


def _capture(fn):
    """Warm up on a side stream, then capture ``fn`` (returns the graph and
    the tensors ``fn`` returned while captured)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    torch.cuda.synchronize()
    return g, out


def test_align_capture_and_replay(dev):
    M, k, E, bs = 64, 8, 48, 16
    ids = uniform_topk(M, k, E, 0).to(dev)
    ws = MoeAlignWorkspace.allocate(M, k, E, bs, device=dev)
    g, (s_g, e_g, n_g) = _capture(lambda: moe_align_block_size(ids, bs, E, truncate=False, workspace=ws,
                                                               backend=Backend.HIP))
    assert s_g.data_ptr() == ws.sorted_ids.data_ptr()
    for r in range(REPLAYS):
        print(f"align replay {r}", flush=True)
        ids.copy_(zipf_topk(M, k, E, 1.1, 10 + r).to(dev))
        g.replay()
        s_ref, e_ref, n_ref = moe_align_block_size(ids, bs, E, truncate=False, backend=Backend.HIP)
        torch.cuda.synchronize()
        assert torch.equal(n_g, n_ref)
        assert torch.equal(s_g, s_ref)
        n_blocks = int(n_ref.item()) // bs
        assert torch.equal(e_g[:n_blocks], e_ref[:n_blocks])


@pytest.mark.parametrize("M,E,N,K,k", [(64, 48, 4096, 7168, 8), (16, 8, 1024, 2048, 2), (512, 16, 512, 1024, 4)])
def test_int4_capture_and_replay(M, E, N, K, k, dev):
    print(f"int4 graph M={M} E={E} N={N} K={K} k={k}", flush=True)
    packed, scale, _ = make_w4a16_weights(E, N, K, 32, device=dev, seed=3, scale_hi=0.02)
    A = torch.empty(M, K, dtype=torch.bfloat16, device=dev)
    ids = torch.empty(M, k, dtype=torch.int32, device=dev)
    w = torch.empty(M, k, dtype=torch.float32, device=dev)

    def load(seed):
        g = torch.Generator(device=dev).manual_seed(seed)
        A.copy_(torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16))
        ids.copy_(zipf_topk(M, k, E, 1.2, seed).to(dev))
        w.copy_(softmax_weights(M, k, seed).to(dev))

    load(1)
    ws = MoeInt4Workspace.allocate(M, k, N, dtype=torch.bfloat16, device=dev, num_experts=E, K=K)

    def call(wsp=None):
        return fused_moe_int4_w4a16(A, packed, scale, ids, w, workspace=wsp, backend=Backend.HIP)

    graph, out = _capture(lambda: call(ws))
    assert out.data_ptr() == ws.out.data_ptr()
    for r in range(REPLAYS):
        print(f"  replay {r}", flush=True)
        load(100 + r)
        graph.replay()
        eager = call()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r} differs from the eager call"
        if r in (0, REPLAYS - 1):
            assert_close(out, moe_w4a16_ref(A, packed, scale, ids, w), 2e-2, 2e-2, f"replay {r}")


def test_int4_fp32_activations_capture_and_replay(dev):
    """fp32 activations (the stream kernel's split-bf16 variant) captured and
    replayed with new inputs, equal to the eager call every time."""
    M, E, N, K, k = 64, 48, 4096, 7168, 8
    packed, scale, _ = make_w4a16_weights(E, N, K, 32, device=dev, seed=4, scale_hi=0.02)
    A = torch.empty(M, K, dtype=torch.float32, device=dev)
    ids = torch.empty(M, k, dtype=torch.int32, device=dev)
    w = torch.empty(M, k, dtype=torch.float32, device=dev)

    def load(seed):
        g = torch.Generator(device=dev).manual_seed(seed)
        A.copy_(torch.randn(M, K, generator=g, device=dev))
        ids.copy_(uniform_topk(M, k, E, seed).to(dev))
        w.copy_(softmax_weights(M, k, seed).to(dev))

    load(1)
    ws = MoeInt4Workspace.allocate(M, k, N, dtype=torch.float32, device=dev, num_experts=E, K=K)
    call = lambda wsp=None: fused_moe_int4_w4a16(A, packed, scale, ids, w, workspace=wsp,  # noqa: E731
                                                 backend=Backend.HIP)
    graph, out = _capture(lambda: call(ws))
    for r in range(REPLAYS):
        print(f"int4 fp32 replay {r}", flush=True)
        load(300 + r)
        graph.replay()
        eager = call()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r} differs from the eager call"
    assert_close(out, moe_w4a16_ref(A, packed, scale, ids, w), 1e-3, 1e-3, "fp32 replay")


def test_mxfp4_capture_and_replay(dev):
    M, E, hidden, ispp, k = 48, 32, 512, 128, 6
    wts = make_mxfp4_moe_weights(E, hidden, ispp, with_bias=True, device=dev, seed=5)
    keys = ("w13", "w13_scale", "w2", "w2_scale")
    A = torch.empty(M, hidden, dtype=torch.bfloat16, device=dev)
    ids = torch.empty(M, k, dtype=torch.int32, device=dev)
    w = torch.empty(M, k, dtype=torch.float32, device=dev)

    def load(seed):
        g = torch.Generator(device=dev).manual_seed(seed)
        A.copy_(torch.randn(M, hidden, generator=g, device=dev).to(torch.bfloat16))
        ids.copy_(uniform_topk(M, k, E, seed).to(dev))
        w.copy_(softmax_weights(M, k, seed).to(dev))

    load(2)
    ws = MoeMxfp4Workspace.allocate(M, k, E, 16, ispp, hidden, dtype=torch.bfloat16, device=dev)
    call = lambda wsp=None: fused_moe_mxfp4(A, *(wts[x] for x in keys), ids, w, b13=wts["b13"],  # noqa: E731
                                            b2=wts["b2"], swiglu_limit=7.0, workspace=wsp,
                                            backend=Backend.HIP)
    graph, out = _capture(lambda: call(ws))
    assert out.data_ptr() == ws.out.data_ptr()
    for r in range(REPLAYS):
        print(f"mxfp4 replay {r}", flush=True)
        load(200 + r)
        graph.replay()
        eager = call()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r} differs from the eager call"
        ref = moe_mxfp4_ref(A, *(wts[x] for x in keys), ids, w, b13=wts["b13"], b2=wts["b2"],
                            swiglu_limit=7.0)
        assert_close(out, ref, 2e-2, 2e-2, f"mxfp4 replay {r}")
