"""xk_moe_int4_w4a16_noalloc (the fused INT4 call with the library's fixed
device scratch) against xk_moe_int4_w4a16 with a caller workspace: bit-exact
on two calls in a row, the second with a smaller input, so the second call
runs over the first call's leftovers in the shared scratch."""
from __future__ import annotations

import pytest
import torch

from tests._helpers import softmax_weights, uniform_topk, zipf_topk
from xkernels_amd import _lib, make_w4a16_weights

pytestmark = pytest.mark.gpu


def _inputs(M, E, N, K, k, seed, routing="uniform"):
    packed, scale, _ = make_w4a16_weights(E, N, K, 32, device="cuda", seed=seed, scale_hi=0.02)
    g = torch.Generator(device="cuda").manual_seed(seed + 1)
    A = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
    ids = uniform_topk(M, k, E, seed + 2) if routing == "uniform" else zipf_topk(M, k, E, 1.2, seed + 2)
    return A, packed, scale, ids.cuda(), softmax_weights(M, k, seed + 3).cuda()


def _args(A, packed, scale, ids, w, flags):
    M, K = A.shape
    E, N, _ = packed.shape
    dt = _lib.XK_DT_FP32 if A.dtype == torch.float32 else _lib.XK_DT_BF16
    return [A.data_ptr(), dt, M, K, packed.data_ptr(), scale.data_ptr(), E, N, 32,
            ids.data_ptr(), w.data_ptr(), ids.shape[1], None, 0, 1, flags]


def _with_workspace(A, packed, scale, ids, w, flags=0):
    M, K = A.shape
    E, N, _ = packed.shape
    out = torch.empty(M, N, dtype=A.dtype, device="cuda")
    ws = torch.empty(_lib.query("xk_moe_int4_w4a16_workspace_bytes", M, ids.shape[1], E, N, K),
                     dtype=torch.uint8, device="cuda")
    _lib.call("xk_moe_int4_w4a16", *_args(A, packed, scale, ids, w, flags), out.data_ptr(),
              ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
    return out


def _no_alloc(A, packed, scale, ids, w, flags=0):
    out = torch.empty(A.shape[0], packed.shape[1], dtype=A.dtype, device="cuda")
    _lib.call("xk_moe_int4_w4a16_noalloc", *_args(A, packed, scale, ids, w, flags), out.data_ptr(),
              torch.cuda.current_stream().cuda_stream)
    return out


def test_no_alloc_matches_workspace_entry():
    flags = 0
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    cases = [(64, 48, 4096, 7168, 8, "uniform"),   # C2
             (5, 8, 1024, 2048, 2, "zipf")]       # smaller, over the first call's leftovers
    for M, E, N, K, k, routing in cases:
        print(f"noalloc flags={flags} M={M} E={E} N={N} K={K} k={k}", flush=True)
        x = _inputs(M, E, N, K, k, seed=M, routing=routing)
        need = _lib.query("xk_moe_int4_w4a16_workspace_bytes", M, k, E, N, K)
        assert need <= _lib.query("xk_moe_int4_w4a16_noalloc_max_bytes")
        got = _no_alloc(*x, flags=flags)
        want = _with_workspace(*x, flags=flags)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"M={M}: noalloc result differs from the workspace entry point"


def test_no_alloc_matches_workspace_entry_fp32_activations():
    """The same with fp32 activations (the stream kernel's split-bf16 variant,
    four K slices at K = 7168)."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    for M, E, N, K, k, routing in [(64, 48, 4096, 7168, 8, "uniform"), (7, 8, 1024, 2048, 2, "zipf")]:
        print(f"noalloc fp32 M={M} E={E} N={N} K={K} k={k}", flush=True)
        A, packed, scale, ids, w = _inputs(M, E, N, K, k, seed=M + 50, routing=routing)
        A = A.float()
        got = _no_alloc(A, packed, scale, ids, w)
        want = _with_workspace(A, packed, scale, ids, w)
        torch.cuda.synchronize()
        assert got.dtype == torch.float32
        assert torch.equal(got, want), f"M={M}: noalloc fp32 result differs from the workspace entry point"


def test_no_alloc_rejects_oversized_call():
    """Sizes whose scratch would exceed the fixed array fail before any launch."""
    M, E, N, K, k = 4096, 48, 4096, 7168, 8
    need = _lib.query("xk_moe_int4_w4a16_workspace_bytes", M, k, E, N, K)
    assert need > _lib.query("xk_moe_int4_w4a16_noalloc_max_bytes")
    fake = 0x1000
    rc = _lib.load().xk_moe_int4_w4a16_noalloc(fake, _lib.XK_DT_BF16, M, K, fake, fake, E, N, 32, fake,
                                               fake, k, None, 0, 1, 0, fake, None)
    assert rc == _lib.XK_ERR_INVALID
    assert "noalloc" in _lib.last_error()
