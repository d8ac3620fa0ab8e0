"""The prefill-regime INT4 tile kernel (MFMA tiles of 256 routed rows x 256
columns) against the oracle and against the decode stream kernel.

Both kernels dequantise to the reference's bf16-rounded weights, so their fp32
per-slot rows differ only by fp32 summation order (checked at 1e-4 relative);
the fused outputs meet the op spec's bf16 tolerance against the oracle. Cases
cover skewed (Zipf) routing with partial and empty row blocks, experts with no
tokens, more tiles than workgroups, expert parallelism and the unweighted sum,
and fixed per-expert row counts that give every tile height (256, 192, 128 and
64 rows) and every tile order class.
"""
from __future__ import annotations

import pytest
import torch

from oracle.torch_ref import moe_w4a16_ref
from tests._helpers import assert_close, softmax_weights, uniform_topk, zipf_topk
from xkernels_amd import _lib, make_w4a16_weights

pytestmark = pytest.mark.gpu


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _fused(A, packed, scale, ids, w, flags, emap=None, mul=1):
    M, K = A.shape
    E, N, _ = packed.shape
    k = ids.shape[1]
    out = torch.empty(M, N, dtype=torch.bfloat16, device=A.device)
    nb = _lib.query("xk_moe_int4_w4a16_workspace_bytes", M, k, E, N, K)
    ws = torch.empty(nb, dtype=torch.uint8, device=A.device)
    _lib.call("xk_moe_int4_w4a16", A.data_ptr(), _lib.XK_DT_BF16, M, K, packed.data_ptr(),
              scale.data_ptr(), E, N, 32, ids.data_ptr(), w.data_ptr(), k,
              None if emap is None else emap.data_ptr(), 0 if emap is None else emap.numel(), mul,
              flags, out.data_ptr(), ws.data_ptr(), ws.numel(), _stream())
    return out


def _slot_rows(A, packed, scale, ids, flags, gws=None):
    """Align (block 16) then the GEMM stage alone: fp32 rows per routed slot
    (gws: the GEMM's workspace, which holds the tile kernel's queue; without
    one the tiles are dealt statically)."""
    M, K = A.shape
    E, N, _ = packed.shape
    k = ids.shape[1]
    numel = M * k
    bs = _lib.query("xk_moe_int4_block_size", M, k, E)
    max_pad = numel + (E + 1) * (bs - 1)
    dev = A.device
    sorted_ids = torch.empty(max_pad, dtype=torch.int32, device=dev)
    expert_ids = torch.empty((max_pad + bs - 1) // bs, dtype=torch.int32, device=dev)
    num_post = torch.empty(1, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    ws = torch.empty(max(1, _lib.query("xk_moe_align_workspace_bytes", numel, E)), dtype=torch.uint8,
                     device=dev)
    _lib.call("xk_moe_align_block_size", ids.data_ptr(), numel, E, bs, None, 0, sorted_ids.data_ptr(),
              expert_ids.data_ptr(), num_post.data_ptr(), offsets.data_ptr(), ws.data_ptr(), ws.numel(),
              _stream())
    parts = _lib.query("xk_moe_int4_gemm_parts", M, k, E, N, K, _lib.XK_DT_BF16, 32, flags)
    slot_out = torch.full((parts, numel, N), float("nan"), dtype=torch.float32, device=dev)
    _lib.call("xk_moe_int4_w4a16_gemm", A.data_ptr(), _lib.XK_DT_BF16, M, K, packed.data_ptr(),
              scale.data_ptr(), E, N, 32, ids.data_ptr(), k, None, 0, sorted_ids.data_ptr(),
              offsets.data_ptr(), slot_out.data_ptr(), flags, None if gws is None else gws.data_ptr(),
              0 if gws is None else gws.numel(), _stream())
    return slot_out.sum(0)


def _inputs(M, E, N, K, ids, seed, scale_hi=0.02):
    packed, scale, _ = make_w4a16_weights(E, N, K, 32, device="cuda", seed=seed, scale_hi=scale_hi)
    g = torch.Generator(device="cuda").manual_seed(seed + 1)
    A = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
    w = softmax_weights(M, ids.shape[1], seed + 2).cuda()
    return A, packed, scale, ids.to(torch.int32).cuda(), w


# Routed rows per expert for the "classes" routing (top_k = 1; the align pads
# each expert to 16 rows): 608 = two full blocks + a 96-row tail, 176 and 144
# (129-192-row tails), 256 (exactly one full block), 32, none, 240 (a tail above
# 192 rows, ordered with the full blocks), 80 (65-128), 704 = two full blocks +
# a 192-row tail.
CLASS_ROWS = [600, 170, 250, 30, 0, 230, 129, 65, 700]


def _ids(M, top_k, E, routing, seed):
    if routing == "zipf":
        return zipf_topk(M, top_k, E, 1.2, seed)
    if routing == "classes":
        assert top_k == 1 and E == len(CLASS_ROWS) and M == sum(CLASS_ROWS)
        ids = torch.cat([torch.full((n,), e, dtype=torch.int32) for e, n in enumerate(CLASS_ROWS)])
        g = torch.Generator().manual_seed(seed)
        return ids[torch.randperm(M, generator=g)].reshape(M, 1)
    return uniform_topk(M, top_k, E, seed)


CASES = [  # M, E, N, K, top_k, routing
    (300, 8, 512, 512, 4, "zipf"),      # partial row blocks, skew
    (1024, 16, 256, 1024, 2, "zipf"),   # some experts empty
    (96, 6, 768, 256, 3, "uniform"),    # one step pair, 3 column blocks
    (2048, 48, 1024, 2048, 8, "zipf"),  # more tiles than workgroups
    (16, 8, 1024, 2048, 2, "uniform"),  # C1 shape, forced onto the tile kernel
    (sum(CLASS_ROWS), len(CLASS_ROWS), 512, 512, 1, "classes"),  # every tile height and order class
    (600, 1, 256, 512, 1, "uniform"),   # one expert: three row blocks, the last a tail
    (512, 1024, 256, 256, 4, "zipf"),   # the most experts the tile kernel takes, most of them empty
]


@pytest.mark.parametrize("M,E,N,K,top_k,routing", CASES)
def test_tile_kernel_rows_match_stream_kernel(M, E, N, K, top_k, routing, dev):
    print(f"tile vs stream M={M} E={E} N={N} K={K} k={top_k} {routing}", flush=True)
    ids = _ids(M, top_k, E, routing, M)
    A, packed, scale, ids, _ = _inputs(M, E, N, K, ids, seed=M + 3)
    tile = _slot_rows(A, packed, scale, ids, _lib._XK_INT4_TEST_FORCE_TILE)
    stream = _slot_rows(A, packed, scale, ids, _lib._XK_INT4_TEST_FORCE_STREAM)
    torch.cuda.synchronize()
    assert not torch.isnan(tile).any(), "a routed slot row was not written"
    assert_close(tile, stream, 1e-4, 1e-4 * float(stream.abs().mean()), "tile vs stream rows")


@pytest.mark.parametrize("M,E,N,K,top_k,routing", CASES)
def test_tile_queue_equals_static_deal(M, E, N, K, top_k, routing, dev):
    """The tile queue (workgroups take tiles atomically, then the other XCDs'
    ranges) computes every tile exactly once: its rows equal the static deal's
    bit for bit, from a buffer of NaNs, over two calls with one workspace."""
    print(f"tile queue M={M} E={E} N={N} K={K} k={top_k} {routing}", flush=True)
    ids = _ids(M, top_k, E, routing, M + 7)
    A, packed, scale, ids, _ = _inputs(M, E, N, K, ids, seed=M + 9)
    need = _lib.query("xk_moe_int4_gemm_workspace_bytes", M, K)
    assert need > 0
    gws = torch.randint(0, 256, (need,), dtype=torch.uint8, device=dev)  # the queue is cleared per call
    static = _slot_rows(A, packed, scale, ids, _lib._XK_INT4_TEST_FORCE_TILE)
    for _ in range(2):
        queued = _slot_rows(A, packed, scale, ids, _lib._XK_INT4_TEST_FORCE_TILE, gws)
        torch.cuda.synchronize()
        assert not torch.isnan(queued).any(), "a routed slot row was not written"
        assert torch.equal(queued, static)


@pytest.mark.parametrize("M,E,N,K,top_k,routing", CASES)
def test_tile_kernel_matches_oracle(M, E, N, K, top_k, routing, dev):
    print(f"tile vs oracle M={M} E={E} N={N} K={K} k={top_k} {routing}", flush=True)
    ids = _ids(M, top_k, E, routing, M + 1)
    A, packed, scale, ids, w = _inputs(M, E, N, K, ids, seed=M + 5)
    got = _fused(A, packed, scale, ids, w, _lib._XK_INT4_TEST_FORCE_TILE)
    assert_close(got, moe_w4a16_ref(A, packed, scale, ids, w), 2e-2, 2e-2, "tile fused")


def test_tile_kernel_unweighted_and_expert_parallel(dev):
    M, E, N, K, k = 512, 16, 512, 1024, 4
    ids = zipf_topk(M, k, E, 1.1, 77)
    A, packed, scale, ids, w = _inputs(M, E, N, K, ids, seed=78)
    got = _fused(A, packed, scale, ids, w, _lib._XK_INT4_TEST_FORCE_TILE, mul=0)
    assert_close(got, moe_w4a16_ref(A, packed, scale, ids, w, mul_routed_weight=False), 2e-2, 2e-2,
                 "tile unweighted")
    dense = moe_w4a16_ref(A, packed, scale, ids, w).float()
    total = torch.zeros_like(dense)
    for r in range(2):
        emap = torch.full((E,), -1, dtype=torch.int32, device="cuda")
        emap[r * 8:(r + 1) * 8] = torch.arange(8, dtype=torch.int32, device="cuda")
        lp, ls = packed[r * 8:(r + 1) * 8].contiguous(), scale[r * 8:(r + 1) * 8].contiguous()
        part = _fused(A, lp, ls, ids, w, _lib._XK_INT4_TEST_FORCE_TILE, emap=emap)
        total += part.float()
    assert_close(total, dense, 3e-2, 3e-2, "tile EP partials")


def test_default_choice_uses_tile_kernel_at_prefill_sizes(dev):
    """numel >= 17 E selects the tile kernel by default; its result equals the
    forced tile kernel's bit for bit."""
    M, E, N, K, k = 1024, 16, 512, 512, 4
    ids = zipf_topk(M, k, E, 1.2, 5)
    A, packed, scale, ids, _ = _inputs(M, E, N, K, ids, seed=6)
    default = _slot_rows(A, packed, scale, ids, 0)
    tile = _slot_rows(A, packed, scale, ids, _lib._XK_INT4_TEST_FORCE_TILE)
    assert torch.equal(default, tile)


def test_batch_past_buffer_reach_runs_in_token_chunks(dev):
    """150,000 tokens at K = 7168: 2.15 GB of activations, past what the MFMA
    kernels address through 32-bit buffer offsets (one launch would take the
    scalar kernel). The fused call runs token chunks on the MFMA kernels, and a
    token's output depends only on its own slots, so it equals two calls over
    another split of the batch bit for bit."""
    M, E, N, K, k = 150_000, 4, 256, 7168, 1
    print(f"token chunks M={M} E={E} N={N} K={K}", flush=True)
    kern = lambda m: _lib.query("xk_moe_int4_kernel", m, k, E, N, K, _lib.XK_DT_BF16, 32, 0, 0)
    assert kern(M) == 0 and kern(M // 2) == 2
    ids = uniform_topk(M, k, E, 41)
    A, packed, scale, ids, w = _inputs(M, E, N, K, ids, seed=43)
    whole = _fused(A, packed, scale, ids, w, 0)
    cut = 100_000
    parts = torch.cat([_fused(A[:cut], packed, scale, ids[:cut], w[:cut], 0),
                       _fused(A[cut:], packed, scale, ids[cut:], w[cut:], 0)])
    torch.cuda.synchronize()
    assert torch.isfinite(whole.float()).all()
    assert torch.equal(whole, parts)
