"""The INT4 grouped GEMM's per-slot rows against an error-bounded reference.

The reference rounds every dequantised weight to bf16 before the contraction
(w4a16.py:42-50: ``(nibble - 8) * scale`` in fp32, then ``.to(bf16)``). The
spec's 2e-2 tolerance cannot tell rounded weights from exact ones, so these
tests call the GEMM stage (``xk_moe_int4_w4a16_gemm``) directly and compare
its fp32 row of every routed slot with a float64 contraction over the
oracle's bf16-rounded weights, allowing only fp32 summation error:

    |got - want| <= 2^-20 * sum_k |a_k * w_k| + 1e-30

(K <= 7168 terms summed in fp32 add at most about K * 2^-24 relative to the
absolute sum; the kernels sum in groups, which is far tighter). A kernel that
contracted the exact (n - 8) * s products instead differs by the weights'
rounding, about 2^-9 of each term, and fails the bound: a negative control
checks that rows computed from the exact products are told apart.
"""
from __future__ import annotations

import pytest
import torch

from oracle.torch_ref import dequant_w4a16
from tests._helpers import uniform_topk, zipf_topk
from xkernels_amd import _lib, make_w4a16_weights

pytestmark = pytest.mark.gpu

REL = 2.0 ** -20


def _gemm_rows(A, packed, scale, ids, flags=0, self_route=False, emap=None, gs=32):
    """fp32 per-slot rows of the grouped GEMM (align with the library's block size,
    or none: the decode kernel then routes the slots itself)."""
    M, K = A.shape
    E, N, _ = packed.shape
    top_k = ids.shape[1]
    numel = M * top_k
    dev = A.device
    dt = _lib.XK_DT_FP32 if A.dtype == torch.float32 else _lib.XK_DT_BF16
    bs = _lib.query("xk_moe_int4_block_size", M, top_k, E)
    max_pad = numel + (E + 1) * (bs - 1)
    sorted_ids = torch.empty(max_pad, dtype=torch.int32, device=dev)
    expert_ids = torch.empty((max_pad + bs - 1) // bs, dtype=torch.int32, device=dev)
    num_post = torch.empty(1, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    aws = torch.empty(max(1, _lib.query("xk_moe_align_workspace_bytes", numel, E)), dtype=torch.uint8,
                      device=dev)
    s = torch.cuda.current_stream().cuda_stream
    ng = 0 if emap is None else emap.numel()
    ep = None if emap is None else emap.data_ptr()
    _lib.call("xk_moe_align_block_size", ids.data_ptr(), numel, E, bs, ep, ng, sorted_ids.data_ptr(),
              expert_ids.data_ptr(), num_post.data_ptr(), offsets.data_ptr(), aws.data_ptr(),
              aws.numel(), s)
    parts = _lib.query("xk_moe_int4_gemm_parts", M, top_k, E, N, K, dt, gs, flags)
    out = torch.full((parts, numel, N), float("nan"), dtype=torch.float32, device=dev)
    gws = torch.empty(max(256, _lib.query("xk_moe_int4_gemm_workspace_bytes", M, K)), dtype=torch.uint8,
                      device=dev)
    _lib.call("xk_moe_int4_w4a16_gemm", A.data_ptr(), dt, M, K, packed.data_ptr(),
              scale.data_ptr(), E, N, gs, ids.data_ptr(), top_k, ep, ng,
              None if self_route else sorted_ids.data_ptr(), None if self_route else offsets.data_ptr(),
              out.data_ptr(), flags, gws.data_ptr(), gws.numel(), s)
    torch.cuda.synchronize()
    return out.sum(0)


def _bounded_check(A, packed, scale, ids, rows, rel=REL, w_dtype=torch.bfloat16, emap=None, gs=32):
    """Compares every routed slot's row, one expert at a time (float64 reference
    over the weights dequantised to ``w_dtype``: bf16-rounded for bf16
    activations, the exact fp32 products for fp32 ones)."""
    top_k = ids.shape[1]
    flat = ids.reshape(-1).long()
    if emap is not None:
        flat = emap.long()[flat]
    worst = 0.0
    for e in flat.unique().tolist():
        if e < 0:
            continue
        slots = (flat == e).nonzero().reshape(-1)
        W = dequant_w4a16(packed[e:e + 1], scale[e:e + 1], gs, out_dtype=w_dtype)[0].double()
        a = A[slots // top_k].double()
        want = a @ W.T
        bound = rel * (a.abs() @ W.abs().T) + 1e-30
        err = (rows[slots].double() - want).abs()
        ratio = float((err / bound).max())
        worst = max(worst, ratio)
        assert ratio <= 1.0, f"expert {e}: error {ratio:.3g} x the fp32-summation bound"
    return worst


def _device_inputs(M, E, N, K, ids, seed, gs=32):
    packed, scale, _ = make_w4a16_weights(E, N, K, gs, device="cuda", seed=seed, scale_hi=0.02)
    g = torch.Generator(device="cuda").manual_seed(seed + 1)
    A = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
    return A, packed, scale, ids.cuda()


@pytest.mark.parametrize("M,E,N,K,top_k,routing", [
    (64, 48, 4096, 7168, 8, "uniform"),    # C2, the headline (most experts one 16-row tile)
    (16, 8, 1024, 2048, 2, "uniform"),     # C1
    (64, 48, 7168, 2048, 8, "uniform"),    # the down projection of the same layer
    (16, 48, 7168, 2048, 8, "uniform"),    # ... at M = 16 and M = 1
    (1, 48, 7168, 2048, 8, "uniform"),
    (64, 16, 512, 1024, 4, "zipf"),        # experts with several 16-row passes (stream kernel)
    (192, 16, 512, 1024, 4, "zipf"),       # 48 rows per expert: the tile kernel
    (40, 6, 160, 768, 3, "zipf"),          # K / 256 odd: one-tile passes only
    (64, 48, 2880, 2880, 8, "uniform"),    # K % 256 != 0: the last 256-k line zero-padded
    (1, 16, 256, 320, 4, "uniform"),       # ... 64 k in the last line
    (200, 8, 256, 1344, 4, "zipf"),        # ... experts with several 16-row passes
    (16, 8, 512, 2080, 2, "zipf"),         # K % 64 != 0: 65 scales a row (2-byte scale loads)
    (37, 8, 48, 96, 3, "zipf"),            # the spec's sweep point: K = 96, N = 48 (a half column pair)
    (20, 6, 80, 160, 2, "uniform"),        # N % 32 == 16, 5 scales a row
    (2, 4, 16, 32, 2, "uniform"),          # one 16-column tile, one 32-k group
    (16, 384, 256, 512, 8, "uniform"),     # 384 local experts (the stream kernel takes up to 512)
    (5, 4, 96, 512, 2, "uniform"),         # N not a multiple of 128
    (1024, 8, 512, 1024, 4, "zipf"),       # prefill regime: the MFMA tile kernel
    (300, 16, 512, 512, 4, "zipf"),        # ... experts of < 128, 129-255 and > 256 rows
    (4096, 48, 4096, 7168, 8, "zipf"),     # C5 at full size, every row (tile kernel)
])
def test_rows_within_fp32_summation_error(M, E, N, K, top_k, routing):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    ids = uniform_topk(M, top_k, E, 3) if routing == "uniform" else zipf_topk(M, top_k, E, 1.2, 3)
    print(f"case M={M} E={E} N={N} K={K} top_k={top_k} {routing}", flush=True)
    A, packed, scale, ids = _device_inputs(M, E, N, K, ids, 11)
    rows = _gemm_rows(A, packed, scale, ids)
    assert not torch.isnan(rows).any(), "a routed slot's row was not written"
    _bounded_check(A, packed, scale, ids, rows)


KERNEL = {0: "scalar", 1: "stream", 2: "tile"}


@pytest.mark.parametrize("M,E,N,K,top_k,gs,routing,kernel", [
    (64, 48, 4096, 7168, 8, 128, "uniform", "stream"),  # C2 shapes with 128-wide groups
    (64, 48, 7168, 2048, 8, 64, "uniform", "stream"),   # the down projection, 64-wide groups
    (1, 16, 256, 1024, 4, 128, "uniform", "stream"),
    (64, 16, 512, 1024, 4, 64, "zipf", "stream"),       # several 16-row passes per expert
    (48, 8, 256, 1152, 2, 64, "zipf", "stream"),        # K % 256 != 0: 4-byte scale loads, padded line
    (40, 6, 160, 1536, 3, 128, "zipf", "stream"),       # 12 scales a row: 4-byte scale loads
    (1024, 8, 512, 1024, 4, 128, "zipf", "tile"),       # prefill regime
    (300, 16, 512, 2048, 4, 64, "zipf", "tile"),
    (16, 8, 512, 1344, 2, 64, "uniform", "stream"),     # 21 scales a row (odd): 2-byte scale loads
    (16, 8, 256, 1280, 2, 256, "uniform", "scalar"),    # groups of 256: the scalar kernel
])
def test_group_sizes_64_128_on_mfma_kernels(M, E, N, K, top_k, gs, routing, kernel):
    """Groups of 64 and 128 run on the MFMA kernels (the decode stream kernel
    and the prefill tile kernel; the query reports which) and every routed
    slot's row meets the fp32-summation bound over the bf16-rounded weights of
    that group size."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from xkernels_amd import _lib
    assert KERNEL[_lib.query("xk_moe_int4_kernel", M, top_k, E, N, K, _lib.XK_DT_BF16, gs, 0, 0)] == kernel
    ids = uniform_topk(M, top_k, E, 7) if routing == "uniform" else zipf_topk(M, top_k, E, 1.2, 7)
    print(f"group {gs} M={M} E={E} N={N} K={K} top_k={top_k} {routing} -> {kernel}", flush=True)
    A, packed, scale, ids = _device_inputs(M, E, N, K, ids, 17, gs=gs)
    rows = _gemm_rows(A, packed, scale, ids, gs=gs)
    assert not torch.isnan(rows).any(), "a routed slot's row was not written"
    _bounded_check(A, packed, scale, ids, rows, gs=gs)
    if kernel == "stream":  # fp32 activations on the same kernel, exact products
        rows32 = _gemm_rows(A.float(), packed, scale, ids, gs=gs)
        _bounded_check(A.float(), packed, scale, ids, rows32, rel=2.0 ** -15, w_dtype=torch.float32, gs=gs)


def test_bound_tells_unrounded_weights_apart():
    """Negative control: rows contracted over the exact (n - 8) * s products
    (no bf16 rounding of the weights) break the bound the kernels' rows meet."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    M, E, N, K, top_k = 64, 48, 4096, 7168, 8
    ids = uniform_topk(M, top_k, E, 3)
    A, packed, scale, ids = _device_inputs(M, E, N, K, ids, 11)
    flat = ids.reshape(-1).long()
    rows = torch.empty(M * top_k, N, dtype=torch.float64, device=A.device)
    for e in flat.unique().tolist():
        slots = (flat == e).nonzero().reshape(-1)
        W = dequant_w4a16(packed[e:e + 1], scale[e:e + 1], 32, out_dtype=torch.float32)[0].double()
        rows[slots] = A[slots // top_k].double() @ W.T
    with pytest.raises(AssertionError, match="fp32-summation bound"):
        _bounded_check(A, packed, scale, ids, rows)


@pytest.mark.parametrize("M,E,N,K,top_k,routing,ep", [
    (64, 48, 4096, 7168, 8, "uniform", False),  # C2
    (64, 16, 512, 1024, 4, "zipf", False),      # several 16-row passes per expert
    (32, 48, 7168, 2048, 8, "zipf", True),      # expert map: half the experts local
    (1, 48, 4096, 7168, 8, "uniform", False),
])
def test_self_routed_rows_equal_aligned_rows(M, E, N, K, top_k, routing, ep):
    """Without align outputs the decode kernel routes the slots itself; every
    written row equals the align-fed kernel's bit for bit (same kernel, same
    per-row arithmetic), dropped slots stay untouched."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    print(f"self-route M={M} E={E} N={N} K={K} k={top_k} {routing} ep={ep}", flush=True)
    ids = uniform_topk(M, top_k, E, 5) if routing == "uniform" else zipf_topk(M, top_k, E, 1.2, 5)
    A, packed, scale, ids = _device_inputs(M, E, N, K, ids, 13)
    emap = None
    if ep:
        E_loc = E // 2
        emap = torch.full((E,), -1, dtype=torch.int32, device="cuda")
        emap[E_loc:] = torch.arange(E_loc, dtype=torch.int32, device="cuda")
        packed, scale = packed[E_loc:].contiguous(), scale[E_loc:].contiguous()
    aligned = _gemm_rows(A, packed, scale, ids, emap=emap)
    routed = _gemm_rows(A, packed, scale, ids, emap=emap, self_route=True)
    assert torch.equal(torch.isnan(aligned), torch.isnan(routed))
    assert torch.equal(torch.nan_to_num(aligned), torch.nan_to_num(routed))
    if ep:
        local = (ids.reshape(-1) >= E // 2)
        assert not torch.isnan(routed[local]).any() and torch.isnan(routed[~local]).all()


# fp32 activations: the reference contracts them with the exact (n - 8) * s
# products in fp32 (w4a16.py:21-50 dequantises to the activation dtype). The
# MFMA stream kernel splits both operands into bf16 pairs (the weight split is
# exact, the activation split leaves 2^-17 of |a|) and drops the lo * lo
# product (2^-18 of |a w|), so every row is within 2^-15 of sum |a w|; a
# kernel that rounded the activations to bf16 (2^-9 of each term) fails it.
REL_F32 = 2.0 ** -15


@pytest.mark.parametrize("M,E,N,K,top_k,routing", [
    (64, 48, 4096, 7168, 8, "uniform"),    # C2 shape with fp32 activations
    (16, 8, 1024, 2048, 2, "uniform"),     # C1 shape
    (64, 16, 512, 1024, 4, "zipf"),        # experts with several 16-row passes
    (1024, 8, 512, 1024, 4, "zipf"),       # prefill regime: fp32 stays on the stream kernel
    (64, 48, 2880, 2880, 8, "uniform"),    # K % 256 != 0: the padded variant
    (1, 16, 256, 320, 4, "uniform"),
    (16, 8, 512, 2080, 2, "zipf"),         # K % 64 != 0: 65 scales a row (2-byte scale loads)
    (37, 8, 48, 96, 3, "zipf"),            # the spec's sweep point: K = 96, N = 48 (a half column pair)
    (20, 6, 80, 160, 2, "uniform"),        # N % 32 == 16, 5 scales a row
    (2, 4, 16, 32, 2, "uniform"),          # one 16-column tile, one 32-k group
    (16, 384, 256, 512, 8, "uniform"),     # 384 local experts
])
def test_fp32_rows_within_split_error(M, E, N, K, top_k, routing):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    ids = uniform_topk(M, top_k, E, 3) if routing == "uniform" else zipf_topk(M, top_k, E, 1.2, 3)
    print(f"fp32 case M={M} E={E} N={N} K={K} top_k={top_k} {routing}", flush=True)
    A, packed, scale, ids = _device_inputs(M, E, N, K, ids, 11)
    g = torch.Generator(device="cuda").manual_seed(17)
    A = torch.randn(M, K, generator=g, device="cuda")  # full fp32 mantissas
    rows = _gemm_rows(A, packed, scale, ids)
    assert not torch.isnan(rows).any(), "a routed slot's row was not written"
    _bounded_check(A, packed, scale, ids, rows, rel=REL_F32, w_dtype=torch.float32)


def test_fp32_bound_tells_bf16_activations_apart():
    """Negative control: the same kernel fed the activations rounded to bf16
    breaks the fp32 bound against the unrounded activations."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    M, E, N, K, top_k = 16, 8, 1024, 2048, 2
    ids = uniform_topk(M, top_k, E, 3)
    _, packed, scale, ids = _device_inputs(M, E, N, K, ids, 11)
    A = torch.randn(M, K, generator=torch.Generator(device="cuda").manual_seed(17), device="cuda")
    rows = _gemm_rows(A.to(torch.bfloat16).float(), packed, scale, ids)
    with pytest.raises(AssertionError, match="fp32-summation bound"):
        _bounded_check(A, packed, scale, ids, rows, rel=REL_F32, w_dtype=torch.float32)


@pytest.mark.parametrize("M,E,N,K,top_k,ep", [(64, 48, 4096, 7168, 8, False), (64, 48, 7168, 2048, 8, True)])
def test_fp32_self_routed_rows_equal_aligned_rows(M, E, N, K, top_k, ep):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    print(f"fp32 self-route M={M} E={E} N={N} K={K} k={top_k} ep={ep}", flush=True)
    ids = zipf_topk(M, top_k, E, 1.2, 5)
    _, packed, scale, ids = _device_inputs(M, E, N, K, ids, 13)
    A = torch.randn(M, K, generator=torch.Generator(device="cuda").manual_seed(19), device="cuda")
    emap = None
    if ep:
        E_loc = E // 2
        emap = torch.full((E,), -1, dtype=torch.int32, device="cuda")
        emap[E_loc:] = torch.arange(E_loc, dtype=torch.int32, device="cuda")
        packed, scale = packed[E_loc:].contiguous(), scale[E_loc:].contiguous()
    aligned = _gemm_rows(A, packed, scale, ids, emap=emap)
    routed = _gemm_rows(A, packed, scale, ids, emap=emap, self_route=True)
    assert torch.equal(torch.isnan(aligned), torch.isnan(routed))
    assert torch.equal(torch.nan_to_num(aligned), torch.nan_to_num(routed))
    _bounded_check(A, packed, scale, ids, torch.nan_to_num(routed), rel=REL_F32, w_dtype=torch.float32,
                   emap=emap)


def _sweep_cases(n=24, seed=2026):
    """Seeded random shapes over the kernels' eligibility boundaries: K a
    multiple of 64 (stream kernel; K % 256 != 0 takes the padded variant), N a
    multiple of 32, 1..64 and a few hundred experts, 1..300 tokens (stream and
    tile kernels), bf16 and fp32 activations, align-fed or self-routed, with or
    without an expert map."""
    import random
    rng = random.Random(seed)
    cases = []
    for i in range(n):
        E = rng.choice([2, 3, 5, 8, 16, 33, 48, 64, 200])
        top_k = rng.randint(1, min(8, E))
        cases.append(dict(M=rng.choice([1, 2, 7, 16, 37, 64, 130, 300]), E=E,
                          N=32 * rng.randint(1, 32), K=64 * rng.randint(1, 48), top_k=top_k,
                          routing=rng.choice(["uniform", "zipf"]),
                          fp32=rng.random() < 0.3, self_route=rng.random() < 0.5,
                          ep=rng.random() < 0.25, seed=100 + i))
    return cases


@pytest.mark.parametrize("case", _sweep_cases(), ids=lambda c: "M{M}-E{E}-N{N}-K{K}-k{top_k}".format(**c))
def test_random_shapes_within_bound(case):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    c = case
    print(f"sweep {c}", flush=True)
    M, E, N, K, top_k = c["M"], c["E"], c["N"], c["K"], c["top_k"]
    ids = (uniform_topk(M, top_k, E, c["seed"]) if c["routing"] == "uniform"
           else zipf_topk(M, top_k, E, 1.2, c["seed"]))
    A, packed, scale, ids = _device_inputs(M, E, N, K, ids, c["seed"])
    if c["fp32"]:
        A = torch.randn(M, K, generator=torch.Generator(device="cuda").manual_seed(c["seed"]), device="cuda")
    emap = None
    if c["ep"] and E >= 2:
        E_loc = E // 2
        emap = torch.full((E,), -1, dtype=torch.int32, device="cuda")
        emap[E - E_loc:] = torch.arange(E_loc, dtype=torch.int32, device="cuda")
        packed, scale = packed[E - E_loc:].contiguous(), scale[E - E_loc:].contiguous()
    # without align outputs only the decode kernel runs (it routes for itself);
    # the others refuse the call
    rows = None
    if c["self_route"]:
        try:
            rows = _gemm_rows(A, packed, scale, ids, emap=emap, self_route=True)
        except RuntimeError as err:
            assert "align outputs" in str(err), err
    if rows is None:
        rows = _gemm_rows(A, packed, scale, ids, emap=emap)
    flat = ids.reshape(-1).long()
    local = torch.ones_like(flat, dtype=torch.bool) if emap is None else emap.long()[flat] >= 0
    assert not torch.isnan(rows[local]).any(), "a routed local slot's row was not written"
    if c["fp32"]:
        _bounded_check(A, packed, scale, ids, torch.nan_to_num(rows), rel=REL_F32, w_dtype=torch.float32,
                       emap=emap)
    else:
        _bounded_check(A, packed, scale, ids, torch.nan_to_num(rows), emap=emap)


def _sweep_cases_groups(n=16, seed=2027):
    """Seeded random shapes over the eligibility added for groups of 64 and
    128: K a multiple of 32 and of the group (odd scale counts per row load 2
    bytes at a time), N a multiple of 16 (a half column pair), groups of 32, 64
    or 128, some shapes large enough for the prefill tile kernel (N and K
    multiples of 256), bf16 and fp32 activations, align-fed or self-routed,
    with or without an expert map."""
    import random
    rng = random.Random(seed)
    cases = []
    for i in range(n):
        E = rng.choice([2, 5, 8, 16, 33, 48])
        gs = rng.choice([32, 64, 128])
        N = 256 * rng.randint(1, 3) if rng.random() < 0.35 else 16 * rng.randint(1, 40)
        K = 256 * rng.randint(1, 12) if rng.random() < 0.35 else gs * rng.randint(1, 4096 // gs)
        cases.append(dict(M=rng.choice([1, 3, 16, 40, 64, 200, 600]), E=E, N=N, K=K,
                          top_k=rng.randint(1, min(8, E)), gs=gs,
                          routing=rng.choice(["uniform", "zipf"]), fp32=rng.random() < 0.25,
                          self_route=rng.random() < 0.5, ep=rng.random() < 0.25, seed=300 + i))
    return cases


@pytest.mark.parametrize("case", _sweep_cases_groups(),
                         ids=lambda c: "M{M}-E{E}-N{N}-K{K}-k{top_k}-g{gs}".format(**c))
def test_random_group_shapes_within_bound(case):
    c = case
    M, E, N, K, top_k, gs = c["M"], c["E"], c["N"], c["K"], c["top_k"], c["gs"]
    dt = _lib.XK_DT_FP32 if c["fp32"] else _lib.XK_DT_BF16
    kern = _lib.query("xk_moe_int4_kernel", M, top_k, E, N, K, dt, gs, 0, 0)
    print(f"group sweep {c} kernel {kern}", flush=True)
    ids = (uniform_topk(M, top_k, E, c["seed"]) if c["routing"] == "uniform"
           else zipf_topk(M, top_k, E, 1.2, c["seed"]))
    A, packed, scale, ids = _device_inputs(M, E, N, K, ids, c["seed"], gs)
    if c["fp32"]:
        A = torch.randn(M, K, generator=torch.Generator(device="cuda").manual_seed(c["seed"]), device="cuda")
    emap = None
    if c["ep"] and E >= 2:
        E_loc = E // 2
        emap = torch.full((E,), -1, dtype=torch.int32, device="cuda")
        emap[E - E_loc:] = torch.arange(E_loc, dtype=torch.int32, device="cuda")
        packed, scale = packed[E - E_loc:].contiguous(), scale[E - E_loc:].contiguous()
    rows = None
    if c["self_route"]:
        try:
            rows = _gemm_rows(A, packed, scale, ids, emap=emap, self_route=True, gs=gs)
        except RuntimeError as err:
            assert "align outputs" in str(err), err
    if rows is None:
        rows = _gemm_rows(A, packed, scale, ids, emap=emap, gs=gs)
    flat = ids.reshape(-1).long()
    local = torch.ones_like(flat, dtype=torch.bool) if emap is None else emap.long()[flat] >= 0
    assert not torch.isnan(rows[local]).any(), "a routed local slot's row was not written"
    if c["fp32"]:
        _bounded_check(A, packed, scale, ids, torch.nan_to_num(rows), rel=REL_F32, w_dtype=torch.float32,
                       emap=emap, gs=gs)
    else:
        _bounded_check(A, packed, scale, ids, torch.nan_to_num(rows), emap=emap, gs=gs)
