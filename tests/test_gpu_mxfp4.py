"""fused_moe_mxfp4 on the GPU against the oracle (mxfp4_reference.py:28-112).

Tolerance 2e-2 / 2e-2 (bf16). Follows the reference's tests/test_moe_mxfp4.py:
with and without bias and routing weight, swiglu_limit disabled, EP partials,
fp32 activations, plus the BASELINE config C4 (E=256, hidden=4096, ispp=512,
top_k=6, M=48) at full size and an exactness probe of the e2m1 decode.
"""
from __future__ import annotations

import pytest
import torch

from oracle import c_oracle
from oracle.torch_ref import moe_mxfp4_ref
from tests._helpers import assert_close, softmax_weights, uniform_topk
from xkernels_amd import Backend, MoeMxfp4Workspace, fused_moe_mxfp4, make_mxfp4_moe_weights

pytestmark = pytest.mark.gpu
KEYS = ("w13", "w13_scale", "w2", "w2_scale")


def _case(M, E, hidden, ispp, top_k, bias=False, dtype=torch.bfloat16, seed=0, **wkw):
    wts = make_mxfp4_moe_weights(E, hidden, ispp, with_bias=bias, device="cpu", seed=seed, **wkw)
    g = torch.Generator().manual_seed(seed + 1)
    A = torch.randn(M, hidden, generator=g).to(dtype)
    ids = uniform_topk(M, top_k, E, seed + 2)
    w = softmax_weights(M, top_k, seed + 3)
    return A, wts, ids, w


def _run(A, wts, ids, w, dev, **kw):
    d = lambda t: None if t is None else t.to(dev)  # noqa: E731
    return fused_moe_mxfp4(d(A), *(d(wts[k]) for k in KEYS), d(ids), d(w), b13=d(wts["b13"]),
                           b2=d(wts["b2"]), backend=Backend.HIP, **kw)


def _ref(A, wts, ids, w, **kw):
    return moe_mxfp4_ref(A, *(wts[k] for k in KEYS), ids, w, b13=wts["b13"], b2=wts["b2"], **kw)


# bf16 A and fewer than 20 routed rows per expert on average: both projections
# run the stream kernel (fp32 partial planes, SwiGLU and combine kernels);
# other shapes the per-stage kernels. Hidden 384 / ispp 640: K not a multiple
# of 256 (but of 128), the last 256-k line zero-padded.
# 600 x 8 = 4800 routed slots on 256 experts: more than the stream kernel
# routes itself, so the align outputs feed it; 200 x 8 on 64 experts (25 rows
# per expert) runs the per-stage kernels.
STREAM_SHAPES = [(4, 8, 256, 256, 2), (1, 16, 512, 256, 6), (48, 32, 512, 512, 6),
                 (33, 4, 256, 512, 2), (100, 64, 256, 256, 8), (600, 256, 256, 256, 8),
                 (200, 64, 256, 256, 8), (8, 16, 384, 640, 4), (8, 384, 256, 256, 6)]


@pytest.mark.parametrize("M,E,hidden,ispp,top_k", [(4, 8, 256, 64, 2), (1, 16, 512, 128, 6),
                                                   (7, 8, 256, 96, 3), (48, 32, 512, 64, 6),
                                                   (40, 4, 128, 32, 2)] + STREAM_SHAPES)
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("mul_routed", [True, False])
def test_matches_oracle(M, E, hidden, ispp, top_k, bias, mul_routed, dev):
    """Elementwise 2e-2 at the reference tests' input scale (A x 0.1,
    tests/test_moe_mxfp4.py:62-68 upstream). At A ~ N(0, 1) a gate/up or down
    sum that lands within an fp32 summation-order difference of a bf16 rounding
    tie rounds one ulp apart in any two implementations, and that ulp (0.125 -
    0.25 at those magnitudes) can exceed the elementwise bound downstream;
    test_full_scale_inputs covers that scale with a relative-L2 bound."""
    A, wts, ids, w = _case(M, E, hidden, ispp, top_k, bias=bias)
    A = (A.float() * 0.1).to(A.dtype)
    got = _run(A, wts, ids, w, dev, mul_routed_weight=mul_routed)
    assert got.dtype == torch.bfloat16 and got.shape == (M, hidden)
    assert_close(got, _ref(A, wts, ids, w, mul_routed_weight=mul_routed), 2e-2, 2e-2, "mxfp4")


@pytest.mark.parametrize("M,E,hidden,ispp,top_k", STREAM_SHAPES)
def test_full_scale_inputs(M, E, hidden, ispp, top_k, dev):
    """A ~ N(0, 1): the output against the oracle in relative L2, and every
    element within 2e-2 of the output's own scale."""
    A, wts, ids, w = _case(M, E, hidden, ispp, top_k, bias=True, seed=12)
    got = _run(A, wts, ids, w, dev).float().cpu()
    want = _ref(A, wts, ids, w).float()
    rel_l2 = float((got - want).norm() / want.norm())
    assert rel_l2 < 2e-3, rel_l2
    assert_close(got, want, 2e-2, 2e-2 * float(want.abs().mean()) * 8, "full scale")


@pytest.mark.parametrize("ispp", [64, 256])
@pytest.mark.parametrize("limit", [None, 0.0, 1.5])
def test_swiglu_limit(limit, ispp, dev):
    A, wts, ids, w = _case(6, 8, 256, ispp, 2, seed=4)
    got = _run(A, wts, ids, w, dev, swiglu_limit=limit)
    assert_close(got, _ref(A, wts, ids, w, swiglu_limit=limit), 2e-2, 2e-2, f"limit={limit}")


def test_fp32_activations(dev):
    A, wts, ids, w = _case(5, 8, 256, 64, 2, dtype=torch.float32, seed=5)
    got = _run(A, wts, ids, w, dev)
    assert got.dtype == torch.float32
    assert_close(got, _ref(A, wts, ids, w), 2e-2, 2e-2, "fp32 A")


@pytest.mark.parametrize("ispp", [64, 256])
def test_full_scale_range_and_special_codes(ispp, dev):
    """Scale bytes across [110, 135) plus 0xFF (reads as 0) and 0 (2^-127) in both
    the 256-k stream kernel and the generic kernel (ispp 64)."""
    A, wts, ids, w = _case(6, 4, 256, ispp, 2, seed=6, scale_lo=110, scale_hi=135)
    wts["w2_scale"][0, :3, 0] = 255
    wts["w13_scale"][1, 5, 2] = 255
    wts["w13_scale"][2, 7, 1] = 0
    wts["w2_scale"][3, 9, 1] = 0
    got = _run(A, wts, ids, w, dev)
    assert_close(got, _ref(A, wts, ids, w), 2e-2, 2e-2, "scale range")


def test_decode_is_exact_single_slot(dev):
    """One token, one expert, weight 1, no clamp: out = bf16-exact pipeline of the C oracle."""
    A, wts, _, _ = _case(1, 2, 128, 32, 1, seed=8)
    ids = torch.tensor([[1]], dtype=torch.int32)
    w = torch.ones(1, 1)
    got = _run(A, wts, ids, w, dev, swiglu_limit=None)
    want = c_oracle.mxfp4_moe(A, *(wts[k] for k in KEYS), ids, w, swiglu_limit=None)
    assert_close(got, want, 1e-2, 1e-2, "single slot")


@pytest.mark.parametrize("ispp", [64, 256])
@pytest.mark.parametrize("ep_size", [2, 4])
def test_expert_parallel_partials(ep_size, ispp, dev):
    E, M = 16, 10
    A, wts, ids, w = _case(M, E, 256, ispp, 4, seed=9)
    dense = _run(A, wts, ids, w, dev).float()
    per = E // ep_size
    total = torch.zeros_like(dense)
    for r in range(ep_size):
        emap = torch.full((E,), -1, dtype=torch.int32)
        emap[r * per:(r + 1) * per] = torch.arange(per, dtype=torch.int32)
        local = {k: (v[r * per:(r + 1) * per] if v is not None else None) for k, v in wts.items()}
        part = _run(A, local, ids, w, dev, expert_map=emap)
        assert_close(part, _ref(A, local, ids, w, expert_map=emap), 2e-2, 2e-2, f"EP rank {r}")
        total += part.float()
    assert_close(total, dense, 3e-2, 3e-2, "EP sum")


@pytest.mark.parametrize("ispp", [64, 256])
def test_workspace(ispp, dev):
    """One workspace, sized for M=16, serves M=16 and then M=3 (the stream path
    uses more K slices at M=3)."""
    ws = MoeMxfp4Workspace.allocate(16, 2, 8, 16, ispp, 256, dtype=torch.bfloat16, device=dev)
    for M in (16, 3):
        A, wts, ids, w = _case(M, 8, 256, ispp, 2, seed=M)
        got = _run(A, wts, ids, w, dev, workspace=ws)
        assert_close(got, _ref(A, wts, ids, w), 2e-2, 2e-2, f"ws M={M}")


def _c4(scale_lo, scale_hi, a_scale=1.0, with_f64=False):
    wts = make_mxfp4_moe_weights(256, 4096, 512, device="cuda", seed=40, scale_lo=scale_lo,
                                 scale_hi=scale_hi)
    g = torch.Generator(device="cuda").manual_seed(41)
    A = (torch.randn(48, 4096, generator=g, device="cuda") * a_scale).to(torch.bfloat16)
    ids = uniform_topk(48, 6, 256, 42).cuda()
    w = softmax_weights(48, 6, 43).cuda()
    got = fused_moe_mxfp4(A, *(wts[k] for k in KEYS), ids, w, backend=Backend.HIP)
    want = moe_mxfp4_ref(A, *(wts[k] for k in KEYS), ids, w)  # oracle on the device copy
    if not with_f64:
        return got.float(), want.float()
    from tests._orderings import moe_mxfp4_f64
    return got.float(), want.float(), moe_mxfp4_f64(A, *(wts[k] for k in KEYS), ids, w).float()


def test_config4_full_size_reference_test_scale(dev):
    """C4 shape at the reference test's input scale (A * 0.1, scale bytes 119..124,
    tests/test_moe_mxfp4.py:62-68 upstream): the op spec's elementwise 2e-2."""
    got, want = _c4(119, 125, a_scale=0.1)
    assert_close(got, want, 2e-2, 2e-2, "C4 reference-test scale")


def test_config4_full_size(dev):
    """C4 exactly as specified: E=256, hidden=4096, ispp=512, top_k=6, M=48, scale
    exponents uniform in [-8, 0].

    With scales up to 2^0 the gate_up sums reach ~50 and the down sums ~500, so
    one bf16 ulp of those intermediates (the reference rounds both) is 0.25-4.
    Two correct implementations that accumulate in different orders then differ
    by such ulps wherever the final sum cancels; the check therefore bounds the
    relative L2 error and each element against the spread that summation order
    alone produces on these inputs: the oracle against the same pipeline with
    float64 contractions (tests/_orderings.py; on the CPU copy of this config
    that spread is rel-L2 8.9e-5 with 12 elements beyond the spec's 2e-2, see
    tests/test_oracle.py). The kernel is held to 4x that spread: a kernel error
    of 10x the ordering noise fails."""
    from tests._orderings import rel_l2
    got, want, alt = _c4(119, 128, with_f64=True)
    spread = rel_l2(want, alt)
    assert 1e-5 < spread < 1e-3, spread
    assert rel_l2(got, want) <= 4 * spread, (rel_l2(got, want), spread)
    worst = float((want - alt).abs().max())
    assert float((got - want).abs().max()) <= 4 * worst, (float((got - want).abs().max()), worst)


def test_known_answer_clamp_and_bias(dev):
    """The hand-computed answer of tests/_mxfp4_kat.py: one-sided gate clamp,
    two-sided up clamp, b13 before the clamp, b2 before the routing weight."""
    from tests import _mxfp4_kat as kat
    x = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in kat.inputs().items()}
    out = fused_moe_mxfp4(x["A"], *(x[k] for k in KEYS), x["topk_ids"], x["topk_w"], b13=x["b13"],
                          b2=x["b2"], swiglu_limit=x["swiglu_limit"], backend=Backend.HIP)
    kat.check(out)


def _sweep_cases(n=16, seed=2027):
    """Seeded random shapes: hidden and ispp multiples of 128 (stream kernels,
    the last 256-k line zero-padded when not a multiple of 256) or of 32 (the
    per-stage kernels), 1..300 tokens on 2..300 experts, bias and SwiGLU limit
    on or off."""
    import random
    rng = random.Random(seed)
    cases = []
    for i in range(n):
        unit = rng.choice([128, 128, 32])
        E = rng.choice([2, 5, 16, 64, 130, 300])
        cases.append(dict(M=rng.choice([1, 3, 16, 48, 100, 300]), E=E,
                          hidden=unit * rng.randint(1, 8), ispp=unit * rng.randint(1, 6),
                          top_k=rng.randint(1, min(8, E)), bias=rng.random() < 0.5,
                          limit=rng.choice([None, 7.0]), seed=200 + i))
    return cases


@pytest.mark.parametrize("case", _sweep_cases(),
                         ids=lambda c: "M{M}-E{E}-h{hidden}-i{ispp}-k{top_k}".format(**c))
def test_random_shapes_match_oracle(case, dev):
    c = case
    print(f"sweep {c}", flush=True)
    A, wts, ids, w = _case(c["M"], c["E"], c["hidden"], c["ispp"], c["top_k"], bias=c["bias"],
                           seed=c["seed"])
    A = (A.float() * 0.1).to(A.dtype)
    got = _run(A, wts, ids, w, dev, swiglu_limit=c["limit"])
    assert_close(got, _ref(A, wts, ids, w, swiglu_limit=c["limit"]), 2e-2, 2e-2, "mxfp4 sweep")
