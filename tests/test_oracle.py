"""Pins the CPU oracle (oracle/torch_ref.py and oracle/moe_oracle.c) before it is
trusted as the parity reference. The xkernels reference commits no golden
vectors for this path, so every function is pinned by checks that do not
restate its own formula:

* align: a brute-force definition on tiny inputs (for each expert, its slots in
  ascending order, padded), structural invariants (the reference's
  tests/test_moe_align_block_size.py:35-71), torch vs C restatements bit-exact;
* dequant_w4a16: hand-computed known answers (nibble order, -8 offset, group
  broadcast, one bf16 round-to-nearest-even) and the generator's chosen values;
* moe_w4a16_ref: the literal per-(token, slot) loop, a dense matmul over the
  generator's chosen weights, linearity in the routing weights, EP partitions;
* moe_sum_reduce_ref: one-hot weights select a row exactly, integer closed form;
* dequant_mxfp4: e2m1 decoded from its sign / exponent / mantissa bit fields,
  e8m0 special code 0xFF;
* moe_mxfp4_ref: independent C restatement, single-expert dense recomputation,
  EP partitions, limit disabled vs huge limit, and a hand-computed answer for
  the clamp and bias branches (tests/_mxfp4_kat.py);
* topk_softmax_ref: float64 brute force (sort by (-p, id)) on tiny rows with
  exact ties, the reference test's tie-break answer, closed forms (equal pair
  = 1/2 each, underflowed probabilities tie at 0), invariants.
"""
from __future__ import annotations

import struct

import pytest
import torch

from oracle import c_oracle
from oracle import torch_ref as R
from xkernels_amd import make_mxfp4_moe_weights, make_w4a16_weights


# ------------------------------------------------------------------ align ----

def _brute_align(ids: list[list[int]], bs: int, E: int):
    flat = [e for row in ids for e in row]
    n = len(flat)
    sorted_ids, expert_ids = [], []
    for e in range(E):
        slots = [t for t, x in enumerate(flat) if x == e]
        if not slots:
            continue
        nb = -(-len(slots) // bs)
        sorted_ids += slots + [n] * (nb * bs - len(slots))
        expert_ids += [e] * nb
    num_post = len(sorted_ids)
    max_pad = n + (E + 1) * (bs - 1)
    sorted_ids += [n] * (max_pad - num_post)
    return sorted_ids, expert_ids, num_post


@pytest.mark.parametrize("seed", range(12))
def test_align_matches_brute_force(seed):
    g = torch.Generator().manual_seed(seed)
    M = int(torch.randint(1, 9, (1,), generator=g))
    k = int(torch.randint(1, 5, (1,), generator=g))
    E = int(torch.randint(1, 7, (1,), generator=g))
    bs = int(torch.randint(1, 6, (1,), generator=g))
    ids = torch.randint(0, E, (M, k), generator=g, dtype=torch.int32)
    s_want, e_want, n_want = _brute_align(ids.tolist(), bs, E)
    s, e, n = R.moe_align_block_size_ref(ids, bs, E, truncate=True)
    assert s.tolist() == s_want
    assert e.tolist() == (e_want or [0])
    assert int(n) == n_want
    cs, ce, cn = c_oracle.align(ids, bs, E)
    assert cs.tolist() == s_want and int(cn) == n_want
    assert ce.tolist()[: len(e_want)] == e_want and all(x == 0 for x in ce.tolist()[len(e_want):])


def test_align_known_answer():
    # slots: 0->e1 1->e0 2->e1 3->e2 4->e1 5->e0 ; bs = 2, pad id 6
    ids = torch.tensor([[1, 0], [1, 2], [1, 0]], dtype=torch.int32)
    s, e, n = R.moe_align_block_size_ref(ids, 2, 3)
    assert s.tolist()[:8] == [1, 5, 0, 2, 4, 6, 3, 6]
    assert e.tolist() == [0, 1, 1, 2]
    assert int(n) == 8
    assert s.numel() == 6 + 4 * 1


@pytest.mark.parametrize("M,k,E,bs", [(8, 2, 4, 4), (16, 8, 48, 16), (1, 8, 48, 16), (32, 4, 8, 8),
                                      (300, 8, 48, 16), (64, 6, 256, 16)])
def test_align_invariants_and_restatements_agree(M, k, E, bs):
    ids = torch.randint(0, E, (M, k), generator=torch.Generator().manual_seed(M), dtype=torch.int32)
    s, e, n = R.moe_align_block_size_ref(ids, bs, E)
    total, n = M * k, int(n)
    assert n % bs == 0 and s.numel() == total + (E + 1) * (bs - 1)
    assert e.numel() == max(n // bs, 1)
    used = s[:n]
    real = used[used != total]
    assert torch.equal(real.sort().values, torch.arange(total, dtype=torch.int32))
    flat = ids.flatten()
    for b in range(n // bs):
        blk = s[b * bs:(b + 1) * bs]
        toks = blk[blk != total]
        assert torch.all(flat[toks.long()] == e[b])
        assert torch.all(toks[1:] > toks[:-1])  # ascending slot order inside an expert
    for x, y in zip(R.moe_align_block_size_ref(ids, bs, E, truncate=False), c_oracle.align(ids, bs, E)):
        assert torch.equal(x, y)


def test_align_truncate_false_and_empty():
    ids = torch.zeros((0, 4), dtype=torch.int32)
    s, e, n = R.moe_align_block_size_ref(ids, 8, 5)
    assert e.tolist() == [0] and int(n) == 0 and torch.all(s == 0)
    s, e, n = R.moe_align_block_size_ref(ids, 8, 5, truncate=False)
    assert e.numel() == -(-(6 * 7) // 8) and torch.all(e == 0)


def test_align_ep_drops_non_local():
    ids = torch.tensor([[0, 3], [2, 1], [3, 3]], dtype=torch.int32)
    emap = torch.tensor([-1, -1, 0, 1], dtype=torch.int32)  # this rank holds experts 2, 3
    s, e, n = R.moe_align_block_size_ep(ids, 2, 4, emap)
    # local rows: slot 1 (e3->1), slot 2 (e2->0), slot 4 (e3->1), slot 5 (e3->1)
    assert e.tolist() == [0, 1, 1]
    assert s.tolist()[:6] == [2, 6, 1, 4, 5, 6]
    cs, ce, cn = c_oracle.align(ids, 2, 2, expert_map=emap)
    assert cs.tolist()[:6] == s.tolist()[:6] and int(cn) == int(n)


# ------------------------------------------------------------------ int4 ----

def _bf16_rne(x: float) -> float:
    u = struct.unpack("<I", struct.pack("<f", x))[0]
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return struct.unpack("<f", struct.pack("<I", u))[0]


def test_dequant_w4a16_known_answer():
    # one row, K = 64: word 0 holds nibbles 0..7, word 1 holds 15,14,...,8
    packed = torch.zeros(1, 1, 8, dtype=torch.int32)
    packed[0, 0, 0] = 0x76543210
    packed[0, 0, 1] = int(0x89ABCDEF - (1 << 32))
    scale = torch.tensor([[[0.0117, 3.0]]]).to(torch.bfloat16)  # groups of 32
    w = R.dequant_w4a16(packed, scale, 32, out_dtype=torch.float32)
    s0 = float(scale[0, 0, 0])
    assert [float(x) for x in w[0, 0, :8]] == [(n - 8) * s0 for n in range(8)]
    assert [float(x) for x in w[0, 0, 8:16]] == [(n - 8) * s0 for n in range(15, 7, -1)]
    assert torch.all(w[0, 0, 16:32] == -8 * s0) and torch.all(w[0, 0, 32:] == -8 * 3.0)
    wb = R.dequant_w4a16(packed, scale, 32)  # bf16: one RNE of the exact product
    assert [float(x) for x in wb[0, 0, :8]] == [_bf16_rne((n - 8) * s0) for n in range(8)]
    assert torch.equal(c_oracle.dequant_int4(packed, scale).view(1, 1, 64), wb.float())


def test_dequant_matches_generator_choice():
    packed, scale, w_ref = make_w4a16_weights(3, 16, 128, 32, device="cpu", seed=5)
    assert torch.equal(R.dequant_w4a16(packed, scale, 32), w_ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("mul", [True, False])
def test_int4_ref_vs_loop_and_dense(dtype, mul):
    M, E, N, K, k = 6, 5, 24, 96, 3
    packed, scale, w_ref = make_w4a16_weights(E, N, K, 32, device="cpu", seed=2)
    g = torch.Generator().manual_seed(3)
    A = torch.randn(M, K, generator=g).to(dtype)
    ids = torch.randint(0, E, (M, k), generator=g, dtype=torch.int32)
    ids[0, 1] = ids[0, 0]  # a duplicated expert counts twice
    w = torch.rand(M, k, generator=g)
    got = R.moe_w4a16_ref(A, packed, scale, ids, w, mul_routed_weight=mul)
    loop = R.moe_w4a16_ref_loop(A, packed, scale, ids, w, mul_routed_weight=mul)
    torch.testing.assert_close(got.float(), loop.float(), rtol=1e-2 if dtype == torch.bfloat16 else 1e-5,
                               atol=1e-2 if dtype == torch.bfloat16 else 1e-5)
    # dense recomputation from the generator's chosen weights
    W = w_ref.float() if dtype == torch.bfloat16 else R.dequant_w4a16(packed, scale, 32, out_dtype=torch.float32)
    dense = torch.zeros(M, N)
    for m in range(M):
        for j in range(k):
            dense[m] += (w[m, j] if mul else 1.0) * (W[int(ids[m, j])] @ A[m].float())
    torch.testing.assert_close(got.float(), dense.to(dtype).float(), rtol=1e-2, atol=1e-2)
    c = c_oracle.int4_moe(A, packed, scale, ids, w, mul_routed_weight=mul)
    torch.testing.assert_close(got.float(), c.to(dtype).float(), rtol=1e-2, atol=1e-2)


def test_int4_ref_linear_in_routing_weights():
    packed, scale, _ = make_w4a16_weights(4, 16, 64, 32, device="cpu", seed=8)
    A = torch.randn(5, 64, generator=torch.Generator().manual_seed(1))
    ids = torch.randint(0, 4, (5, 2), generator=torch.Generator().manual_seed(2), dtype=torch.int32)
    w = torch.rand(5, 2, generator=torch.Generator().manual_seed(3))
    one = R.moe_w4a16_ref(A, packed, scale, ids, torch.ones_like(w))
    plain = R.moe_w4a16_ref(A, packed, scale, ids, w, mul_routed_weight=False)
    torch.testing.assert_close(one, plain)
    twice = R.moe_w4a16_ref(A, packed, scale, ids, 2 * w)
    torch.testing.assert_close(twice, 2 * R.moe_w4a16_ref(A, packed, scale, ids, w), rtol=1e-6, atol=1e-6)


def test_int4_ref_ep_partition_sums_to_dense():
    E, M, k = 8, 7, 3
    packed, scale, _ = make_w4a16_weights(E, 32, 64, 32, device="cpu", seed=11)
    A = torch.randn(M, 64, generator=torch.Generator().manual_seed(4))
    ids = torch.randint(0, E, (M, k), generator=torch.Generator().manual_seed(5), dtype=torch.int32)
    w = torch.rand(M, k, generator=torch.Generator().manual_seed(6))
    dense = R.moe_w4a16_ref(A, packed, scale, ids, w)
    total = torch.zeros_like(dense)
    for r in range(2):
        emap = torch.full((E,), -1, dtype=torch.int32)
        emap[r * 4:(r + 1) * 4] = torch.arange(4, dtype=torch.int32)
        part = R.moe_w4a16_ref(A, packed[r * 4:(r + 1) * 4], scale[r * 4:(r + 1) * 4], ids, w, expert_map=emap)
        total += part
        cpart = c_oracle.int4_moe(A, packed[r * 4:(r + 1) * 4], scale[r * 4:(r + 1) * 4], ids, w, expert_map=emap)
        torch.testing.assert_close(part, cpart, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(total, dense, rtol=1e-5, atol=1e-5)


# ------------------------------------------------------------ sum_reduce ----

def test_sum_reduce_one_hot_and_integers():
    y = torch.arange(2 * 3 * 4, dtype=torch.float32).view(2, 3, 4)
    w = torch.tensor([[0.0, 1.0, 0.0], [1.0, 0.0, 0.0]])
    out = R.moe_sum_reduce_ref(y, w)
    assert torch.equal(out, torch.stack([y[0, 1], y[1, 0]]))
    plain = R.moe_sum_reduce_ref(y, None, 2.0)
    # closed form: 2 * sum_k (12 m + 4 k + h) = 2 * (36 m + 12 + 3 h)
    m = torch.arange(2).view(2, 1).float()
    h = torch.arange(4).view(1, 4).float()
    assert torch.equal(plain, 2 * (36 * m + 12 + 3 * h))
    yb = torch.randn(5, 4, 33, generator=torch.Generator().manual_seed(0))
    wb = torch.randn(5, 4, generator=torch.Generator().manual_seed(1))
    torch.testing.assert_close(R.moe_sum_reduce_ref(yb, wb, 0.5), c_oracle.sum_reduce(yb, wb, 0.5),
                               rtol=1e-5, atol=1e-5)


# ----------------------------------------------------------------- mxfp4 ----

def _e2m1_from_bits(code: int) -> float:
    sign = -1.0 if code & 8 else 1.0
    e, m = (code >> 1) & 3, code & 1
    mag = m * 0.5 if e == 0 else 2.0 ** (e - 1) * (1 + m / 2)
    return sign * mag


def test_dequant_mxfp4_bit_fields_and_specials():
    # every byte value once: every (lo, hi) nibble pair, 4 rows x 128 values
    packed = torch.arange(256, dtype=torch.uint8).view(1, 4, 64)
    sc = torch.tensor([[[127, 126, 255, 0], [130, 127, 127, 127], [1, 127, 127, 127], [127, 127, 127, 127]]],
                      dtype=torch.uint8)
    w = R.dequant_mxfp4(packed, sc)
    for r in range(4):
        for kk in range(128):
            byte = int(packed[0, r, kk // 2])
            code = byte & 0xF if kk % 2 == 0 else byte >> 4
            sb = int(sc[0, r, kk // 32])
            mult = 0.0 if sb == 255 else 2.0 ** (sb - 127)
            assert float(w[0, r, kk]) == _e2m1_from_bits(code) * mult
    torch.testing.assert_close(c_oracle.dequant_mxfp4(packed, sc), w)


def test_mxfp4_dequant_matches_generator():
    wts = make_mxfp4_moe_weights(2, 64, 32, device="cpu", seed=3)
    assert torch.equal(R.dequant_mxfp4_weight(wts["w13"], wts["w13_scale"]), wts["w13_ref"])
    assert torch.equal(R.dequant_mxfp4_weight(wts["w2"], wts["w2_scale"]), wts["w2_ref"])


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("limit", [10.0, None])
def test_mxfp4_ref_vs_c_restatement(bias, limit):
    M, E, hidden, ispp, k = 5, 6, 64, 32, 2
    wts = make_mxfp4_moe_weights(E, hidden, ispp, with_bias=bias, device="cpu", seed=7)
    g = torch.Generator().manual_seed(8)
    A = torch.randn(M, hidden, generator=g).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(M)]).to(torch.int32)
    w = torch.softmax(torch.randn(M, k, generator=g), -1)
    keys = ("w13", "w13_scale", "w2", "w2_scale")
    got = R.moe_mxfp4_ref(A, *(wts[x] for x in keys), ids, w, b13=wts["b13"], b2=wts["b2"], swiglu_limit=limit)
    c = c_oracle.mxfp4_moe(A, *(wts[x] for x in keys), ids, w, b13=wts["b13"], b2=wts["b2"], swiglu_limit=limit)
    torch.testing.assert_close(got.float(), c.to(torch.bfloat16).float(), rtol=2e-2, atol=2e-2)


def test_mxfp4_ref_single_expert_dense():
    wts = make_mxfp4_moe_weights(3, 64, 32, device="cpu", seed=9)
    A = torch.randn(2, 64, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    ids = torch.tensor([[2], [2]], dtype=torch.int32)
    w = torch.tensor([[0.5], [2.0]])
    got = R.moe_mxfp4_ref(A, wts["w13"], wts["w13_scale"], wts["w2"], wts["w2_scale"], ids, w,
                          swiglu_limit=None)
    gu = (A.float() @ wts["w13_ref"][2].float().T).to(torch.bfloat16).float()
    g_, u_ = gu[:, :32], gu[:, 32:]
    act = (g_ * torch.sigmoid(g_) * u_).to(torch.bfloat16).float()
    down = (act @ wts["w2_ref"][2].float().T).to(torch.bfloat16).float()
    torch.testing.assert_close(got.float(), (down * w).to(torch.bfloat16).float(), rtol=1e-2, atol=1e-2)


def test_mxfp4_ref_limit_none_equals_huge_limit_and_ep():
    E = 4
    wts = make_mxfp4_moe_weights(E, 64, 32, device="cpu", seed=10)
    keys = ("w13", "w13_scale", "w2", "w2_scale")
    A = torch.randn(3, 64, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    ids = torch.tensor([[0, 3], [1, 2], [3, 1]], dtype=torch.int32)
    w = torch.rand(3, 2, generator=torch.Generator().manual_seed(3))
    a = R.moe_mxfp4_ref(A, *(wts[x] for x in keys), ids, w, swiglu_limit=None)
    b = R.moe_mxfp4_ref(A, *(wts[x] for x in keys), ids, w, swiglu_limit=1e30)
    assert torch.equal(a, b)
    total = torch.zeros(3, 64)
    for r in range(2):
        emap = torch.full((E,), -1, dtype=torch.int32)
        emap[2 * r:2 * r + 2] = torch.arange(2, dtype=torch.int32)
        local = [wts[x][2 * r:2 * r + 2] for x in keys]
        total += R.moe_mxfp4_ref(A.float(), *local, ids, w, swiglu_limit=None, expert_map=emap)
    torch.testing.assert_close(total, R.moe_mxfp4_ref(A.float(), *(wts[x] for x in keys), ids, w,
                                                      swiglu_limit=None), rtol=1e-5, atol=1e-5)


def test_c4_spec_tolerance_is_below_the_summation_order_spread():
    """BASELINE config C4 (E=256, hidden=4096, ispp=512, top_k=6, M=48, A ~ N(0,1),
    e8m0 exponents in [-8, 0]): the oracle against the same pipeline with float64
    contractions (bf16 roundings at the same points, mxfp4_reference.py:90-110)
    already differs beyond the op spec's elementwise 2e-2 / 2e-2. The gate/up sums
    reach ~50 and the down sums ~500, so one bf16 ulp of those rounded
    intermediates is 0.25-4, and wherever the weighted output cancels that ulp is
    large against the result. Measured on these seeded inputs: 12 of 196,608
    elements beyond the spec tolerance, max |diff| 16.0, relative L2 8.9e-5 (the
    GPU test of C4 bounds the kernel by a small multiple of the same spread on its
    own inputs)."""
    from tests._helpers import softmax_weights, uniform_topk
    from tests._orderings import moe_mxfp4_f64, rel_l2
    wts = make_mxfp4_moe_weights(256, 4096, 512, device="cpu", seed=40, scale_lo=119, scale_hi=128)
    A = torch.randn(48, 4096, generator=torch.Generator().manual_seed(41)).to(torch.bfloat16)
    ids = uniform_topk(48, 6, 256, 42)
    w = softmax_weights(48, 6, 43)
    keys = ("w13", "w13_scale", "w2", "w2_scale")
    ref = R.moe_mxfp4_ref(A, *(wts[k] for k in keys), ids, w).float()
    alt = moe_mxfp4_f64(A, *(wts[k] for k in keys), ids, w).float()
    diff = (ref - alt).abs()
    # (the exact counts can move with the CPU matmul's blocking; the claims
    # below are what the tolerance choice rests on)
    beyond = int((diff > 2e-2 + 2e-2 * alt.abs()).sum())
    assert beyond >= 1, "the spec tolerance holds between orderings here"
    assert float(diff.max()) >= 4.0
    assert 3e-5 < rel_l2(ref, alt) < 3e-4, rel_l2(ref, alt)


def test_mxfp4_ref_known_answer_clamp_and_bias():
    """Hand-computed values pin the one-sided gate clamp, the two-sided up
    clamp, b13 before the clamp and b2 before the routing weight (see
    tests/_mxfp4_kat.py for the arithmetic)."""
    from tests import _mxfp4_kat as kat
    x = kat.inputs()
    kat.check(R.moe_mxfp4_ref(x["A"], x["w13"], x["w13_scale"], x["w2"], x["w2_scale"], x["topk_ids"],
                              x["topk_w"], b13=x["b13"], b2=x["b2"], swiglu_limit=x["swiglu_limit"]))
    c = c_oracle.mxfp4_moe(x["A"], x["w13"], x["w13_scale"], x["w2"], x["w2_scale"], x["topk_ids"],
                           x["topk_w"], b13=x["b13"], b2=x["b2"], swiglu_limit=x["swiglu_limit"])
    kat.check(c.to(torch.bfloat16))


# ----------------------------------------------------------- topk_softmax ----

def _brute_topk_softmax(rows: list[list[float]], k: int, renorm: bool):
    """Float64 softmax per row, experts ordered by (-probability, id)."""
    import math
    ws, ids = [], []
    for r in rows:
        m = max(r)
        ex = [math.exp(x - m) for x in r]
        s = sum(ex)
        p = [x / s for x in ex]
        order = sorted(range(len(r)), key=lambda e: (-p[e], e))[:k]
        w = [p[e] for e in order]
        if renorm:
            t = sum(w)
            w = [x / t for x in w]
        ws.append(w)
        ids.append(order)
    return torch.tensor(ws, dtype=torch.float64), torch.tensor(ids, dtype=torch.int32)


@pytest.mark.parametrize("renorm", [True, False])
@pytest.mark.parametrize("M,E,k", [(6, 7, 3), (5, 16, 4), (3, 64, 8), (4, 9, 9), (2, 5, 1)])
def test_topk_softmax_ref_vs_brute_force(M, E, k, renorm):
    # bf16 logits: distinct values are far apart, equal values tie exactly
    g = torch.Generator().manual_seed(M * 100 + E)
    logits = (torch.randn(M, E, generator=g) * 2).to(torch.bfloat16)
    logits[0, 1] = logits[0, E - 1]  # a forced exact tie in row 0
    w, ids = R.topk_softmax_ref(logits, k, renorm)
    bw, bids = _brute_topk_softmax(logits.float().tolist(), k, renorm)
    assert ids.dtype == torch.int32 and w.dtype == torch.float32
    assert torch.equal(ids, bids)
    torch.testing.assert_close(w.double(), bw, rtol=1e-6, atol=1e-7)


def test_topk_softmax_ref_known_answers():
    # the reference's own tie-break case (tests/test_topk_softmax.py:62-74)
    g = torch.tensor([[0.1, 0.2, 0.7, 0.3, 0.0, 0.7, -1.0]])
    w, ids = R.topk_softmax_ref(g, 3, renormalize=False)
    assert ids[0].tolist() == [2, 5, 3]
    assert w[0, 0].item() == w[0, 1].item()
    # two equal logits and the rest far below: each of the pair gets 1/2
    g = torch.tensor([[3.0, -30.0, 3.0, -30.0]])
    w, ids = R.topk_softmax_ref(g, 2, renormalize=False)
    assert ids[0].tolist() == [0, 2]
    torch.testing.assert_close(w, torch.tensor([[0.5, 0.5]]), rtol=1e-6, atol=1e-6)
    # probabilities that underflow to 0 tie and keep ascending ids
    g = torch.tensor([[0.0, -200.0, 5.0, -300.0, -250.0]])
    w, ids = R.topk_softmax_ref(g, 5, renormalize=True)
    assert ids[0].tolist() == [2, 0, 1, 3, 4]
    assert w[0, 2:].tolist() == [0.0, 0.0, 0.0]
    # k = E with renorm is the full softmax, sorted
    g = torch.tensor([[1.0, 2.0, 0.0]])
    w, ids = R.topk_softmax_ref(g, 3, renormalize=True)
    assert ids[0].tolist() == [1, 0, 2]
    torch.testing.assert_close(w[0], torch.softmax(torch.tensor([2.0, 1.0, 0.0]), 0))


def test_topk_softmax_ref_non_finite_rows():
    """torch's softmax turns a row with a NaN or +inf logit, or with only -inf
    logits, into all NaN (the NaN, or inf - inf, reaches the sum), and its
    stable descending sort keeps NaN keys in ascending id order: such rows
    select experts 0 .. k-1 with NaN weights. Some -inf logits alone are only
    zero probabilities."""
    nan, inf = float("nan"), float("inf")
    g = torch.tensor([[0.5, 1.0, nan, 2.0, 0.0],
                      [1.0, 2.0, 0.0, inf, 3.0],
                      [-inf, -inf, -inf, -inf, -inf],
                      [1.0, -inf, 3.0, -inf, 2.0]])
    for renorm in (True, False):
        w, ids = R.topk_softmax_ref(g, 3, renorm)
        assert ids[:3].tolist() == [[0, 1, 2]] * 3
        assert torch.isnan(w[:3]).all()
        assert ids[3].tolist() == [2, 4, 0]
        assert not torch.isnan(w[3]).any()


def test_topk_softmax_ref_invariants_and_errors():
    g = torch.randn(32, 48, generator=torch.Generator().manual_seed(4))
    w, ids = R.topk_softmax_ref(g, 6, renormalize=True)
    torch.testing.assert_close(w.sum(1), torch.ones(32), rtol=1e-6, atol=1e-6)
    assert bool((w[:, :-1] >= w[:, 1:]).all())
    w2, ids2 = R.topk_softmax_ref(g, 6, renormalize=False)
    assert torch.equal(ids, ids2)
    torch.testing.assert_close(w2, torch.softmax(g, 1).gather(1, ids2.long()))
    assert all(len(set(r)) == 6 for r in ids.tolist())
    with pytest.raises(ValueError):
        R.topk_softmax_ref(g, 0)
    with pytest.raises(ValueError):
        R.topk_softmax_ref(g, 49)
