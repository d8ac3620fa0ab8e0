"""topk_softmax on the GPU against the oracle (topk_softmax.py:33-95 upstream).

ids must match exactly, including the ascending-id order of tied
probabilities (bf16/fp16 logits tie often); weights within the Op Spec's
per-dtype tolerance. Cases follow the reference's tests/test_topk_softmax.py
(:88-116) plus the edges of this kernel: E not a multiple of 64, E = 2048 (the
largest register-resident row) and above it (the streaming kernel), k = E,
k > 64, rows with many exact ties, with probabilities that underflow to 0 and
with NaN / +-inf logits, and the reference's measured shape (M=4096, E=256,
k=8).
"""
from __future__ import annotations

import pytest
import torch

from oracle.torch_ref import topk_softmax_ref
from xkernels_amd import Backend, topk_softmax

pytestmark = pytest.mark.gpu
TOL = {torch.float32: (1e-5, 1e-6), torch.bfloat16: (1e-2, 1e-2), torch.float16: (1e-2, 1e-2)}
DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def _check(g, k, renorm):
    w, ids = topk_softmax(g, k, renormalize=renorm, backend=Backend.HIP)
    rw, rids = topk_softmax_ref(g, k, renorm)
    assert w.dtype == torch.float32 and ids.dtype == torch.int32
    assert w.shape == ids.shape == (g.shape[0], k)
    bad = (ids != rids).any(dim=1)
    assert not bad.any(), f"ids differ in {int(bad.sum())} rows; first {int(bad.nonzero()[0])}: " \
                          f"{ids[bad][0].tolist()} vs {rids[bad][0].tolist()}"
    rtol, atol = TOL[g.dtype]
    torch.testing.assert_close(w, rw, rtol=rtol, atol=atol, equal_nan=True)


@pytest.mark.parametrize("M,E,k", [(8, 16, 4), (64, 256, 8), (37, 8, 2), (1, 256, 8), (8, 4, 1)])
@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("renorm", [True, False])
def test_matches_oracle(M, E, k, dt, renorm, dev):
    g = torch.randn(M, E, generator=torch.Generator(device=dev).manual_seed(M * E + k), device=dev).to(dt)
    _check(g, k, renorm)


@pytest.mark.parametrize("M,E,k", [(33, 65, 7), (5, 2048, 64), (3, 2048, 100), (4, 130, 130),
                                   (9, 1, 1), (17, 384, 12), (2, 1000, 999),
                                   (6, 2049, 8), (3, 5000, 70), (2, 3000, 300)])  # E > 2048: streaming kernel
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_edge_shapes(M, E, k, dt, dev):
    print(f"topk_softmax M={M} E={E} k={k} {dt}", flush=True)
    g = torch.randn(M, E, generator=torch.Generator(device=dev).manual_seed(E + k), device=dev).to(dt)
    _check(g, k, True)
    _check(g, k, False)


@pytest.mark.parametrize("dt", DTYPES)
def test_exact_ties_keep_ascending_ids(dev, dt):
    """Integer logits in a small range: most experts tie with several others."""
    g = torch.randint(-3, 4, (64, 256), generator=torch.Generator(device=dev).manual_seed(1),
                      device=dev).to(dt)
    _check(g, 16, True)
    _check(g, 200, False)


def test_underflowed_probabilities_tie_at_zero(dev):
    g = torch.full((4, 96), -500.0, device=dev)
    g[:, 7] = 0.0
    g[:, 50] = 1.0
    g[1, 3] = -80.0
    _check(g, 12, True)
    w, ids = topk_softmax(g, 5, renormalize=False, backend=Backend.HIP)
    assert ids[0].tolist() == [50, 7, 0, 1, 2]


def test_reference_measured_shape(dev):
    g = torch.randn(4096, 256, generator=torch.Generator(device=dev).manual_seed(2), device=dev)
    _check(g.to(torch.bfloat16), 8, True)


def test_rejects_bad_topk_and_cpu(dev):
    g = torch.randn(4, 8, device=dev)
    with pytest.raises(ValueError):
        topk_softmax(g, 0, backend=Backend.HIP)
    with pytest.raises(ValueError):
        topk_softmax(g, 9, backend=Backend.HIP)
    with pytest.raises(RuntimeError):
        topk_softmax(g.cpu(), 2, backend=Backend.HIP)


def test_empty_batch(dev):
    w, ids = topk_softmax(torch.empty(0, 64, device=dev), 4, backend=Backend.HIP)
    assert w.shape == ids.shape == (0, 4)


@pytest.mark.parametrize("dt", DTYPES)
def test_non_finite_rows(dev, dt):
    """Rows with a NaN or +inf logit, or only -inf logits, softmax to all NaN in
    the reference and select experts 0 .. k-1 (NaN keys rank first, ties to the
    lower id); rows with some -inf logits select normally. Every id stays in
    [0, E)."""
    nan, inf = float("nan"), float("inf")
    E = 130
    g = torch.randn(8, E, generator=torch.Generator(device=dev).manual_seed(5), device=dev)
    g[0, 77] = nan
    g[1, 129] = inf
    g[2] = -inf
    g[3, ::2] = -inf
    g[4, :] = -inf
    g[4, 100] = 0.0
    g[5, 64] = nan
    g[5, 3] = inf
    g = g.to(dt)
    for k in (1, 5, 70):
        # against the oracle on the CPU: torch's device softmax does not turn
        # a row holding both a NaN and a +inf (row 5) into all NaN
        for renorm in (True, False):
            w, ids = topk_softmax(g, k, renormalize=renorm, backend=Backend.HIP)
            rw, rids = topk_softmax_ref(g.cpu(), k, renorm)
            assert torch.equal(ids.cpu(), rids)
            rtol, atol = TOL[dt]
            torch.testing.assert_close(w.cpu(), rw, rtol=rtol, atol=atol, equal_nan=True)
        w, ids = topk_softmax(g, k, renormalize=True, backend=Backend.HIP)
        assert int(ids.min()) >= 0 and int(ids.max()) < E
        for r in (0, 1, 2, 5):
            assert ids[r].tolist() == list(range(k))
            assert torch.isnan(w[r]).all()
        assert int(ids[4, 0]) == 100


def test_auto_dispatch_above_2048_experts(dev):
    """backend='auto' picks the HIP kernel for any E (rows beyond 2048 experts
    stream), including the non-finite row semantics."""
    g = torch.randn(5, 4100, generator=torch.Generator(device=dev).manual_seed(8), device=dev)
    g[1, 4099] = float("nan")
    w, ids = topk_softmax(g, 6, renormalize=True)
    rw, rids = topk_softmax_ref(g.cpu(), 6, True)
    assert torch.equal(ids.cpu(), rids)
    torch.testing.assert_close(w.cpu(), rw, rtol=1e-5, atol=1e-6, equal_nan=True)
    assert ids[1].tolist() == list(range(6))
