"""moe_sum_reduce on the GPU against the oracle (sum_reduce.py:20-39).

Tolerances are the op spec's: bf16 rtol 1.6e-2 / atol 1e-2, fp32 rtol 1e-5 /
atol 1e-4. Includes the BASELINE config ([8192, 8, 7168] bf16) and an exact
known-answer case (one-hot weights select a row without rounding).
"""
from __future__ import annotations

import pytest
import torch

from oracle import c_oracle
from oracle.torch_ref import moe_sum_reduce_ref
from tests._helpers import assert_close
from xkernels_amd import Backend, moe_sum_reduce

pytestmark = pytest.mark.gpu
TOL = {torch.bfloat16: (1.6e-2, 1e-2), torch.float32: (1e-5, 1e-4)}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,top_k,H", [(128, 8, 7168), (1, 8, 7168), (37, 4, 96), (5, 3, 7),
                                       (9, 1, 64), (3, 9, 40), (16, 6, 4096), (4, 2, 12),
                                       (640, 2, 7168)])  # 2^22 outputs or more: fp32 8-wide path
@pytest.mark.parametrize("wkind", ["fp32", "bf16", "none"])
def test_matches_oracle(dtype, M, top_k, H, wkind, dev):
    g = torch.Generator().manual_seed(M * 31 + H)
    y = torch.randn(M, top_k, H, generator=g).to(dtype)
    w = None if wkind == "none" else torch.randn(M, top_k, generator=g).to(
        torch.float32 if wkind == "fp32" else torch.bfloat16)
    got = moe_sum_reduce(y.to(dev), None if w is None else w.to(dev), routed_scaling_factor=2.5,
                         backend=Backend.HIP)
    assert got.dtype == dtype and got.shape == (M, H)
    want = moe_sum_reduce_ref(y, w, 2.5)
    rtol, atol = TOL[dtype]
    assert_close(got, want, rtol, atol, "sum_reduce")


def test_one_hot_weights_select_exactly(dev):
    g = torch.Generator().manual_seed(3)
    y = torch.randn(6, 4, 256, generator=g).to(torch.bfloat16)
    w = torch.zeros(6, 4)
    pick = torch.tensor([0, 3, 1, 2, 2, 0])
    w[torch.arange(6), pick] = 1.0
    got = moe_sum_reduce(y.to(dev), w.to(dev), backend=Backend.HIP).cpu()
    assert torch.equal(got, y[torch.arange(6), pick])


def test_baseline_config_full_size(dev):
    """C3 sum_reduce: y bf16 [8192, 8, 7168], softmax fp32 weights."""
    g = torch.Generator(device=dev).manual_seed(5)
    y = torch.randn(8192, 8, 7168, generator=g, device=dev).to(torch.bfloat16)
    w = torch.softmax(torch.randn(8192, 8, generator=g, device=dev), -1)
    got = moe_sum_reduce(y, w, backend=Backend.HIP)
    want = moe_sum_reduce_ref(y, w)  # oracle evaluated on the device copy
    assert_close(got, want, 1.6e-2, 1e-2, "C3 sum_reduce")
    rows = torch.tensor([0, 1, 4095, 8191])
    c = c_oracle.sum_reduce(y[rows].cpu(), w[rows].cpu())
    assert_close(got[rows], c, 1.6e-2, 1e-2, "C3 rows vs C oracle")
