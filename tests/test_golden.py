"""Committed golden fixtures (tests/golden/moe_golden.npz, written by
tests/golden/make_golden.py from the pinned oracle). CPU: both oracle
restatements still reproduce them bit-for-bit. GPU: the HIP path, called
through the C ABI, reproduces the align fixtures bit-exactly (including the
expert-parallel remap) and the int4 and mxfp4 fixtures within one or two bf16 ulp and the reduce
fixtures within the op spec's tolerance."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import c_oracle
from oracle import torch_ref as R
from tests._helpers import assert_within_bf16_ulps

G = np.load(Path(__file__).resolve().parent / "golden" / "moe_golden.npz")
ALIGN = ["tiny", "decode", "skew", "bs1", "ep", "grid", "grid_wide", "grid_ep"]


def _t(key):
    return torch.from_numpy(G[key].copy())


def _bf16(key):
    return _t(key).view(torch.bfloat16)


# ------------------------------------------------------------------- CPU ----

@pytest.mark.parametrize("name", ALIGN)
def test_oracles_reproduce_align_fixture(name):
    ids = _t(f"align_{name}_ids")
    bs, nl = (int(x) for x in G[f"align_{name}_meta"])
    if name in ("ep", "grid_ep"):
        emap = _t(f"align_{name}_emap")
        s, e, n = R.moe_align_block_size_ep(ids, bs, emap.numel(), emap)
        cs, ce, cn = c_oracle.align(ids, bs, nl, expert_map=emap)
        assert torch.equal(cs, s)
    else:
        s, e, n = R.moe_align_block_size_ref(ids, bs, nl, truncate=False)
        cs, ce, cn = c_oracle.align(ids, bs, nl)
        assert torch.equal(cs, s) and torch.equal(ce, e) and int(cn) == int(n)
    assert np.array_equal(s.numpy(), G[f"align_{name}_sorted"])
    assert np.array_equal(e.numpy(), G[f"align_{name}_expert_ids"])
    assert int(n) == int(G[f"align_{name}_num_post"][0])


# Floating-point fixtures are compared at one bf16 ulp (bf16 outputs) and 1e-5
# (fp32): the CPU matmul's summation order differs between hosts and BLAS
# builds, which can move an fp32 sum by a few ulps and, rarely, a bf16 rounding.
BF16_ULP = dict(rtol=2 ** -7, atol=1e-6)
F32_TOL = dict(rtol=1e-5, atol=1e-6)


def test_oracle_reproduces_int4_fixture():
    args = (_bf16("int4_A"), _t("int4_packed"), _bf16("int4_scale"), _t("int4_ids"), _t("int4_w"))
    torch.testing.assert_close(R.moe_w4a16_ref(*args).float(), _bf16("int4_out").float(), **BF16_ULP)
    torch.testing.assert_close(R.moe_w4a16_ref(args[0].float(), *args[1:]), _t("int4_out_f32"), **F32_TOL)


def test_oracle_reproduces_mxfp4_fixture():
    out = R.moe_mxfp4_ref(_bf16("mx_A"), _t("mx_w13"), _t("mx_w13_scale"), _t("mx_w2"),
                          _t("mx_w2_scale"), _t("mx_ids"), _t("mx_w"), b13=_bf16("mx_b13"),
                          b2=_bf16("mx_b2"), swiglu_limit=7.0)
    torch.testing.assert_close(out.float(), _bf16("mx_out").float(), **BF16_ULP)


def test_oracle_reproduces_sum_reduce_fixture():
    torch.testing.assert_close(R.moe_sum_reduce_ref(_t("sr_y"), _t("sr_w"), 1.5), _t("sr_out"), **F32_TOL)
    torch.testing.assert_close(R.moe_sum_reduce_ref(_bf16("sr_y_bf16"), _t("sr_w"), 1.5).float(),
                               _bf16("sr_out_bf16").float(), **BF16_ULP)


# ------------------------------------------------------------------- GPU ----

@pytest.mark.gpu
@pytest.mark.parametrize("name", ALIGN)
def test_hip_align_matches_fixture(name, dev):
    from xkernels_amd import _lib

    ids = _t(f"align_{name}_ids").to(dev)
    bs, nl = (int(x) for x in G[f"align_{name}_meta"])
    numel = ids.numel()
    max_pad = numel + (nl + 1) * (bs - 1)
    sorted_ids = torch.full((max_pad,), -7, dtype=torch.int32, device=dev)
    expert_ids = torch.full(((max_pad + bs - 1) // bs,), -7, dtype=torch.int32, device=dev)
    num_post = torch.empty(1, dtype=torch.int32, device=dev)
    ws = torch.full((max(1, _lib.query("xk_moe_align_workspace_bytes", numel, nl)),), 0x7F,
                    dtype=torch.uint8, device=dev)  # stale scratch must not matter
    emap = _t(f"align_{name}_emap").to(dev) if name in ("ep", "grid_ep") else None
    stream = torch.cuda.current_stream().cuda_stream
    _lib.call("xk_moe_align_block_size", ids.data_ptr(), numel, nl, bs,
              None if emap is None else emap.data_ptr(), 0 if emap is None else emap.numel(),
              sorted_ids.data_ptr(), expert_ids.data_ptr(), num_post.data_ptr(), None,
              ws.data_ptr(), ws.numel(), stream)
    torch.cuda.synchronize()
    assert np.array_equal(sorted_ids.cpu().numpy(), G[f"align_{name}_sorted"])
    n = int(G[f"align_{name}_num_post"][0])
    assert int(num_post.item()) == n
    want = G[f"align_{name}_expert_ids"]
    assert np.array_equal(expert_ids.cpu().numpy()[: len(want)], want)


@pytest.mark.gpu
def test_hip_int4_matches_fixture(dev):
    from xkernels_amd import fused_moe_int4_w4a16

    out = fused_moe_int4_w4a16(_bf16("int4_A").to(dev), _t("int4_packed").to(dev),
                               _bf16("int4_scale").to(dev), _t("int4_ids").to(dev),
                               _t("int4_w").to(dev), backend="hip")
    # the kernel and the fixture round the same fp32 sums to bf16; only the
    # summation order differs, so at most one bf16 ulp apart
    assert_within_bf16_ulps(out, _bf16("int4_out"), 1, "int4 fixture")
    out32 = fused_moe_int4_w4a16(_bf16("int4_A").float().to(dev), _t("int4_packed").to(dev),
                                 _bf16("int4_scale").to(dev), _t("int4_ids").to(dev),
                                 _t("int4_w").to(dev), backend="hip")
    torch.testing.assert_close(out32.cpu(), _t("int4_out_f32"), rtol=1e-5, atol=1e-5)


@pytest.mark.gpu
def test_hip_mxfp4_matches_fixture(dev):
    from xkernels_amd import fused_moe_mxfp4

    out = fused_moe_mxfp4(_bf16("mx_A").to(dev), _t("mx_w13").to(dev), _t("mx_w13_scale").to(dev),
                          _t("mx_w2").to(dev), _t("mx_w2_scale").to(dev), _t("mx_ids").to(dev),
                          _t("mx_w").to(dev), b13=_bf16("mx_b13").to(dev), b2=_bf16("mx_b2").to(dev),
                          swiglu_limit=7.0, backend="hip")
    # one ulp of the output, plus what one bf16 ulp of an intermediate activation
    # moves a down-projection sum (bounded by 2^-8 of the sum of magnitudes)
    assert_within_bf16_ulps(out, _bf16("mx_out"), 2, "mxfp4 fixture")


@pytest.mark.gpu
def test_hip_sum_reduce_matches_fixture(dev):
    from xkernels_amd import moe_sum_reduce

    out = moe_sum_reduce(_t("sr_y").to(dev), _t("sr_w").to(dev), routed_scaling_factor=1.5, backend="hip")
    torch.testing.assert_close(out.cpu(), _t("sr_out"), rtol=1e-6, atol=1e-5)
    outb = moe_sum_reduce(_bf16("sr_y_bf16").to(dev), _t("sr_w").to(dev), routed_scaling_factor=1.5,
                          backend="hip")
    torch.testing.assert_close(outb.float().cpu(), _bf16("sr_out_bf16").float(), rtol=8e-3, atol=8e-3)
