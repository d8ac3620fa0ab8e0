"""Writes the small golden fixtures under tests/golden/ (numpy .npz, no pickles).

The xkernels reference commits no vectors for the MoE path, so these fixtures
are produced by this repository's own oracle (oracle/torch_ref.py) after the
oracle has been pinned by tests/test_oracle.py. Their job is to freeze the
oracle: a later edit of the oracle that changes any output fails
tests/test_golden.py, and the GPU tests compare the HIP kernels with the same
bytes. Inputs are stored, not regenerated, so the fixtures do not depend on the
weight generators either.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import torch_ref as R  # noqa: E402
from xkernels_amd import make_mxfp4_moe_weights, make_w4a16_weights  # noqa: E402


def _bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy()


def align_cases() -> dict[str, np.ndarray]:
    out = {}
    # the last three exceed one workgroup (numel > 8192): the grid path
    cases = [("tiny", 3, 2, 3, 2, 0), ("decode", 64, 8, 48, 16, 1), ("skew", 40, 6, 8, 16, 2),
             ("bs1", 9, 3, 5, 1, 3), ("ep", 32, 4, 16, 8, 4), ("grid", 1500, 8, 48, 16, 5),
             ("grid_wide", 1100, 8, 600, 4, 6), ("grid_ep", 1300, 8, 64, 64, 7)]
    for name, M, k, E, bs, seed in cases:
        g = torch.Generator().manual_seed(seed)
        if name == "skew":  # every slot on experts 0/1: most blocks pad-only tails
            ids = torch.randint(0, 2, (M, k), generator=g, dtype=torch.int32)
        elif name.startswith("grid"):  # Zipf-like expert popularity
            p = 1.0 / torch.arange(1, E + 1, dtype=torch.float64) ** 1.1
            ids = torch.multinomial(p.expand(M, E), k, replacement=False, generator=g).to(torch.int32)
        else:
            ids = torch.randint(0, E, (M, k), generator=g, dtype=torch.int32)
        emap = None
        nl = E
        if name in ("ep", "grid_ep"):
            nl = 8 if name == "ep" else 24
            emap = torch.full((E,), -1, dtype=torch.int32)
            emap[4:4 + nl] = torch.arange(nl, dtype=torch.int32)
            s, e, n = R.moe_align_block_size_ep(ids, bs, E, emap)
        else:
            s, e, n = R.moe_align_block_size_ref(ids, bs, E, truncate=False)
        out[f"align_{name}_ids"] = ids.numpy()
        out[f"align_{name}_meta"] = np.array([bs, nl], dtype=np.int32)
        if emap is not None:
            out[f"align_{name}_emap"] = emap.numpy()
        out[f"align_{name}_sorted"] = s.numpy()
        out[f"align_{name}_expert_ids"] = e.numpy()
        out[f"align_{name}_num_post"] = np.array([int(n)], dtype=np.int32)
    return out


def int4_case() -> dict[str, np.ndarray]:
    M, E, N, K, k = 8, 4, 64, 256, 2
    packed, scale, _ = make_w4a16_weights(E, N, K, 32, device="cpu", seed=31)
    g = torch.Generator().manual_seed(32)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(M)]).to(torch.int32)
    w = torch.softmax(torch.randn(M, k, generator=g), -1)
    out = R.moe_w4a16_ref(A, packed, scale, ids, w)
    return {"int4_A": _bf16_bits(A), "int4_packed": packed.numpy(), "int4_scale": _bf16_bits(scale),
            "int4_ids": ids.numpy(), "int4_w": w.numpy(), "int4_out": _bf16_bits(out),
            "int4_out_f32": R.moe_w4a16_ref(A.float(), packed, scale, ids, w).numpy()}


def mxfp4_case() -> dict[str, np.ndarray]:
    M, E, hidden, ispp, k = 6, 4, 128, 64, 2
    wts = make_mxfp4_moe_weights(E, hidden, ispp, with_bias=True, device="cpu", seed=41)
    g = torch.Generator().manual_seed(42)
    A = (torch.randn(M, hidden, generator=g) * 0.5).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(M)]).to(torch.int32)
    w = torch.softmax(torch.randn(M, k, generator=g), -1)
    out = R.moe_mxfp4_ref(A, wts["w13"], wts["w13_scale"], wts["w2"], wts["w2_scale"], ids, w,
                          b13=wts["b13"], b2=wts["b2"], swiglu_limit=7.0)
    d = {"mx_A": _bf16_bits(A), "mx_ids": ids.numpy(), "mx_w": w.numpy(), "mx_out": _bf16_bits(out)}
    for key in ("w13", "w13_scale", "w2", "w2_scale"):
        d[f"mx_{key}"] = wts[key].numpy()
    d["mx_b13"] = _bf16_bits(wts["b13"])
    d["mx_b2"] = _bf16_bits(wts["b2"])
    return d


def sum_reduce_case() -> dict[str, np.ndarray]:
    g = torch.Generator().manual_seed(51)
    y = torch.randn(5, 4, 96, generator=g)
    w = torch.rand(5, 4, generator=g)
    return {"sr_y": y.numpy(), "sr_w": w.numpy(), "sr_out": R.moe_sum_reduce_ref(y, w, 1.5).numpy(),
            "sr_y_bf16": _bf16_bits(y), "sr_out_bf16": _bf16_bits(R.moe_sum_reduce_ref(y.bfloat16(), w, 1.5))}


def build() -> dict[str, np.ndarray]:
    d = {}
    for part in (align_cases(), int4_case(), mxfp4_case(), sum_reduce_case()):
        d.update(part)
    return d


if __name__ == "__main__":
    np.savez_compressed(HERE / "moe_golden.npz", **build())
    print("wrote", HERE / "moe_golden.npz")
