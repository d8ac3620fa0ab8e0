"""A hand-computed known answer for the MXFP4 MoE (mxfp4_reference.py:90-110):
tiny e2m1 weights whose products are exact, chosen so that every branch of the
expert body shows up in its own output column.

One expert, hidden 64, ispp 32, swiglu_limit 10. Only column 0 of the w13
rows 0..4 (gate) and 32..36 (up) is non-zero, scale byte 129 (x4); w2 is the
identity on columns 0..4 (scale byte 127). Token 0 is e_0 with routing weight
0.5, token 1 is 0.5 e_0 with routing weight 2. Output column j then reads
``bf16(bf16(silu(clamp(g_j)) * clamp(u_j)) + b2_j) * r`` for one (g_j, u_j):

  col 0  gate 24 - 2 (b13) = 22 is clamped to 10 (bias before the clamp)
  col 1  gate -24 stays: the gate clamp is one-sided (max only)
  col 2  up -24 is clamped to -10 (the up clamp is two-sided)
  col 3  up 24 is clamped to 10
  col 4  b13 on both halves, no clamp: gate 8 + 0.5, up 2 - 0.25
  col 5  no expert output, only b2 = -1: b2 is added before the routing weight

Each expected value below is worked out by hand, with the bf16 rounding of
the activation at the step size of its binade. The alternatives a plausible
misreading would give are listed beside them; every one is off by more than
one bf16 ulp.
"""
from __future__ import annotations

import math

import torch

E2M1 = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)
HIDDEN, ISPP, LIMIT = 64, 32, 10.0


def _code(v: float) -> int:
    return E2M1.index(abs(v)) | (8 if v < 0 else 0)


def _pack(rows: torch.Tensor) -> torch.Tensor:
    """[..., K] e2m1 values -> [..., K/2] bytes, element 2i in the low nibble."""
    codes = rows.clone().apply_(lambda v: _code(v)).to(torch.uint8)
    return codes[..., 0::2] | (codes[..., 1::2] << 4)


def inputs():
    w13 = torch.zeros(1, 2 * ISPP, HIDDEN)
    # (gate, up) per intermediate column j, before the x4 scale
    for j, (g, u) in enumerate([(6.0, 1.0), (-6.0, 2.0), (1.0, -6.0), (0.5, 6.0), (2.0, 0.5)]):
        w13[0, j, 0], w13[0, ISPP + j, 0] = g, u
    w2 = torch.zeros(1, HIDDEN, ISPP)
    for j in range(5):
        w2[0, j, j] = 1.0
    b13 = torch.zeros(1, 2 * ISPP)
    b13[0, 0] = -2.0
    b13[0, 4], b13[0, ISPP + 4] = 0.5, -0.25
    b2 = torch.zeros(1, HIDDEN)
    b2[0, [0, 2, 3, 4]] = 2.0
    b2[0, 5] = -1.0
    A = torch.zeros(2, HIDDEN)
    A[0, 0], A[1, 0] = 1.0, 0.5
    return dict(
        A=A.to(torch.bfloat16),
        w13=_pack(w13), w13_scale=torch.full((1, 2 * ISPP, HIDDEN // 32), 129, dtype=torch.uint8),
        w2=_pack(w2), w2_scale=torch.full((1, HIDDEN, ISPP // 32), 127, dtype=torch.uint8),
        topk_ids=torch.zeros(2, 1, dtype=torch.int32), topk_w=torch.tensor([[0.5], [2.0]]),
        b13=b13.to(torch.bfloat16), b2=b2.to(torch.bfloat16), swiglu_limit=LIMIT)


def _tiny(gate: float, up: float, r: float) -> float:
    """Column 1: silu of a large negative gate, far below one bf16 ulp of 1."""
    return gate / (1.0 + math.exp(-gate)) * up * r


# token 0 (x = 1, r = 0.5):
#   c0: silu(10) * 4  = 39.98 -> 40.0  (step 1/4);  +2 -> 42     * 0.5 = 21
#       [bias after clamp: silu(8)*4 = 31.99 -> 16.99; no gate clamp: 87.99 -> 44.99]
#   c1: silu(-24) * 8 = -7.25e-9 * 0.5                 [two-sided gate clamp: -1.8e-3]
#   c2: silu(4) * -10 = -39.28 -> -39.25;  +2 -> -37.25  * 0.5 = -18.625   [no clamp: -46.1]
#   c3: silu(2) * 10  = 17.616 -> 17.625 (step 1/8); +2 -> 19.625 * 0.5 = 9.8125
#   c4: silu(8.5) * 1.75 = 14.872 -> 14.875 (1/16); +2 -> 16.875 * 0.5 = 8.4375
#       [b13 dropped: silu(8)*2 = 15.99 -> 8.99]
#   c5: -1 * 0.5 = -0.5                                [b2 after the weight: -1]
# token 1 (x = 0.5, r = 2):
#   c0: gate 12 - 2 = 10 (at the limit): silu(10) * 2 = 19.99 -> 20; +2 -> 22 * 2 = 44
#   c1: silu(-12) * 4 * 2
#   c2: silu(2) * -10 = -17.616 -> -17.625; +2 -> -15.625 * 2 = -31.25
#   c3: silu(1) * 10 = 7.3106 -> 7.3125 (1/32); +2 -> 9.3125 * 2 = 18.625
#   c4: silu(4.5) * 0.75 = 3.3379 -> 3.34375 (1/64); +2 -> 5.34375 * 2 = 10.6875
#   c5: -1 * 2 = -2
EXPECTED_EXACT = {  # (token, column) -> value, exact in bf16
    (0, 0): 21.0, (0, 2): -18.625, (0, 3): 9.8125, (0, 4): 8.4375, (0, 5): -0.5,
    (1, 0): 44.0, (1, 2): -31.25, (1, 3): 18.625, (1, 4): 10.6875, (1, 5): -2.0,
}
EXPECTED_TINY = {(0, 1): _tiny(-24.0, 8.0, 0.5), (1, 1): _tiny(-12.0, 4.0, 2.0)}


def check(out: torch.Tensor) -> None:
    """Asserts the known answer on a [2, 64] output."""
    out = out.float().cpu()
    assert out.shape == (2, HIDDEN)
    for (t, c), v in EXPECTED_EXACT.items():
        assert float(out[t, c]) == v, f"token {t} column {c}: {float(out[t, c])} != {v}"
    for (t, c), v in EXPECTED_TINY.items():
        assert abs(float(out[t, c]) - v) <= 1e-2 * abs(v), f"token {t} column {c}: {float(out[t, c])} vs {v}"
    rest = out.clone()
    rest[:, :6] = 0
    assert torch.count_nonzero(rest) == 0
