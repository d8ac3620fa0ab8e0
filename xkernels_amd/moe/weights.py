"""Seeded synthetic weight generators (data creation only; no op math).

Same names, shapes and value ranges as the reference's generators
(src/xkernels/ops/moe/w4a16.py:158-176 and mxfp4.py:59-124). The ``*_ref``
tensors are the values the generator chose, written out directly from the
chosen integer codes (not decoded from the packed bytes), so a test can compare
a kernel's decode against them.
"""
from __future__ import annotations

import torch

E2M1_VALUES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)


def make_w4a16_weights(E: int, N: int, K: int, group_size: int = 32, *, device="cuda", seed=0,
                       scale_lo: float = 0.005, scale_hi: float = 0.025):
    """Random ``uint4b8`` weights.

    Returns ``(packed [E,N,K//8] int32, scale [E,N,K//g] bf16, w_ref [E,N,K] bf16)``;
    ``w_ref = bf16((q - 8) * scale)`` for the chosen nibbles ``q``. Scales are
    ``U(scale_lo, scale_hi)`` (the reference generator uses 0.005..0.025).
    """
    if K % 8 or K % group_size:
        raise ValueError("K must be a multiple of 8 and of group_size")
    g = torch.Generator(device=device).manual_seed(seed)
    q = torch.randint(0, 16, (E, N, K), generator=g, device=device, dtype=torch.int32)
    shifts = torch.arange(8, device=device, dtype=torch.int32) * 4
    packed = (q.view(E, N, K // 8, 8) << shifts).sum(dim=-1).to(torch.int32)
    scale = (
        torch.rand((E, N, K // group_size), generator=g, device=device, dtype=torch.float32)
        * (scale_hi - scale_lo) + scale_lo
    ).to(torch.bfloat16)
    w_ref = ((q.float() - 8.0).view(E, N, K // group_size, group_size)
             * scale.float().unsqueeze(-1)).view(E, N, K).to(torch.bfloat16)
    return packed, scale, w_ref


def make_mxfp4_moe_weights(E: int, hidden: int, ispp: int, *, group_size: int = 32,
                           with_bias: bool = False, device="cuda", seed: int = 0,
                           scale_lo: int = 119, scale_hi: int = 125):
    """Random MXFP4 expert weights (any byte is a valid e2m1 pair).

    Returns a dict with ``w13 [E,2*ispp,hidden//2]``, ``w13_scale``, ``w2
    [E,hidden,ispp//2]``, ``w2_scale`` (uint8; scale bytes in
    ``[scale_lo, scale_hi)``), ``b13`` / ``b2`` (bf16 or None) and the chosen
    values ``w13_ref`` / ``w2_ref`` (bf16).
    """
    if hidden % group_size or ispp % group_size:
        raise ValueError("hidden and ispp must be multiples of group_size")
    g = torch.Generator(device=device).manual_seed(seed)
    lut = torch.tensor(E2M1_VALUES, device=device, dtype=torch.float32)

    def _make(rows: int, cols: int):
        codes = torch.randint(0, 256, (E, rows, cols // 2), generator=g, device=device, dtype=torch.uint8)
        sc = torch.randint(scale_lo, scale_hi, (E, rows, cols // group_size), generator=g,
                           device=device, dtype=torch.uint8)
        c = codes.to(torch.int64)
        vals = torch.stack((lut[c & 0xF], lut[c >> 4]), dim=-1).reshape(E, rows, cols)
        mult = torch.where(sc == 255, torch.zeros((), device=device),
                           torch.exp2(sc.float() - 127.0))
        ref = (vals * mult.repeat_interleave(group_size, dim=-1)).to(torch.bfloat16)
        return codes, sc, ref

    w13, w13_scale, w13_ref = _make(2 * ispp, hidden)
    w2, w2_scale, w2_ref = _make(hidden, ispp)
    out = {"w13": w13, "w13_scale": w13_scale, "w2": w2, "w2_scale": w2_scale,
           "w13_ref": w13_ref, "w2_ref": w2_ref, "b13": None, "b2": None}
    if with_bias:
        out["b13"] = (torch.rand(E, 2 * ispp, generator=g, device=device) * 0.2 - 0.1).to(torch.bfloat16)
        out["b2"] = (torch.rand(E, hidden, generator=g, device=device) * 0.2 - 0.1).to(torch.bfloat16)
    return out
