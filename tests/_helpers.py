"""Input builders shared by the tests (seeded, CPU generators, moved to device)."""
from __future__ import annotations

import torch


def zipf_topk(M: int, top_k: int, E: int, s: float, seed: int) -> torch.Tensor:
    """top_k distinct experts per token with Zipf(s) popularity (no repeats per token)."""
    g = torch.Generator().manual_seed(seed)
    p = 1.0 / torch.arange(1, E + 1, dtype=torch.float64) ** s
    perm = torch.randperm(E, generator=g)  # which expert gets which popularity rank
    probs = torch.zeros(E, dtype=torch.float64)
    probs[perm] = p / p.sum()
    ids = torch.multinomial(probs.expand(M, E), top_k, replacement=False, generator=g)
    return ids.to(torch.int32)


def uniform_topk(M: int, top_k: int, E: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.stack([torch.randperm(E, generator=g)[:top_k] for _ in range(M)]).to(torch.int32)


def softmax_weights(M: int, top_k: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.softmax(torch.randn(M, top_k, generator=g), dim=-1).float()


def assert_close(got: torch.Tensor, want: torch.Tensor, rtol: float, atol: float, msg: str = ""):
    got, want = got.detach().float().cpu(), want.detach().float().cpu()
    assert got.shape == want.shape, (got.shape, want.shape, msg)
    assert not torch.isnan(got).any(), f"NaN in result {msg}"
    bad = (got - want).abs() > atol + rtol * want.abs()
    if bad.any():
        i = int(bad.reshape(-1).nonzero()[0])
        raise AssertionError(
            f"{msg}: {int(bad.sum())}/{bad.numel()} elements out of tolerance "
            f"(rtol={rtol}, atol={atol}); first at {i}: got {got.reshape(-1)[i]:.6g} "
            f"want {want.reshape(-1)[i]:.6g}; max abs err {(got - want).abs().max():.3g}"
        )


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 values at |x| (8 significant bits), floored at the
    smallest normal's spacing."""
    a = x.detach().float().abs().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


def assert_within_bf16_ulps(got: torch.Tensor, want: torch.Tensor, ulps: float, msg: str = ""):
    """|got - want| <= ulps * (bf16 spacing at want), element by element."""
    got, want = got.detach().float().cpu(), want.detach().float().cpu()
    assert got.shape == want.shape, (got.shape, want.shape, msg)
    err = (got - want).abs()
    lim = ulps * bf16_ulp(want)
    bad = ~(err <= lim)
    if bad.any():
        i = int(bad.reshape(-1).nonzero()[0])
        raise AssertionError(f"{msg}: {int(bad.sum())}/{bad.numel()} elements beyond {ulps} bf16 ulp; "
                             f"first at {i}: got {got.reshape(-1)[i]:.8g} want {want.reshape(-1)[i]:.8g}; "
                             f"max err in ulps {float((err / bf16_ulp(want)).max()):.3g}")
