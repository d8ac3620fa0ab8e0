"""Analytical FLOP / byte models per sweep point and per-arch roofline ceilings.

Same role as the reference's registry/cost_model.py:38-151: ``verify(...,
measure_perf=True)`` divides these by the measured time to report TFLOP/s and
% of DRAM bandwidth. Bytes are ALGORITHMIC (each input read once, each output
written once); for the grouped GEMMs the weight bytes count the experts that
can be active, ``min(E, M*top_k)``.
"""
from __future__ import annotations

from collections.abc import Callable
from typing import Any

from .dtypes import dtype_bytes

# fp32_tflops: vector fp32 ceiling (reference convention); dram_bw_gbs: HBM peak;
# mfma_bf16_tflops: dense bf16 matrix-core peak (no sparsity).
_ARCH_PEAKS: dict[str, dict[str, float]] = {
    "nvidia_sm121": {"fp32_tflops": 29.5, "dram_bw_gbs": 243.0},
    "nvidia_sm80": {"fp32_tflops": 19.5, "dram_bw_gbs": 1550.0},
    "nvidia_sm90": {"fp32_tflops": 67.0, "dram_bw_gbs": 3000.0},
    "nvidia_sm100": {"fp32_tflops": 28.0, "dram_bw_gbs": 8000.0},
    "amd_cdna2": {"fp32_tflops": 24.0, "dram_bw_gbs": 3276.0},
    "amd_cdna3": {"fp32_tflops": 80.0, "dram_bw_gbs": 5300.0},
    # MI355X (gfx950): 256 CUs, HBM3E 8 TB/s, bf16 MFMA 2.5 PFLOP/s dense.
    "amd_cdna4": {"fp32_tflops": 157.3, "dram_bw_gbs": 8000.0, "mfma_bf16_tflops": 2500.0},
    "any": {"fp32_tflops": 0.0, "dram_bw_gbs": 0.0},
}


def arch_peaks(arch: str) -> dict[str, float]:
    return _ARCH_PEAKS.get(arch, {"fp32_tflops": 0.0, "dram_bw_gbs": 0.0})


def int4_weight_bytes(E_active: int, N: int, K: int, group_size: int = 32) -> int:
    """Packed nibbles + bf16 group scales of ``E_active`` experts."""
    return E_active * N * (K // 2) + E_active * N * (K // group_size) * 2


def mxfp4_expert_bytes(hidden: int, ispp: int) -> int:
    """w13 + w13_scale + w2 + w2_scale bytes of one expert."""
    return (2 * ispp * hidden // 2 + 2 * ispp * hidden // 32
            + hidden * ispp // 2 + hidden * ispp // 32)


def _moe_int4_w4a16(p: dict[str, Any]) -> tuple[int, int]:
    M, K, N, E, k = (int(p[x]) for x in ("M", "K", "N", "E", "top_k"))
    ab = dtype_bytes(p.get("dtype", "bf16"))
    flops = 2 * M * k * N * K
    e_act = min(E, M * k)
    return flops, int4_weight_bytes(e_act, N, K) + ab * (M * K + M * N) + 8 * M * k


def _moe_sum_reduce(p: dict[str, Any]) -> tuple[int, int]:
    M, k, H = int(p["M"]), int(p["top_k"]), int(p["H"])
    yb = dtype_bytes(p.get("dtype", "fp32"))
    return 2 * M * k * H, yb * M * k * H + 4 * M * k + yb * M * H


def _moe_align(p: dict[str, Any]) -> tuple[int, int]:
    M, k, E, bs = int(p["M"]), int(p["top_k"]), int(p["num_experts"]), int(p["block_size"])
    max_pad = M * k + (E + 1) * (bs - 1)
    return 0, 4 * (M * k + max_pad + (max_pad + bs - 1) // bs + 1)


def _moe_mxfp4(p: dict[str, Any]) -> tuple[int, int]:
    M, k, E = int(p["M"]), int(p["top_k"]), int(p["E"])
    hidden, ispp = int(p["hidden"]), int(p["ispp"])
    ab = dtype_bytes(p.get("dtype", "bf16"))
    flops = 2 * M * k * (2 * ispp * hidden + hidden * ispp)
    e_act = min(E, M * k)
    return flops, e_act * mxfp4_expert_bytes(hidden, ispp) + 2 * ab * M * hidden + 8 * M * k


_MODELS: dict[str, Callable[[dict[str, Any]], tuple[int, int]]] = {
    "moe_int4_w4a16@1.0.0": _moe_int4_w4a16,
    "moe_sum_reduce@1.0.0": _moe_sum_reduce,
    "moe_align_block_size@1.0.0": _moe_align,
    "moe_mxfp4@1.0.0": _moe_mxfp4,
}


def has_model(op_id: str) -> bool:
    return op_id in _MODELS


def cost_model(op_id: str, point: dict[str, Any]) -> tuple[int, int] | None:
    fn = _MODELS.get(op_id)
    return None if fn is None else fn(point)
