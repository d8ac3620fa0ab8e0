"""Correctness / parity / perf harness (contract of the reference's
src/xkernels/verify.py:169-452).

``verify(card_id, arch)`` runs one Impl Card over its Op Spec's shape sweep and
compares with the spec's reference callable under ``|a-e| <= atol + rtol*|e|``
(per-dtype tolerances), re-runs point 0 for determinism and optionally times
the last point. ``verify_parity(op_id, archs)`` runs every card of an op on the
same inputs and checks pairwise agreement with ``cross_backend_rtol``; fewer than
two runnable backends is reported as inconclusive, never as agreement.
"""
from __future__ import annotations

import hashlib
import inspect
import traceback
import warnings
from collections.abc import Callable
from typing import Any

import torch

from .registry import backend_callable, get_card, get_spec, load_shape_sweep, reference_callable
from .registry.archs import vendor_of
from .registry.input_gen import generate_inputs
from .registry.catalog import ImplCard, OpSpec

DEFAULT_SEED = 1729


def _as_device(arch: str, fallback: str = "cpu") -> str:
    if arch in ("any", ""):
        return fallback
    if torch.cuda.is_available():
        vendor = vendor_of(arch)
        if vendor == "nvidia" and getattr(torch.version, "hip", None):
            warnings.warn(f"arch {arch!r} is an NVIDIA target but the device is AMD; running anyway",
                          stacklevel=2)
        return "cuda"
    return fallback


def _normalize(out: Any) -> list[torch.Tensor]:
    if isinstance(out, (tuple, list)):
        return [t for t in out if isinstance(t, torch.Tensor)]
    if isinstance(out, torch.Tensor):
        return [out]
    raise TypeError(f"unsupported op output type {type(out).__name__}")


def _accepted(fn: Callable, inputs: dict) -> tuple[set[str], bool]:
    try:
        sig = inspect.signature(fn)
    except (TypeError, ValueError):
        return set(), False
    names, var_kw = set(), False
    for name, prm in sig.parameters.items():
        if prm.kind is inspect.Parameter.VAR_KEYWORD:
            var_kw = True
        elif prm.kind is not inspect.Parameter.VAR_POSITIONAL and name not in inputs:
            names.add(name)
    return names, var_kw


def _apply_knobs(fn: Callable, inputs: dict, knobs: dict) -> tuple[Any, dict]:
    names, var_kw = _accepted(fn, inputs)
    applied = dict(knobs) if var_kw else {k: v for k, v in knobs.items() if k in names}
    return fn(**inputs, **applied), applied


def _errors(actual, expected) -> tuple[float, float]:
    mabs = mrel = 0.0
    for a, e in zip(actual, expected, strict=True):
        a, e = a.detach().float().cpu(), e.detach().float().cpu()
        if a.shape != e.shape:
            return float("inf"), float("inf")
        if a.numel() == 0:
            continue
        d = (a - e).abs()
        mabs = max(mabs, float(d.max()))
        mrel = max(mrel, float((d / e.abs().clamp_min(1e-8)).max()))
    return mabs, mrel


def _within(actual, expected, rtol: float, atol: float) -> bool:
    for a, e in zip(actual, expected, strict=True):
        a, e = a.detach().float().cpu(), e.detach().float().cpu()
        if a.shape != e.shape:
            return False
        if bool(((a - e).abs() > atol + rtol * e.abs()).any()) or bool(torch.isnan(a).ne(torch.isnan(e)).any()):
            return False
    return True


def _points(shapes) -> list[dict]:
    if isinstance(shapes, str):
        return load_shape_sweep(shapes)
    if isinstance(shapes, list):
        return shapes
    raise TypeError("shapes must be a sweep id or a list of points")


def _run(card: ImplCard, op: OpSpec, point: dict, seed: int, device: str, knobs=None):
    inputs = generate_inputs(op.id, point, seed, device)
    fn = backend_callable(op.id, card.backend.name)
    return _apply_knobs(fn, inputs, knobs)[0] if knobs else fn(**inputs)


def _run_id(card: ImplCard, arch: str, seed: int, sweep) -> str:
    return "run:" + hashlib.sha1(f"{card.id}|{arch}|{seed}|{sweep}".encode()).hexdigest()[:12]


def verify(impl_card_id: str, arch: str = "any", *, knobs: dict | None = None, shapes=None,
           seed: int = DEFAULT_SEED, measure_perf: bool = False) -> dict[str, Any]:
    """Check one card against its spec's reference over the shape sweep."""
    card = get_card(impl_card_id)
    op = get_spec(card.implements)
    sweep = shapes if shapes is not None else op.shape_sweep
    points = _points(sweep)
    device = _as_device(arch)
    knobs = knobs or {}
    compiled, error, tb = True, None, None
    failing: list[dict] = []
    mabs = mrel = 0.0
    applied: dict = {}
    determinism = False
    try:
        outs = []
        for p in points:
            ref = _normalize(reference_callable(op.id)(**generate_inputs(op.id, p, seed, device)))
            got, applied = _apply_knobs(backend_callable(op.id, card.backend.name),
                                        generate_inputs(op.id, p, seed, device), knobs)
            outs.append((p, ref, _normalize(got)))
        try:
            again = _normalize(_run(card, op, points[0], seed, device, knobs))
            determinism = _errors(again, outs[0][2])[1] <= op.rtol
        except Exception:  # noqa: BLE001
            determinism = False
        for p, ref, got in outs:
            rtol, atol = op.tolerance(p.get("dtype", "fp32"))
            a, r = _errors(got, ref)
            mabs, mrel = max(mabs, a), max(mrel, r)
            if not _within(got, ref, rtol, atol):
                failing.append({"point": p, "abs_err": a, "rel_err": r, "rtol": rtol, "atol": atol})
        passed = not failing
    except Exception as e:  # noqa: BLE001 - reported in the blob
        compiled, passed = False, False
        error, tb = f"{type(e).__name__}: {e}", traceback.format_exc(limit=4)
    result: dict[str, Any] = {
        "impl_card_id": impl_card_id, "implements": card.implements, "backend": card.backend.name,
        "arch": arch, "compiled": compiled,
        "correctness": {"passed": passed, "max_abs_err": mabs, "max_rel_err": mrel,
                        "failing_shapes": failing, "n_points": len(points)},
        "determinism_check": determinism, "knobs_requested": knobs, "knobs_applied": applied,
        "knobs_unapplied": sorted(set(knobs) - set(applied)),
        "artifacts": {"run_id": _run_id(card, arch, seed, sweep)},
    }
    if error is not None:
        result["artifacts"].update(error=error, traceback=tb)
    if measure_perf and compiled and passed and device != "cpu":
        result["perf"] = _measure_perf(card, op, points[-1], seed, device, knobs)
    else:
        result["perf"] = {"ms": None, "tflops": None, "achieved_bw_pct": None,
                          "note": "perf not measured (set measure_perf=True on a GPU device)"}
    return result


def _measure_perf(card: ImplCard, op: OpSpec, point: dict, seed: int, device: str, knobs) -> dict:
    from .registry.cost_model import arch_peaks, cost_model
    from .utils.benchmarking import benchmark_repeat

    inputs = generate_inputs(op.id, point, seed, device)
    fn = backend_callable(op.id, card.backend.name)
    call = (lambda: _apply_knobs(fn, inputs, knobs)[0]) if knobs else (lambda: fn(**inputs))
    b = benchmark_repeat(call)
    ms = b["ms"]
    tflops = bw = None
    note = "ms measured; no cost model for this op"
    model = cost_model(op.id, point)
    if model is not None:
        flops, nbytes = model
        arch = card.arch_family
        peaks = arch_peaks(arch)
        if ms > 0 and flops > 0 and peaks["fp32_tflops"] > 0:
            tflops = round(flops / (ms * 1e-3) / 1e12, 3)
        if ms > 0 and nbytes > 0 and peaks["dram_bw_gbs"] > 0:
            bw = round(nbytes / (ms * 1e-3) / 1e9 / peaks["dram_bw_gbs"] * 100, 2)
        note = f"derived from cost model (flops={flops}, bytes={nbytes}) vs {arch!r} peaks {peaks}"
    return {"ms": ms, "tflops": tflops, "achieved_bw_pct": bw, "note": note,
            "median": b["median"], "ms_p10": b["p10"], "ms_p90": b["p90"],
            "ms_spread_ratio": b["spread_ratio"], "ms_n_repeat": b["n_repeat"]}


def _parity_device(archs) -> str:
    if not archs:
        return "cpu"
    if any(vendor_of(a) in ("amd", "nvidia") for a in archs) and torch.cuda.is_available():
        return "cuda"
    return "cpu"


def verify_parity(op_id: str, archs: list[str] | None = None, *, shapes=None,
                  seed: int = DEFAULT_SEED, device: str | None = None) -> dict[str, Any]:
    """Pairwise agreement of every runnable card of ``op_id`` on the same inputs."""
    from .registry import cards_for

    op = get_spec(op_id)
    points = _points(shapes if shapes is not None else op.shape_sweep)
    device = device or _parity_device(archs)
    outputs: dict[str, list] = {}
    errors: dict[str, str] = {}
    for name, card in cards_for(op_id).items():
        try:
            outputs[name] = [_normalize(_run(card, op, p, seed, device)) for p in points]
        except Exception as e:  # noqa: BLE001
            errors[name] = f"{type(e).__name__}: {e}"
    names = list(outputs)
    worst, diverging = 0.0, []
    for i in range(len(names)):
        for j in range(i + 1, len(names)):
            a, b = names[i], names[j]
            for idx, (oa, ob) in enumerate(zip(outputs[a], outputs[b], strict=True)):
                _, atol = op.tolerance(points[idx].get("dtype", "fp32"))
                ae, re_ = _errors(oa, ob)
                worst = max(worst, re_)
                if not _within(oa, ob, op.cross_backend_rtol, atol):
                    diverging.append({"pair": [a, b], "point": points[idx], "abs_err": ae, "rel_err": re_})
    inconclusive = len(names) < 2
    return {
        "op_id": op_id, "cross_backend_rtol": op.cross_backend_rtol, "device": device,
        "agree": None if inconclusive else not diverging, "inconclusive": inconclusive,
        "n_runnable": len(names), "max_pairwise_rel_err": worst, "diverging": diverging,
        "per_backend_runnable": {k: k in outputs for k in cards_for(op_id)}, "errors": errors,
        "n_points": len(points),
    }
