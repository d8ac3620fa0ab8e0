"""Structured retrieval over the registry (contract of the reference's
src/xkernels/retrieval.py:25-205): filter Op Specs by canonical op, decidable
constraints and fusions, then rank Impl Cards by arch fit and measurements.
Every candidate carries ``reject_reasons``."""
from __future__ import annotations

from typing import Any

from .registry import all_specs, cards_for
from .registry.archs import vendor_of
from .registry.constraints import UndecidableConstraintError, evaluate
from .registry.catalog import ImplCard, OpSpec


def _arch_reasons(card: ImplCard, target: str, features: set[str]) -> list[str]:
    r: list[str] = []
    fam = card.arch_family
    if fam != "any" and fam != target:
        r.append(f"arch.family {fam!r} != target {target!r}")
    r += [f"missing required feature {x!r}" for x in card.arch_requires if x not in features]
    if card.backend.name == "CUDA" and vendor_of(target) == "amd":
        r.append("cuda backend on an amd target")
    if card.backend.name == "HIP" and vendor_of(target) == "nvidia":
        r.append("hip backend on an nvidia target")
    return r


def _bindings(op: OpSpec, specs: dict[str, dict]) -> dict[str, Any]:
    b: dict[str, Any] = {}
    for arg, contract in op.inputs.items():
        q = specs.get(arg)
        if q is None:
            continue
        syms, shape = contract.get("shape_symbols", []), q.get("shape")
        if shape is not None and len(shape) == len(syms):
            b.update({s: int(v) for s, v in zip(syms, shape)})
        if q.get("dtype") is not None:
            b[f"dtype:{arg}"] = q["dtype"]
    return b


def _constraint_reasons(op: OpSpec, b: dict[str, Any]) -> list[str]:
    r = []
    for c in op.constraints:
        try:
            if not evaluate(c, b):
                r.append(f"constraint violated: {c!r}")
        except UndecidableConstraintError:
            continue
    return r


def _matched(card: ImplCard, specs: dict[str, dict], arch: str):
    dtype = next((q["dtype"] for q in specs.values() if q.get("dtype")), None)
    if dtype is None:
        return None
    return next((m for m in card.measured if m["arch"] == arch and m["dtype"] == dtype), None)


def _score(card: ImplCard, ok: bool, matched, objective: str) -> float:
    if not ok:
        return 0.0
    s = 1.0 if matched is not None else (0.5 if card.backend.name != "REFERENCE" else 0.1)
    if objective in ("memory", "bandwidth") and card.roofline == "memory_bound":
        s += 0.05
    if objective == "throughput" and card.roofline == "compute_bound":
        s += 0.05
    if objective == "latency" and card.backend.name == "REFERENCE":
        s -= 0.05
    return round(s, 3)


def find_impl(canonical_op: str, input_specs: dict[str, dict] | None = None,
              target_arch: str = "any", available_features: list[str] | None = None,
              required_fusions: list[str] | None = None,
              objective: str = "throughput") -> list[dict[str, Any]]:
    """Ranked candidates (applicable first, then by score) with reject reasons."""
    specs = input_specs or {}
    features = set(available_features or [])
    fusions = set(required_fusions or [])
    results: list[dict[str, Any]] = []
    for op in all_specs().values():
        if op.canonical_op != canonical_op:
            continue
        op_rej = _constraint_reasons(op, _bindings(op, specs))
        op_rej += [f"missing required fusion {f!r}" for f in sorted(fusions - set(op.fusions))]
        bucket = cards_for(op.id)
        if not bucket:
            results.append({"op_id": op.id, "impl_card_id": None, "backend": None,
                            "arch": target_arch, "applicable": not op_rej,
                            "reject_reasons": op_rej or ["no implementation cards registered"],
                            "score": 0.0, "matched_measurement": None, "missing_backend": True})
            continue
        any_ok = False
        for card in bucket.values():
            reasons = op_rej + _arch_reasons(card, target_arch, features)
            ok = not reasons
            any_ok |= ok
            m = _matched(card, specs, target_arch) if specs else None
            results.append({
                "op_id": op.id, "impl_card_id": card.id, "backend": card.backend.name,
                "arch": target_arch, "applicable": ok, "reject_reasons": reasons,
                "score": _score(card, ok, m, objective),
                "matched_measurement": None if m is None else {
                    "arch": m["arch"], "shape": dict(m["shape"]), "dtype": m["dtype"],
                    "tflops": m.get("tflops"), "ms": m.get("ms"),
                    "achieved_bw_pct": m.get("achieved_bw_pct"), "source": m["source"]},
            })
        if not op_rej and not any_ok:
            results[-1]["missing_backend"] = True
    results.sort(key=lambda r: (r["applicable"], r["score"]), reverse=True)
    return results
