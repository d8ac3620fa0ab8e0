"""Dataclass views of Op Spec / Impl Card documents (fields of the reference's
registry/models.py)."""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

from .._backends import Backend


@dataclass(frozen=True)
class Numerics:
    reference: str
    rtol: float
    atol: float
    cross_backend_rtol: float
    reduce_dtype: str | None = None
    notes: str | None = None
    by_dtype: dict[str, dict[str, float]] = field(default_factory=dict)

    def tolerance_for(self, dtype: str) -> tuple[float, float]:
        e = self.by_dtype.get(dtype)
        if e:
            return float(e["rtol"]), float(e["atol"])
        return self.rtol, self.atol


@dataclass(frozen=True)
class OpSpec:
    id: str
    name: str
    version: str
    kernel: str
    signature: str
    canonical_op: str
    fusions: tuple[str, ...]
    inputs: dict[str, dict]
    outputs: dict[str, dict]
    constraints: tuple[str, ...]
    preconditions: tuple[str, ...]
    numerics: Numerics
    shape_sweep: str
    composes_with: tuple[str, ...]
    doc: dict

    @property
    def short_name(self) -> str:
        return self.id.split("@", 1)[0]


@dataclass(frozen=True)
class ArchSpec:
    family: str
    requires: tuple[str, ...] = ()
    wave_size: int = 0
    scratch: dict[str, Any] = field(default_factory=lambda: {"kind": "none", "bytes": 0})


@dataclass(frozen=True)
class Measurement:
    arch: str
    shape: dict[str, int]
    dtype: str
    knobs: dict[str, Any]
    source: str
    tflops: float | None = None
    achieved_bw_pct: float | None = None
    ms: float | None = None


@dataclass(frozen=True)
class ImplCard:
    id: str
    implements: str
    backend: Backend
    arch: ArchSpec
    specialization_knobs: dict[str, dict]
    perf_regime: str
    roofline: str
    measured: tuple[Measurement, ...]
    uses_primitives: tuple[str, ...]
    supersedes: tuple[str, ...]
    provenance: dict[str, Any]
    doc: dict

    @classmethod
    def from_doc(cls, doc: dict) -> "ImplCard":
        a = doc["arch"]
        perf = doc.get("perf", {})
        return cls(
            id=doc["id"],
            implements=doc["implements"],
            backend=Backend(doc["backend"]),
            arch=ArchSpec(a["family"], tuple(a.get("requires", [])), a.get("wave_size", 0),
                          a.get("scratch") or {"kind": "none", "bytes": 0}),
            specialization_knobs=doc.get("specialization_knobs", {}),
            perf_regime=perf.get("regime", ""),
            roofline=perf.get("roofline", "unknown"),
            measured=tuple(
                Measurement(m["arch"], m["shape"], m["dtype"], m["knobs"], m["source"],
                            m.get("tflops"), m.get("achieved_bw_pct"), m.get("ms"))
                for m in perf.get("measured", [])
            ),
            uses_primitives=tuple(doc.get("uses_primitives", [])),
            supersedes=tuple(doc.get("supersedes", [])),
            provenance=doc["provenance"],
            doc=doc,
        )

    @property
    def short_name(self) -> str:
        return self.id.split("@", 1)[0]

    def matches_measurement(self, arch: str, shape: dict, dtype: str) -> Measurement | None:
        want = {str(k): v for k, v in shape.items()}
        for m in self.measured:
            if m.arch == arch and m.dtype == dtype and dict(m.shape) == want:
                return m
        return None


def op_spec_from_doc(doc: dict) -> OpSpec:
    n = doc["numerics"]
    rtol = float(n["rtol"])
    return OpSpec(
        id=doc["id"], name=doc["name"], version=doc["version"], kernel=doc["kernel"],
        signature=doc["op"]["signature"], canonical_op=doc["op"]["canonical_op"],
        fusions=tuple(doc["op"].get("fusions", [])), inputs=doc["inputs"],
        outputs=doc["outputs"], constraints=tuple(doc.get("constraints", [])),
        preconditions=tuple(doc.get("preconditions", [])),
        numerics=Numerics(n["reference"], rtol, float(n["atol"]),
                          float(n.get("cross_backend_rtol", rtol)), n.get("reduce_dtype"),
                          n.get("notes"), n.get("by_dtype", {}) or {}),
        shape_sweep=doc["shape_sweep"], composes_with=tuple(doc.get("composes_with", [])),
        doc=doc,
    )
