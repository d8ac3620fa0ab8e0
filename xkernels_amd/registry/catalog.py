"""The registry of Op Specs, Impl Cards and shape sweeps under ``registry/``.

Same documents and lookups as the reference's registry (Op Spec / Impl Card
JSON, registry/loader.py:63-202 for the lookup names ``get_spec``, ``get_card``,
``cards_for``, ``load_shape_sweep``, ``reference_callable``, ``backend_callable``).
Here the documents stay JSON: ``OpSpec`` and ``ImplCard`` are read-only views
with properties for the fields the harness and ``find_impl`` read, and one
``_Catalog`` is built (and validated) on first use.

The Op Specs name their reference callable as the reference repository does
(``xkernels.ops.moe.*``). Where that module is not importable (this standalone
checkout), a caller may bind the path to an equivalent function with
``bind_reference``; the test harness binds the CPU oracle that way. The
package itself never imports an oracle.
"""
from __future__ import annotations

import importlib
import json
from collections.abc import Callable
from pathlib import Path
from typing import Any

from .._backends import Backend
from .constraints import UndecidableConstraintError, validate_decidable
from .schemas import registry_root, validate_impl_card, validate_op_spec


class RegistryError(ValueError):
    """A document under registry/ is malformed or inconsistent."""


class OpSpec:
    """Read-only view of one Op Spec document."""

    __slots__ = ("doc",)

    def __init__(self, doc: dict) -> None:
        self.doc = doc

    id = property(lambda self: self.doc["id"])
    kernel = property(lambda self: self.doc["kernel"])
    inputs = property(lambda self: self.doc["inputs"])
    outputs = property(lambda self: self.doc["outputs"])
    shape_sweep = property(lambda self: self.doc["shape_sweep"])
    canonical_op = property(lambda self: self.doc["op"]["canonical_op"])
    fusions = property(lambda self: tuple(self.doc["op"].get("fusions", ())))
    constraints = property(lambda self: tuple(self.doc.get("constraints", ())))
    reference = property(lambda self: self.doc["numerics"]["reference"])

    @property
    def short_name(self) -> str:
        return self.id.split("@", 1)[0]

    @property
    def rtol(self) -> float:
        return float(self.doc["numerics"]["rtol"])

    @property
    def cross_backend_rtol(self) -> float:
        n = self.doc["numerics"]
        return float(n.get("cross_backend_rtol", n["rtol"]))

    def tolerance(self, dtype: str) -> tuple[float, float]:
        """(rtol, atol) for outputs of ``dtype`` (the spec's per-dtype table, else
        its default)."""
        n = self.doc["numerics"]
        per = (n.get("by_dtype") or {}).get(dtype) or n
        return float(per["rtol"]), float(per["atol"])

    def __repr__(self) -> str:
        return f"OpSpec({self.id})"


class ImplCard:
    """Read-only view of one Impl Card document."""

    __slots__ = ("doc", "_measured")

    def __init__(self, doc: dict) -> None:
        self.doc = doc
        # measurements without a source or an arch carry no evidence
        self._measured = tuple(m for m in doc.get("perf", {}).get("measured", ())
                               if m.get("source") and m.get("arch"))

    id = property(lambda self: self.doc["id"])
    implements = property(lambda self: self.doc["implements"])
    backend = property(lambda self: Backend(self.doc["backend"]))
    arch_family = property(lambda self: self.doc["arch"]["family"])
    arch_requires = property(lambda self: tuple(self.doc["arch"].get("requires", ())))
    roofline = property(lambda self: self.doc.get("perf", {}).get("roofline", "unknown"))
    measured = property(lambda self: self._measured)

    @property
    def short_name(self) -> str:
        return self.id.split("@", 1)[0]

    def __repr__(self) -> str:
        return f"ImplCard({self.id})"


def _read_json(path: Path) -> dict:
    try:
        return json.loads(path.read_text())
    except json.JSONDecodeError as e:
        raise RegistryError(f"{path}: invalid JSON ({e})") from e


class _Catalog:
    """Every spec, card and sweep of registry/, validated once."""

    def __init__(self, root: Path) -> None:
        self.root = root
        self.specs: dict[str, OpSpec] = {}
        self.cards: dict[str, dict[str, ImplCard]] = {}  # op id -> backend NAME -> card
        for path in sorted((root / "ops").glob("*.spec.json")):
            doc = _read_json(path)
            try:
                validate_op_spec(doc)
                for expr in doc.get("constraints", ()):
                    validate_decidable(expr)
            except (ValueError, UndecidableConstraintError) as e:
                raise RegistryError(f"{path.name}: {e}") from e
            if doc["id"] in self.specs:
                raise RegistryError(f"{path.name}: Op Spec id {doc['id']!r} defined twice")
            self.specs[doc["id"]] = OpSpec(doc)
        for path in sorted((root / "impls").glob("*.card.json")):
            doc = _read_json(path)
            try:
                validate_impl_card(doc)
            except ValueError as e:
                raise RegistryError(f"{path.name}: {e}") from e
            card = ImplCard(doc)
            if card.implements not in self.specs:
                raise RegistryError(f"{path.name}: implements unknown Op Spec {card.implements!r}")
            per_op = self.cards.setdefault(card.implements, {})
            if card.backend.name in per_op:
                raise RegistryError(f"{path.name}: second {card.backend.name} card for "
                                    f"{card.implements!r}")
            per_op[card.backend.name] = card


_catalog: _Catalog | None = None
_bound_references: dict[str, Callable] = {}


def _cat() -> _Catalog:
    global _catalog
    if _catalog is None:
        _catalog = _Catalog(registry_root())
    return _catalog


def reset_cache() -> None:
    """Re-reads registry/ on the next lookup."""
    global _catalog
    _catalog = None


def all_specs() -> dict[str, OpSpec]:
    return dict(_cat().specs)


def all_cards() -> dict[str, dict[str, ImplCard]]:
    return {k: dict(v) for k, v in _cat().cards.items()}


def get_spec(op_id: str) -> OpSpec:
    try:
        return _cat().specs[op_id]
    except KeyError:
        raise KeyError(f"unknown Op Spec {op_id!r}; have {sorted(_cat().specs)}") from None


def cards_for(op_id: str) -> dict[str, ImplCard]:
    return dict(_cat().cards.get(op_id, {}))


def get_card(card_id: str) -> ImplCard:
    for per_op in _cat().cards.values():
        for card in per_op.values():
            if card.id == card_id:
                return card
    raise KeyError(f"unknown Impl Card {card_id!r}")


def load_shape_sweep(sweep_id: str) -> list[dict[str, Any]]:
    """The sweep's points, each with an explicit dtype."""
    path = _cat().root / "shape_sweeps" / f"{sweep_id}.sweep.json"
    if not path.is_file():
        raise KeyError(f"no shape sweep {sweep_id!r} ({path})")
    doc = _read_json(path)
    fallback = doc.get("default_dtype", "fp32")
    return [dict(point, dtype=point.get("dtype", fallback)) for point in doc.get("points", ())]


def bind_reference(path: str, fn: Callable) -> None:
    """Resolves the spec reference ``module:attr`` to ``fn`` when the module
    itself cannot be imported (a standalone checkout without the reference)."""
    _bound_references[path] = fn


def reference_callable(op_id: str) -> Callable:
    """The callable the Op Spec names as its numerical reference."""
    path = get_spec(op_id).reference
    module, sep, attr = path.partition(":")
    if not sep or not attr:
        raise RegistryError(f"reference {path!r} of {op_id} is not 'module:attr'")
    try:
        return getattr(importlib.import_module(module), attr)
    except ImportError:
        if path in _bound_references:
            return _bound_references[path]
        raise


def backend_callable(op_id: str, backend: str) -> Callable:
    """The function registered for the spec's kernel on ``backend``."""
    from .. import _dispatch  # the package registers its backends on import

    importlib.import_module("xkernels_amd")
    kernel = get_spec(op_id).kernel
    try:
        b = Backend(backend.lower())
    except ValueError:
        raise KeyError(f"unknown backend {backend!r}") from None
    if b not in _dispatch.registered_backends(kernel):
        raise KeyError(f"backend {backend!r} not registered for kernel {kernel!r}; have "
                       f"{sorted(x.name for x in _dispatch.registered_backends(kernel))}")
    return _dispatch._TABLE[kernel].impls[b]
