"""Loads Op Specs, Impl Cards and shape sweeps from ``registry/`` and ties them
to the dispatch registry (API of the reference's registry/loader.py:63-202).
"""
from __future__ import annotations

import importlib
import json
from collections.abc import Callable
from functools import lru_cache
from pathlib import Path
from typing import Any

from .._backends import Backend
from .._dispatch import _REGISTRY, registered_backends
from .constraints import UndecidableConstraintError, validate_decidable
from .models import ImplCard, OpSpec, op_spec_from_doc
from .schemas import registry_root, validate_impl_card, validate_op_spec


class RegistryError(ValueError):
    """An artifact in registry/ is malformed or inconsistent."""


def _read(path: Path) -> dict:
    try:
        with path.open() as f:
            return json.load(f)
    except json.JSONDecodeError as e:
        raise RegistryError(f"invalid JSON in {path}: {e}") from e


def _load_spec(path: Path) -> OpSpec:
    doc = _read(path)
    try:
        validate_op_spec(doc)
    except ValueError as e:
        raise RegistryError(f"{path.name}: {e}") from e
    for c in doc.get("constraints", []):
        try:
            validate_decidable(c)
        except UndecidableConstraintError as e:
            raise RegistryError(f"{path.name}: {e}") from e
    return op_spec_from_doc(doc)


def _load_card(path: Path) -> ImplCard:
    doc = _read(path)
    try:
        validate_impl_card(doc)
    except ValueError as e:
        raise RegistryError(f"{path.name}: {e}") from e
    measured = doc.get("perf", {}).get("measured", [])
    kept = [m for m in measured if m.get("source") and m.get("arch")]
    if len(kept) != len(measured):  # un-sourced / arch-less entries are dropped
        doc = {**doc, "perf": {**doc["perf"], "measured": kept}}
    return ImplCard.from_doc(doc)


@lru_cache(maxsize=1)
def load() -> tuple[dict[str, OpSpec], dict[str, dict[str, ImplCard]]]:
    """(specs by id, cards by op id then backend NAME)."""
    root = registry_root()
    specs: dict[str, OpSpec] = {}
    for p in sorted((root / "ops").glob("*.spec.json")):
        s = _load_spec(p)
        if s.id in specs:
            raise RegistryError(f"duplicate Op Spec id {s.id!r}")
        specs[s.id] = s
    cards: dict[str, dict[str, ImplCard]] = {}
    for p in sorted((root / "impls").glob("*.card.json")):
        c = _load_card(p)
        if c.implements not in specs:
            raise RegistryError(f"{p.name}: implements unknown Op Spec {c.implements!r}")
        bucket = cards.setdefault(c.implements, {})
        if c.backend.name in bucket:
            raise RegistryError(f"duplicate card for {c.implements!r} backend {c.backend.name}")
        bucket[c.backend.name] = c
    return specs, cards


def reset_cache() -> None:
    load.cache_clear()


def all_specs() -> dict[str, OpSpec]:
    return load()[0]


def all_cards() -> dict[str, dict[str, ImplCard]]:
    return load()[1]


def get_spec(op_id: str) -> OpSpec:
    specs = all_specs()
    if op_id not in specs:
        raise KeyError(f"unknown Op Spec {op_id!r}; have {sorted(specs)}")
    return specs[op_id]


def cards_for(op_id: str) -> dict[str, ImplCard]:
    return all_cards().get(op_id, {})


def get_card(card_id: str) -> ImplCard:
    for bucket in all_cards().values():
        for c in bucket.values():
            if c.id == card_id:
                return c
    raise KeyError(f"unknown Impl Card {card_id!r}")


def card_by_short_name(op_id: str, backend: str) -> ImplCard:
    bucket = cards_for(op_id)
    if backend.upper() in bucket:
        return bucket[backend.upper()]
    short = f"{op_id.split('@')[0]}.{backend.lower()}"
    for c in bucket.values():
        if c.short_name == short:
            return c
    raise KeyError(f"no {backend!r} card for {op_id!r}")


def _import_attr(path: str) -> Callable:
    module, _, attr = path.partition(":")
    if not attr:
        raise RegistryError(f"reference path must be 'module:attr', got {path!r}")
    return getattr(importlib.import_module(module), attr)


def reference_callable(op_id: str) -> Callable:
    """The spec's numerics.reference callable (the CPU oracle named in the spec)."""
    return _import_attr(get_spec(op_id).numerics.reference)


def backend_callable(op_id: str, backend: str) -> Callable:
    """The dispatch callable registered for (spec.kernel, backend)."""
    importlib.import_module("xkernels_amd")
    spec = get_spec(op_id)
    try:
        key = Backend(backend.lower())
    except ValueError as e:
        raise KeyError(f"unknown backend {backend!r}: {e}") from e
    impls = _REGISTRY.get(spec.kernel, {})
    if key not in impls:
        raise KeyError(
            f"backend {backend!r} not registered for kernel {spec.kernel!r}; "
            f"have {sorted(b.name for b in registered_backends(spec.kernel))}"
        )
    return impls[key]


def load_shape_sweep(sweep_id: str) -> list[dict[str, Any]]:
    path = registry_root() / "shape_sweeps" / f"{sweep_id}.sweep.json"
    if not path.exists():
        raise KeyError(f"no shape sweep {sweep_id!r} at {path}")
    doc = _read(path)
    default = doc.get("default_dtype", "fp32")
    return [{**p, "dtype": p.get("dtype", default)} for p in doc.get("points", [])]
