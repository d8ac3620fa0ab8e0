"""Op Spec / Impl Card / shape-sweep registry (public surface of the reference's
xkernels.registry restricted to the MoE path)."""
from __future__ import annotations

from .archs import ALL_ARCHS, AMD_ARCHS, NVIDIA_ARCHS, vendor_of
from .constraints import UndecidableConstraintError, evaluate, validate_decidable
from .loader import (
    RegistryError,
    all_cards,
    all_specs,
    backend_callable,
    card_by_short_name,
    cards_for,
    get_card,
    get_spec,
    load,
    load_shape_sweep,
    reference_callable,
    reset_cache,
)
from .models import ArchSpec, ImplCard, Numerics, OpSpec, op_spec_from_doc
from .schemas import have_validator, impl_card_schema, op_spec_schema, registry_root

__all__ = [
    "ALL_ARCHS", "AMD_ARCHS", "NVIDIA_ARCHS", "vendor_of", "UndecidableConstraintError",
    "evaluate", "validate_decidable", "RegistryError", "all_cards", "all_specs",
    "backend_callable", "card_by_short_name", "cards_for", "get_card", "get_spec", "load",
    "load_shape_sweep", "reference_callable", "reset_cache", "ArchSpec", "ImplCard", "Numerics",
    "OpSpec", "op_spec_from_doc", "have_validator", "impl_card_schema", "op_spec_schema",
    "registry_root",
]
