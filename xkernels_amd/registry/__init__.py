"""Op Spec / Impl Card / shape-sweep registry of the MoE path (the lookups the
reference's harness and retrieval use)."""
from __future__ import annotations

from .archs import ALL_ARCHS, AMD_ARCHS, NVIDIA_ARCHS, vendor_of
from .catalog import (
    ImplCard,
    OpSpec,
    RegistryError,
    all_cards,
    all_specs,
    backend_callable,
    bind_reference,
    cards_for,
    get_card,
    get_spec,
    load_shape_sweep,
    reference_callable,
    reset_cache,
)
from .constraints import UndecidableConstraintError, evaluate, validate_decidable
from .schemas import have_validator, impl_card_schema, op_spec_schema, registry_root

__all__ = [
    "ALL_ARCHS", "AMD_ARCHS", "NVIDIA_ARCHS", "vendor_of", "ImplCard", "OpSpec",
    "RegistryError", "all_cards", "all_specs", "backend_callable", "bind_reference",
    "cards_for", "get_card", "get_spec", "load_shape_sweep", "reference_callable",
    "reset_cache", "UndecidableConstraintError", "evaluate", "validate_decidable",
    "have_validator", "impl_card_schema", "op_spec_schema", "registry_root",
]
