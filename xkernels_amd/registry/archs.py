"""Architecture vocabulary (mirror of the Impl Card schema's ``arch.family`` enum).

Same contract as the reference's registry/archs.py:17-31, extended with
``amd_cdna4`` (MI350/MI355X, gfx950). ``tests/test_registry.py`` checks that this
set and the schema enum agree.
"""
from __future__ import annotations

AMD_ARCHS = frozenset({"amd_cdna2", "amd_cdna3", "amd_cdna4"})
NVIDIA_ARCHS = frozenset({"nvidia_sm80", "nvidia_sm90", "nvidia_sm100", "nvidia_sm121"})
ALL_ARCHS = AMD_ARCHS | NVIDIA_ARCHS


def vendor_of(arch: str) -> str:
    """'amd' | 'nvidia' | 'any'."""
    if arch in AMD_ARCHS:
        return "amd"
    if arch in NVIDIA_ARCHS:
        return "nvidia"
    return "any"
