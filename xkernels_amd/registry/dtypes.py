"""Dtype short names <-> torch dtypes (the names used by specs and sweeps)."""
from __future__ import annotations

import torch

_MAP: dict[str, torch.dtype] = {
    "fp32": torch.float32,
    "fp16": torch.float16,
    "bf16": torch.bfloat16,
    "int32": torch.int32,
    "int8": torch.int8,
    "uint8": torch.uint8,
    "bool": torch.bool,
}
_BYTES = {k: torch.empty(0, dtype=v).element_size() for k, v in _MAP.items()}


def to_torch_dtype(short) -> torch.dtype:
    if isinstance(short, torch.dtype):
        return short
    try:
        return _MAP[short.lower()]
    except KeyError:
        raise KeyError(f"unknown dtype short name {short!r}; have {sorted(_MAP)}") from None


def to_short_dtype(dtype: torch.dtype) -> str:
    for k, v in _MAP.items():
        if v == dtype:
            return k
    raise KeyError(f"no short name for {dtype}")


def dtype_bytes(short: str) -> int:
    try:
        return _BYTES[short.lower()]
    except KeyError:
        raise KeyError(f"unknown dtype short name {short!r}") from None
