"""Backend identifiers and vendor detection.

Same names and values as the reference's ``xkernels._backends``
(src/xkernels/_backends.py:9-27) so Impl Cards and ``XKERNELS_BACKEND`` values
carry over unchanged.
"""
from __future__ import annotations

import enum

import torch


class Backend(enum.Enum):
    REFERENCE = "reference"
    TRITON = "triton"
    CUDA = "cuda"
    HIP = "hip"


def detect_vendor() -> str:
    """'amd' on a ROCm build of torch, 'nvidia' on a CUDA build with a GPU, else 'none'."""
    if getattr(torch.version, "hip", None):
        return "amd"
    if getattr(torch.version, "cuda", None) and torch.cuda.is_available():
        return "nvidia"
    return "none"


def device_of(tensor: torch.Tensor) -> str:
    """'cpu' or 'cuda' (ROCm devices report 'cuda')."""
    return tensor.device.type
