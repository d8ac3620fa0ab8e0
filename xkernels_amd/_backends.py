"""Backend identifiers and the vendor of the running torch build.

The ``Backend`` names and values are the reference's plugin vocabulary
(src/xkernels/_backends.py:9-18): Impl Cards and ``XKERNELS_BACKEND`` use
them, so they are kept as they are.
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
    """Which preference list the dispatcher uses: a ROCm build of torch is
    'amd' (HIP first) whether or not a device is visible, a CUDA build with a
    device is 'nvidia', anything else 'none' (CPU only)."""
    if torch.version.hip:
        return "amd"
    return "nvidia" if (torch.version.cuda and torch.cuda.is_available()) else "none"
