"""Shared pytest setup.

* registers the ``gpu`` marker (tests that need an MI355X; run with ``-m gpu``);
* puts the repository root on ``sys.path`` so ``oracle`` and ``xkernels_amd``
  import from the checkout;
* installs the CPU oracle as the REFERENCE backend, so ``verify_parity`` has a
  second backend to compare the HIP cards with (the package itself registers
  only HIP).
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU (gfx950) and libxk_moe.so")


def pytest_sessionstart(session):
    from oracle.torch_ref import register_reference_backends

    import xkernels_amd  # noqa: F401  (registers HIP)

    register_reference_backends()


@pytest.fixture
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return "cuda"
