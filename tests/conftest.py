"""Test configuration.

Two tiers, as in the reference's suite (tests/test_kernels.py +
tests/test_kernel_math.py):
  * CPU tier (default, `-m "not gpu"`): the oracle against finite differences,
    autograd, known answers and golden fixtures; the C ABI's exports and
    host-side argument validation; the eager formulations.
  * GPU tier (`-m gpu`): the HIP kernels through the C ABI against the oracle.
    These fail (not skip) when the library is missing on a machine with a GPU.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X / gfx950)")


def _ensure_built() -> None:
    """Build libnf_hip.so only when nothing is built (the GPU box gets it prebuilt)."""
    from nuvla_forge_amd import build

    if not build.LIB.exists():
        build.build()


_ensure_built()


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from nuvla_forge_amd import _lib

    _lib.lib()  # raises if the HIP library is missing or stale: no silent fallback
    return torch.device("cuda", 0)
