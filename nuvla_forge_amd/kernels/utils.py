"""Shared helpers for the kernel package.

Mirrors ``nuvla_forge/kernels/utils.py``: the reference exports ``HAS_TRITON``
(is the fused backend importable).  Here the fused backend is the HIP library,
so ``HAS_HIP`` is the probe and ``HAS_TRITON`` is kept as the same flag under
the reference's name, so callers that test it keep working.

Dispatch follows the reference's rule (adaln_rmsnorm.py:258-267,
swiglu.py:104, chunked_ce.py:133): host tensors and ``force_reference=True``
take the eager PyTorch formulation.  Device tensors take the HIP kernels; a
missing or stale library raises there instead of silently running the eager
path on the GPU.

``NUVLA_FORGE_DISABLE_TRITON=1`` in the environment when the package is
imported is the reference's escape hatch (utils.py:16-20, set by its
train.py:112-113 to time the baseline): ``HAS_TRITON`` is then False and every
op takes its eager formulation, on the device too.  It selects the reference
path, not another GPU backend.
"""

from __future__ import annotations

import os

import torch

from .. import _lib

# The reference's switch, read once at import (reference utils.py:16-20).
FUSED_DISABLED: bool = os.environ.get("NUVLA_FORGE_DISABLE_TRITON", "0") == "1"

HAS_HIP: bool = _lib.available()
# compatibility name (reference utils.py:7-20): the fused path is usable
HAS_TRITON: bool = HAS_HIP and not FUSED_DISABLED


class DeviceMismatchError(ValueError, RuntimeError):
    """A tensor argument of a fused op is not on the primary tensor's device.

    Raised before any launch, so a host pointer never reaches a HIP kernel.
    A ValueError (a bad argument) and a RuntimeError (what the reference's
    Triton launch or torch op raises for the same call)."""


def check_devices(op: str, primary: str, tensors: dict, device: torch.device | None = None
                  ) -> None:
    """Raise DeviceMismatchError unless every tensor in ``tensors`` (name ->
    tensor or None) is on ``device``, by default the device of
    ``tensors[primary]`` (``primary`` names what sets the device)."""
    dev = tensors[primary].device if device is None else device
    for name, t in tensors.items():
        if t is not None and t.device != dev:
            raise DeviceMismatchError(
                f"{op}: {name} is on {t.device}, but {primary} is on {dev}; every tensor "
                f"argument must be on one device")


def next_power_of_2(n: int) -> int:
    """Smallest power of two >= n (reference utils.py:23-27)."""
    if n <= 1:
        return 1
    return 1 << (n - 1).bit_length()


def warps_for_block(block_n: int) -> int:
    """Wavefronts per row for a row of ``block_n`` elements (reference
    utils.py:30-44, where it picks Triton warps for single-row reductions).

    On MI355X the row kernels place a row on 64-lane wavefronts: the adaLN
    forward gives each lane one or two 16-byte chunks (8 elements each) and
    splits rows of N >= 1024 over at least two wavefronts, so the count is the
    smallest power of two with 64 * w * 16 >= N, at least 2 from N = 1024 on.
    The C++ launch plan (``make_plan`` in csrc/adaln_impl.h) applies the same
    rule; this function only reports it."""
    w = 1
    while 64 * w * 8 * 2 < block_n:
        w *= 2
    if block_n >= 1024 and w < 2:
        w = 2
    return w


def use_fused(t: torch.Tensor, op: str, force_reference: bool = False) -> bool:
    """True when ``op`` runs the HIP kernels on ``t``: a device tensor, no
    ``force_reference`` and no ``NUVLA_FORGE_DISABLE_TRITON=1``.  Host
    tensors take the eager formulation, as the reference's dispatch does for
    tensors that are not on the GPU.  On a device tensor the HIP library must
    load (RuntimeError otherwise)."""
    if force_reference or FUSED_DISABLED or not t.is_cuda:
        return False
    if torch.version.hip is None:
        raise RuntimeError(f"{op}: this build targets ROCm (gfx950); torch has no HIP")
    _lib.lib()  # raises RuntimeError naming the problem if the library cannot load
    return True


class device_of:
    """Make t's device current for the launch (no-op when it already is).

    Reads the current device with torch's raw accessor: the public
    ``torch.cuda.current_device()`` re-checks lazy initialisation on every
    call, and a device tensor implies an initialised runtime."""

    def __init__(self, t: torch.Tensor):
        self.idx = t.get_device()
        self.prev = None

    def __enter__(self):
        cur = torch._C._cuda_getDevice()
        if cur != self.idx:
            self.prev = cur
            torch.cuda.set_device(self.idx)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False
