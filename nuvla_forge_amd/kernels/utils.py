"""Shared helpers for the kernel package.

Mirrors ``nuvla_forge/kernels/utils.py``: the reference exports ``HAS_TRITON``
(is the fused backend importable).  Here the fused backend is the HIP library,
so ``HAS_HIP`` is the probe and ``HAS_TRITON`` is kept as the same flag under
the reference's name, so callers that test it keep working.  There is no
Triton and no escape hatch that silently swaps backends: the eager formulation
runs only when a caller passes ``force_reference=True``.
"""

from __future__ import annotations

import torch

from .. import _lib

HAS_HIP: bool = _lib.available()
HAS_TRITON: bool = HAS_HIP  # compatibility name (reference utils.py:7-20)


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


def require_device(t: torch.Tensor, op: str) -> None:
    """The fused ops run only on ROCm device tensors; say so instead of falling back."""
    if not t.is_cuda:
        raise RuntimeError(
            f"{op}: the fused HIP path needs a ROCm device tensor (got {t.device}); "
            "pass force_reference=True for the eager PyTorch formulation"
        )
    if torch.version.hip is None:
        raise RuntimeError(f"{op}: this build targets ROCm (gfx950); torch has no HIP")


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
