"""Fused SwiGLU on MI355X: ``out = silu(a) * b`` in one HBM pass.

Drop-in for ``nuvla_forge/kernels/swiglu.py``: the same ``_FusedSwiGLU``
autograd Function (``forward(ctx, a, b)``, ``backward`` returning ``(da, db)``,
swiglu.py:66-92) and the same ``fused_swiglu(a, b, force_reference=False)``
entry point (swiglu.py:95-106).  The forward and backward are the HIP kernels
``nf_swiglu_fwd`` / ``nf_swiglu_bwd``; the backward recomputes the sigmoid
from ``a`` instead of storing it.
"""

from __future__ import annotations

import torch

from .. import _lib
from .reference import swiglu_ref
from .utils import device_of, require_device


def _check(a: torch.Tensor, b: torch.Tensor) -> None:
    if a.shape != b.shape:
        raise ValueError(f"fused_swiglu: shape mismatch {tuple(a.shape)} vs {tuple(b.shape)}")
    if a.dtype != b.dtype:
        raise TypeError(f"fused_swiglu: dtype mismatch {a.dtype} vs {b.dtype}")
    if a.device != b.device:
        raise ValueError("fused_swiglu: a and b are on different devices")
    _lib.dtype_code(a)


class _FusedSwiGLU(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, b):
        _check(a, b)
        a = a.contiguous()
        b = b.contiguous()
        out = torch.empty_like(a)
        L = _lib.lib()
        with device_of(a):
            _lib.check(
                L.nf_swiglu_fwd(a.data_ptr(), b.data_ptr(), out.data_ptr(), a.numel(),
                                _lib.dtype_code(a), _lib.stream_of(a)),
                "nf_swiglu_fwd",
            )
        ctx.save_for_backward(a, b)
        return out

    @staticmethod
    def backward(ctx, dout):
        a, b = ctx.saved_tensors
        dout = dout.contiguous()
        if dout.dtype != a.dtype:
            dout = dout.to(a.dtype)
        da = torch.empty_like(a)
        db = torch.empty_like(b)
        L = _lib.lib()
        with device_of(a):
            _lib.check(
                L.nf_swiglu_bwd(dout.data_ptr(), a.data_ptr(), b.data_ptr(), da.data_ptr(),
                                db.data_ptr(), a.numel(), _lib.dtype_code(a), _lib.stream_of(a)),
                "nf_swiglu_bwd",
            )
        return da, db


def fused_swiglu(a: torch.Tensor, b: torch.Tensor, force_reference: bool = False) -> torch.Tensor:
    """SwiGLU: ``silu(a) * b``, fused into a single pass.

    Args:
        a: gate projection, any shape, on a ROCm device.
        b: up projection, same shape and dtype as ``a``.
        force_reference: run the eager PyTorch formulation instead.
    """
    if force_reference:
        return swiglu_ref(a, b)
    require_device(a, "fused_swiglu")
    return _FusedSwiGLU.apply(a, b)
