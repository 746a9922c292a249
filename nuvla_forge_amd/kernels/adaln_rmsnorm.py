"""Fused gated residual + RMSNorm + adaLN-Zero modulation on MI355X.

Drop-in for ``nuvla_forge/kernels/adaln_rmsnorm.py``: the same
``_FusedAdaLNResidualRMSNorm`` autograd Function (``forward(ctx, x, y, gate,
weight, scale, shift, tokens_per_sample, eps) -> (h, out)``; ``backward``
returns 8 values, adaln_rmsnorm.py:165-236) and the same public
``fused_adaln_residual_rmsnorm(x, y, gate, weight, scale, shift,
tokens_per_sample, eps=1e-6, force_reference=False)`` (adaln_rmsnorm.py:239-270).

    h   = x + gate * y                                (residual stream, x.dtype)
    out = rmsnorm(h) * weight * (1 + scale) + shift   (next branch input, x.dtype)

Dispatch as in the reference (adaln_rmsnorm.py:258-267): host tensors, rows
wider than ``MAX_N`` and ``force_reference=True`` run the eager formulation
(``reference.adaln_residual_rmsnorm_ref``); device tensors run the HIP kernels.

Differences from the reference's launch code, none visible in results beyond
fp32 rounding:
  * the conditioning tensors are read through their row stride, so the
    ``chunk(6)`` views and stride-0 ``expand`` views of the DiT block are not
    copied; x/y need only a unit-stride last dimension;
  * x may be fp32 with y bf16/fp16 (the autocast mix of the DiT seams): each
    is read in its own type and dy is written in y's type directly;
  * the backward recomputes h in fp32 from x and y (same traffic as reading
    h) and skips the reductions for inputs that need no gradient.
"""

from __future__ import annotations

import torch

from .. import _lib
from .reference import adaln_residual_rmsnorm_ref
from .utils import check_devices, device_of, use_fused

MAX_N = 16384  # widest row the kernels take (the reference's own limit, :262)


def _rows(t: torch.Tensor) -> torch.Tensor:
    """2-D view with unit-stride columns (copy only if the last dim is strided)."""
    return t if t.stride(-1) == 1 else t.contiguous()


def _cond(c: torch.Tensor, b: int, n: int, name: str) -> torch.Tensor:
    if c.dim() != 2 or c.shape[0] != b or c.shape[1] != n:
        raise ValueError(f"{name} must be [B={b}, N={n}], got {tuple(c.shape)}")
    return _rows(c)


class _FusedAdaLNResidualRMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, y, gate, weight, scale, shift, tokens_per_sample, eps):
        if x.dim() != 2 or y.shape != x.shape:
            raise ValueError(f"x and y must be the same [M, N]; got {tuple(x.shape)}, {tuple(y.shape)}")
        m, n = x.shape
        t = int(tokens_per_sample)
        if t <= 0 or m % t != 0:
            raise ValueError(f"M={m} is not a multiple of tokens_per_sample={t}")
        if n > MAX_N:
            raise ValueError(f"N={n} exceeds {MAX_N}")
        check_devices("fused_adaln_residual_rmsnorm", "x",
                      dict(x=x, y=y, gate=gate, weight=weight, scale=scale, shift=shift))
        b = m // t
        x = _rows(x)
        y = _rows(y)
        gate = _cond(gate, b, n, "gate")
        scale = _cond(scale, b, n, "scale")
        shift = _cond(shift, b, n, "shift")
        if weight.shape != (n,):
            raise ValueError(f"weight must be [N={n}], got {tuple(weight.shape)}")
        weight = weight.contiguous()

        h = torch.empty((m, n), dtype=x.dtype, device=x.device)
        out = torch.empty((m, n), dtype=x.dtype, device=x.device)
        rstd = torch.empty(m, dtype=torch.float32, device=x.device)
        L = _lib.lib()
        dc = _lib.dtype_code
        with device_of(x):
            _lib.check(
                L.nf_adaln_fwd(
                    x.data_ptr(), x.stride(0), y.data_ptr(), y.stride(0),
                    gate.data_ptr(), gate.stride(0), weight.data_ptr(),
                    scale.data_ptr(), scale.stride(0), shift.data_ptr(), shift.stride(0),
                    h.data_ptr(), out.data_ptr(), rstd.data_ptr(),
                    m, n, t, float(eps),
                    dc(x), dc(y), dc(gate), dc(weight), dc(scale), dc(shift),
                    _lib.stream_of(x),
                ),
                "nf_adaln_fwd",
            )
        ctx.save_for_backward(x, y, gate, weight, scale, rstd)
        ctx.tokens_per_sample = t
        ctx.shift_dtype = shift.dtype
        ctx.set_materialize_grads(False)
        return h, out

    @staticmethod
    def backward(ctx, dh_up, dout):
        x, y, gate, weight, scale, rstd = ctx.saved_tensors
        t = ctx.tokens_per_sample
        m, n = x.shape
        b = m // t
        need = ctx.needs_input_grad
        if dh_up is None and dout is None:
            return (None,) * 8
        check_devices("fused_adaln_residual_rmsnorm backward", "x",
                      dict(x=x, dh_up=dh_up, dout=dout))
        dh_up = None if dh_up is None else dh_up.to(x.dtype).contiguous()
        dout = None if dout is None else dout.to(x.dtype).contiguous()

        dev = x.device
        dx = torch.empty((m, n), dtype=x.dtype, device=dev)
        dy = torch.empty((m, n), dtype=y.dtype, device=dev)
        dgate = torch.empty((b, n), dtype=gate.dtype, device=dev) if need[2] else None
        dweight = torch.empty((n,), dtype=weight.dtype, device=dev) if need[3] else None
        dscale = torch.empty((b, n), dtype=scale.dtype, device=dev) if need[4] else None
        dshift = torch.empty((b, n), dtype=ctx.shift_dtype, device=dev) if need[5] else None
        L = _lib.lib()
        dc = _lib.dtype_code
        ws_bytes = L.nf_adaln_bwd_workspace(m, n, t)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        with device_of(x):
            stream = _lib.stream_of(x)
            _lib.check(
                L.nf_adaln_bwd(
                    _lib.ptr(dh_up), _lib.ptr(dout),
                    x.data_ptr(), x.stride(0), y.data_ptr(), y.stride(0),
                    gate.data_ptr(), gate.stride(0), weight.data_ptr(),
                    scale.data_ptr(), scale.stride(0), rstd.data_ptr(),
                    dx.data_ptr(), dy.data_ptr(), ws.data_ptr(), ws_bytes, m, n, t,
                    dc(x), dc(y), dc(gate), dc(weight), dc(scale), stream,
                ),
                "nf_adaln_bwd",
            )
            _lib.check(
                L.nf_adaln_bwd_reduce(
                    ws.data_ptr(), ws_bytes, weight.data_ptr(), scale.data_ptr(),
                    scale.stride(0), _lib.ptr(dgate), _lib.ptr(dweight), _lib.ptr(dscale),
                    _lib.ptr(dshift), m, n, t, dc(gate), dc(weight), dc(scale),
                    dc(ctx.shift_dtype), stream,
                ),
                "nf_adaln_bwd_reduce",
            )
        return (dx if need[0] else None, dy if need[1] else None,
                dgate, dweight, dscale, dshift, None, None)


def fused_adaln_residual_rmsnorm(
    x: torch.Tensor,
    y: torch.Tensor,
    gate: torch.Tensor,
    weight: torch.Tensor,
    scale: torch.Tensor,
    shift: torch.Tensor,
    tokens_per_sample: int,
    eps: float = 1e-6,
    force_reference: bool = False,
):
    """Fused gated residual + RMSNorm + adaLN-Zero modulation.

    Falls back to the eager PyTorch formulation for host tensors, for rows
    wider than 16384 and under ``force_reference=True``, as the reference does.

    Returns:
        (h, out) — the updated residual stream and the modulated branch input,
        both [M, N] in x.dtype.
    """
    if x.shape[-1] > MAX_N or not use_fused(x, "fused_adaln_residual_rmsnorm",
                                             force_reference):
        return adaln_residual_rmsnorm_ref(x, y, gate, weight, scale, shift, tokens_per_sample, eps)
    return _FusedAdaLNResidualRMSNorm.apply(x, y, gate, weight, scale, shift, tokens_per_sample, eps)
