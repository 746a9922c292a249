"""Fused SwiGLU on MI355X: ``out = silu(a) * b`` in one HBM pass.

Drop-in for ``nuvla_forge/kernels/swiglu.py``: the same ``_FusedSwiGLU``
autograd Function (``forward(ctx, a, b)``, ``backward`` returning ``(da, db)``,
swiglu.py:66-92) and the same ``fused_swiglu(a, b, force_reference=False)``
entry point (swiglu.py:95-106).  The forward and backward are the HIP kernels
``nf_swiglu_fwd`` / ``nf_swiglu_bwd``; the backward recomputes the sigmoid
from ``a`` instead of storing it.

Beyond the reference: ``fused_gate_up_swiglu`` moves the SwiGLU into the
epilogue of the gate/up projection GEMM (``nf_gemm_swiglu``), so a and b
never make the HBM round trip between the projections and the activation.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .. import _lib
from .reference import swiglu_ref
from .utils import check_devices, device_of, use_fused


def _check(a: torch.Tensor, b: torch.Tensor) -> None:
    if a.shape != b.shape:
        raise ValueError(f"fused_swiglu: shape mismatch {tuple(a.shape)} vs {tuple(b.shape)}")
    if a.dtype != b.dtype:
        raise TypeError(f"fused_swiglu: dtype mismatch {a.dtype} vs {b.dtype}")
    check_devices("fused_swiglu", "a", dict(a=a, b=b))
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
        check_devices("fused_swiglu backward", "a", dict(a=a, dout=dout))
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


class _FusedGateUpSwiGLU(torch.autograd.Function):
    """act = silu(x W_gate^T) * (x W_up^T) with the SwiGLU in the GEMM epilogue.

    forward: one ``nf_gemm_swiglu`` launch writes act and the bf16 a, b the
    backward needs.  backward: ``nf_swiglu_bwd`` forms da, db from a, b and
    dact (sigmoid recomputed); ``nf_gemm_swiglu_wgrad`` computes dW_gate =
    da^T x and dW_up = db^T x in one split-K launch (a token sum added in a
    fixed order); dx = da W_gate + db W_up runs as library GEMMs.
    """

    @staticmethod
    def forward(ctx, x, w_gate, w_up):
        check_devices("fused_gate_up_swiglu", "x", dict(x=x, w_gate=w_gate, w_up=w_up))
        m, d = x.shape
        h = w_gate.shape[0]
        a = torch.empty((m, h), dtype=torch.bfloat16, device=x.device)
        b = torch.empty_like(a)
        act = torch.empty_like(a)
        L = _lib.lib()
        with device_of(x):
            _lib.check(
                L.nf_gemm_swiglu(x.data_ptr(), x.stride(0), w_gate.data_ptr(), w_gate.stride(0),
                                 w_up.data_ptr(), w_up.stride(0), a.data_ptr(), b.data_ptr(),
                                 act.data_ptr(), h, m, d, h, _lib.dtype_code(torch.bfloat16),
                                 _lib.stream_of(x)),
                "nf_gemm_swiglu",
            )
        ctx.save_for_backward(x, w_gate, w_up, a, b)
        return act

    @staticmethod
    def backward(ctx, dact):
        x, w_gate, w_up, a, b = ctx.saved_tensors
        check_devices("fused_gate_up_swiglu backward", "x", dict(x=x, dact=dact))
        dact = dact.to(torch.bfloat16).contiguous()
        da, db = torch.empty_like(a), torch.empty_like(b)
        L = _lib.lib()
        with device_of(a):
            _lib.check(
                L.nf_swiglu_bwd(dact.data_ptr(), a.data_ptr(), b.data_ptr(), da.data_ptr(),
                                db.data_ptr(), a.numel(), _lib.dtype_code(a), _lib.stream_of(a)),
                "nf_swiglu_bwd",
            )
        need = ctx.needs_input_grad
        dx = torch.addmm(torch.mm(da, w_gate), db, w_up) if need[0] else None
        dwg = dwu = None
        if need[1] or need[2]:
            m, d = x.shape
            h = a.shape[1]
            dwg = torch.empty((h, d), dtype=torch.bfloat16, device=x.device)
            dwu = torch.empty_like(dwg)
            with device_of(x):
                nbytes = L.nf_gemm_swiglu_wgrad_workspace(m, d, h)
                ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
                _lib.check(
                    L.nf_gemm_swiglu_wgrad(da.data_ptr(), db.data_ptr(), da.stride(0),
                                           x.data_ptr(), x.stride(0), dwg.data_ptr(),
                                           dwu.data_ptr(), dwg.stride(0), m, d, h,
                                           _lib.dtype_code(torch.bfloat16), ws.data_ptr(),
                                           nbytes, _lib.stream_of(x)),
                    "nf_gemm_swiglu_wgrad",
                )
        return dx, dwg if need[1] else None, dwu if need[2] else None


def _gate_up_eager(x, w_gate, w_up):
    return F.silu(F.linear(x, w_gate)) * F.linear(x, w_up)


def fused_gate_up_swiglu(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor,
                         force_reference: bool = False) -> torch.Tensor:
    """``silu(x @ w_gate.T) * (x @ w_up.T)``: the gate/up half of a SwiGLU MLP
    (the reference's ``SwiGLUMLP``, model/dit.py:96-110) with the SwiGLU fused
    into the projection GEMM's epilogue.

    Args:
        x: [..., D] activations.
        w_gate, w_up: [H, D] projection weights (``nn.Linear.weight``); each
            may have its own row stride.
        force_reference: run the eager formulation (two Linears + silu * mul).

    The fused kernel computes in bf16 with fp32 accumulation: it runs when
    the inputs are bf16, or under bf16 autocast (as the Linears would); other
    dtypes take the two Linears and the fused SwiGLU kernel.  Host tensors
    take the eager formulation.  Gradients come back in each input's dtype.
    """
    if not use_fused(x, "fused_gate_up_swiglu", force_reference):
        return _gate_up_eager(x, w_gate, w_up)
    if w_gate.shape != w_up.shape or w_gate.dim() != 2 or x.shape[-1] != w_gate.shape[1]:
        raise ValueError(f"fused_gate_up_swiglu: x [..., D] and weights [H, D] expected, got "
                         f"{tuple(x.shape)}, {tuple(w_gate.shape)}, {tuple(w_up.shape)}")
    autocast_bf16 = (torch.is_autocast_enabled(x.device.type)
                     and torch.get_autocast_dtype(x.device.type) == torch.bfloat16)
    all_bf16 = x.dtype == w_gate.dtype == w_up.dtype == torch.bfloat16
    if not (all_bf16 or autocast_bf16):
        return fused_swiglu(F.linear(x, w_gate), F.linear(x, w_up))
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    with torch.autocast(x.device.type, enabled=False):
        act = _FusedGateUpSwiGLU.apply(
            _rows_bf16(x2), _rows_bf16(w_gate), _rows_bf16(w_up))
    return act.reshape(*lead, w_gate.shape[0])


def _rows_bf16(t: torch.Tensor) -> torch.Tensor:
    """bf16 with unit-stride rows (a differentiable cast / copy only when needed)."""
    t = t.to(torch.bfloat16)
    return t if t.stride(-1) == 1 else t.contiguous()


def fused_swiglu(a: torch.Tensor, b: torch.Tensor, force_reference: bool = False) -> torch.Tensor:
    """SwiGLU: ``silu(a) * b``, fused into a single pass.

    Args:
        a: gate projection, any shape.
        b: up projection, same shape and dtype as ``a``.
        force_reference: run the eager PyTorch formulation instead.

    Host tensors take the eager formulation, as in the reference (swiglu.py:104).
    """
    if not use_fused(a, "fused_swiglu", force_reference):
        return swiglu_ref(a, b)
    return _FusedSwiGLU.apply(a, b)
