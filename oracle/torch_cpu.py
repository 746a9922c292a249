"""PyTorch-CPU restatement of the reference's eager path (test oracle; see __init__).

This is what ``bench.py``'s ``cpu_baseline`` times on the GPU host's cores:
the reference's non-fused formulation (``kernels/reference.py:22-96``) run
forward plus ``torch.autograd.backward``, and, for the cross entropy, the
reference's CPU row-chunk loop (``kernels/chunked_ce.py:101-182``) with its
gradient formed during the forward pass.  It also serves the CPU tests as an
autograd cross-check of ``numerics``.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def _rows(c: torch.Tensor, t: int) -> torch.Tensor:
    return c.repeat_interleave(t, dim=0)


def _wide(t: torch.Tensor) -> torch.Tensor:
    """The reference's `.float()`, except that fp64 stays fp64 (for the fp64 checks)."""
    return t.to(torch.promote_types(t.dtype, torch.float32))


def adaln_fwd_bwd(x, y, gate, weight, scale, shift, t, dh_up, dout, eps=1e-6):
    """Forward (reference.py:22-66) and autograd backward of <h,dh_up> + <out,dout>.

    Returns (h, out, grads) with grads keyed x, y, gate, weight, scale, shift.
    """
    leaves = {k: v.detach().clone().requires_grad_(True)
              for k, v in dict(x=x, y=y, gate=gate, weight=weight, scale=scale, shift=shift).items()}
    lv = leaves
    h = lv["x"] + _rows(lv["gate"], t) * lv["y"]
    hf = _wide(h)
    rstd = torch.rsqrt(hf.pow(2).mean(dim=-1, keepdim=True) + eps)
    out = (hf * rstd * _wide(lv["weight"]) * (1.0 + _wide(_rows(lv["scale"], t)))
           + _wide(_rows(lv["shift"], t))).to(x.dtype)
    torch.autograd.backward([h, out], [dh_up, dout])
    return h.detach(), out.detach(), {k: v.grad for k, v in leaves.items()}


def swiglu_fwd_bwd(a, b, dout):
    """(silu(a.float()) * b.float()).to(a.dtype) (reference.py:69-74) and its autograd grads."""
    a = a.detach().clone().requires_grad_(True)
    b = b.detach().clone().requires_grad_(True)
    out = (F.silu(_wide(a)) * _wide(b)).to(a.dtype)
    out.backward(dout)
    return out.detach(), a.grad, b.grad


def chunked_ce_fwd_bwd(hidden, weight, targets, chunk_size=1024, ignore_index=-100):
    """The reference's CPU chunk loop: loss, dH, dW (fp32), chunked_ce.py:101-172."""
    m = hidden.shape[0]
    valid_all = targets != ignore_index
    inv = 1.0 / max(int(valid_all.sum()), 1)
    w = weight.float()
    loss = torch.zeros((), dtype=torch.float32)
    d_hidden = torch.zeros(hidden.shape, dtype=torch.float32)
    d_weight = torch.zeros(weight.shape, dtype=torch.float32)
    for start in range(0, m, chunk_size):
        stop = min(start + chunk_size, m)
        hc = hidden[start:stop].float()
        tc = targets[start:stop]
        valid = tc != ignore_index
        z = F.linear(hc, w)
        lse = torch.logsumexp(z, dim=-1)
        safe = tc.clamp(min=0)
        zt = z.gather(1, safe.unsqueeze(1)).squeeze(1)
        loss += torch.where(valid, lse - zt, torch.zeros_like(lse)).sum() * inv
        p = torch.softmax(z, dim=-1)
        p.scatter_add_(1, safe.unsqueeze(1), -torch.ones_like(zt).unsqueeze(1))
        p = p * valid.unsqueeze(1) * inv
        d_hidden[start:stop] = p @ w
        d_weight += p.T @ hc
    return loss, d_hidden, d_weight


def ce_autograd(hidden, weight, targets, ignore_index=-100):
    """Textbook F.cross_entropy(mean) with autograd (reference.py:77-96), any dtype."""
    h = hidden.detach().clone().requires_grad_(True)
    w = weight.detach().clone().requires_grad_(True)
    loss = F.cross_entropy(h @ w.T, targets, ignore_index=ignore_index, reduction="mean")
    loss.backward()
    return loss.detach(), h.grad, w.grad
