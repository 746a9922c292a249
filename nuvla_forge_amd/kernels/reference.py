"""Eager PyTorch formulations of the three fused ops (``force_reference=True``).

Same names and semantics as ``nuvla_forge/kernels/reference.py``: the
reference's own non-fused path, which its ``force_reference`` switch selects
and its DiT/nuVLA models run with ``fused=False``.  These run on whatever
device the inputs live on, through ATen; they are never chosen implicitly.
The parity oracle the tests use is a separate NumPy restatement (``oracle/``).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def _expand_cond(c: torch.Tensor, tokens_per_sample: int) -> torch.Tensor:
    """[B, N] -> [B*T, N]; row m belongs to sample m // T (reference.py:17-19)."""
    return c.repeat_interleave(tokens_per_sample, dim=0)


def adaln_residual_rmsnorm_ref(x, y, gate, weight, scale, shift, tokens_per_sample, eps=1e-6):
    """h = x + gate*y;  out = rmsnorm(h) * w * (1 + scale) + shift  (reference.py:22-66).

    Returns (h, out); out is cast to x.dtype, h keeps the promoted dtype of
    ``x + gate * y`` exactly as the reference's eager expression does.
    """
    t = tokens_per_sample
    g = _expand_cond(gate, t)
    s = _expand_cond(scale, t)
    sh = _expand_cond(shift, t)
    h = x + g * y
    hf = h.float()
    rstd = torch.rsqrt(hf.pow(2).mean(dim=-1, keepdim=True) + eps)
    out = hf * rstd * weight.float() * (1.0 + s.float()) + sh.float()
    return h, out.to(x.dtype)


def swiglu_ref(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """silu(a) * b in fp32, cast to a.dtype (reference.py:69-74)."""
    return (F.silu(a.float()) * b.float()).to(a.dtype)


def chunked_cross_entropy_ref(hidden, lm_weight, targets, ignore_index=-100):
    """Unchunked mean cross entropy over hidden @ lm_weight.T (reference.py:77-96)."""
    logits = F.linear(hidden.float(), lm_weight.float())
    return F.cross_entropy(logits, targets, ignore_index=ignore_index, reduction="mean")
