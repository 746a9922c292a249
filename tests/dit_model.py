"""A compact adaLN-Zero DiT block for the seam integration tests.

It exercises the two fused seams exactly as the reference's caller drives
them (nuvla_forge/model/dit.py:113-175):

  * conditioning from one Linear(dim, 6 dim) split with ``chunk(6)``, so
    gate/scale/shift reach the kernel as row-strided views (stride 6 * dim);
  * seam 1 passes stride-0 ``expand`` zeros as scale and shift (an
    unmodulated norm for the cross-attention input), seam 2 passes ``expand``
    ones as the gate;
  * [B, T, dim] activations flattened to [B * T, dim] with T as
    ``tokens_per_sample``;
  * under bf16 autocast the residual stream is fp32 while the branch outputs
    and the conditioning are bf16 and the norm weights fp32.

``fused=False`` is the eager formulation of the same function
(dit.py:169-172), which is what the fused path is compared against.
Attention is computed in fp32 on contiguous operands (the test is about the
seams; it keeps clear of bf16 batched products on transposed views).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from nuvla_forge_amd.kernels import fused_adaln_residual_rmsnorm, fused_swiglu


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x):
        xf = x.float()
        r = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return (xf * r).to(x.dtype) * self.weight


def modulate(x, shift, scale):
    return x * (1 + scale.unsqueeze(1)) + shift.unsqueeze(1)


class Attention(nn.Module):
    """Multi-head attention with the math in fp32 (self or cross)."""

    def __init__(self, dim: int, heads: int):
        super().__init__()
        self.heads = heads
        self.q = nn.Linear(dim, dim, bias=False)
        self.kv = nn.Linear(dim, 2 * dim, bias=False)
        self.proj = nn.Linear(dim, dim, bias=False)

    def forward(self, x, context=None):
        b, t, c = x.shape
        ctx = x if context is None else context
        s = ctx.shape[1]
        hd = c // self.heads
        q = self.q(x.reshape(b * t, c)).float().reshape(b, t, self.heads, hd)
        kv = self.kv(ctx.reshape(b * s, c)).float().reshape(b, s, 2, self.heads, hd)
        q = q.permute(0, 2, 1, 3).contiguous()                 # [b, H, t, hd]
        k = kv[:, :, 0].permute(0, 2, 3, 1).contiguous()       # [b, H, hd, s]
        v = kv[:, :, 1].permute(0, 2, 1, 3).contiguous()       # [b, H, s, hd]
        w = torch.softmax(torch.matmul(q, k) / hd ** 0.5, dim=-1)
        o = torch.matmul(w, v).permute(0, 2, 1, 3).reshape(b * t, c).contiguous()
        return self.proj(o).reshape(b, t, c)


class SwiGLUMLP(nn.Module):
    def __init__(self, dim: int, hidden: int, fused: bool):
        super().__init__()
        self.w_gate = nn.Linear(dim, hidden, bias=False)
        self.w_up = nn.Linear(dim, hidden, bias=False)
        self.w_down = nn.Linear(hidden, dim, bias=False)
        self.fused = fused

    def forward(self, x):
        b, t, c = x.shape
        x2 = x.reshape(b * t, c)
        a, g = self.w_gate(x2), self.w_up(x2)
        act = fused_swiglu(a, g) if self.fused else F.silu(a) * g
        return self.w_down(act).reshape(b, t, c)


class DiTBlock(nn.Module):
    def __init__(self, dim: int, heads: int, fused: bool, mlp_ratio: float = 4.0):
        super().__init__()
        self.dim = dim
        self.fused = fused
        self.norm1 = RMSNorm(dim)
        self.norm2 = RMSNorm(dim)
        self.norm_cross = RMSNorm(dim)
        self.attn = Attention(dim, heads)
        self.cross = Attention(dim, heads)
        self.mlp = SwiGLUMLP(dim, int(dim * mlp_ratio), fused)
        self.cond = nn.Sequential(nn.SiLU(), nn.Linear(dim, 6 * dim))
        self.register_buffer("_zeros", torch.zeros(1, dim), persistent=False)
        self.register_buffer("_ones", torch.ones(1, dim), persistent=False)
        self.seam_inputs = []  # (gate, scale, shift) views seen by the fused seams

    def forward(self, x, c, context):
        b, t, _ = x.shape
        shift1, scale1, gate1, shift2, scale2, gate2 = self.cond(c).chunk(6, dim=-1)
        if not self.fused:
            x = x + gate1.unsqueeze(1) * self.attn(modulate(self.norm1(x), shift1, scale1))
            x = x + self.cross(self.norm_cross(x), context)
            return x + gate2.unsqueeze(1) * self.mlp(modulate(self.norm2(x), shift2, scale2))

        attn_out = self.attn(modulate(self.norm1(x), shift1, scale1))
        zeros = self._zeros.to(x.dtype).expand(b, self.dim)
        self.seam_inputs.append((gate1, zeros, zeros))
        x2, h = fused_adaln_residual_rmsnorm(
            x.reshape(b * t, -1), attn_out.reshape(b * t, -1), gate1,
            self.norm_cross.weight, zeros, zeros, tokens_per_sample=t)
        cross_out = self.cross(h.reshape(b, t, -1), context)
        ones = self._ones.to(x.dtype).expand(b, self.dim)
        self.seam_inputs.append((ones, scale2, shift2))
        x2, h = fused_adaln_residual_rmsnorm(
            x2, cross_out.reshape(b * t, -1), ones, self.norm2.weight, scale2, shift2,
            tokens_per_sample=t)
        x = x2.reshape(b, t, -1)
        return x + gate2.unsqueeze(1) * self.mlp(h.reshape(b, t, -1))


class SmallDiT(nn.Module):
    """in_proj + pos -> depth DiT blocks -> out, conditioned on c and context."""

    def __init__(self, dim=384, depth=2, heads=6, horizon=6, fused=True):
        super().__init__()
        self.in_proj = nn.Linear(2, dim)
        self.pos = nn.Parameter(torch.zeros(1, horizon, dim))
        self.blocks = nn.ModuleList([DiTBlock(dim, heads, fused) for _ in range(depth)])
        self.norm_out = RMSNorm(dim)
        self.out = nn.Linear(dim, 2)

    def forward(self, z, c, context):
        x = self.in_proj(z) + self.pos
        for blk in self.blocks:
            x = blk(x, c, context)
        return self.out(self.norm_out(x))


def make_pair(dim=384, depth=2, heads=6, horizon=6, seed=0):
    """A fused and an eager model with identical random weights (the
    conditioning projection is random rather than adaLN-Zero's zeros, so the
    gates, scales and shifts are not trivial)."""
    torch.manual_seed(seed)
    fused = SmallDiT(dim, depth, heads, horizon, fused=True)
    for p in fused.parameters():
        with torch.no_grad():
            p.normal_(0.0, 0.05)
    for blk in fused.blocks:
        for norm in (blk.norm1, blk.norm2, blk.norm_cross):
            with torch.no_grad():
                norm.weight.normal_(1.0, 0.02)
    eager = SmallDiT(dim, depth, heads, horizon, fused=False)
    eager.load_state_dict(fused.state_dict())
    return fused, eager
