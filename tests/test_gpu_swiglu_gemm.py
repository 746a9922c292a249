"""SwiGLU fused into the gate/up projection GEMM (GPU).

``fused_gate_up_swiglu(x, w_gate, w_up)`` computes what the reference's
SwiGLUMLP computes before its down projection, ``silu(x W_gate^T) *
(x W_up^T)`` (model/dit.py:96-110), with one MFMA kernel whose epilogue
applies the activation.  Checked against the fp64 oracle on the same
bf16-rounded operands, forward and all three gradients, at 2e-2 norm-wise
relative error (the bf16 criterion), across tile-aligned, ragged (M, H not
multiples of the 256 x 128 tile), unaligned-D (register-copy loader) and
single-row shapes; against the eager composition; under bf16 autocast with
fp32 activations and weights; and fp32 inputs without autocast, which take
the two Linears and the fused SwiGLU kernel (1e-5).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from nuvla_forge_amd.kernels import fused_gate_up_swiglu
from oracle import numerics as on
from tests.helpers import gen, note, np64, randn

pytestmark = pytest.mark.gpu


def _oracle(x, wg, wu, dact):
    """fp64: a = x Wg^T, b = x Wu^T, act = silu(a) b and its gradients."""
    a, b = x @ wg.T, x @ wu.T
    act = on.swiglu_forward(a, b)
    da, db = on.swiglu_backward(a, b, dact)
    return act, da @ wg + db @ wu, da.T @ x, db.T @ x


def _inputs(m, d, h, dtype, dev, seed=0):
    g = gen(seed)
    x = randn((m, d), g, dtype, dev)
    wg = randn((h, d), g, dtype, dev, std=d ** -0.5)
    wu = randn((h, d), g, dtype, dev, std=d ** -0.5)
    dact = randn((m, h), g, dtype, dev)
    return x, wg, wu, dact


def _run(x, wg, wu, dact, **kw):
    leaves = [t.detach().requires_grad_(True) for t in (x, wg, wu)]
    act = fused_gate_up_swiglu(*leaves, **kw)
    act.backward(dact)
    torch.cuda.synchronize()
    return act.detach(), [t.grad for t in leaves]


@pytest.mark.parametrize("m,d,h", [(512, 384, 1536), (300, 200, 333), (64, 36, 100), (1, 8, 1),
                                   (2048, 1024, 2816)])
def test_gate_up_swiglu_matches_oracle(cuda, m, d, h):
    note(f"gemm swiglu m={m} d={d} h={h}")
    x, wg, wu, dact = _inputs(m, d, h, torch.bfloat16, cuda)
    act, (dx, dwg, dwu) = _run(x, wg, wu, dact)
    assert act.dtype == dx.dtype == dwg.dtype == torch.bfloat16
    ref = _oracle(np64(x), np64(wg), np64(wu), np64(dact))
    errs = {k: on.rel_err(np64(v), r)
            for k, v, r in zip(("act", "dx", "dwg", "dwu"), (act, dx, dwg, dwu), ref)}
    assert all(e <= 2e-2 for e in errs.values()), errs


def test_gate_up_swiglu_agrees_with_eager_composition(cuda):
    note("gemm swiglu vs eager composition")
    x, wg, wu, dact = _inputs(1024, 512, 1024, torch.bfloat16, cuda, seed=1)
    act, grads = _run(x, wg, wu, dact)
    act_e, grads_e = _run(x, wg, wu, dact, force_reference=True)
    assert on.rel_err(np64(act), np64(act_e)) < 1e-2
    for g, ge in zip(grads, grads_e):
        assert on.rel_err(np64(g), np64(ge)) < 2e-2


def test_gate_up_swiglu_under_autocast_keeps_input_dtypes(cuda):
    """fp32 activations and fp32 nn.Linear weights under bf16 autocast run
    the fused bf16 kernel; the gradients come back in fp32."""
    note("gemm swiglu autocast fp32 -> bf16")
    x, wg, wu, dact = _inputs(256, 384, 768, torch.float32, cuda, seed=2)
    leaves = [t.detach().requires_grad_(True) for t in (x, wg, wu)]
    with torch.autocast("cuda", dtype=torch.bfloat16):
        act = fused_gate_up_swiglu(*leaves)
    assert act.dtype == torch.bfloat16
    act.backward(dact.to(torch.bfloat16))
    torch.cuda.synchronize()
    assert all(t.grad.dtype == torch.float32 for t in leaves)
    xb, wgb, wub = (np64(t.to(torch.bfloat16)) for t in (x, wg, wu))
    ref = _oracle(xb, wgb, wub, np64(dact.to(torch.bfloat16)))
    got = [act] + [t.grad for t in leaves]
    assert all(on.rel_err(np64(v), r) <= 2e-2 for v, r in zip(got, ref))


def test_gate_up_swiglu_fp32_takes_the_composed_path(cuda):
    note("gemm swiglu fp32 without autocast")
    x, wg, wu, dact = _inputs(128, 64, 96, torch.float32, cuda, seed=3)
    act, (dx, dwg, dwu) = _run(x, wg, wu, dact)
    ref = _oracle(np64(x), np64(wg), np64(wu), np64(dact))
    for v, r in zip((act, dx, dwg, dwu), ref):
        assert on.rel_err(np64(v), r) <= 1e-5


def test_gate_up_swiglu_forward_is_deterministic_and_3d(cuda):
    note("gemm swiglu determinism, [B, T, D] input")
    x, wg, wu, _ = _inputs(4 * 96, 256, 640, torch.bfloat16, cuda, seed=4)
    x3 = x.view(4, 96, 256)
    a1 = fused_gate_up_swiglu(x3, wg, wu)
    a2 = fused_gate_up_swiglu(x3, wg, wu)
    assert a1.shape == (4, 96, 640) and torch.equal(a1, a2)
    ref = F.silu(x.float() @ wg.float().T) * (x.float() @ wu.float().T)
    assert on.rel_err(np64(a1.reshape(-1, 640)), np64(ref)) < 2e-2
