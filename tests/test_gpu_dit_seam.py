"""DiT block integration of the fused seams (GPU).

The reference's real caller of fused_adaln_residual_rmsnorm and fused_swiglu
is the adaLN-Zero DiT block (nuvla_forge/model/dit.py:113-175), whose fused
and eager paths compute the same function (dit.py:113-118).  A two-block DiT
at the reference's model shape (dim 384, 6 heads, horizon 6, batch 8, 32
scene tokens; NuVLAConfig, model/nuvla.py:26-44) is run through both paths
with identical weights:

  * fp32: the fused model's output and every parameter gradient match the
    eager model's at 1e-5 norm-wise relative error;
  * bf16 autocast (fp32 residual, bf16 branch outputs and conditioning, fp32
    norm weights): against the eager model run in fp32, the fused model is
    as accurate as the eager model under the same autocast.  Through two
    blocks of bf16 Linears the eager path itself exceeds the per-op 2e-2 on
    some gradients (~3.4e-2 measured), so the bound is relative to it: per
    tensor within max(3e-2, 1.5 x the eager-autocast error), and over all
    gradients together within 1.25 x the eager-autocast error + 1e-3 (a
    single cancellation-dominated gradient such as the output bias, a sum of
    residuals, can land anywhere in the bf16 noise);
  * the conditioning reaches the kernel as chunk(6) views (row stride
    6 * dim) and stride-0 expand views, without copies;
  * the fused model's backward is bit-identical run to run.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from nuvla_forge_amd.kernels.adaln_rmsnorm import _cond
from oracle import numerics as on
from tests.dit_model import make_pair
from tests.helpers import gen, note, np64

pytestmark = pytest.mark.gpu

B, T, DIM, CTX = 8, 6, 384, 32


def _data(dev, seed=3):
    g = gen(seed)
    z = torch.randn(B, T, 2, generator=g).to(dev)
    c = torch.randn(B, DIM, generator=g).to(dev)
    ctx = torch.randn(B, CTX, DIM, generator=g).to(dev)
    tgt = torch.randn(B, T, 2, generator=g).to(dev)
    return z, c, ctx, tgt


def _step(model, data, autocast):
    z, c, ctx, tgt = data
    model.zero_grad(set_to_none=True)
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        out = model(z, c, ctx)
    loss = ((out.float() - tgt) ** 2).mean()
    loss.backward()
    torch.cuda.synchronize()
    grads = {n: p.grad.detach().clone() for n, p in model.named_parameters()}
    return out.detach().float(), grads


def _errors(out_a, grads_a, out_b, grads_b):
    errs = {"out": on.rel_err(np64(out_a), np64(out_b))}
    for n in grads_b:
        errs[n] = on.rel_err(np64(grads_a[n]), np64(grads_b[n]))
    return errs


def test_dit_seams_fp32_match_eager(cuda):
    note("dit seams fp32: fused vs eager, B=8 T=6 dim=384 depth=2")
    fused, eager = (m.to(cuda) for m in make_pair())
    data = _data(cuda)
    out_f, g_f = _step(fused, data, autocast=False)
    out_e, g_e = _step(eager, data, autocast=False)
    errs = _errors(out_f, g_f, out_e, g_e)
    worst = max(errs, key=errs.get)
    print(f"worst {worst}: {errs[worst]:.2e}", flush=True)
    assert all(v <= 1e-5 for v in errs.values()), {k: f"{v:.2e}" for k, v in errs.items() if v > 1e-5}


def test_dit_seams_bf16_autocast_as_accurate_as_eager(cuda):
    note("dit seams bf16 autocast: fused vs fp32 eager")
    fused, eager = (m.to(cuda) for m in make_pair(seed=1))
    data = _data(cuda, seed=4)
    out_f, g_f = _step(fused, data, autocast=True)
    out_e, g_e = _step(eager, data, autocast=False)
    errs = _errors(out_f, g_f, out_e, g_e)
    # eager under the same autocast: the rounding floor of the bf16 Linears
    out_a, g_a = _step(eager, data, autocast=True)
    floor = _errors(out_a, g_a, out_e, g_e)
    worst = max(errs, key=errs.get)
    print(f"worst {worst}: fused {errs[worst]:.2e}, eager-autocast {floor[worst]:.2e}", flush=True)
    for k in sorted(errs, key=lambda k: -errs[k] / max(floor[k], 1e-12))[:12]:
        print(f"  {k:40s} fused {errs[k]:.2e}  eager-autocast {floor[k]:.2e}", flush=True)
    bad = {k: f"{v:.2e} (eager-autocast {floor[k]:.2e})" for k, v in errs.items()
           if v > max(3e-2, 1.5 * floor[k])}
    assert not bad, bad
    cat = lambda g: np.concatenate([np64(g[k]).ravel() / np.abs(np64(g_e[k])).max() for k in g_e])
    total_f, total_a = on.rel_err(cat(g_f), cat(g_e)), on.rel_err(cat(g_a), cat(g_e))
    print(f"all gradients: fused {total_f:.2e}, eager-autocast {total_a:.2e}", flush=True)
    assert total_f <= 1.25 * total_a + 1e-3


def test_dit_seam_conditioning_views_reach_the_kernel_uncopied(cuda):
    note("dit seams: conditioning views")
    fused, _ = (m.to(cuda) for m in make_pair(seed=2))
    data = _data(cuda, seed=5)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        fused(*data[:3])
    seen = [v for blk in fused.blocks for triple in blk.seam_inputs for v in triple]
    assert any(v.stride() == (6 * DIM, 1) for v in seen)   # chunk(6) views
    assert any(v.stride() == (0, 1) for v in seen)         # expand(b, dim) zeros / ones
    for v in seen:
        assert _cond(v, B, DIM, "cond") is v  # read through its stride, never copied


def test_dit_seams_backward_is_deterministic(cuda):
    note("dit seams: determinism of the fused backward")
    fused, _ = (m.to(cuda) for m in make_pair(seed=6))
    data = _data(cuda, seed=7)
    _, g1 = _step(fused, data, autocast=True)
    _, g2 = _step(fused, data, autocast=True)
    for n in g1:
        assert torch.equal(g1[n], g2[n]), n
