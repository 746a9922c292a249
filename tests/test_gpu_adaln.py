"""adaLN seam HIP kernels vs the oracle (GPU).

Covers BASELINE cfg1 (fp32 [2,64,256], all six gradients at 1e-5) and cfg2
(bf16 [8,1024,1024], 10 bit-identical backward passes), the reference's test
shapes (tests/test_kernels.py:85-115, incl. the N=1000 masked tail), odd N
(element-wise kernel variant), wide N (multi-wavefront rows) in fp32, bf16
and fp16, mixed autocast dtypes (fp32 residual with a bf16 or fp16 branch), strided / broadcast conditioning views as the DiT block passes them
(model/dit.py:146-166), missing upstream gradients, and the large seam stress
shape [32,2048,2048]; many samples with one row each (several reduction
rounds) and single-row inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from nuvla_forge_amd.kernels import fused_adaln_residual_rmsnorm
from oracle import numerics as on
from tests.helpers import TOL, gen, note, np64, randn

pytestmark = pytest.mark.gpu

NAMES = ("x", "y", "gate", "weight", "scale", "shift")


def _inputs(b, t, n, dtype, dev, seed=0, cond_dtype=None, y_dtype=None):
    """BASELINE distributions: x, y ~ N(0,1); cond ~ N(0, 0.1); w = 1 + N(0, 0.02)."""
    g = gen(seed)
    cd = cond_dtype or dtype
    return {
        "x": randn((b * t, n), g, dtype, dev),
        "y": randn((b * t, n), g, y_dtype or dtype, dev),
        "gate": randn((b, n), g, cd, dev, std=0.1),
        "weight": randn((n,), g, cd, dev, std=0.02, mean=1.0),
        "scale": randn((b, n), g, cd, dev, std=0.1),
        "shift": randn((b, n), g, cd, dev, std=0.1),
    }


def _upstream(m, n, dtype, dev, seed=1):
    g = gen(seed)
    return randn((m, n), g, dtype, dev), randn((m, n), g, dtype, dev)


def _run(inp, t, dh, dout):
    leaves = {k: v.detach().requires_grad_(True) for k, v in inp.items()}
    h, out = fused_adaln_residual_rmsnorm(**leaves, tokens_per_sample=t)
    torch.autograd.backward([h, out], [dh, dout])
    torch.cuda.synchronize()
    return h.detach(), out.detach(), {k: v.grad for k, v in leaves.items()}


def _check(inp, t, dh, dout, h, out, grads, tol, label, eps=1e-6):
    a = {k: np64(v) for k, v in inp.items()}
    hw, ow, _ = on.adaln_forward(**a, t=t, eps=eps)
    gw = on.adaln_backward(**a, t=t, dh_up=np64(dh), dout=np64(dout), eps=eps)
    errs = {"h": on.rel_err(np64(h), hw), "out": on.rel_err(np64(out), ow)}
    for k in NAMES:
        errs["d" + k] = on.rel_err(np64(grads[k]), gw[k])
    bad = {k: v for k, v in errs.items() if not v <= tol}
    assert not bad, f"{label}: rel err above {tol}: {bad}"
    return errs


def test_cfg1_fp32_all_six_gradients(cuda):
    note("adaln cfg1 fp32 [2,64,256]")
    b, t, n = 2, 64, 256
    inp = _inputs(b, t, n, torch.float32, cuda)
    dh, dout = _upstream(b * t, n, torch.float32, cuda)
    h, out, grads = _run(inp, t, dh, dout)
    _check(inp, t, dh, dout, h, out, grads, 1e-5, "cfg1")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("b,t,n", [(2, 16, 256), (4, 32, 1024), (3, 7, 768), (1, 64, 1536),
                                   (2, 8, 1000), (2, 3, 333), (1, 5, 8), (2, 4, 4096),
                                   (1, 2, 16384), (300, 1, 64), (1, 1, 1024), (5, 3, 2048),
                                   (3, 700, 512), (24, 96, 1024)])
def test_adaln_matches_oracle(cuda, dtype, b, t, n):
    note(f"adaln dtype={dtype} b={b} t={t} n={n}")
    inp = _inputs(b, t, n, dtype, cuda)
    dh, dout = _upstream(b * t, n, dtype, cuda)
    h, out, grads = _run(inp, t, dh, dout)
    assert h.dtype == dtype and out.dtype == dtype
    for k in NAMES:
        assert grads[k].dtype == inp[k].dtype and grads[k].shape == inp[k].shape
    _check(inp, t, dh, dout, h, out, grads, TOL[dtype], f"{dtype} ({b},{t},{n})")


@pytest.mark.parametrize("dtype,b,t,n", [
    (torch.bfloat16, 8, 128, 8192),   # 4 rows per forward group, 8 wavefronts x 2 chunks back
    (torch.bfloat16, 2, 256, 16384),  # 2 rows per forward group, 16 wavefronts, no prefetch
    (torch.bfloat16, 4, 64, 6000),    # 8 wavefronts x 2 chunks with a partial last chunk
    (torch.float16, 3, 100, 5000),    # wide rows whose groups cross samples
    (torch.float32, 2, 256, 8192),
    (torch.float32, 1, 64, 16384),
    (torch.bfloat16, 2, 40, 10001),   # odd N: element-wise path, 16 wavefronts, LDS factors
    (torch.float32, 3, 30, 5001),     # odd N: element-wise path, 8 wavefronts x 2 chunks
    (torch.bfloat16, 4, 129, 12000),  # odd T: the one-row forward on 1024-thread blocks
    (torch.float16, 3, 75, 16384),    # fewer than 2 rows per forward group
])
def test_adaln_wide_rows(cuda, dtype, b, t, n):
    """Rows of 5000-16384 elements with enough rows for the wide-row launch
    plans (several rows per forward row group, two chunks per lane in the
    backward), against the oracle, and a second backward bit-identical."""
    note(f"adaln wide rows dtype={dtype} b={b} t={t} n={n}")
    inp = _inputs(b, t, n, dtype, cuda)
    dh, dout = _upstream(b * t, n, dtype, cuda)
    h, out, grads = _run(inp, t, dh, dout)
    _check(inp, t, dh, dout, h, out, grads, TOL[dtype], f"wide {dtype} ({b},{t},{n})")
    _, _, again = _run(inp, t, dh, dout)
    for k in NAMES:
        assert torch.equal(again[k], grads[k]), f"d{k} differs between runs"


def test_cfg2_bf16_and_bitwise_deterministic_backward(cuda):
    note("adaln cfg2 bf16 [8,1024,1024] x10 backward")
    b, t, n = 8, 1024, 1024
    inp = _inputs(b, t, n, torch.bfloat16, cuda)
    dh, dout = _upstream(b * t, n, torch.bfloat16, cuda)
    h, out, grads = _run(inp, t, dh, dout)
    _check(inp, t, dh, dout, h, out, grads, 2e-2, "cfg2")
    for _ in range(9):
        _, _, again = _run(inp, t, dh, dout)
        for k in NAMES:
            assert torch.equal(again[k], grads[k]), f"d{k} differs between runs"


def test_mixed_autocast_dtypes(cuda):
    """x fp32 residual, y bf16 branch output, bf16 conditioning, fp32 weight."""
    note("adaln mixed dtypes")
    b, t, n = 2, 32, 512
    inp = _inputs(b, t, n, torch.float32, cuda, cond_dtype=torch.bfloat16, y_dtype=torch.bfloat16)
    inp["weight"] = inp["weight"].float()
    dh, dout = _upstream(b * t, n, torch.float32, cuda)
    h, out, grads = _run(inp, t, dh, dout)
    assert h.dtype == torch.float32 and grads["y"].dtype == torch.bfloat16
    assert grads["gate"].dtype == torch.bfloat16 and grads["weight"].dtype == torch.float32
    _check(inp, t, dh, dout, h, out, grads, 2e-2, "mixed")


def test_mixed_fp32_residual_fp16_branch(cuda):
    """x fp32 residual with an fp16 branch output, fp16 conditioning and weight
    (the fp16 autocast form of the seam)."""
    note("adaln mixed fp32 / fp16")
    b, t, n = 3, 40, 768
    inp = _inputs(b, t, n, torch.float32, cuda, cond_dtype=torch.float16, y_dtype=torch.float16)
    dh, dout = _upstream(b * t, n, torch.float32, cuda)
    h, out, grads = _run(inp, t, dh, dout)
    assert h.dtype == torch.float32 and grads["y"].dtype == torch.float16
    assert grads["gate"].dtype == torch.float16 and grads["shift"].dtype == torch.float16
    _check(inp, t, dh, dout, h, out, grads, 2e-2, "mixed fp16")


def test_strided_and_broadcast_conditioning(cuda):
    """chunk(6) views (row stride 6N) and expand()-ed zeros/ones (row stride 0)."""
    note("adaln strided cond")
    b, t, n = 4, 16, 256
    g = gen(5)
    x = randn((b * t, n), g, torch.float32, cuda)
    y = randn((b * t, n), g, torch.float32, cuda)
    w = randn((n,), g, torch.float32, cuda, std=0.02, mean=1.0)
    cond = randn((b, 6 * n), g, torch.float32, cuda, std=0.1).requires_grad_(True)
    shift1, scale1, gate1, shift2, scale2, gate2 = cond.chunk(6, dim=-1)
    zeros = torch.zeros(1, n, device=cuda).expand(b, n)
    ones = torch.ones(1, n, device=cuda).expand(b, n)
    dh, dout = _upstream(b * t, n, torch.float32, cuda)
    for gate, scale, shift in ((gate1, zeros, zeros), (ones, scale2, shift2)):
        cond.grad = None
        xs = x.detach().requires_grad_(True)
        ws = w.detach().requires_grad_(True)
        h, out = fused_adaln_residual_rmsnorm(xs, y, gate, ws, scale, shift, tokens_per_sample=t)
        torch.autograd.backward([h, out], [dh, dout])
        a = dict(x=np64(x), y=np64(y), gate=np64(gate), weight=np64(w), scale=np64(scale),
                 shift=np64(shift))
        hw, ow, _ = on.adaln_forward(**a, t=t)
        gw = on.adaln_backward(**a, t=t, dh_up=np64(dh), dout=np64(dout))
        assert on.rel_err(np64(out), ow) < 1e-5 and on.rel_err(np64(h), hw) < 1e-5
        assert on.rel_err(np64(xs.grad), gw["x"]) < 1e-5
        assert on.rel_err(np64(ws.grad), gw["weight"]) < 1e-5
        # gradients land in the right sixth of the cond projection
        cg = np64(cond.grad).reshape(b, 6, n)
        if gate is gate1:
            assert on.rel_err(cg[:, 2], gw["gate"]) < 1e-5
            assert not cg[:, [0, 1, 3, 4, 5]].any()
        else:
            assert on.rel_err(cg[:, 4], gw["scale"]) < 1e-5
            assert on.rel_err(cg[:, 3], gw["shift"]) < 1e-5
            assert not cg[:, [0, 1, 2, 5]].any()


@pytest.mark.parametrize("which", ["h_only", "out_only"])
def test_missing_upstream_gradient(cuda, which):
    note(f"adaln upstream {which}")
    b, t, n = 2, 8, 512
    inp = _inputs(b, t, n, torch.float32, cuda)
    leaves = {k: v.detach().requires_grad_(True) for k, v in inp.items()}
    h, out = fused_adaln_residual_rmsnorm(**leaves, tokens_per_sample=t)
    g = randn((b * t, n), gen(3), torch.float32, cuda)
    (h if which == "h_only" else out).backward(g)
    torch.cuda.synchronize()
    a = {k: np64(v) for k, v in inp.items()}
    gw = on.adaln_backward(**a, t=t, dh_up=np64(g) if which == "h_only" else None,
                           dout=np64(g) if which == "out_only" else None)
    for k in NAMES:
        got = leaves[k].grad
        want = gw[k]
        if got is None:
            assert not np.any(want), k
        else:
            assert on.rel_err(np64(got), want) < 1e-5, k


@pytest.mark.parametrize("want", [("weight",), ("gate", "shift"), ("scale",),
                                  ("x", "y"), ("gate", "weight", "scale", "shift")])
@pytest.mark.parametrize("b,t,n", [(8, 64, 1024), (2, 16, 333), (40, 3, 256)])
def test_only_some_parameter_gradients(cuda, want, b, t, n):
    """Leaves that do not require grad get no reduction output: the partial
    reduction runs without its dweight blocks, or without its dgate / dshift /
    dscale blocks, and the requested sums are unchanged."""
    note(f"adaln grads {want} b={b} t={t} n={n}")
    inp = _inputs(b, t, n, torch.float32, cuda, seed=5)
    leaves = {k: v.detach().requires_grad_(k in want) for k, v in inp.items()}
    h, out = fused_adaln_residual_rmsnorm(**leaves, tokens_per_sample=t)
    dh, dout = _upstream(b * t, n, torch.float32, cuda, seed=6)
    torch.autograd.backward([h, out], [dh, dout])
    torch.cuda.synchronize()
    a = {k: np64(v) for k, v in inp.items()}
    gw = on.adaln_backward(**a, t=t, dh_up=np64(dh), dout=np64(dout))
    for k in NAMES:
        got = leaves[k].grad
        if k not in want:
            assert got is None, k
        else:
            assert on.rel_err(np64(got), gw[k]) < 1e-5, (k, on.rel_err(np64(got), gw[k]))


def test_zero_gate_keeps_residual_exact(cuda):
    note("adaln zero gate")
    b, t, n = 2, 16, 1024
    inp = _inputs(b, t, n, torch.bfloat16, cuda)
    inp["gate"] = torch.zeros_like(inp["gate"])
    h, _ = fused_adaln_residual_rmsnorm(**inp, tokens_per_sample=t)
    assert torch.equal(h, inp["x"])


def test_rejects_bad_shapes(cuda):
    x = torch.zeros(10, 64, device=cuda)
    c = torch.zeros(2, 64, device=cuda)
    with pytest.raises(ValueError):
        fused_adaln_residual_rmsnorm(x, x, c, torch.ones(64, device=cuda), c, c, 3)
    c3 = torch.zeros(3, 64, device=cuda)
    with pytest.raises(ValueError):  # T = 5 gives B = 2, not 3
        fused_adaln_residual_rmsnorm(x, x, c3, torch.ones(64, device=cuda), c3, c3, 5)


def test_rows_wider_than_the_kernels_take_the_eager_path(cuda):
    """N = 16385: the reference's eager fallback on the device (adaln_rmsnorm.py:262),
    checked against the oracle (the eager path normalises in fp32)."""
    note("adaln N=16385 eager fallback")
    b, t, n = 1, 2, 16385
    inp = _inputs(b, t, n, torch.float32, cuda, seed=9)
    dh, dout = _upstream(b * t, n, torch.float32, cuda, seed=10)
    h, out, grads = _run(inp, t, dh, dout)
    _check(inp, t, dh, dout, h, out, grads, 1e-5, "N=16385")


def test_eps_placement_rows_near_eps(cuda):
    """Rows whose mean square is comparable to eps (x, y ~ N(0, 1e-3), eps =
    1e-6), where eps inside the square root (reference.py:62,
    adaln_rmsnorm.py:85-86) and any other placement differ by percents: fp32
    at 1e-5 against the oracle, for the forward and all six gradients."""
    note("adaln eps placement fp32 rows ~1e-3")
    b, t, n = 2, 64, 1024
    g = gen(11)
    inp = {
        "x": randn((b * t, n), g, torch.float32, cuda, std=1e-3),
        "y": randn((b * t, n), g, torch.float32, cuda, std=1e-3),
        "gate": randn((b, n), g, torch.float32, cuda, std=0.1),
        "weight": randn((n,), g, torch.float32, cuda, std=0.02, mean=1.0),
        "scale": randn((b, n), g, torch.float32, cuda, std=0.1),
        "shift": randn((b, n), g, torch.float32, cuda, std=0.1),
    }
    dh, dout = _upstream(b * t, n, torch.float32, cuda, seed=12)
    h, out, grads = _run(inp, t, dh, dout)
    _check(inp, t, dh, dout, h, out, grads, 1e-5, "eps rows")
    # the rows really sit where eps matters: moving eps outside the root
    # changes the oracle's output by far more than the tolerance
    a = {k: np64(v) for k, v in inp.items()}
    hh = a["x"] + np.repeat(a["gate"], t, axis=0) * a["y"]
    ms = np.mean(hh * hh, axis=1)
    assert 0.3 < float(np.median(ms)) / 1e-6 < 3.0
    _, ow, _ = on.adaln_forward(**a, t=t)
    wrong = 1.0 / (np.sqrt(ms) + 1e-6)
    out_wrong = (hh * wrong[:, None]) * a["weight"] * (1 + np.repeat(a["scale"], t, 0)) + \
        np.repeat(a["shift"], t, 0)
    assert on.rel_err(out_wrong, ow) > 1e-2


def test_stress_shape(cuda):
    """BASELINE cfg5 seam: bf16 [32, 2048, 2048], oracle evaluated in fp32 on the host."""
    note("adaln stress bf16 [32,2048,2048]")
    b, t, n = 32, 2048, 2048
    inp = _inputs(b, t, n, torch.bfloat16, cuda, seed=7)
    dh, dout = _upstream(b * t, n, torch.bfloat16, cuda, seed=8)
    h, out, grads = _run(inp, t, dh, dout)

    def f32(v):
        return v.to("cpu", torch.float32).numpy()

    a = {k: f32(v) for k, v in inp.items()}
    hw, ow, _ = on.adaln_forward(**a, t=t)
    gw = on.adaln_backward(**a, t=t, dh_up=f32(dh), dout=f32(dout))
    errs = {"h": on.rel_err(f32(h), hw), "out": on.rel_err(f32(out), ow)}
    for k in NAMES:
        errs["d" + k] = on.rel_err(f32(grads[k]), gw[k])
    bad = {k: v for k, v in errs.items() if not v <= 2e-2}
    assert not bad, bad


@pytest.mark.parametrize("b,t,n,dt", [(8, 1024, 1024, torch.bfloat16), (8, 6, 384, None)])
def test_fwd_bwd_replays_in_a_graph(cuda, b, t, n, dt):
    """Forward + backward captured in a HIP graph (as bench.py times it):
    every replay matches the eager step bit for bit.  dt None: the DiT
    block's autocast mix (fp32 x, bf16 y and conditioning, fp32 weight)."""
    from tests.helpers import assert_graph_replays_match

    note(f"adaln graph replay b={b} t={t} n={n} dt={dt}")
    if dt is None:
        inp = _inputs(b, t, n, torch.float32, cuda, cond_dtype=torch.bfloat16,
                      y_dtype=torch.bfloat16)
        inp["weight"] = inp["weight"].float()
        dh, dout = _upstream(b * t, n, torch.float32, cuda)
    else:
        inp = _inputs(b, t, n, dt, cuda)
        dh, dout = _upstream(b * t, n, dt, cuda)

    def make():
        leaves = {k: v.detach().requires_grad_(True) for k, v in inp.items()}

        def step():
            h, out = fused_adaln_residual_rmsnorm(**leaves, tokens_per_sample=t)
            grads = torch.autograd.grad([h, out], list(leaves.values()), [dh, dout])
            return (h, out, *grads)

        return step

    assert_graph_replays_match(make)
