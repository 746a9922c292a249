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


def test_gate_up_swiglu_weights_with_different_row_strides(cuda):
    """w_gate a column-slice view of a wider [H, 2D + 8] tensor (row stride
    2D + 8), w_up contiguous (row stride D): each weight is read through its
    own row stride."""
    note("gemm swiglu w_gate strided view, w_up contiguous")
    m, d, h = 300, 128, 384
    g = gen(7)
    x = randn((m, d), g, torch.bfloat16, cuda)
    wide = randn((h, 2 * d + 8), g, torch.bfloat16, cuda, std=d ** -0.5)
    wg = wide[:, 8:8 + d]
    wu = randn((h, d), g, torch.bfloat16, cuda, std=d ** -0.5)
    dact = randn((m, h), g, torch.bfloat16, cuda)
    assert wg.stride(0) == 2 * d + 8 and wu.stride(0) == d
    act, (dx, dwg, dwu) = _run(x, wg, wu, dact)
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


def _wgrad(da, db, x, ldw=None):
    """Call nf_gemm_swiglu_wgrad on [M, H] views da, db and [M, D] view x."""
    from nuvla_forge_amd import _lib

    m, h = da.shape
    d = x.shape[1]
    ldw = ldw or d
    dwg_buf = torch.full((h, ldw), 7.0, dtype=torch.bfloat16, device=x.device)
    dwu_buf = torch.full_like(dwg_buf, 7.0)
    L = _lib.lib()
    nbytes = L.nf_gemm_swiglu_wgrad_workspace(m, d, h)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
    _lib.check(L.nf_gemm_swiglu_wgrad(da.data_ptr(), db.data_ptr(), da.stride(0), x.data_ptr(),
                                      x.stride(0), dwg_buf.data_ptr(), dwu_buf.data_ptr(), ldw,
                                      m, d, h, 1, ws.data_ptr(), nbytes, _lib.stream_of(x)),
               "nf_gemm_swiglu_wgrad")
    torch.cuda.synchronize()
    return dwg_buf, dwu_buf


# (M, D, H, row pad of da/db, row pad of x, row pad of dW): the headline DiT MLP
# (10 token slices), ragged H and D (the element-wise transpose), fewer tokens
# than one 8-token pad, and strided views with untouched pad columns.
@pytest.mark.parametrize("m,d,h,pab,px,pw", [
    (9408, 384, 1536, 0, 0, 0), (1000, 200, 333, 0, 0, 0), (5, 64, 96, 0, 0, 0),
    (777, 136, 264, 8, 16, 8), (3000, 1024, 2816, 0, 0, 0)])
def test_gate_up_wgrad_entry_matches_fp64(cuda, m, d, h, pab, px, pw):
    """dW_gate = da^T x, dW_up = db^T x from the same bf16 operands in fp64.
    The only rounding is fp32 accumulation and the final bf16 store, so the
    norm-wise error stays under 2^-8 (round-to-nearest bf16 is within 2^-9
    of each element); the gradients are bit-identical on a second call and
    the pad columns of dW keep their contents."""
    note(f"gate/up wgrad entry m={m} d={d} h={h} pads={pab},{px},{pw}")
    g = gen(11)
    dab = randn((m, h + pab), g, torch.bfloat16, cuda)
    dbb = randn((m, h + pab), g, torch.bfloat16, cuda)
    xb = randn((m, d + px), g, torch.bfloat16, cuda)
    da, db, x = dab[:, :h], dbb[:, :h], xb[:, :d]
    dwg, dwu = _wgrad(da, db, x, d + pw)
    ref_g, ref_u = np64(da).T @ np64(x), np64(db).T @ np64(x)
    assert on.rel_err(np64(dwg[:, :d]), ref_g) < 2.0 ** -8
    assert on.rel_err(np64(dwu[:, :d]), ref_u) < 2.0 ** -8
    if pw:
        assert bool((dwg[:, d:] == 7.0).all()) and bool((dwu[:, d:] == 7.0).all())
    dwg2, dwu2 = _wgrad(da, db, x, d + pw)
    assert torch.equal(dwg, dwg2) and torch.equal(dwu, dwu2)


def test_gate_up_wgrad_entry_without_tokens_zeroes(cuda):
    note("gate/up wgrad entry m=0")
    e = torch.empty((0, 64), dtype=torch.bfloat16, device=cuda)
    x = torch.empty((0, 32), dtype=torch.bfloat16, device=cuda)
    dwg, dwu = _wgrad(e, e, x, 40)
    assert bool((dwg[:, :32] == 0).all()) and bool((dwu[:, :32] == 0).all())
    assert bool((dwg[:, 32:] == 7.0).all())


def test_gate_up_fwd_bwd_replays_in_a_graph(cuda):
    """The encoder-MLP gate/up step (GEMM with the SwiGLU epilogue, SwiGLU
    backward, split-K weight gradients with their transposes and reduce, dx)
    captured in a HIP graph: every replay matches the eager step bit for bit."""
    from tests.helpers import assert_graph_replays_match

    note("gate/up graph replay m=9408 d=384 h=1536")
    x, wg, wu, dact = _inputs(9408, 384, 1536, torch.bfloat16, cuda, seed=12)

    def make():
        leaves = [t.detach().requires_grad_(True) for t in (x, wg, wu)]

        def step():
            act = fused_gate_up_swiglu(*leaves)
            return (act, *torch.autograd.grad(act, leaves, dact))

        return step

    assert_graph_replays_match(make)
