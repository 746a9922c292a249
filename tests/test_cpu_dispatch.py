"""The reference's CPU cases through the public functions (CPU only).

The reference dispatches host tensors to its eager PyTorch path
(adaln_rmsnorm.py:258-267, swiglu.py:104, chunked_ce.py:133), and its CPU CI
(.github/workflows/ci.yml:21-24) runs tests/test_kernels.py on exactly that
path.  These are those cases, called the way the reference's tests call them
-- no ``force_reference`` -- and checked against the fp64 oracle:
  * test_kernels.py:118-133  adaLN on [2, 4, 32] against a hand transcription;
  * test_kernels.py:182-201  CE M512 H64 V1000 at chunk 128 and 4096;
  * test_kernels.py:204-224  CE with every third target ignored;
  * test_kernels.py:227-237  CE with every target ignored;
plus SwiGLU on the reference's shapes, the gate/up projection, and adaLN rows
wider than the kernels' 16384 (the reference's eager fallback, :262).
"""

from __future__ import annotations

import pytest
import torch

from nuvla_forge_amd import kernels as K
from nuvla_forge_amd.kernels import reference
from oracle import numerics as on


def _np(t):
    return t.detach().double().numpy()


def _adaln_inputs(b, t, n, seed=0):
    g = torch.Generator().manual_seed(seed)
    m = b * t
    return {
        "x": torch.randn(m, n, generator=g), "y": torch.randn(m, n, generator=g),
        "gate": torch.randn(b, n, generator=g), "weight": torch.randn(n, generator=g),
        "scale": torch.randn(b, n, generator=g), "shift": torch.randn(b, n, generator=g),
    }


def test_adaln_on_host_tensors_matches_transcription_and_oracle():
    """test_kernels.py:118-133 through the public op (fp32, [2, 4, 32])."""
    b, t, n = 2, 4, 32
    inp = _adaln_inputs(b, t, n)
    leaves = {k: v.clone().requires_grad_(True) for k, v in inp.items()}
    h, out = K.fused_adaln_residual_rmsnorm(**leaves, tokens_per_sample=t)
    gate = inp["gate"].repeat_interleave(t, 0)
    manual_h = inp["x"] + gate * inp["y"]
    rms = manual_h.pow(2).mean(-1, keepdim=True).add(1e-6).rsqrt()
    manual_out = (manual_h * rms * inp["weight"] * (1 + inp["scale"].repeat_interleave(t, 0))
                  + inp["shift"].repeat_interleave(t, 0))
    torch.testing.assert_close(h, manual_h)
    torch.testing.assert_close(out, manual_out, atol=1e-5, rtol=1e-5)
    g = torch.Generator().manual_seed(1)
    dh, dout = torch.randn(b * t, n, generator=g), torch.randn(b * t, n, generator=g)
    torch.autograd.backward([h, out], [dh, dout])
    a = {k: _np(v) for k, v in inp.items()}
    hw, ow, _ = on.adaln_forward(**a, t=t)
    gw = on.adaln_backward(**a, t=t, dh_up=_np(dh), dout=_np(dout))
    assert on.rel_err(_np(h), hw) < 1e-6 and on.rel_err(_np(out), ow) < 1e-5
    for k, v in leaves.items():
        assert on.rel_err(_np(v.grad), gw[k]) < 1e-5, k


def test_adaln_wider_than_the_kernels_takes_the_eager_path():
    """N = 16385 > 16384: the reference's own fallback condition (:262)."""
    b, t, n = 1, 2, 16385
    inp = _adaln_inputs(b, t, n, seed=2)
    h, out = K.fused_adaln_residual_rmsnorm(**inp, tokens_per_sample=t)
    hw, ow, _ = on.adaln_forward(**{k: _np(v) for k, v in inp.items()}, t=t)
    assert on.rel_err(_np(h), hw) < 1e-6 and on.rel_err(_np(out), ow) < 1e-5


@pytest.mark.parametrize("shape", [(64, 512), (17, 333)])
def test_swiglu_on_host_tensors(shape):
    g = torch.Generator().manual_seed(0)
    a, b, dout = (torch.randn(*shape, generator=g) for _ in range(3))
    la, lb = a.clone().requires_grad_(True), b.clone().requires_grad_(True)
    out = K.fused_swiglu(la, lb)
    out.backward(dout)
    da, db = on.swiglu_backward(_np(a), _np(b), _np(dout))
    assert on.rel_err(_np(out), on.swiglu_forward(_np(a), _np(b))) < 1e-6
    assert on.rel_err(_np(la.grad), da) < 1e-5 and on.rel_err(_np(lb.grad), db) < 1e-5


def test_gate_up_swiglu_on_host_tensors():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(12, 16, generator=g)
    wg, wu = torch.randn(24, 16, generator=g), torch.randn(24, 16, generator=g)
    act = K.fused_gate_up_swiglu(x, wg, wu)
    want = on.swiglu_forward(_np(x) @ _np(wg).T, _np(x) @ _np(wu).T)
    assert on.rel_err(_np(act), want) < 1e-5


def _ce_case(m, h, v, seed):
    g = torch.Generator().manual_seed(seed)
    hid = torch.randn(m, h, generator=g)
    w = torch.randn(v, h, generator=g) * 0.02
    tgt = torch.randint(0, v, (m,), generator=g)
    return hid, w, tgt


def _ce_run(hid, w, tgt, chunk):
    lh, lw = hid.clone().requires_grad_(True), w.clone().requires_grad_(True)
    loss = K.chunked_cross_entropy(lh, lw, tgt, chunk_size=chunk)
    loss.backward()
    return loss, lh.grad, lw.grad


@pytest.mark.parametrize("chunk", [128, 4096])
def test_chunked_ce_on_host_tensors_matches_oracle(chunk):
    """test_kernels.py:182-201: M512 H64 V1000, 1e-4 against the unchunked loss."""
    hid, w, tgt = _ce_case(512, 64, 1000, 0)
    loss, dh, dw = _ce_run(hid, w, tgt, chunk)
    lo, dho, dwo = on.ce_forward_backward(_np(hid), _np(w), tgt.numpy())
    assert loss.dtype == torch.float32 and loss.dim() == 0
    assert float(loss.detach()) == pytest.approx(lo, rel=1e-5)
    assert on.rel_err(_np(dh), dho) < 1e-5 and on.rel_err(_np(dw), dwo) < 1e-5
    want = reference.chunked_cross_entropy_ref(hid, w, tgt)
    torch.testing.assert_close(loss, want, atol=1e-4, rtol=1e-4)


def test_chunked_ce_on_host_tensors_ignores_every_third_row():
    """test_kernels.py:204-224: ignored rows add no loss, no gradient, no count."""
    hid, w, tgt = _ce_case(64, 32, 200, 3)
    tgt[::3] = -100
    loss, dh, dw = _ce_run(hid, w, tgt, 16)
    lo, dho, dwo = on.ce_forward_backward(_np(hid), _np(w), tgt.numpy())
    assert float(loss.detach()) == pytest.approx(lo, rel=1e-5)
    assert on.rel_err(_np(dh), dho) < 1e-5 and on.rel_err(_np(dw), dwo) < 1e-5
    assert torch.all(dh[::3] == 0)


def test_chunked_ce_on_host_tensors_all_ignored():
    """test_kernels.py:227-237: a fully masked batch gives loss 0 and zero grads."""
    hid, w, _ = _ce_case(16, 8, 50, 4)
    tgt = torch.full((16,), -100, dtype=torch.long)
    loss, dh, dw = _ce_run(hid, w, tgt, 4)
    assert torch.isfinite(loss) and float(loss.detach()) == 0.0
    assert torch.all(dh == 0) and torch.all(dw == 0)
