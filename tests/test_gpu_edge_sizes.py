"""Degenerate sizes through the public ops on the device (GPU): empty
inputs, one-element rows, a one-word vocabulary, one-wide hidden states, and
an ignore_index other than -100 (inside the vocabulary, or -1); every result
checked against the oracle (or the closed form where the oracle's answer is
trivially 0)."""

from __future__ import annotations

import pytest
import torch

from nuvla_forge_amd.kernels import (chunked_cross_entropy, fused_adaln_residual_rmsnorm,
                                     fused_swiglu)
from oracle import numerics as on
from tests.helpers import gen, note, np64, randn

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,d,v", [(5, 1, 1), (1, 1, 2), (3, 8, 1), (7, 1, 50)])
def test_ce_tiny_vocabulary_and_width(cuda, m, d, v):
    note(f"ce edge m={m} d={d} v={v}")
    g = gen(m * 100 + d * 10 + v)
    hid = randn((m, d), g, torch.float32, cuda)
    w = randn((v, d), g, torch.float32, cuda)
    tgt = torch.randint(0, v, (m,), generator=g).to(cuda)
    lh, lw = hid.detach().requires_grad_(True), w.detach().requires_grad_(True)
    loss = chunked_cross_entropy(lh, lw, tgt, chunk_size=2)
    loss.backward()
    torch.cuda.synchronize()
    lo, dho, dwo = on.ce_forward_backward(np64(hid), np64(w), tgt.cpu().numpy())
    assert abs(float(loss) - lo) <= 1e-5 * max(1.0, abs(lo))
    assert on.rel_err(np64(lh.grad), dho) <= 1e-5
    assert on.rel_err(np64(lw.grad), dwo) <= 1e-5
    if v == 1:  # one class: probability 1, loss 0, no gradient
        assert float(loss) == 0.0 and not lh.grad.any() and not lw.grad.any()


def test_ce_no_rows(cuda):
    note("ce m=0")
    hid = torch.zeros(0, 16, device=cuda, requires_grad=True)
    w = torch.randn(10, 16, device=cuda, requires_grad=True)
    tgt = torch.zeros(0, dtype=torch.int64, device=cuda)
    loss = chunked_cross_entropy(hid, w, tgt)
    loss.backward()
    torch.cuda.synchronize()
    assert float(loss) == 0.0
    assert hid.grad.shape == (0, 16) and not w.grad.any()


@pytest.mark.parametrize("b,t,n", [(1, 1, 1), (3, 1, 1), (2, 5, 1), (1, 1, 7)])
def test_adaln_one_element_rows(cuda, b, t, n):
    note(f"adaln edge b={b} t={t} n={n}")
    g = gen(b * 100 + t * 10 + n)
    inp = {"x": randn((b * t, n), g, torch.float32, cuda), "y": randn((b * t, n), g, torch.float32, cuda),
           "gate": randn((b, n), g, torch.float32, cuda, std=0.1),
           "weight": randn((n,), g, torch.float32, cuda, std=0.02, mean=1.0),
           "scale": randn((b, n), g, torch.float32, cuda, std=0.1),
           "shift": randn((b, n), g, torch.float32, cuda, std=0.1)}
    dh, dout = randn((b * t, n), g, torch.float32, cuda), randn((b * t, n), g, torch.float32, cuda)
    leaves = {k: v.detach().requires_grad_(True) for k, v in inp.items()}
    h, out = fused_adaln_residual_rmsnorm(**leaves, tokens_per_sample=t)
    torch.autograd.backward([h, out], [dh, dout])
    torch.cuda.synchronize()
    a = {k: np64(v) for k, v in inp.items()}
    hw, ow, _ = on.adaln_forward(**a, t=t)
    gw = on.adaln_backward(**a, t=t, dh_up=np64(dh), dout=np64(dout))
    assert on.rel_err(np64(h), hw) <= 1e-5 and on.rel_err(np64(out), ow) <= 1e-5
    for k in inp:
        assert on.rel_err(np64(leaves[k].grad), gw[k]) <= 1e-5, k


def test_adaln_no_rows(cuda):
    note("adaln m=0")
    n = 64
    x = torch.zeros(0, n, device=cuda, requires_grad=True)
    y = torch.zeros(0, n, device=cuda, requires_grad=True)
    cond = [torch.zeros(0, n, device=cuda, requires_grad=True) for _ in range(3)]
    w = torch.ones(n, device=cuda, requires_grad=True)
    h, out = fused_adaln_residual_rmsnorm(x, y, cond[0], w, cond[1], cond[2], tokens_per_sample=4)
    assert h.shape == (0, n) and out.shape == (0, n)
    (h.sum() + out.sum()).backward()
    torch.cuda.synchronize()
    assert w.grad is not None and not w.grad.any()


@pytest.mark.parametrize("shape", [(0,), (0, 5), (1,), (3, 1)])
def test_swiglu_empty_and_single(cuda, shape):
    note(f"swiglu edge {shape}")
    g = gen(3)
    a, b, dout = (randn(shape, g, torch.float32, cuda) for _ in range(3))
    la, lb = a.detach().requires_grad_(True), b.detach().requires_grad_(True)
    out = fused_swiglu(la, lb)
    out.backward(dout)
    torch.cuda.synchronize()
    assert out.shape == a.shape
    if a.numel():
        A, B, G = np64(a), np64(b), np64(dout)
        da, db = on.swiglu_backward(A, B, G)
        assert on.rel_err(np64(out), on.swiglu_forward(A, B)) <= 1e-5
        assert on.rel_err(np64(la.grad), da) <= 1e-5 and on.rel_err(np64(lb.grad), db) <= 1e-5


@pytest.mark.parametrize("ignore_index", [3, -1, 0])
def test_ce_custom_ignore_index(cuda, ignore_index):
    """An ignore_index inside the vocabulary (3, 0) ignores the rows whose
    target is that class; -1 ignores rows marked -1; against the oracle with
    the same rows dropped."""
    note(f"ce ignore_index={ignore_index}")
    m, d, v = 64, 16, 10
    g = gen(40 + ignore_index)
    hid = randn((m, d), g, torch.float32, cuda)
    w = randn((v, d), g, torch.float32, cuda)
    tgt = torch.randint(0, v, (m,), generator=g)
    if ignore_index < 0:
        tgt[::5] = ignore_index
    tgt = tgt.to(cuda)
    lh, lw = hid.detach().requires_grad_(True), w.detach().requires_grad_(True)
    loss = chunked_cross_entropy(lh, lw, tgt, chunk_size=16, ignore_index=ignore_index)
    loss.backward()
    torch.cuda.synchronize()
    t = tgt.cpu().numpy().copy()
    dropped = t == ignore_index
    assert dropped.any()
    t[dropped] = -100  # the oracle's own ignore marker
    lo, dho, dwo = on.ce_forward_backward(np64(hid), np64(w), t)
    assert abs(float(loss) - lo) <= 1e-5 * max(1.0, abs(lo))
    assert on.rel_err(np64(lh.grad), dho) <= 1e-5 and on.rel_err(np64(lw.grad), dwo) <= 1e-5
    assert not lh.grad[torch.from_numpy(dropped).to(cuda)].any()
