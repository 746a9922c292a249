"""Pin the parity oracle (CPU only).

Each oracle function is checked against something that does not share its
code: fp64 central differences of the forward pass, torch fp64 autograd of the
independently written torch_cpu restatement, textbook library routines
(F.cross_entropy, F.silu), hand-computed known answers, invariants the
reference's own tests assert, and golden fixtures written by
tests/golden/make_golden.py.  Tolerances follow the reference's
tests/test_kernel_math.py (norm-wise relative error, RTOL 1e-6 for FD).
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import numerics as on
from oracle import torch_cpu as tc

FD_RTOL = 1e-6
GOLDEN = Path(__file__).parent / "golden" / "golden_small.npz"


def _adaln_args(rng, b, t, n):
    m = b * t
    return {
        "x": rng.standard_normal((m, n)), "y": rng.standard_normal((m, n)),
        "gate": rng.standard_normal((b, n)), "weight": rng.standard_normal(n),
        "scale": rng.standard_normal((b, n)), "shift": rng.standard_normal((b, n)),
    }


# ---------------------------------------------------------------------------
# adaLN
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("b,t,n", [(3, 5, 7), (2, 4, 16), (1, 8, 5)])
def test_adaln_backward_matches_central_differences(b, t, n):
    rng = np.random.default_rng(0)
    args = _adaln_args(rng, b, t, n)
    dh_up = rng.standard_normal((b * t, n))
    dout = rng.standard_normal((b * t, n))

    def loss():
        h, out, _ = on.adaln_forward(**args, t=t)
        return float((h * dh_up).sum() + (out * dout).sum())

    grads = on.adaln_backward(**args, t=t, dh_up=dh_up, dout=dout)
    for name, value in args.items():
        err = on.rel_err(grads[name], on.central_difference(value, loss))
        assert err < FD_RTOL, f"d{name}: {err:.2e}"


def test_adaln_backward_matches_torch_autograd_fp64():
    """cfg1 shape (B=2, T=64, N=256): analytic backward vs autograd of torch_cpu."""
    rng = np.random.default_rng(1)
    b, t, n = 2, 64, 256
    args = _adaln_args(rng, b, t, n)
    dh_up = rng.standard_normal((b * t, n))
    dout = rng.standard_normal((b * t, n))
    h, out, _ = on.adaln_forward(**args, t=t)
    grads = on.adaln_backward(**args, t=t, dh_up=dh_up, dout=dout)
    T = {k: torch.from_numpy(v) for k, v in args.items()}
    th, tout, tg = tc.adaln_fwd_bwd(**T, t=t, dh_up=torch.from_numpy(dh_up),
                                    dout=torch.from_numpy(dout))
    assert on.rel_err(h, th.numpy()) < 1e-14
    assert on.rel_err(out, tout.numpy()) < 1e-13
    for k in args:
        assert on.rel_err(grads[k], tg[k].numpy()) < 1e-12, k


def test_adaln_known_answer_hand_computed():
    """x = [[3, 4]], y = [[1, -2]], gate = 0.5 -> h = [3.5, 3]; mean(h^2) = 10.625."""
    x = np.array([[3.0, 4.0]])
    y = np.array([[1.0, -2.0]])
    gate = np.array([[0.5, 0.5]])
    w = np.array([2.0, 1.0])
    scale = np.array([[0.0, 1.0]])
    shift = np.array([[0.25, -1.0]])
    h, out, rstd = on.adaln_forward(x, y, gate, w, scale, shift, 1, eps=0.0)
    assert np.array_equal(h, [[3.5, 3.0]])
    r = 1.0 / math.sqrt(10.625)
    assert rstd[0] == pytest.approx(r, rel=1e-15)
    assert out[0, 0] == pytest.approx(3.5 * r * 2.0 * 1.0 + 0.25, rel=1e-15)
    assert out[0, 1] == pytest.approx(3.0 * r * 1.0 * 2.0 - 1.0, rel=1e-15)


def test_adaln_eps_known_answer_where_eps_matters():
    """mean(h^2) = 3e-6 next to eps = 1e-6: rstd = 1/sqrt(3e-6 + 1e-6) = 500
    exactly, so out = h * 500.  eps outside the root (1/(sqrt(3e-6) + 1e-6) =
    576.99...), eps dropped (577.35...), or a sum instead of the mean over N
    (1/sqrt(9e-6 + 1e-6) = 316.2...) all miss by more than 10%."""
    x = np.array([[1e-3, 2e-3, 2e-3]])
    zero = np.zeros((1, 3))
    h, out, rstd = on.adaln_forward(x, zero, zero, np.ones(3), zero, zero, 1, eps=1e-6)
    assert rstd[0] == pytest.approx(500.0, rel=1e-12)
    np.testing.assert_allclose(out, [[0.5, 1.0, 1.0]], rtol=1e-12)
    # the same through a second sample with gate and modulation in play:
    # h = 0.5 * y, w = 2, scale = 0.5, shift = 0.25
    y = np.array([[2e-3, 4e-3, 4e-3]])
    h2, out2, rstd2 = on.adaln_forward(zero, y, np.full((1, 3), 0.5), np.full(3, 2.0),
                                       np.full((1, 3), 0.5), np.full((1, 3), 0.25), 1, eps=1e-6)
    np.testing.assert_allclose(h2, x, rtol=1e-15)
    assert rstd2[0] == pytest.approx(500.0, rel=1e-12)
    np.testing.assert_allclose(out2, [[0.5 * 3 + 0.25, 1.0 * 3 + 0.25, 1.0 * 3 + 0.25]],
                               rtol=1e-12)
    for wrong in (1.0 / (math.sqrt(3e-6) + 1e-6), 1.0 / math.sqrt(3e-6),
                  1.0 / math.sqrt(9e-6 + 1e-6)):
        assert abs(wrong - rstd[0]) / rstd[0] > 0.1


def test_adaln_zero_gate_is_identity_on_residual():
    """adaLN-Zero init: gate = 0 gives h == x exactly (reference test_kernel_math.py:111-121)."""
    rng = np.random.default_rng(2)
    b, t, n = 2, 3, 8
    args = _adaln_args(rng, b, t, n)
    args["gate"] = np.zeros((b, n))
    h, _, _ = on.adaln_forward(**args, t=t)
    assert np.array_equal(h, args["x"])


def test_adaln_unit_modulation_normalises_rows():
    rng = np.random.default_rng(3)
    b, t, n = 2, 5, 64
    args = _adaln_args(rng, b, t, n)
    args.update(weight=np.ones(n), scale=np.zeros((b, n)), shift=np.zeros((b, n)))
    _, out, _ = on.adaln_forward(**args, t=t, eps=0.0)
    np.testing.assert_allclose(np.sqrt((out ** 2).mean(axis=1)), 1.0, rtol=1e-12)


def test_adaln_shift_is_additive_and_rows_are_independent():
    rng = np.random.default_rng(4)
    b, t, n = 2, 6, 16
    args = _adaln_args(rng, b, t, n)
    _, out0, _ = on.adaln_forward(**args, t=t)
    bump = rng.standard_normal((b, n))
    _, out1, _ = on.adaln_forward(**{**args, "shift": args["shift"] + bump}, t=t)
    np.testing.assert_allclose(out1 - out0, np.repeat(bump, t, axis=0), atol=1e-12)
    perm = np.concatenate([rng.permutation(t) + s * t for s in range(b)])
    _, out_p, _ = on.adaln_forward(**{**args, "x": args["x"][perm], "y": args["y"][perm]}, t=t)
    np.testing.assert_allclose(out_p, out0[perm], rtol=1e-13, atol=1e-13)


def test_adaln_backward_mistakes_are_caught():
    """A plausible slip (dropping the mean term of the RMSNorm backward) fails the FD check."""
    rng = np.random.default_rng(5)
    b, t, n = 1, 3, 6
    args = _adaln_args(rng, b, t, n)
    dout = rng.standard_normal((b * t, n))

    def loss():
        return float((on.adaln_forward(**args, t=t)[1] * dout).sum())

    h, _, rstd = on.adaln_forward(**args, t=t)
    wrong = rstd[:, None] * dout * args["weight"] * (1 + args["scale"])  # no mean term
    assert on.rel_err(wrong, on.central_difference(args["x"], loss)) > 1e-2


# ---------------------------------------------------------------------------
# SwiGLU
# ---------------------------------------------------------------------------
def test_swiglu_backward_matches_central_differences():
    rng = np.random.default_rng(6)
    a, b, dout = (rng.standard_normal((4, 5)) for _ in range(3))

    def loss():
        return float((on.swiglu_forward(a, b) * dout).sum())

    da, db = on.swiglu_backward(a, b, dout)
    assert on.rel_err(da, on.central_difference(a, loss)) < FD_RTOL
    assert on.rel_err(db, on.central_difference(b, loss)) < FD_RTOL


def test_swiglu_matches_torch_silu_autograd_fp64():
    rng = np.random.default_rng(7)
    a, b, dout = (rng.standard_normal((17, 333)) * 4 for _ in range(3))
    out, ta, tb = tc.swiglu_fwd_bwd(*(torch.from_numpy(v) for v in (a, b, dout)))
    da, db = on.swiglu_backward(a, b, dout)
    assert on.rel_err(on.swiglu_forward(a, b), out.numpy()) < 1e-14
    assert on.rel_err(da, ta.numpy()) < 1e-13
    assert on.rel_err(db, tb.numpy()) < 1e-13


def test_swiglu_known_values():
    a = np.array([0.0, 60.0, -60.0, 1.0])
    b = np.array([3.0, 2.0, 5.0, 1.0])
    out = on.swiglu_forward(a, b)
    assert out[0] == 0.0
    assert out[1] == pytest.approx(120.0, rel=1e-15)
    assert abs(out[2]) < 1e-20
    assert out[3] == pytest.approx(1.0 / (1.0 + math.exp(-1.0)), rel=1e-15)
    da, db = on.swiglu_backward(a, b, np.ones(4))
    assert da[0] == pytest.approx(3.0 * 0.5)  # silu'(0) = 1/2
    assert db[0] == 0.0


# ---------------------------------------------------------------------------
# cross entropy
# ---------------------------------------------------------------------------
def test_ce_gradients_match_central_differences():
    rng = np.random.default_rng(8)
    m, d, v = 9, 4, 6
    hidden = rng.standard_normal((m, d))
    weight = rng.standard_normal((v, d))
    targets = rng.integers(0, v, m)
    targets[::4] = -100

    def loss():
        return on.ce_forward_backward(hidden, weight, targets)[0]

    _, dh, dw = on.ce_forward_backward(hidden, weight, targets)
    assert on.rel_err(dh, on.central_difference(hidden, loss)) < FD_RTOL
    assert on.rel_err(dw, on.central_difference(weight, loss)) < FD_RTOL
    assert np.all(dh[::4] == 0.0), "ignored rows must carry zero gradient"


@pytest.mark.parametrize("ignore_every", [0, 3])
def test_ce_matches_torch_cross_entropy_fp64(ignore_every):
    g = torch.Generator().manual_seed(9)
    m, d, v = 64, 32, 200
    hid = torch.randn(m, d, generator=g, dtype=torch.float64)
    w = torch.randn(v, d, generator=g, dtype=torch.float64) * 0.5
    tgt = torch.randint(0, v, (m,), generator=g)
    if ignore_every:
        tgt[::ignore_every] = -100
    loss_t, dh_t, dw_t = tc.ce_autograd(hid, w, tgt)
    loss, dh, dw = on.ce_forward_backward(hid.numpy(), w.numpy(), tgt.numpy())
    assert loss == pytest.approx(float(loss_t), rel=1e-13)
    assert on.rel_err(dh, dh_t.numpy()) < 1e-12
    assert on.rel_err(dw, dw_t.numpy()) < 1e-12


def test_ce_brute_force_rows():
    """Per-row textbook loop: -log(softmax)[t], mean over valid rows."""
    rng = np.random.default_rng(10)
    m, d, v = 7, 3, 5
    hidden, weight = rng.standard_normal((m, d)), rng.standard_normal((v, d))
    targets = np.array([0, 4, -100, 2, 2, -100, 1])
    total, n = 0.0, 0
    for i in range(m):
        if targets[i] == -100:
            continue
        z = [sum(hidden[i, k] * weight[j, k] for k in range(d)) for j in range(v)]
        total += -math.log(math.exp(z[targets[i]]) / sum(math.exp(q) for q in z))
        n += 1
    loss, _, _ = on.ce_forward_backward(hidden, weight, targets)
    assert loss == pytest.approx(total / n, rel=1e-13)


def test_ce_all_ignored_is_zero():
    rng = np.random.default_rng(11)
    hidden, weight = rng.standard_normal((16, 8)), rng.standard_normal((50, 8))
    loss, dh, dw = on.ce_forward_backward(hidden, weight, np.full(16, -100))
    assert loss == 0.0 and not dh.any() and not dw.any()


def test_ce_mean_uses_valid_count():
    """Denominator = non-ignored tokens (reference test_kernel_math.py:188-206)."""
    rng = np.random.default_rng(12)
    hidden, weight = rng.standard_normal((8, 3)), rng.standard_normal((5, 3))
    targets = rng.integers(0, 5, 8)
    full, _, _ = on.ce_forward_backward(hidden[:4], weight, targets[:4])
    targets[4:] = -100
    half, _, _ = on.ce_forward_backward(hidden, weight, targets)
    assert half == pytest.approx(full, rel=1e-14)


def test_ce_large_logits_are_stable():
    hidden = np.array([[1000.0, 0.0], [-1000.0, 5.0]])
    weight = np.array([[1.0, 0.0], [0.0, 1.0], [0.5, 0.5]])
    loss, dh, dw = on.ce_forward_backward(hidden, weight, np.array([0, 1]))
    assert np.isfinite(loss) and np.isfinite(dh).all() and np.isfinite(dw).all()


@pytest.mark.parametrize("chunk", [128, 4096])
def test_torch_cpu_chunk_loop_matches_oracle(chunk):
    """The timed CPU baseline computes the same quantities (fp32 vs fp64 oracle)."""
    g = torch.Generator().manual_seed(13)
    m, d, v = 512, 64, 1000
    hid = torch.randn(m, d, generator=g)
    w = torch.randn(v, d, generator=g) * 0.02
    tgt = torch.randint(0, v, (m,), generator=g)
    tgt[::5] = -100
    loss, dh, dw = tc.chunked_ce_fwd_bwd(hid, w, tgt, chunk_size=chunk)
    lo, dho, dwo = on.ce_forward_backward(hid.double().numpy(), w.double().numpy(), tgt.numpy())
    assert float(loss) == pytest.approx(lo, rel=1e-5)
    assert on.rel_err(dh.numpy(), dho) < 1e-5
    assert on.rel_err(dw.numpy(), dwo) < 1e-5


# ---------------------------------------------------------------------------
# golden fixtures (tests/golden/make_golden.py, torch fp64 autograd)
# ---------------------------------------------------------------------------
def test_golden_fixtures():
    z = np.load(GOLDEN, allow_pickle=False)
    t = int(z["adaln_t"])
    args = {k: z["adaln_" + k] for k in ("x", "y", "gate", "weight", "scale", "shift")}
    h, out, _ = on.adaln_forward(**args, t=t, eps=float(z["adaln_eps"]))
    grads = on.adaln_backward(**args, t=t, dh_up=z["adaln_dh"], dout=z["adaln_dout"],
                              eps=float(z["adaln_eps"]))
    assert on.rel_err(h, z["adaln_h"]) < 1e-13
    assert on.rel_err(out, z["adaln_out"]) < 1e-13
    for k in args:
        assert on.rel_err(grads[k], z["adaln_d" + k]) < 1e-12, k

    out = on.swiglu_forward(z["swiglu_a"], z["swiglu_b"])
    da, db = on.swiglu_backward(z["swiglu_a"], z["swiglu_b"], z["swiglu_dout"])
    assert on.rel_err(out, z["swiglu_out"]) < 1e-14
    assert on.rel_err(da, z["swiglu_da"]) < 1e-13
    assert on.rel_err(db, z["swiglu_db"]) < 1e-13

    loss, dh, dw = on.ce_forward_backward(z["ce_hidden"], z["ce_weight"], z["ce_targets"])
    assert loss == pytest.approx(float(z["ce_loss"]), rel=1e-13)
    assert on.rel_err(dh, z["ce_dhidden"]) < 1e-12
    assert on.rel_err(dw, z["ce_dweight"]) < 1e-12
