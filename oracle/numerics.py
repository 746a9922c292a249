"""NumPy restatement of the fused ops' mathematics (test oracle; see __init__).

Every function works in the dtype of its inputs (fp64 for the parity checks;
callers upcast bf16/fp16 inputs first) and follows the reference file:line it
cites.  Nothing here imports torch or the product package.
"""

from __future__ import annotations

import numpy as np


def rel_err(got, want) -> float:
    """Norm-wise relative error max|got - want| / max|want| (the reference's
    tests/test_kernel_math.py:41-43 definition; 0/0 counts as 0)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    if got.shape != want.shape:
        raise ValueError(f"shape mismatch {got.shape} vs {want.shape}")
    if want.size == 0:
        return 0.0
    scale = float(np.abs(want).max())
    diff = float(np.abs(got - want).max())
    if scale == 0.0:
        return diff
    return diff / scale


def central_difference(array: np.ndarray, loss_fn, h: float = 1e-6) -> np.ndarray:
    """d loss / d array by symmetric differences, perturbing `array` in place."""
    grad = np.zeros_like(array)
    flat, gflat = array.reshape(-1), grad.reshape(-1)
    for i in range(flat.size):
        keep = flat[i]
        flat[i] = keep + h
        plus = loss_fn()
        flat[i] = keep - h
        minus = loss_fn()
        flat[i] = keep
        gflat[i] = (plus - minus) / (2.0 * h)
    return grad


# ---------------------------------------------------------------------------
# adaLN-Zero seam
# ---------------------------------------------------------------------------
def _per_row(c: np.ndarray, t: int) -> np.ndarray:
    """[B, N] conditioning -> [B*T, N] (row m is sample m // T); reference.py:17-19."""
    return np.repeat(c, t, axis=0)


def adaln_forward(x, y, gate, weight, scale, shift, t: int, eps: float = 1e-6):
    """h = x + gate*y; rstd = 1/sqrt(mean(h^2) + eps); out = h*rstd*w*(1+scale) + shift.

    reference.py:22-66 (eps inside the sqrt, mean over the true N) and the fused
    kernel adaln_rmsnorm.py:61-95 (rstd from the unrounded h).
    Returns (h, out, rstd[M]).
    """
    g = _per_row(gate, t)
    s = _per_row(scale, t)
    sh = _per_row(shift, t)
    h = x + g * y
    rstd = 1.0 / np.sqrt(np.mean(h * h, axis=1) + eps)
    out = (h * rstd[:, None]) * weight[None, :] * (1.0 + s) + sh
    return h, out, rstd


def adaln_backward(x, y, gate, weight, scale, shift, t: int, dh_up, dout, eps: float = 1e-6):
    """All six gradients of L = <h, dh_up> + <out, dout>.

    Same algebra as the fused backward (adaln_rmsnorm.py:135-162):
      xhat = h*rstd, dxhat = dout*w*(1+s), c = mean(dxhat*xhat)
      dh = dh_up + rstd*(dxhat - xhat*c);  dx = dh;  dy = dh*gate
      dgate = sum_t dh*y;  dscale = sum_t dout*xhat*w;  dshift = sum_t dout
      dweight = sum_m dout*xhat*(1+s)
    dh_up / dout may be None (zero).
    """
    m, n = x.shape
    b = m // t
    h, _, rstd = adaln_forward(x, y, gate, weight, scale, shift, t, eps)
    dh_up = np.zeros_like(x) if dh_up is None else dh_up
    dout = np.zeros_like(x) if dout is None else dout
    g = _per_row(gate, t)
    ops = 1.0 + _per_row(scale, t)
    xhat = h * rstd[:, None]
    dxhat = dout * weight[None, :] * ops
    c = np.mean(dxhat * xhat, axis=1)
    dh = dh_up + rstd[:, None] * (dxhat - xhat * c[:, None])

    def per_sample(rows):
        return rows.reshape(b, t, n).sum(axis=1)

    return {
        "x": dh,
        "y": dh * g,
        "gate": per_sample(dh * y),
        "weight": (dout * xhat * ops).sum(axis=0),
        "scale": per_sample(dout * xhat * weight[None, :]),
        "shift": per_sample(dout),
    }


# ---------------------------------------------------------------------------
# SwiGLU
# ---------------------------------------------------------------------------
def sigmoid(z):
    """1 / (1 + exp(-z)), evaluated without overflow for either sign."""
    z = np.asarray(z)
    e = np.exp(-np.abs(z))
    return np.where(z >= 0, 1.0 / (1.0 + e), e / (1.0 + e))


def swiglu_forward(a, b):
    """silu(a) * b = a * sigmoid(a) * b (reference.py:69-74, swiglu.py:35-46)."""
    return a * sigmoid(a) * b


def swiglu_backward(a, b, dout):
    """da = dout*b*s*(1 + a*(1 - s)), db = dout*a*s with s = sigmoid(a) (swiglu.py:48-63)."""
    s = sigmoid(a)
    return dout * b * (s * (1.0 + a * (1.0 - s))), dout * (a * s)


# ---------------------------------------------------------------------------
# cross entropy with the gradient formed in the forward pass
# ---------------------------------------------------------------------------
def ce_forward_backward(hidden, weight, targets, ignore_index: int = -100):
    """Mean CE over non-ignored rows of hidden @ weight.T, with dH and dW.

    reference.py:77-96 for the loss and chunked_ce.py:120-182 for the
    gradient-during-forward and the denominators: inv = 1/max(n_valid, 1), so
    an all-ignored batch gives loss 0 and zero gradients (chunked_ce.py:126-127).
    Returns (loss, dH[M, D], dW[V, D]).
    """
    targets = np.asarray(targets)
    m = hidden.shape[0]
    valid = targets != ignore_index
    inv = 1.0 / max(int(valid.sum()), 1)
    safe = np.where(valid, targets, 0)
    z = hidden @ weight.T
    zmax = z.max(axis=1, keepdims=True)
    p = np.exp(z - zmax)
    ssum = p.sum(axis=1, keepdims=True)
    lse = (zmax + np.log(ssum))[:, 0]
    loss = float(np.where(valid, lse - z[np.arange(m), safe], 0.0).sum() * inv)
    dz = p / ssum
    dz[np.arange(m), safe] -= 1.0
    dz *= valid[:, None] * inv
    return loss, dz @ weight, dz.T @ hidden
