"""Write tests/golden/golden_small.npz: small seeded inputs and their expected
outputs and gradients for the three ops, computed by torch fp64 autograd of
the reference's eager formulation (oracle/torch_cpu.py).  The fixtures pin the
NumPy oracle (tests/test_oracle.py::test_golden_fixtures) and double as
seeded GPU parity cases (tests/test_gpu_golden.py runs them through the
fused ops in fp32).

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import torch_cpu as tc  # noqa: E402

OUT = Path(__file__).with_name("golden_small.npz")


def main() -> None:
    g = torch.Generator().manual_seed(20260101)
    f64 = torch.float64
    rec: dict[str, np.ndarray] = {}

    # adaLN: B=3, T=5, N=40 (N not a power of two)
    b, t, n, eps = 3, 5, 40, 1e-6
    x = torch.randn(b * t, n, generator=g, dtype=f64)
    y = torch.randn(b * t, n, generator=g, dtype=f64)
    gate = torch.randn(b, n, generator=g, dtype=f64) * 0.1
    weight = 1 + torch.randn(n, generator=g, dtype=f64) * 0.02
    scale = torch.randn(b, n, generator=g, dtype=f64) * 0.1
    shift = torch.randn(b, n, generator=g, dtype=f64) * 0.1
    dh = torch.randn(b * t, n, generator=g, dtype=f64)
    dout = torch.randn(b * t, n, generator=g, dtype=f64)
    h, out, grads = tc.adaln_fwd_bwd(x, y, gate, weight, scale, shift, t, dh, dout, eps)
    for k, v in dict(x=x, y=y, gate=gate, weight=weight, scale=scale, shift=shift,
                     dh=dh, dout=dout, h=h, out=out).items():
        rec["adaln_" + k] = v.numpy()
    for k, v in grads.items():
        rec["adaln_d" + k] = v.numpy()
    rec["adaln_t"] = np.array(t)
    rec["adaln_eps"] = np.array(eps)

    # SwiGLU: 7 x 19 (odd sizes)
    a = torch.randn(7, 19, generator=g, dtype=f64) * 3
    bb = torch.randn(7, 19, generator=g, dtype=f64)
    d = torch.randn(7, 19, generator=g, dtype=f64)
    o, da, db = tc.swiglu_fwd_bwd(a, bb, d)
    rec.update(swiglu_a=a.numpy(), swiglu_b=bb.numpy(), swiglu_dout=d.numpy(),
               swiglu_out=o.numpy(), swiglu_da=da.numpy(), swiglu_db=db.numpy())

    # CE: M=24, D=16, V=40, every 5th row ignored
    m, dd, v = 24, 16, 40
    hid = torch.randn(m, dd, generator=g, dtype=f64)
    w = torch.randn(v, dd, generator=g, dtype=f64) * 0.3
    tgt = torch.randint(0, v, (m,), generator=g)
    tgt[::5] = -100
    loss, dhid, dw = tc.ce_autograd(hid, w, tgt)
    rec.update(ce_hidden=hid.numpy(), ce_weight=w.numpy(), ce_targets=tgt.numpy(),
               ce_loss=np.array(float(loss)), ce_dhidden=dhid.numpy(), ce_dweight=dw.numpy())

    np.savez_compressed(OUT, **rec)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, torch {torch.__version__})")


if __name__ == "__main__":
    main()
