"""The committed golden fixtures (tests/golden/golden_small.npz: torch fp64
autograd of the eager formulation) as seeded GPU parity cases: each fused op
runs the fixture's inputs in fp32 on the device and must reproduce its
outputs and gradients at the fp32 tolerance (1e-5 relative, norm-wise).

The fixtures' shapes are small and ragged (adaLN [3 x 5, 40]: rows not a
multiple of 8, the element-wise path; SwiGLU [7, 19]; CE M24 D16 V40 with
ignored rows), so they also cover the kernels' edge handling.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from nuvla_forge_amd.kernels import (chunked_cross_entropy, fused_adaln_residual_rmsnorm,
                                     fused_swiglu)
from oracle import numerics as on
from tests.helpers import TOL, note, np64

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).parent / "golden" / "golden_small.npz"
TOL32 = TOL[torch.float32]


@pytest.fixture(scope="module")
def fx():
    with np.load(GOLDEN, allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


def _dev(a, dev):
    return torch.tensor(a, dtype=torch.float32, device=dev).requires_grad_(True)


def test_golden_adaln(cuda, fx):
    note("golden adaln fp32 [15, 40] T=5")
    names = ["x", "y", "gate", "weight", "scale", "shift"]
    ins = [_dev(fx[f"adaln_{k}"], cuda) for k in names]
    t = int(fx["adaln_t"])
    h, out = fused_adaln_residual_rmsnorm(*ins, tokens_per_sample=t, eps=float(fx["adaln_eps"]))
    dh = torch.tensor(fx["adaln_dh"], dtype=torch.float32, device=cuda)
    dout = torch.tensor(fx["adaln_dout"], dtype=torch.float32, device=cuda)
    torch.autograd.backward([h, out], [dh, dout])
    torch.cuda.synchronize()
    errs = {"h": on.rel_err(np64(h), fx["adaln_h"]), "out": on.rel_err(np64(out), fx["adaln_out"])}
    for k, v in zip(names, ins):
        errs["d" + k] = on.rel_err(np64(v.grad), fx["adaln_d" + k])
    bad = {k: e for k, e in errs.items() if not e <= TOL32}
    assert not bad, bad


def test_golden_swiglu(cuda, fx):
    note("golden swiglu fp32 [7, 19]")
    a, b = _dev(fx["swiglu_a"], cuda), _dev(fx["swiglu_b"], cuda)
    out = fused_swiglu(a, b)
    out.backward(torch.tensor(fx["swiglu_dout"], dtype=torch.float32, device=cuda))
    torch.cuda.synchronize()
    assert on.rel_err(np64(out), fx["swiglu_out"]) <= TOL32
    assert on.rel_err(np64(a.grad), fx["swiglu_da"]) <= TOL32
    assert on.rel_err(np64(b.grad), fx["swiglu_db"]) <= TOL32


@pytest.mark.parametrize("chunk", [1024, 8])
def test_golden_ce(cuda, fx, chunk):
    note(f"golden ce fp32 M24 D16 V40 chunk={chunk}")
    hid, w = _dev(fx["ce_hidden"], cuda), _dev(fx["ce_weight"], cuda)
    tgt = torch.tensor(fx["ce_targets"], dtype=torch.int64, device=cuda)
    loss = chunked_cross_entropy(hid, w, tgt, chunk_size=chunk)
    loss.backward()
    torch.cuda.synchronize()
    lo = float(fx["ce_loss"])
    assert abs(float(loss.detach()) - lo) <= TOL32 * abs(lo)
    assert on.rel_err(np64(hid.grad), fx["ce_dhidden"]) <= TOL32
    assert on.rel_err(np64(w.grad), fx["ce_dweight"]) <= TOL32
