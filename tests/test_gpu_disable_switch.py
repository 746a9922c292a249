"""NUVLA_FORGE_DISABLE_TRITON=1 on the device (reference utils.py:16-20): with
the switch set at import, the three public ops on device tensors give exactly
what ``force_reference=True`` gives (the eager formulation on the device) and
never call the HIP library.  Run in a child interpreter, since the switch is
read when the package is imported; the child replaces the library entry with
one that fails if anything reaches it."""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

from tests.helpers import note

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]

CHILD = r"""
import torch
from nuvla_forge_amd import _lib
from nuvla_forge_amd import kernels as K
from nuvla_forge_amd.kernels import utils

assert utils.FUSED_DISABLED and not K.HAS_TRITON
def no_library(*a, **k):
    raise AssertionError("the HIP library was called with NUVLA_FORGE_DISABLE_TRITON=1")
_lib.lib = no_library

dev = torch.device("cuda", 0)
g = torch.Generator().manual_seed(5)
def r(*s, std=1.0, mean=0.0):
    return (torch.randn(*s, generator=g) * std + mean).to(torch.bfloat16).to(dev)

b, t, n = 2, 16, 128
args = (r(b * t, n), r(b * t, n), r(b, n, std=0.1), r(n, std=0.02, mean=1.0),
        r(b, n, std=0.1), r(b, n, std=0.1))
got = K.fused_adaln_residual_rmsnorm(*args, tokens_per_sample=t)
want = K.fused_adaln_residual_rmsnorm(*args, tokens_per_sample=t, force_reference=True)
assert all(torch.equal(x, y) for x, y in zip(got, want)), "adaLN"

a, bb = r(64, 256), r(64, 256)
assert torch.equal(K.fused_swiglu(a, bb), K.fused_swiglu(a, bb, force_reference=True)), "swiglu"

hid, w = r(96, 64), r(500, 64, std=0.05)
tgt = torch.randint(0, 500, (96,), generator=g)
tgt[::4] = -100
tgt = tgt.to(dev)
lg = K.chunked_cross_entropy(hid, w, tgt, chunk_size=32)
lr = K.chunked_cross_entropy(hid, w, tgt, chunk_size=32, force_reference=True)
assert torch.equal(lg, lr), "ce"
torch.cuda.synchronize()
print("eager path on the device, library untouched")
"""


def test_disable_switch_sends_device_tensors_to_the_eager_path(cuda):
    note("NUVLA_FORGE_DISABLE_TRITON=1 on device tensors (child interpreter)")
    env = dict(os.environ, NUVLA_FORGE_DISABLE_TRITON="1")
    res = subprocess.run([sys.executable, "-c", CHILD], cwd=ROOT, env=env, capture_output=True,
                         text=True, timeout=110)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "library untouched" in res.stdout
