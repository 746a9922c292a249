"""Host-side dispatch checks, CPU only: the reference's environment switch and
the device check every fused op runs before any launch.

No GPU is needed: a ``meta`` tensor stands for the device tensor and a host
tensor for the caller's mistake, and the library entry point is replaced by
one that fails the test, so each check is shown to fire before anything could
reach a kernel.
"""

from __future__ import annotations

import os
import subprocess
import sys
import types
from pathlib import Path

import pytest
import torch

from nuvla_forge_amd import _lib
from nuvla_forge_amd.kernels import adaln_rmsnorm, chunked_ce, swiglu, utils

ROOT = Path(__file__).resolve().parents[1]


def _probe(env_value: str | None) -> list[str]:
    """HAS_TRITON, FUSED_DISABLED and use_fused on a stand-in device tensor,
    read in a fresh interpreter (the switch is read at import)."""
    env = dict(os.environ)
    env.pop("NUVLA_FORGE_DISABLE_TRITON", None)
    if env_value is not None:
        env["NUVLA_FORGE_DISABLE_TRITON"] = env_value
    code = (
        "import types, torch\n"
        "from nuvla_forge_amd import kernels\n"
        "from nuvla_forge_amd.kernels import utils\n"
        "fake = types.SimpleNamespace(is_cuda=True)\n"
        "torch.version.hip = torch.version.hip or 'stand-in'\n"
        "print(kernels.HAS_TRITON, utils.FUSED_DISABLED, utils.use_fused(fake, 'probe'))\n"
    )
    res = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True,
                         text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    return res.stdout.split()


def test_disable_switch_forces_the_eager_path():
    """NUVLA_FORGE_DISABLE_TRITON=1 at import (reference utils.py:16-20): the
    fused path reports unavailable and a device tensor takes the eager path;
    any other value, or none, leaves the fused path on."""
    assert _probe("1") == ["False", "True", "False"]
    assert _probe(None) == ["True", "False", "True"]
    assert _probe("0") == ["True", "False", "True"]


def test_disable_switch_in_process(monkeypatch):
    fake = types.SimpleNamespace(is_cuda=True)
    monkeypatch.setattr(utils, "FUSED_DISABLED", True)
    monkeypatch.setattr(_lib, "lib", _no_launch)
    assert not utils.use_fused(fake, "probe")


def _no_launch(*_a, **_k):
    raise AssertionError("the HIP library was reached before the device check")


def _meta(*shape, dtype=torch.bfloat16):
    return torch.empty(*shape, dtype=dtype, device="meta")


def _host(*shape, dtype=torch.bfloat16):
    return torch.zeros(*shape, dtype=dtype)


@pytest.fixture
def no_library(monkeypatch):
    monkeypatch.setattr(_lib, "lib", _no_launch)


@pytest.mark.parametrize("bad", ["y", "gate", "weight", "scale", "shift"])
def test_adaln_forward_device_check(no_library, bad):
    b, t, n = 2, 4, 64
    args = dict(x=_meta(b * t, n), y=_meta(b * t, n), gate=_meta(b, n), weight=_meta(n),
                scale=_meta(b, n), shift=_meta(b, n))
    args[bad] = _host(*args[bad].shape)
    with pytest.raises(utils.DeviceMismatchError, match=bad):
        adaln_rmsnorm._FusedAdaLNResidualRMSNorm.apply(*args.values(), t, 1e-6)


@pytest.mark.parametrize("bad", ["dh_up", "dout"])
def test_adaln_backward_device_check(no_library, bad):
    b, t, n = 2, 4, 64
    saved = (_meta(b * t, n), _meta(b * t, n), _meta(b, n), _meta(n), _meta(b, n),
             _meta(b * t, dtype=torch.float32))
    ctx = types.SimpleNamespace(saved_tensors=saved, tokens_per_sample=t,
                                needs_input_grad=(True,) * 8, shift_dtype=torch.bfloat16)
    grads = dict(dh_up=_meta(b * t, n), dout=_meta(b * t, n))
    grads[bad] = _host(b * t, n)
    with pytest.raises(utils.DeviceMismatchError, match=bad):
        adaln_rmsnorm._FusedAdaLNResidualRMSNorm.backward(ctx, *grads.values())


def test_swiglu_device_checks(no_library):
    with pytest.raises(utils.DeviceMismatchError, match="b is on cpu"):
        swiglu._FusedSwiGLU.apply(_meta(8, 16), _host(8, 16))
    ctx = types.SimpleNamespace(saved_tensors=(_meta(8, 16), _meta(8, 16)))
    with pytest.raises(utils.DeviceMismatchError, match="dout"):
        swiglu._FusedSwiGLU.backward(ctx, _host(8, 16))
    with pytest.raises(utils.DeviceMismatchError, match="w_up"):
        swiglu._FusedGateUpSwiGLU.apply(_meta(8, 16), _meta(32, 16), _host(32, 16))


@pytest.mark.parametrize("bad", ["lm_weight", "targets"])
def test_ce_forward_device_check(no_library, bad):
    """A host ``targets`` beside a device ``hidden`` is the likely mistake:
    the compaction kernel would read it through a host pointer."""
    args = dict(hidden=_meta(16, 8), lm_weight=_meta(50, 8),
                targets=_meta(16, dtype=torch.int64))
    args[bad] = _host(*args[bad].shape, dtype=args[bad].dtype)
    with pytest.raises(utils.DeviceMismatchError, match=bad):
        chunked_ce._ChunkedCrossEntropy.apply(*args.values(), 1024, -100, False)


def test_ce_backward_device_check(no_library):
    call = chunked_ce._DeviceCall(16, 8, 50, 1024, torch.bfloat16)
    with pytest.raises(utils.DeviceMismatchError, match="grad_output"):
        chunked_ce._backward_hip(call, _meta(64, dtype=torch.uint8), torch.ones(()),
                                 torch.bfloat16, torch.bfloat16, torch.device("meta"))


def test_error_is_value_and_runtime_error():
    """ValueError for a bad argument, RuntimeError as the reference's launch
    raises for the same call."""
    assert issubclass(utils.DeviceMismatchError, ValueError)
    assert issubclass(utils.DeviceMismatchError, RuntimeError)
