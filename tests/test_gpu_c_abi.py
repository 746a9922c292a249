"""The C ABI from C (GPU): tests/c/abi_smoke, built by nuvla_forge_amd.build
with gcc against include/nuvla_forge_hip.h and libnf_hip.so, runs the SwiGLU
forward/backward and the adaLN forward on a stream of its own with no Python
or torch in the process, and checks them against host arithmetic in double
(1e-5 norm-wise, fp32)."""

from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

from tests.helpers import note

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent / "c" / "abi_smoke"


def test_c_program_drives_the_library():
    note("C ABI smoke program")
    assert EXE.exists(), f"{EXE} is not built; run `python -m nuvla_forge_amd.build`"
    res = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "c abi smoke OK" in res.stdout
