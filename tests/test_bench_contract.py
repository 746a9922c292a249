"""bench.py's contract checks that need no GPU.

* ``--gpus N`` with N > 1 exits with status 2 and says why (one-GPU build),
  before torch is imported;
* the algorithmic byte counts behind ``value`` and ``roofline.achieved``
  match the closed forms quoted for the BASELINE configs: adaLN fwd+bwd
  (10·M·N + 6·B·N + 2·N)·e = 1,325,056 B at cfg1 (fp32 [2, 64, 256]),
  167,874,560 B at cfg2 (bf16 [8, 1024, 1024]) and 2,685,149,184 B at the
  stress shape (bf16 [32, 2048, 2048]); SwiGLU fwd+bwd 8·M·H·e, and the
  cfg5 chain's 8,590,729,216 B.
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


@pytest.mark.parametrize("n", [2, 8])
def test_more_than_one_gpu_is_refused(n):
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", str(n)],
                         capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert res.returncode == 2
    assert "one GPU only" in res.stderr
    assert res.stdout == ""


def test_adaln_algorithmic_bytes_at_the_baseline_configs():
    assert bench.adaln_alg_bytes(2, 64, 256, e=4) == 1_325_056
    assert bench.adaln_alg_bytes(8, 1024, 1024) == 167_874_560
    assert bench.adaln_alg_bytes(32, 2048, 2048) == 2_685_149_184


def test_stress_chain_bytes():
    # the adaLN stress seam plus SwiGLU [65536, 5632] bf16 (8·M·H·e = 5,905,580,032 B)
    assert bench.adaln_alg_bytes(32, 2048, 2048) + 8 * 65536 * 5632 * 2 == 8_590_729_216
