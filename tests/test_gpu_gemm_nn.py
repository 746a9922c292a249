"""nf_gemm_nn (GPU): the MFMA core's N-major-B path (B [K, N] row-major, read
through transposing LDS reads) and its transposed store (C[n * ldc + m]),
which the cross entropy's dW product uses in bf16: against float64 products
at ragged sizes (K, N and M not multiples of the 256 x 256 tile or the
64-wide stage, columns between N and ldb present but excluded, M not a
multiple of 8 for the per-element transposed store, K and ldb not multiples
of 8 for the register-staged operand copies).  The hook's argument
checks run on the CPU (tests/test_abi.py)."""

from __future__ import annotations

import pytest
import torch

from nuvla_forge_amd import _lib, _measure
from oracle import numerics as on
from tests.helpers import gen, note, np64, randn

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,n,k,ldb", [(256, 256, 64, 256), (300, 1000, 264, 1008),
                                       (513, 777, 1000, 784), (264, 1000, 200, 1000),
                                       (2048, 300, 64, 304), (1, 8, 8, 8), (40, 16, 2000, 24),
                                       (2048, 4000, 1024, 4000),
                                       # K and ldb not multiples of 8: operands through registers
                                       (100, 200, 37, 203), (300, 257, 300, 261)])
@pytest.mark.parametrize("ct", [0, 1])
def test_gemm_nn_matches_numpy(cuda, m, n, k, ldb, ct):
    note(f"gemm_nn m={m} n={n} k={k} ldb={ldb} ct={ct}")
    g = gen(m + n + k)
    a = randn((m, k), g, torch.bfloat16, cuda)
    b = randn((k, ldb), g, torch.bfloat16, cuda)
    c = torch.full((n, m) if ct else (m, n), float("nan"), device=cuda)
    L = _measure.lib()
    _lib.check(L.nf_gemm_nn(a.data_ptr(), k, b.data_ptr(), ldb, c.data_ptr(), c.stride(0), m, n,
                            k, ct, _lib.stream_of(a)), "nf_gemm_nn")
    torch.cuda.synchronize()
    want = np64(a) @ np64(b)[:, :n]
    got = np64(c).T if ct else np64(c)
    assert on.rel_err(got, want) < 1e-5

