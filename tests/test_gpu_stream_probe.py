"""nf_stream_probe, the streaming ceiling bench.py sets the row kernels
against (GPU): every output vector is the xor of the input vectors plus the
output's index in each 32-bit lane, for each supported (reads, writes) pair,
at a size that fits one pass of the grid and ones that need the grid-stride
loop (more vectors than 8192 blocks x 256 threads x 2), the largest with
4 x 96 MB of input, past the non-temporal-load threshold (320 MiB)."""

from __future__ import annotations

import pytest
import torch

from nuvla_forge_amd import _lib, _measure
from tests.helpers import note

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("reads,writes", [(1, 1), (2, 2), (4, 2)])
@pytest.mark.parametrize("n16", [1000, 4_500_001, 6_000_001])
def test_stream_probe_values(cuda, reads, writes, n16):
    note(f"stream probe reads={reads} writes={writes} n16={n16}")
    g = torch.Generator().manual_seed(reads * 10 + writes)
    ins = [torch.randint(-2**31, 2**31 - 1, (n16, 4), generator=g, dtype=torch.int64)
           .to(torch.int32).to(cuda) for _ in range(reads)]
    outs = [torch.full((n16, 4), -1, dtype=torch.int32, device=cuda) for _ in range(writes)]
    ptrs = [t.data_ptr() for t in ins] + [None] * (4 - reads)
    ptrs += [t.data_ptr() for t in outs] + [None] * (2 - writes)
    L = _measure.lib()
    _lib.check(L.nf_stream_probe(reads, writes, *ptrs, n16, _lib.stream_of(ins[0])),
               "nf_stream_probe")
    torch.cuda.synchronize()
    want = ins[0].clone()
    for t in ins[1:]:
        want ^= t
    for w, t in enumerate(outs):
        # unsigned 32-bit lanes: +w wraps modulo 2^32, as int32 addition does
        assert torch.equal(t, want + w), w


@pytest.mark.parametrize("n16", [1000, 4_500_001])
def test_stream_probe_read_only_pass(cuda, n16):
    """The (1, 0) form reads in0 and writes nothing for data without the
    marker value (its one possible store goes to out0[0] only)."""
    note(f"stream probe read-only n16={n16}")
    g = torch.Generator().manual_seed(7)
    src = torch.randint(-2**31, 2**31 - 1, (n16, 4), generator=g, dtype=torch.int64)
    src = src.to(torch.int32).to(cuda)
    sink = torch.full((2, 4), -1, dtype=torch.int32, device=cuda)
    L = _measure.lib()
    _lib.check(L.nf_stream_probe(1, 0, src.data_ptr(), None, None, None, sink.data_ptr(), None,
                                 n16, _lib.stream_of(src)), "nf_stream_probe")
    torch.cuda.synchronize()
    assert torch.all(sink == -1)
