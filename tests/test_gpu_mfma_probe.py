"""nf_mfma_probe, the MFMA ceiling bench.py sets the cross entropy's products
against (GPU): with every A operand a and every B operand b (bf16), each of a
thread's 256 accumulators receives iters products of 32-term dot products
(form 0, 16x16x32) or 2 * iters of 16-term ones (form 1, 32x32x16), so its
sum is 256 * 32 * iters * a * b either way, exact in fp32 at these sizes;
zero operands (a null `ops`) give 0; the stamps count forward.  Likewise
nf_mainloop_probe in each mode: with every operand c, each of a thread's 128
accumulators receives 2 * iters 32-term dot products, so its sum is
128 * 64 * iters * c * c."""

from __future__ import annotations

import pytest
import torch

from nuvla_forge_amd import _lib, _measure
from tests.helpers import note

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("form", [0, 1])
@pytest.mark.parametrize("a,b,iters,blocks", [(1.0, 1.0, 10, 3), (0.5, 0.25, 7, 300),
                                              (0.0, 3.0, 5, 1), (None, None, 4, 2)])
def test_mfma_probe_values(cuda, a, b, iters, blocks, form):
    note(f"mfma probe form={form} a={a} b={b} iters={iters} blocks={blocks}")
    L = _measure.lib()
    ops = None
    if a is not None:
        ops = torch.empty(16, 256, 8, dtype=torch.bfloat16, device=cuda)
        ops[0:4].fill_(a)
        ops[8:12].fill_(a)
        ops[4:8].fill_(b)
        ops[12:16].fill_(b)
    out = torch.full((blocks, 256), -1.0, device=cuda)
    stamps = torch.zeros(blocks, 4, dtype=torch.int64, device=cuda)
    _lib.check(L.nf_mfma_probe(None if ops is None else ops.data_ptr(), iters, blocks, form,
                               out.data_ptr(), stamps.data_ptr(), _lib.stream_of(out)),
               "nf_mfma_probe")
    torch.cuda.synchronize()
    want = 0.0 if a is None else 256 * 32 * iters * a * b
    assert torch.equal(out, torch.full_like(out, want))
    st = stamps.cpu()
    assert bool((st[:, 1] >= st[:, 0]).all()) and bool((st[:, 3] >= st[:, 2]).all())


@pytest.mark.parametrize("mode", [1, 2, 3, 4, 5])
def test_mainloop_probe_values(cuda, mode):
    iters, blocks, c = 5, 40, 0.5
    note(f"mainloop probe mode={mode} iters={iters} blocks={blocks}")
    L = _measure.lib()
    ops = torch.full((12, 512, 8), c, dtype=torch.bfloat16, device=cuda)
    src_bytes = 64 << 20
    src = torch.zeros(src_bytes // 2, dtype=torch.bfloat16, device=cuda)
    out = torch.full((blocks, 512), -1.0, device=cuda)
    stamps = torch.zeros(blocks, 4, dtype=torch.int64, device=cuda)
    _lib.check(L.nf_mainloop_probe(mode, ops.data_ptr(), src.data_ptr(), src_bytes, iters, blocks,
                                   out.data_ptr(), stamps.data_ptr(), _lib.stream_of(out)),
               "nf_mainloop_probe")
    torch.cuda.synchronize()
    assert torch.equal(out, torch.full_like(out, 128 * 64 * iters * c * c))
    st = stamps.cpu()
    assert bool((st[:, 1] >= st[:, 0]).all()) and bool((st[:, 3] >= st[:, 2]).all())
