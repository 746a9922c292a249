"""Chunked cross entropy and its MFMA GEMM core vs the oracle (GPU).

nf_gemm_nt is driven directly through the C ABI at ragged sizes first: it
checks the MFMA operand/accumulator lane layouts the cross entropy relies on.
Then the op through the autograd Function: the reference's test cases
(tests/test_kernels.py:182-237: M512 H64 V1000 at chunk 128/4096, every 3rd
row ignored, all rows ignored), ragged shapes (non-multiple-of-8 D and V),
bad targets, grad_output scaling, and BASELINE cfg4 (bf16 M4096 D2048 V32000,
10% ignored) against an fp32 host oracle, with a bit-identical rerun; and the
reference's peak-memory test (fused below the eager reference).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from nuvla_forge_amd import _lib, _measure
from nuvla_forge_amd.kernels import chunked_cross_entropy
from oracle import numerics as on
from tests.helpers import TOL, gen, note, np64, randn

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("m,n,k", [(128, 128, 64), (32, 32, 16), (200, 130, 72), (1, 1, 8),
                                   (257, 383, 1000), (64, 96, 36), (96, 64, 1), (512, 256, 2048)])
def test_gemm_nt_matches_numpy(cuda, dtype, m, n, k):
    note(f"gemm_nt dtype={dtype} m={m} n={n} k={k}")
    g = gen(0)
    a = randn((m, k), g, dtype, cuda)
    b = randn((n, k), g, dtype, cuda)
    c = torch.full((m, n), float("nan"), device=cuda)
    L = _measure.lib()
    _lib.check(L.nf_gemm_nt(a.data_ptr(), k, b.data_ptr(), k, c.data_ptr(), n, m, n, k,
                            _lib.dtype_code(dtype), _lib.stream_of(a)), "nf_gemm_nt")
    torch.cuda.synchronize()
    want = np64(a) @ np64(b).T
    assert on.rel_err(np64(c), want) < 1e-5


@pytest.mark.parametrize("m,n,k", [(256, 256, 128), (300, 520, 200), (1024, 768, 2048),
                                   (33, 17, 64), (512, 256, 72)])
def test_gemm_nt_accumulates_onto_c(cuda, m, n, k):
    """nf_gemm_nt_acc: C += A B^T with the accumulator preloaded from C (row
    stride n + 3), so a non-zero accumulator goes through the 16x16x32
    mainloop's layout change on the way in and back on the way out; the
    columns past n stay untouched."""
    note(f"gemm_nt_acc m={m} n={n} k={k}")
    g = gen(7)
    a = randn((m, k), g, torch.bfloat16, cuda)
    b = randn((n, k), g, torch.bfloat16, cuda)
    c0 = randn((m, n + 3), g, torch.float32, cuda)
    c = c0.clone()
    L = _measure.lib()
    _lib.check(L.nf_gemm_nt_acc(a.data_ptr(), k, b.data_ptr(), k, c.data_ptr(), n + 3, m, n, k,
                                _lib.stream_of(a)), "nf_gemm_nt_acc")
    torch.cuda.synchronize()
    want = np64(c0[:, :n]) + np64(a) @ np64(b).T
    assert on.rel_err(np64(c[:, :n]), want) < 1e-5
    assert torch.equal(c[:, n:], c0[:, n:])


def test_gemm_nt_leading_dimensions(cuda):
    note("gemm_nt strided operands")
    g = gen(1)
    base_a = randn((100, 96), g, torch.bfloat16, cuda)
    base_b = randn((70, 80), g, torch.bfloat16, cuda)
    c = torch.zeros(100, 90, device=cuda)
    L = _measure.lib()
    # A = base_a[:, 8:72] (lda 96), B = base_b[:, 16:80] (ldb 80), C = c[:, :70] (ldc 90)
    _lib.check(L.nf_gemm_nt(base_a[:, 8:].data_ptr(), 96, base_b[:, 16:].data_ptr(), 80,
                            c.data_ptr(), 90, 100, 70, 64, 1, _lib.stream_of(c)), "nf_gemm_nt")
    torch.cuda.synchronize()
    want = np64(base_a[:, 8:72]) @ np64(base_b[:, 16:80]).T
    assert on.rel_err(np64(c[:, :70]), want) < 1e-5
    assert not c[:, 70:].any()


def test_gemm_nt_output_over_2gib(cuda):
    """An fp32 C of 2.15 GB is past the 32-bit offsets of a buffer resource:
    the store epilogue takes its plain-store path (ragged last column tile);
    checked against torch's fp32 product on the device."""
    note("gemm_nt C > 2 GiB m=16384 n=32800 k=64")
    m, n, k = 16384, 32800, 64
    g = gen(5)
    a = randn((m, k), g, torch.bfloat16, cuda)
    b = randn((n, k), g, torch.bfloat16, cuda)
    c = torch.full((m, n), float("nan"), device=cuda)
    assert c.numel() * 4 >= 2 ** 31
    L = _measure.lib()
    _lib.check(L.nf_gemm_nt(a.data_ptr(), k, b.data_ptr(), k, c.data_ptr(), n, m, n, k,
                            _lib.dtype_code(torch.bfloat16), _lib.stream_of(a)), "nf_gemm_nt")
    want = a.float() @ b.float().T
    torch.cuda.synchronize()
    err = float((c - want).abs().max() / want.abs().max())
    del want, c
    assert err < 1e-5, err


def _ce_inputs(m, d, v, dtype, dev, seed=0, w_std=0.02, ignore=None):
    g = gen(seed)
    hid = randn((m, d), g, dtype, dev)
    w = randn((v, d), g, dtype, dev, std=w_std)
    tgt = torch.randint(0, v, (m,), generator=g)
    if ignore is not None:
        tgt[ignore] = -100
    return hid, w, tgt.to(dev)


def _run_ce(hid, w, tgt, chunk, scale=1.0):
    h = hid.detach().requires_grad_(True)
    ww = w.detach().requires_grad_(True)
    loss = chunked_cross_entropy(h, ww, tgt, chunk_size=chunk)
    (loss * scale).backward()
    torch.cuda.synchronize()
    return loss.detach(), h.grad, ww.grad


def _check_ce(hid, w, tgt, loss, dh, dw, tol, label, scale=1.0):
    lo, dho, dwo = on.ce_forward_backward(np64(hid), np64(w), tgt.cpu().numpy())
    errs = {"loss": abs(float(loss) - lo) / max(abs(lo), 1e-30) if lo else abs(float(loss)),
            "dh": on.rel_err(np64(dh), scale * dho), "dw": on.rel_err(np64(dw), scale * dwo)}
    bad = {k: v for k, v in errs.items() if not v <= tol}
    assert not bad, f"{label}: {bad}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("chunk", [128, 4096])
def test_ce_reference_case(cuda, dtype, chunk):
    """m, h, v = 512, 64, 1000 (reference tests/test_kernels.py:182-201)."""
    note(f"ce ref case dtype={dtype} chunk={chunk}")
    hid, w, tgt = _ce_inputs(512, 64, 1000, dtype, cuda)
    loss, dh, dw = _run_ce(hid, w, tgt, chunk)
    assert dh.dtype == dtype and dw.dtype == dtype and loss.dtype == torch.float32
    _check_ce(hid, w, tgt, loss, dh, dw, TOL[dtype], f"{dtype} chunk {chunk}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_ce_respects_ignore_index(cuda, dtype):
    note(f"ce ignore_index dtype={dtype}")
    hid, w, tgt = _ce_inputs(64, 32, 200, dtype, cuda, seed=3, ignore=slice(None, None, 3))
    loss, dh, dw = _run_ce(hid, w, tgt, 16)
    _check_ce(hid, w, tgt, loss, dh, dw, TOL[dtype], "ignore")
    assert torch.all(dh[::3] == 0)


def test_ce_all_ignored_is_zero(cuda):
    note("ce all ignored")
    hid, w, _ = _ce_inputs(16, 8, 50, torch.float32, cuda)
    tgt = torch.full((16,), -100, device=cuda)
    loss, dh, dw = _run_ce(hid, w, tgt, 4)
    assert float(loss) == 0.0
    assert not dh.any() and not dw.any()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("chunk", [64, 4096])
def test_ce_rows_far_from_their_reference(cuda, dtype, chunk):
    """Logits of standard deviation ~32 in every other row (hidden rows
    N(0, 1) x 4, weights N(0, 1)), so that in about half of the rows the loss
    plus ln n exceeds 65 nats: E is stored relative to the target logit and
    scaled by a per-row factor exp(mref - lse) / n, and those rows would
    leave the exponent range, so the logits pass keeps their far tiles
    relative to the tile maximum and the statistics pass rescales the row to
    its maximum; the others (loss + ln n under 55) keep the fast path.
    Against the fp64
    oracle on the same rounded inputs.  Tolerances: bf16 2e-2; fp32 1e-4,
    because an fp32 logit of magnitude ~100 carries an absolute rounding
    error of ~1e-5, which exp turns into a relative error of the same size in
    every probability (the fp64 oracle has none)."""
    note(f"ce far-from-reference rows dtype={dtype} chunk={chunk}")
    m, d, v = 300, 64, 1000
    g = gen(21)
    hid = randn((m, d), g, torch.float32, "cpu")
    hid[::2] *= 4.0
    w = randn((v, d), g, torch.float32, "cpu")
    tgt = torch.randint(0, v, (m,), generator=g)
    tgt[::7] = -100
    hid, w, tgt = hid.to(dtype).to(cuda), w.to(dtype).to(cuda), tgt.to(cuda)
    logits = np64(hid) @ np64(w).T
    valid = (tgt != -100).cpu().numpy()
    tcol = np.where(valid, tgt.cpu().numpy(), 0)
    mx = logits.max(axis=1)
    lse = mx + np.log(np.exp(logits - mx[:, None]).sum(axis=1))
    crit = (lse - logits[np.arange(m), tcol] + np.log(valid.sum()))[valid]
    assert (crit > 65).sum() >= 0.3 * valid.sum()  # the rescale is exercised
    assert (crit < 55).sum() >= 0.3 * valid.sum()  # and so is the fast path
    loss, dh, dw = _run_ce(hid, w, tgt, chunk)
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-4
    _check_ce(hid, w, tgt, loss, dh, dw, tol, f"far rows {dtype} chunk {chunk}")


@pytest.mark.parametrize("chunk", [1024, 4096])
def test_ce_tiny_row_factor_keeps_its_weight_gradient(cuda, chunk):
    """bf16, n = 4096 valid rows, and 32 rows whose largest logit lies only
    74.5 above the target's but whose loss is ~82.8 nats (4080 logits share
    that maximum).  On the fast path such a row's factor exp(mref - lse) / n
    is ~3e-40, below bf16's normal range, and its share of the dW operand
    (factor x hidden row, rounded to bf16) would vanish while its dH stayed
    right; the criterion (loss + ln n above 60 nats: rescale the row to its
    maximum) keeps it.
    The 32 rows are the only ones with a nonzero hidden column 0, so dW[:, 0]
    is their contribution alone, checked on its own besides dH row by row."""
    note(f"ce tiny row factor bf16 m=4096 d=64 v=4096 chunk={chunk}")
    m, d, v, nspec, nlow = 4096, 64, 4096, 32, 16
    g = gen(41)
    hid = torch.randn(m, d, generator=g)
    hid[:, 0] = 0.0
    spec = torch.randperm(m, generator=g)[:nspec]
    hid[spec] = 0.0
    hid[spec, 0] = 1.0
    w = torch.randn(v, d, generator=g) * 0.05
    w[:, 0] = 74.5  # bf16-exact
    low = torch.randperm(v, generator=g)[:nlow]
    w[low, 0] = 0.0
    tgt = torch.randint(0, v, (m,), generator=g)
    tgt[spec] = low[torch.randint(0, nlow, (nspec,), generator=g)]
    hid, w = hid.to(torch.bfloat16).to(cuda), w.to(torch.bfloat16).to(cuda)
    tgt = tgt.to(cuda)
    loss, dh, dw = _run_ce(hid, w, tgt, chunk)
    lo, dho, dwo = on.ce_forward_backward(np64(hid), np64(w), tgt.cpu().numpy())
    rows = spec.numpy()
    logits = np64(hid)[rows] @ np64(w).T
    row_loss = np.log(np.exp(logits - logits.max(1, keepdims=True)).sum(1)) + logits.max(1)
    assert np.all(row_loss > 82) and np.all(row_loss < 84)  # fast path before the criterion
    assert abs(float(loss) - lo) / lo < 2e-2
    assert on.rel_err(np64(dw)[:, 0], dwo[:, 0]) < 2e-2, "the 32 rows' dW share"
    for r in rows:
        assert on.rel_err(np64(dh)[r], dho[r]) < 2e-2, f"dH row {r}"
    assert on.rel_err(np64(dh), dho) < 2e-2 and on.rel_err(np64(dw), dwo) < 2e-2


@pytest.mark.parametrize("dtype,m,d,v,chunk", [
    (torch.bfloat16, 512, 384, 32000, 1024),   # the reasoning head's shape, E held once
    (torch.float32, 512, 384, 32000, 1024),
    (torch.bfloat16, 512, 2048, 4096, 4096),   # E in both layouts
    (torch.bfloat16, 1000, 384, 5000, 64),     # chunks of 256 rows with the dW accumulator
])
def test_ce_every_row_far_from_its_reference(cuda, dtype, m, d, v, chunk):
    """Hidden and weights both N(0, 1): logits of standard deviation ~sqrt(D)
    (20-45), so nearly every row's maximum lies far above its target logit
    and most wavefront tiles store E relative to their own maximum; every
    such row is rescaled to its maximum by the statistics pass.  Against the
    fp64 oracle (tolerances as in the far-rows test), and the call stays
    within a few milliseconds (rows like these were once recomputed one at a
    time with scalar dot products, ~0.2 s for the first case)."""
    note(f"ce every row far dtype={dtype} m={m} d={d} v={v} chunk={chunk}")
    g = gen(57)
    hid = randn((m, d), g, torch.float32, "cpu")
    w = randn((v, d), g, torch.float32, "cpu")
    tgt = torch.randint(0, v, (m,), generator=g)
    tgt[::11] = -100
    hid, w, tgt = hid.to(dtype).to(cuda), w.to(dtype).to(cuda), tgt.to(cuda)
    logits = np64(hid) @ np64(w).T
    valid = (tgt != -100).cpu().numpy()
    tcol = np.where(valid, tgt.cpu().numpy(), 0)
    gap = (logits.max(axis=1) - logits[np.arange(m), tcol])[valid]
    assert (gap > 60).mean() > 0.5  # tiles far above the target logit in most rows
    _run_ce(hid, w, tgt, chunk)  # warm
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    loss, dh, dw = _run_ce(hid, w, tgt, chunk)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end)
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-4
    _check_ce(hid, w, tgt, loss, dh, dw, tol, f"every row far {dtype} m={m} d={d} v={v}")
    assert ms < 50.0, f"{ms:.1f} ms for one forward + backward"


@pytest.mark.parametrize("dtype,chunk,d", [(torch.bfloat16, 128, 64), (torch.bfloat16, 4096, 256),
                                           (torch.float32, 128, 256)])
def test_ce_large_vocabulary(cuda, dtype, chunk, d):
    """A Llama-3-sized vocabulary (V = 128256: 1002 statistics tiles per row,
    several load rounds in the lse pass, 501 vocabulary tiles per logits
    launch) with several row chunks and with one, against the oracle.  bf16
    at chunk_size 128 takes two chunks at D = 64 (at D = 256 E for all 300
    rows fits the bytes of the reference's tile and accumulator: one)."""
    m, v = 300, 128256
    note(f"ce large vocabulary dtype={dtype} m={m} d={d} v={v} chunk={chunk}")
    hid, w, tgt = _ce_inputs(m, d, v, dtype, cuda, seed=9, w_std=0.05,
                             ignore=slice(None, None, 7))
    loss, dh, dw = _run_ce(hid, w, tgt, chunk)
    _check_ce(hid, w, tgt, loss, dh, dw, TOL[dtype], f"large vocab {dtype} chunk {chunk}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("m,d,v,chunk", [(17, 36, 333, 7), (300, 40, 1030, 1000), (9, 4, 6, 1),
                                         (130, 264, 129, 64),
                                         # bf16 holds E once here (chunks of 256 / 512 rows):
                                         # the dW product reads it N-major; D = 36 stores dW
                                         # transposed element by element, D = 72 through LDS
                                         (600, 36, 333, 100), (1100, 72, 1000, 200),
                                         # bf16 holds E in both layouts here (D >= 2048, one
                                         # chunk); D = 2050 takes the unaligned loads
                                         (300, 2048, 1030, 1000), (150, 2050, 500, 64)])
def test_ce_ragged_shapes(cuda, dtype, m, d, v, chunk):
    note(f"ce ragged dtype={dtype} m={m} d={d} v={v} chunk={chunk}")
    # logits of standard deviation ~2-4 at every width (0.3 at D = 2048 would
    # give ~14, rows whose fp32 exp rounding alone exceeds the 1e-5 tolerance)
    hid, w, tgt = _ce_inputs(m, d, v, dtype, cuda, seed=4, w_std=0.3 if d < 1024 else 0.05,
                             ignore=slice(None, None, 4))
    loss, dh, dw = _run_ce(hid, w, tgt, chunk)
    _check_ce(hid, w, tgt, loss, dh, dw, TOL[dtype], f"ragged {m},{d},{v}")


def test_ce_wide_rows_in_many_chunks(cuda):
    """bf16 at D = 2048 with chunk_size 256 over 8192 rows: the budget
    2 (256 + 2048) rows of E is under M, so the rows go in 16 chunks of 512
    held once, the fp32 dW^T accumulator carried through 15 of them (every
    other chunk-size test with several chunks has D <= 256); against the
    fp64 oracle."""
    note("ce wide rows many chunks bf16 m=8192 d=2048 v=1000 chunk=256")
    m, d, v = 8192, 2048, 1000
    hid, w, tgt = _ce_inputs(m, d, v, torch.bfloat16, cuda, seed=17, w_std=0.02,
                             ignore=slice(None, None, 9))
    loss, dh, dw = _run_ce(hid, w, tgt, 256)
    _check_ce(hid, w, tgt, loss, dh, dw, TOL[torch.bfloat16], "wide rows, 16 chunks")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("chunk_rows", [256, 100000])
def test_ce_one_call_entry_point(cuda, dtype, chunk_rows):
    """nf_ce_fwd_bwd (the reference's structure: loss and unscaled fp32
    gradients in one call) through the C ABI: parity with the oracle, and
    bit-identical to the two-call path asked for fp32 gradients with
    grad_output 1 (the same kernels in the same order); with 256-row chunks
    (the 500 valid rows of 600, every 6th ignored, in two chunks: the first
    chunk's products in the forward, the second's in the backward) and with
    one chunk holding every row."""
    note(f"ce one-call entry point dtype={dtype} chunk_rows={chunk_rows}")
    m, d, v = 600, 72, 1030
    hid, w, tgt = _ce_inputs(m, d, v, dtype, cuda, seed=11, w_std=0.2,
                             ignore=slice(None, None, 6))
    L = _lib.lib()
    code, s = _lib.dtype_code(dtype), _lib.stream_of(hid)
    loss = torch.empty((), device=cuda)
    dh = torch.empty(m, d, device=cuda)
    dw = torch.empty(v, d, device=cuda)
    bad = torch.empty(1, dtype=torch.int32, device=cuda)
    nb = L.nf_ce_workspace(m, d, v, chunk_rows, code)
    ws = torch.empty(nb, dtype=torch.uint8, device=cuda)
    _lib.check(L.nf_ce_fwd_bwd(hid.data_ptr(), w.data_ptr(), tgt.data_ptr(), m, d, v, -100,
                               chunk_rows, code, loss.data_ptr(), dh.data_ptr(), dw.data_ptr(),
                               bad.data_ptr(), ws.data_ptr(), nb, s), "nf_ce_fwd_bwd")
    torch.cuda.synchronize()
    assert int(bad.item()) == 0
    _check_ce(hid, w, tgt, loss, dh, dw, TOL[dtype], f"one call {dtype}")
    # the same through nf_ce_fwd + nf_ce_bwd
    shape = (m, d, v, chunk_rows, code)
    sb = L.nf_ce_state_bytes(*shape)
    state = torch.empty(sb, dtype=torch.uint8, device=cuda)
    fw, bw = L.nf_ce_fwd_workspace(*shape), L.nf_ce_bwd_workspace(*shape)
    ws1 = torch.empty(fw, dtype=torch.uint8, device=cuda)
    ws2 = torch.empty(bw, dtype=torch.uint8, device=cuda)
    loss2, dh2, dw2 = torch.empty_like(loss), torch.empty_like(dh), torch.empty_like(dw)
    one = torch.ones((), device=cuda)
    _lib.check(L.nf_ce_fwd(hid.data_ptr(), w.data_ptr(), tgt.data_ptr(), m, d, v, -100,
                           chunk_rows, code, loss2.data_ptr(), None, state.data_ptr(), sb,
                           ws1.data_ptr(), fw, s), "nf_ce_fwd")
    f32 = _lib.dtype_code(torch.float32)
    _lib.check(L.nf_ce_bwd(m, d, v, chunk_rows, code, state.data_ptr(), sb, one.data_ptr(),
                           dh2.data_ptr(), f32, dw2.data_ptr(), f32, ws2.data_ptr(), bw, s),
               "nf_ce_bwd")
    torch.cuda.synchronize()
    assert torch.equal(loss, loss2) and torch.equal(dh, dh2) and torch.equal(dw, dw2)


def test_ce_grad_output_scaling(cuda):
    note("ce grad scaling")
    hid, w, tgt = _ce_inputs(128, 64, 500, torch.float32, cuda, seed=5)
    loss, dh, dw = _run_ce(hid, w, tgt, 64, scale=3.0)
    _check_ce(hid, w, tgt, loss, dh, dw, 1e-5, "scaled", scale=3.0)


def test_ce_out_of_range_targets_count_as_ignored_or_raise_on_request(cuda, monkeypatch):
    """By default a target outside [0, V) that is not ignore_index is treated
    as ignored (counted on the device, no host synchronisation); with
    VALIDATE_TARGETS it raises ValueError."""
    from nuvla_forge_amd.kernels import chunked_ce

    note("ce bad target")
    hid, w, tgt = _ce_inputs(32, 16, 40, torch.float32, cuda)
    tgt[5] = 40
    tgt[9] = -7
    loss, dh, dw = _run_ce(hid, w, tgt, 8)
    as_ignored = tgt.clone()
    as_ignored[[5, 9]] = -100
    _check_ce(hid, w, as_ignored, loss, dh, dw, 1e-5, "bad targets as ignored")
    monkeypatch.setattr(chunked_ce, "VALIDATE_TARGETS", True)
    with pytest.raises(ValueError, match="outside"):
        chunked_cross_entropy(hid, w, tgt)


def test_ce_reasoning_head_step_makes_no_host_sync(cuda):
    """Eager forward + backward of the fused CE at the reasoning-head shape
    under torch.cuda.set_sync_debug_mode("error"): any synchronising call
    (the reference's n_valid .item(), chunked_ce.py:126, or a target check)
    would raise."""
    note("ce reasoning head: no host synchronisation")
    hid, lm_head, tgt = _reasoning_head_inputs(cuda, seed=12)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        for _ in range(2):
            with torch.autocast("cuda", dtype=torch.bfloat16):
                loss = chunked_cross_entropy(hid, lm_head, tgt, chunk_size=1024)
            loss.backward()
    finally:
        torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
    lo, _, _ = on.ce_forward_backward(np64(hid), np64(lm_head.detach().to(torch.bfloat16)),
                                      tgt.cpu().numpy())
    assert abs(float(loss.detach()) - lo) / lo < 2e-2


def test_ce_fp32_hidden_and_lm_head_under_autocast_compute_in_bf16(cuda):
    """The reasoning head as the reference model feeds it: the fp32 residual
    stream out of the text blocks and the fp32 lm_head, under bf16 autocast
    (train.py:174-179).  The reference's autocast-ed F.linear computes those
    logits in bf16; so does this path: parity against the fp64 oracle on the
    bf16-rounded operands, gradients in fp32."""
    note("ce fp32 hidden + fp32 lm_head under bf16 autocast")
    g = gen(13)
    hid = randn((512, 384), g, torch.float32, cuda).requires_grad_(True)
    lm_head = torch.nn.Parameter(randn((32000, 384), g, torch.float32, cuda, std=0.02))
    tgt = torch.randint(0, 32000, (512,), generator=g)
    tgt[::5] = -100
    tgt = tgt.to(cuda)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        loss = chunked_cross_entropy(hid, lm_head, tgt, chunk_size=1024)
    loss.backward()
    torch.cuda.synchronize()
    assert hid.grad.dtype == torch.float32 and lm_head.grad.dtype == torch.float32
    Hb = np64(hid.detach().to(torch.bfloat16))
    Wb = np64(lm_head.detach().to(torch.bfloat16))
    lo, dho, dwo = on.ce_forward_backward(Hb, Wb, tgt.cpu().numpy())
    assert abs(float(loss.detach()) - lo) / lo < 2e-2
    assert on.rel_err(np64(hid.grad), dho) < 2e-2
    assert on.rel_err(np64(lm_head.grad), dwo) < 2e-2
    # bf16 products, not fp32: with fp32 accumulation the loss sits on the
    # bf16-rounded operands' value (to ~1e-7), while the unrounded operands'
    # value differs from that by the rounding of 410 target logits (~1e-5)
    lo32, _, _ = on.ce_forward_backward(np64(hid), np64(lm_head), tgt.cpu().numpy())
    assert abs(float(loss.detach()) - lo) < abs(float(loss.detach()) - lo32)


_CFG4_ORACLE: dict = {}


@pytest.mark.parametrize("chunk", [1024, 4096])
def test_ce_cfg4_bf16_full_size_and_deterministic(cuda, chunk):
    """BASELINE cfg4: bf16 M4096 D2048 V32000, 409 rows ignored (M_valid 3687).

    chunk_size 1024 is the reference's default: E held once for every valid
    row in one chunk (262 MB, no fp32 dW accumulator: the reference's
    accumulator alone takes that much), the dW product reading E N-major and
    storing dW transposed; 4096 holds E in both layouts, one chunk.  Both are
    the plans the benchmark reports."""
    note(f"ce cfg4 bf16 M4096 D2048 V32000 chunk={chunk}")
    m, d, v = 4096, 2048, 32000
    g = gen(2)
    hid = randn((m, d), gen(0), torch.bfloat16, cuda)
    w = randn((v, d), gen(1), torch.bfloat16, cuda, std=0.02)
    tgt = torch.randint(0, v, (m,), generator=g)
    tgt[torch.randperm(m, generator=g)[:409]] = -100
    tgt = tgt.to(cuda)
    loss, dh, dw = _run_ce(hid, w, tgt, chunk)
    loss2, dh2, dw2 = _run_ce(hid, w, tgt, chunk)
    assert torch.equal(loss, loss2) and torch.equal(dh, dh2) and torch.equal(dw, dw2)
    if "ref" not in _CFG4_ORACLE:  # the same inputs for both chunk sizes
        H = hid.float().cpu().numpy()
        W = w.float().cpu().numpy()
        _CFG4_ORACLE["ref"] = on.ce_forward_backward(H, W, tgt.cpu().numpy())
    lo, dho, dwo = _CFG4_ORACLE["ref"]
    assert abs(float(loss.detach()) - lo) / lo < 2e-2
    assert on.rel_err(dh.float().cpu().numpy(), dho) < 2e-2
    assert on.rel_err(dw.float().cpu().numpy(), dwo) < 2e-2
    assert np.all(dh.float().cpu().numpy()[(tgt == -100).cpu().numpy()] == 0)


def test_ce_probabilities_over_2gib(cuda):
    """One chunk whose probabilities exceed 2 GiB (bf16 E [8448, 128256],
    2.17 GB, held once at D = 64): the logits launch stores E through 64-bit
    offsets and the gradient products read it through registers.  Checked
    against torch's fp32 cross entropy on the device (the fp64 oracle would
    take minutes at this size) at the bf16 tolerance."""
    note("ce E over 2 GiB m=8448 d=64 v=128256 chunk=100000")
    m, d, v = 8448, 64, 128256
    hid, w, tgt = _ce_inputs(m, d, v, torch.bfloat16, cuda, seed=13, w_std=0.1,
                             ignore=slice(None, None, 5))
    L = _lib.lib()
    assert L.nf_ce_state_bytes(m, d, v, 100000, _lib.dtype_code(torch.bfloat16)) > 2 * m * v
    assert 2 * m * v > 2 ** 31
    loss, dh, dw = _run_ce(hid, w, tgt, 100000)
    h32 = hid.float().requires_grad_(True)
    w32 = w.float().requires_grad_(True)
    ref = torch.nn.functional.cross_entropy(h32 @ w32.t(), tgt, ignore_index=-100)
    ref.backward()
    torch.cuda.synchronize()

    def rel(a, b):
        return float((a.float() - b).norm() / b.norm())

    lo = float(ref.detach())
    assert abs(float(loss) - lo) / lo < 2e-2
    assert rel(dh, h32.grad) < 2e-2 and rel(dw, w32.grad) < 2e-2
    assert not dh[::5].any()


def test_ce_state_is_released_after_backward(cuda):
    """The state nf_ce_fwd leaves for nf_ce_bwd (E, W^T, the scaled Hc^T, the
    fp32 dH rows and, with several chunks, the fp32 dW accumulator) is saved through
    save_for_backward, so autograd frees it once the backward has run, while
    the caller still holds ``loss`` (a training loop keeping the previous
    step's loss for logging must not carry two states)."""
    note("ce state released after backward")
    m, d, v = 1024, 256, 8192
    g = gen(31)
    hid = randn((m, d), g, torch.bfloat16, cuda).requires_grad_(True)
    w = randn((v, d), g, torch.bfloat16, cuda, std=0.05).requires_grad_(True)
    tgt = torch.randint(0, v, (m,), generator=g).to(cuda)
    L = _lib.lib()
    state_bytes = L.nf_ce_state_bytes(m, d, v, 256, _lib.dtype_code(torch.bfloat16))
    assert state_bytes > 2 * m * v  # bf16 E of every row (one chunk at this shape) at least
    loss = chunked_cross_entropy(hid, w, tgt, chunk_size=256)
    torch.cuda.synchronize()
    held = torch.cuda.memory_allocated()
    loss.backward()
    torch.cuda.synchronize()
    grads = hid.grad.numel() * 2 + w.grad.numel() * 2
    after = torch.cuda.memory_allocated()
    assert after <= held + grads - state_bytes, (held, after, grads, state_bytes)
    assert loss.grad_fn is not None  # loss still referenced
    with pytest.raises(RuntimeError):
        loss.backward()  # the saved state is gone: a second backward is refused


def _reasoning_head_inputs(dev, seed=8):
    """The reasoning head at the reference's model shape (model/nuvla.py:150-164,
    NuVLAConfig :26-44): batch 8 x 64 text tokens = 512 rows, width 384,
    vocabulary 32000; hidden states bf16 (autocast activations), lm_head an
    fp32 Parameter, every 7th target ignored."""
    g = gen(seed)
    hid = randn((512, 384), g, torch.bfloat16, dev).requires_grad_(True)
    lm_head = torch.nn.Parameter(randn((32000, 384), g, torch.float32, dev, std=0.02))
    tgt = torch.randint(0, 32000, (512,), generator=g)
    tgt[::7] = -100
    return hid, lm_head, tgt.to(dev)


@pytest.mark.parametrize("chunk", [1024, 128])
def test_ce_reasoning_head_model_shape_under_autocast(cuda, chunk):
    """bf16 hidden with an fp32 lm_head under bf16 autocast computes in bf16
    (as the reference's autocast-ed F.linear does) and returns each gradient
    in its input's dtype; parity against the fp64 oracle on the bf16-rounded
    operands at the bf16 tolerance.  Both chunk sizes take one chunk of the
    512 rows (E for every row, 33 MB, is less than the reference's fp32 dW
    accumulator alone, 49 MB), whose dH product is split over K into fp32
    slices added before the bf16 store."""
    note(f"ce reasoning head M512 D384 V32000 bf16/fp32 autocast chunk={chunk}")
    hid, lm_head, tgt = _reasoning_head_inputs(cuda)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        loss = chunked_cross_entropy(hid, lm_head, tgt, chunk_size=chunk)
    (loss * 0.5).backward()
    torch.cuda.synchronize()
    assert loss.dtype == torch.float32
    assert hid.grad.dtype == torch.bfloat16 and lm_head.grad.dtype == torch.float32
    lo, dho, dwo = on.ce_forward_backward(np64(hid), np64(lm_head.detach().to(torch.bfloat16)),
                                          tgt.cpu().numpy())
    assert abs(float(loss.detach()) - lo) / lo < 2e-2
    assert on.rel_err(np64(hid.grad), 0.5 * dho) < 2e-2
    assert on.rel_err(np64(lm_head.grad), 0.5 * dwo) < 2e-2
    assert not hid.grad[::7].any()


def test_ce_fp16_inputs_give_fp16_gradients(cuda):
    """fp16 hidden and weight are widened to fp32 for the products and the
    gradients come back in fp16, scaled by grad_output (the half-precision
    output path of the gradient epilogues), over several vocabulary chunks."""
    note("ce fp16 inputs m=200 d=72 v=700 chunk=64")
    hid, w, tgt = _ce_inputs(200, 72, 700, torch.float16, cuda, seed=9, w_std=0.2,
                             ignore=slice(None, None, 5))
    loss, dh, dw = _run_ce(hid, w, tgt, 64, scale=2.0)
    assert dh.dtype == torch.float16 and dw.dtype == torch.float16
    _check_ce(hid, w, tgt, loss, dh, dw, 2e-3, "fp16", scale=2.0)


@pytest.mark.parametrize("lm_scale", [1.0, 50.0])
def test_ce_reasoning_head_step_replays_in_a_graph(cuda, lm_scale):
    """The device path needs no host synchronisation (the reference's
    n_valid .item(), chunked_ce.py:126, is gone): forward + backward of the
    reasoning head capture into one HIP graph, and every replay, with eager
    work and synchronisations between replays, reproduces the eager step
    bit for bit.  lm_scale 50 (lm_head N(0, 1)) puts nearly every row far
    from its reference logit, so the replays run the far-row rescale too."""
    note(f"ce reasoning head graph capture lm_scale={lm_scale}")
    hid0, lm0, tgt = _reasoning_head_inputs(cuda, seed=9)
    lm0 = lm0.detach() * lm_scale

    def make():
        h = hid0.detach().requires_grad_(True)
        w = torch.nn.Parameter(lm0.detach().clone())

        def step():
            with torch.autocast("cuda", dtype=torch.bfloat16):
                loss = chunked_cross_entropy(h, w, tgt, chunk_size=1024)
            gh, gw = torch.autograd.grad(loss, [h, w])
            return loss, gh, gw

        return step

    eager = [t.clone() for t in make()()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step = make()
        step()
    side.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        outs = step()
    torch.cuda.current_stream().wait_stream(side)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(outs, eager)), f"replay {i}"
        make()()  # eager work between replays
        torch.cuda.synchronize()


def test_ce_peak_memory_below_the_eager_reference(cuda):
    """The reference's memory test (tests/test_kernels.py:240-262): bf16 hidden
    [4096, 512] and W [32000, 512]; loss + backward through the fused op peaks
    below the eager reference (fp32 logits materialised)."""
    note("ce peak memory bf16 [4096,512] x [32000,512]")
    from nuvla_forge_amd.kernels.reference import chunked_cross_entropy_ref

    m, h, v = 4096, 512, 32000
    g = gen(23)
    hid = randn((m, h), g, torch.bfloat16, cuda).requires_grad_(True)
    w = randn((v, h), g, torch.bfloat16, cuda).requires_grad_(True)
    tgt = torch.randint(0, v, (m,), generator=g).to(cuda)

    def peak(fn):
        hid.grad = w.grad = None
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats()
        fn().backward()
        torch.cuda.synchronize()
        return torch.cuda.max_memory_allocated()

    naive = peak(lambda: chunked_cross_entropy_ref(hid, w, tgt))
    fused = peak(lambda: chunked_cross_entropy(hid, w, tgt, chunk_size=1024))
    note(f"peak MiB: eager {naive / 2**20:.1f}, fused {fused / 2**20:.1f}")
    assert fused < naive
