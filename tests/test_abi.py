"""C ABI and host-side logic, CPU only (no kernel is launched here).

Checks that libnf_hip.so loads, exports every function include/*.h declares,
reports its ABI version, and rejects bad arguments with a status and a
message before touching the GPU; and that ``force_reference=True`` runs the
eager formulation (host tensors take it too: tests/test_cpu_dispatch.py).
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from nuvla_forge_amd import _lib, _measure
from nuvla_forge_amd import kernels as K
from nuvla_forge_amd.kernels import chunked_ce, reference
from oracle import numerics as on

ROOT = Path(__file__).resolve().parents[1]
PRODUCT_HEADER = ROOT / "include" / "nuvla_forge_hip.h"
MEASURE_HEADER = ROOT / "include" / "nuvla_forge_measure.h"

NF_OK, NF_ERR_ARG, NF_ERR_DTYPE, NF_ERR_WORKSPACE = 0, -1, -2, -3
FAKE = 4096  # a non-null pointer value; every call below returns before using it


def _declared(header: Path) -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    return set(re.findall(r"\b(nf_\w+)\s*\(", text))


def _err() -> str:
    return _lib.lib().nf_last_error().decode()


def _exported(path: Path) -> set[str]:
    """Dynamic symbols a shared library defines (nm -D --defined-only)."""
    import shutil
    import subprocess

    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("no nm")
    out = subprocess.run([nm, "-D", "--defined-only", str(path)], capture_output=True,
                         text=True, check=True).stdout
    return {ln.split()[-1] for ln in out.splitlines() if ln.split()}


def test_library_exports_every_declared_symbol():
    """Every include/*.h header belongs to one library: the product header to
    libnf_hip.so, the measurement header to libnf_measure.so; each library
    exports what its header declares, each ctypes table matches its header,
    and the product library exports no nf_ entry point beyond its header."""
    headers = sorted((ROOT / "include").glob("*.h"))
    assert headers == sorted([PRODUCT_HEADER, MEASURE_HEADER]), headers
    for header, path, table in ((PRODUCT_HEADER, _lib.LIB_PATH, _lib.SIGNATURES),
                                (MEASURE_HEADER, _measure.LIB_PATH, _measure.SIGNATURES)):
        declared = _declared(header)
        assert declared, header
        raw = ctypes.CDLL(str(path))
        missing = [n for n in sorted(declared) if not hasattr(raw, n)]
        assert not missing, f"{path.name} does not export {missing}"
        assert declared == set(table), f"ctypes table out of sync with {header.name}"
    product = {n for n in _exported(_lib.LIB_PATH) if n.startswith("nf_")}
    assert product == _declared(PRODUCT_HEADER), product ^ _declared(PRODUCT_HEADER)
    assert not _declared(PRODUCT_HEADER) & _declared(MEASURE_HEADER)
    assert len(_declared(PRODUCT_HEADER)) >= 10


def test_header_is_c_and_the_c_program_links_the_library():
    """include/nuvla_forge_hip.h compiles as C99; tests/c/abi_smoke (built with
    the library) resolves libnf_hip.so through its rpath."""
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no gcc")
    for header in ("nuvla_forge_hip.h", "nuvla_forge_measure.h"):
        src = (f'#include "{header}"\n'
               'int main(void) { return nf_abi_version() != NF_ABI_VERSION; }\n')
        res = subprocess.run([gcc, "-std=c99", "-Wall", "-Wextra", "-Werror", "-fsyntax-only",
                              f"-I{ROOT / 'include'}", "-x", "c", "-"], input=src,
                             capture_output=True, text=True)
        assert res.returncode == 0, (header, res.stderr)
    exe = ROOT / "tests" / "c" / "abi_smoke"
    assert exe.exists(), "tests/c/abi_smoke is built by nuvla_forge_amd.build"
    ldd = subprocess.run(["ldd", str(exe)], capture_output=True, text=True).stdout
    line = [ln for ln in ldd.splitlines() if "libnf_hip.so" in ln]
    assert line and "not found" not in line[0], ldd


def test_abi_version():
    assert _lib.lib().nf_abi_version() == _lib.ABI_VERSION == 3
    assert K.HAS_HIP and K.HAS_TRITON


def test_swiglu_argument_validation():
    L = _lib.lib()
    assert L.nf_swiglu_fwd(FAKE, FAKE, FAKE, -1, 1, None) == NF_ERR_ARG
    assert "n=-1" in _err()
    assert L.nf_swiglu_fwd(None, FAKE, FAKE, 10, 1, None) == NF_ERR_ARG
    assert "null" in _err()
    assert L.nf_swiglu_fwd(FAKE, FAKE, FAKE, 10, 7, None) == NF_ERR_DTYPE
    assert L.nf_swiglu_bwd(FAKE, FAKE, FAKE, FAKE, FAKE, 0, 1, None) == NF_OK  # empty: no launch


def test_gemm_swiglu_argument_validation():
    L = _lib.lib()
    # x, ldx, w_gate, ld_gate, w_up, ld_up, a, b, act, ldo, M, D, H, dtype, stream
    ok = [FAKE, 64, FAKE, 64, FAKE, 128, FAKE, FAKE, FAKE, 128, 16, 64, 128, 1, None]
    bad_dtype = list(ok)
    bad_dtype[13] = 0
    assert L.nf_gemm_swiglu(*bad_dtype) == NF_ERR_DTYPE and "bf16 only" in _err()
    one_saved = list(ok)
    one_saved[7] = None  # a without b
    assert L.nf_gemm_swiglu(*one_saved) == NF_ERR_ARG and "both or neither" in _err()
    short_ldo = list(ok)
    short_ldo[9] = 100  # ldo < H
    assert L.nf_gemm_swiglu(*short_ldo) == NF_ERR_ARG and "leading dimension" in _err()
    for i in (3, 5):  # each weight's own row stride is checked against D
        short_ldw = list(ok)
        short_ldw[i] = 63
        assert L.nf_gemm_swiglu(*short_ldw) == NF_ERR_ARG and "leading dimension" in _err()
    neg = list(ok)
    neg[12] = 0  # H = 0
    assert L.nf_gemm_swiglu(*neg) == NF_ERR_ARG and "bad shape" in _err()
    empty = list(ok)
    empty[10] = 0  # M = 0: nothing to do, no launch
    assert L.nf_gemm_swiglu(*empty) == NF_OK


def _round_up(v: int, m: int) -> int:
    return (v + m - 1) // m * m


def test_gemm_swiglu_wgrad_workspace_and_validation():
    L = _lib.lib()
    assert L.nf_gemm_swiglu_wgrad_workspace(0, 384, 1536) == 0
    # Headline DiT MLP (M = 8 x 1176 tokens, D 384, H 1536): 6 x 2 output tiles of
    # 256 x 256 per product, so the token sum is cut into 256 // 24 = 10 slices of
    # 960 tokens; the workspace is the token-contiguous copies of da, db, x and
    # the fp32 slices of both products.
    m, d, h = 9408, 384, 1536
    slices = 256 // (2 * 6 * 2)
    want = 2 * _round_up(h * m * 2, 256) + _round_up(d * m * 2, 256) + 2 * slices * h * d * 4
    assert L.nf_gemm_swiglu_wgrad_workspace(m, d, h) == want
    # one tile and 100 tokens (padded to 104): no split, no fp32 slices
    assert L.nf_gemm_swiglu_wgrad_workspace(100, 64, 64) == 3 * _round_up(64 * 104 * 2, 256)
    # da, db, ld_ab, x, ldx, dw_gate, dw_up, ldw, M, D, H, dtype, workspace, bytes, stream
    ok = [FAKE, FAKE, h, FAKE, d, FAKE, FAKE, d, m, d, h, 1, FAKE, want, None]
    bad_dtype = list(ok)
    bad_dtype[11] = 0
    assert L.nf_gemm_swiglu_wgrad(*bad_dtype) == NF_ERR_DTYPE and "bf16 only" in _err()
    short_ld = list(ok)
    short_ld[2] = h - 1
    assert L.nf_gemm_swiglu_wgrad(*short_ld) == NF_ERR_ARG and "leading dimension" in _err()
    no_x = list(ok)
    no_x[3] = None
    assert L.nf_gemm_swiglu_wgrad(*no_x) == NF_ERR_ARG and "null" in _err()
    small_ws = list(ok)
    small_ws[13] = want - 1
    assert L.nf_gemm_swiglu_wgrad(*small_ws) == NF_ERR_WORKSPACE and str(want) in _err()
    bad_shape = list(ok)
    bad_shape[9] = 0
    assert L.nf_gemm_swiglu_wgrad(*bad_shape) == NF_ERR_ARG and "bad shape" in _err()
    huge = list(ok)
    huge[8] = 1 << 20  # 1M tokens x 1536 bf16 = 3 GiB per operand
    assert L.nf_gemm_swiglu_wgrad(*huge) == NF_ERR_ARG and "2 GiB" in _err()
    absurd = list(ok)
    absurd[8] = 1 << 62  # the size test divides, so this cannot wrap around
    assert L.nf_gemm_swiglu_wgrad(*absurd) == NF_ERR_ARG and "2 GiB" in _err()
    assert L.nf_gemm_swiglu_wgrad_workspace(1 << 62, d, h) == 0


def test_adaln_argument_validation():
    L = _lib.lib()
    args = [FAKE, 1024, FAKE, 1024, FAKE, 1024, FAKE, FAKE, 1024, FAKE, 1024, FAKE, FAKE, FAKE]
    tail = [1e-6, 1, 1, 1, 1, 1, 1, None]
    assert L.nf_adaln_fwd(*args, 100, 1024, 7, *tail) == NF_ERR_ARG  # M % T != 0
    assert "multiple" in _err()
    assert L.nf_adaln_fwd(*args, 64, 20000, 8, *tail) == NF_ERR_ARG  # N too large
    assert "exceeds" in _err()
    assert L.nf_adaln_fwd(*args, 64, 1024, 8, 1e-6, 1, 0, 1, 1, 1, 1, None) == NF_ERR_DTYPE  # bf16 x, f32 y
    bad_ld = list(args)
    bad_ld[1] = 512
    assert L.nf_adaln_fwd(*bad_ld, 64, 1024, 8, *tail) == NF_ERR_ARG
    assert L.nf_adaln_bwd_workspace(8192, 1024, 1024) > 8 * 1024 * 4
    assert L.nf_adaln_bwd_workspace(10, 1024, 3) == 0
    assert L.nf_adaln_bwd_workspace(1 << 40, 1024, 1) == 0  # beyond any buffer
    assert L.nf_adaln_fwd(*args, 1 << 40, 1024, 8, *tail) == NF_ERR_ARG and "2^40" in _err()
    small = L.nf_adaln_bwd_workspace(64, 1024, 8)
    bwd = [FAKE, FAKE, FAKE, 1024, FAKE, 1024, FAKE, 1024, FAKE, FAKE, 1024, FAKE, FAKE, FAKE,
           FAKE, small - 1, 64, 1024, 8, 1, 1, 1, 1, 1, None]
    assert L.nf_adaln_bwd(*bwd) == NF_ERR_WORKSPACE
    assert "workspace" in _err()
    red = [FAKE, small - 1, FAKE, FAKE, 1024, FAKE, None, None, None, 64, 1024, 8, 1, 1, 1, 1, None]
    assert L.nf_adaln_bwd_reduce(*red) == NF_ERR_WORKSPACE
    red[1] = small
    red[3] = None
    assert L.nf_adaln_bwd_reduce(*red) == NF_ERR_ARG  # scale missing
    assert L.nf_adaln_bwd_reduce(FAKE, small, FAKE, FAKE, 1024, None, None, None, None,
                                 64, 1024, 8, 1, 1, 1, 1, None) == NF_OK  # nothing requested


@pytest.mark.parametrize("b", [1, 2, 3, 5, 6, 7, 8, 12, 24, 32, 40, 100, 255, 256, 300])
@pytest.mark.parametrize("t,n", [(2048, 1024), (2048, 2048), (64, 256)])
def test_adaln_backward_blocks_fit_one_round(b, t, n):
    """The backward's B x J blocks (J read back from the workspace size,
    B * J * 3 * N fp32 partial rows) stay within the 256 CUs that each hold one
    512-thread backward block, unless every sample already runs one block."""
    L = _lib.lib()
    ws = L.nf_adaln_bwd_workspace(b * t, n, t)
    j, rem = divmod(ws, b * 3 * n * 4)
    assert rem == 0 and j >= 1
    assert b * j <= 256 or j == 1, (b, j)
    if b <= 256 and t >= 2048:
        assert b * j > 128, (b, j)  # and still at least half the CUs


def _ceil(a: int, b: int) -> int:
    return -(-a // b)


def _ce_state_closed_form(m, d, v, chunk_rows, es=2):
    """The state nf_ce_fwd leaves for nf_ce_bwd, term by term (each buffer
    256-byte aligned): scalars, pos [M], the fp32 row factors [M], W^T
    [D, V8], the scaled Hc^T [D, M8], one chunk's E, fp32 dH rows [M, D], and
    the fp32 dW accumulator when more than one chunk.  bf16 (es 2) has a
    budget of 2 * (min(chunk_rows, M) + D) rows of E (the bytes of the
    reference's fp32 [chunk_rows, V] tile and fp32 [V, D] accumulator) and
    takes the first of: one chunk in both layouts, E [C, V8] and E^T [V, C]
    (D >= 2048 and 2 C inside the budget); one chunk held once, E [C, V8] (C
    inside the budget); chunks of C = 2 * chunk_rows rows rounded up to 256
    held once, with the accumulator transposed, [D, V8].  fp32 holds chunks
    of C = chunk_rows rows rounded up to 256 in both layouts with the
    accumulator [V, D].  C is at most M rounded up to 256."""
    a = lambda x: _ceil(x, 256) * 256  # noqa: E731
    mcap = _ceil(m, 256) * 256
    want = min(chunk_rows, mcap)
    if es == 2:
        budget = 2 * (min(chunk_rows, m) + d)
        single = d < 2048 or 2 * mcap > budget
        c = min(a(2 * want) if single and mcap > budget else mcap, mcap)
    else:
        single = False
        c = min(a(want), mcap)
    v8, m8 = _ceil(v, 8) * 8, _ceil(m, 8) * 8
    nch = _ceil(m, c)
    e_bytes = a(es * c * v8) + (0 if single else a(es * v * c))
    acc = (a(4 * d * v8) if single else a(4 * v * d)) if nch > 1 else 0
    return (a(64) + a(4 * m) + a(4 * m) + a(es * d * v8) + a(es * d * m8) + e_bytes
            + a(4 * m * d) + acc)


def sb_at(L, chunk_rows):
    return L.nf_ce_state_bytes(16384, 2048, 32000, chunk_rows, 1)


def test_ce_state_and_workspace_sizes():
    L = _lib.lib()
    shapes = [(4096, 2048, 32000, 1024), (4096, 2048, 32000, 4096), (4096, 4096, 32000, 4096),
              (4096, 4096, 32000, 1024), (16384, 2048, 32000, 1024), (16384, 384, 32000, 1024),
              (512, 384, 32000, 1024), (300, 72, 1030, 100), (17, 36, 333, 7)]
    for m, d, v, cr in shapes:
        assert L.nf_ce_state_bytes(m, d, v, cr, 1) == _ce_state_closed_form(m, d, v, cr), (m, cr)
        assert L.nf_ce_state_bytes(m, d, v, cr, 0) == _ce_state_closed_form(m, d, v, cr, es=4)
    # bf16: E and the dW accumulator together stay within what the
    # reference's chunk loop holds for the same roles at the same chunk_size
    # (an fp32 [chunk_size, V] tile, an fp32 [V, D] accumulator), up to the
    # rounding of a chunk to 256 rows
    for m, d, v, cr in shapes:
        a = lambda x: _ceil(x, 256) * 256  # noqa: E731
        v8, m8 = _ceil(v, 8) * 8, _ceil(m, 8) * 8
        rest = a(64) + 2 * a(4 * m) + a(2 * d * v8) + a(2 * d * m8) + a(4 * m * d)
        e_acc = L.nf_ce_state_bytes(m, d, v, cr, 1) - rest
        assert e_acc <= 4 * v8 * (min(cr, m) + d) + 4 * 256 * v8 + 512, (m, d, cr)
    # cfg4 at the reference's default chunk_size holds E once for every row
    # (262 MB) and no accumulator: the reference's accumulator alone is 262 MB
    assert (L.nf_ce_state_bytes(4096, 2048, 32000, 1024, 1)
            == _ce_state_closed_form(4096, 2048, 32000, 4096 * 4, es=2) - 2 * 4096 * 32000)
    # a chunk's E (bf16, 2 * chunk_size rows, once) is the bytes of the
    # reference's [chunk_size, V] fp32 logits tile: each 1024 more rows of
    # chunk_size hold 4 * 1024 * 32000 more bytes
    more = sb_at(L, 2048) - sb_at(L, 1024)
    assert more == 4 * 1024 * 32000
    assert L.nf_ce_state_bytes(4096, 2048, 32000, 1024, 2) == 0  # fp16 unsupported
    assert L.nf_ce_state_bytes(0, 2048, 32000, 1024, 1) == 0
    assert L.nf_ce_state_bytes(4096, 2048, 32000, 0, 1) == 0
    sb = L.nf_ce_state_bytes(4096, 2048, 32000, 1024, 1)
    fws = L.nf_ce_fwd_workspace(4096, 2048, 32000, 1024, 1)
    bws = L.nf_ce_bwd_workspace(4096, 2048, 32000, 1024, 1)
    assert fws > 4096 * 2048 * 2 and bws > 0  # the forward holds the gathered rows
    assert L.nf_ce_workspace(4096, 2048, 32000, 1024, 1) == sb + max(fws, bws)


def test_ce_argument_validation():
    L = _lib.lib()
    # sizes no buffer could have are refused before any byte count is formed
    assert L.nf_ce_workspace(4096, 1 << 40, 32000, 4096, 1) == 0
    assert L.nf_ce_fwd(FAKE, FAKE, FAKE, 16, 1 << 40, 50, -100, 64, 1, FAKE, None, FAKE, 1 << 20,
                       FAKE, 1 << 20, None) == NF_ERR_ARG and "2^40" in _err()
    M_ = _measure.lib()
    assert M_.nf_gemm_nt(FAKE, 1 << 40, FAKE, 1 << 40, FAKE, 16, 16, 16, 1 << 40, 1,
                         None) == NF_ERR_ARG and "int32" in _err()
    # leading dimensions below the extents they hold
    assert M_.nf_gemm_nn(FAKE, 16, FAKE, 16, FAKE, 16, 16, 16, 24, 0,
                         None) == NF_ERR_ARG and "leading dim" in _err()  # lda < K
    assert M_.nf_gemm_nn(FAKE, 24, FAKE, 8, FAKE, 16, 16, 16, 24, 0, None) == NF_ERR_ARG
    assert M_.nf_gemm_nn(FAKE, 24, FAKE, 16, FAKE, 8, 16, 16, 24, 1, None) == NF_ERR_ARG  # ldc < M
    ws = L.nf_ce_workspace(16, 8, 50, 64, 1)
    base = [FAKE, FAKE, FAKE]
    out = [FAKE, FAKE, FAKE, None, FAKE]
    assert L.nf_ce_fwd_bwd(*base, 16, 8, 50, -100, 0, 1, *out, ws, None) == NF_ERR_ARG
    assert L.nf_ce_fwd_bwd(*base, 16, 8, 50, -100, 64, 2, *out, ws, None) == NF_ERR_DTYPE
    assert L.nf_ce_fwd_bwd(*base, 16, 8, 50, -100, 64, 1, *out, 16, None) == NF_ERR_WORKSPACE
    # the two-call form: shapes, chunk rows, dtypes, buffers
    sb = L.nf_ce_state_bytes(16, 8, 50, 64, 1)
    fws = L.nf_ce_fwd_workspace(16, 8, 50, 64, 1)
    bws = L.nf_ce_bwd_workspace(16, 8, 50, 64, 1)
    fwd = [FAKE, FAKE, FAKE, 16, 8, 50, -100, 64, 1, FAKE, None, FAKE, sb, FAKE, fws, None]
    assert L.nf_ce_fwd(*fwd[:3], 0, *fwd[4:]) == NF_ERR_ARG
    assert L.nf_ce_fwd(*fwd[:7], 0, *fwd[8:]) == NF_ERR_ARG and "chunk_rows" in _err()
    assert L.nf_ce_fwd(*fwd[:8], 2, *fwd[9:]) == NF_ERR_DTYPE
    assert L.nf_ce_fwd(*fwd[:12], sb - 1, *fwd[13:]) == NF_ERR_WORKSPACE  # state too small
    assert L.nf_ce_fwd(*fwd[:14], fws - 1, None) == NF_ERR_WORKSPACE
    # M, D, V, chunk_rows, dtype, state, state_bytes, g, dh, dt_h, dw, dt_w, ws, bytes, stream
    bwd = [16, 8, 50, 64, 1, FAKE, sb, None, FAKE, 1, FAKE, 0, FAKE, bws, None]
    assert L.nf_ce_bwd(*bwd[:3], 0, *bwd[4:]) == NF_ERR_ARG  # chunk_rows
    assert L.nf_ce_bwd(*bwd[:8], None, *bwd[9:]) == NF_ERR_ARG  # dhidden
    assert L.nf_ce_bwd(*bwd[:9], 7, *bwd[10:]) == NF_ERR_DTYPE  # gradient dtype
    assert L.nf_ce_bwd(*bwd[:6], sb - 1, *bwd[7:]) == NF_ERR_WORKSPACE
    assert L.nf_ce_bwd(*bwd[:13], bws - 1, None) == NF_ERR_WORKSPACE
    assert M_.nf_gemm_nt(FAKE, 4, FAKE, 4, FAKE, 2, 2, 2, 8, 1, None) == NF_ERR_ARG  # lda < K


def test_stream_probe_argument_validation():
    """The streaming-ceiling entry point refuses what it cannot run before
    any launch (no GPU needed); n16 = 0 is a no-op."""
    L = _measure.lib()
    ptrs = [FAKE] * 6
    assert L.nf_stream_probe(3, 1, *ptrs, 16, None) == NF_ERR_ARG and "(3, 1)" in _err()
    assert L.nf_stream_probe(4, 1, *ptrs, 16, None) == NF_ERR_ARG
    assert L.nf_stream_probe(2, 2, *ptrs, -1, None) == NF_ERR_ARG and "< 0" in _err()
    assert L.nf_stream_probe(2, 2, FAKE, None, None, None, FAKE, FAKE, 16, None) == NF_ERR_ARG
    assert "input 1" in _err()
    assert L.nf_stream_probe(1, 1, FAKE + 8, None, None, None, FAKE, None, 16,
                             None) == NF_ERR_ARG and "aligned" in _err()
    assert L.nf_stream_probe(2, 2, *ptrs, 0, None) == NF_OK


def test_mfma_probe_argument_validation():
    """The MFMA-ceiling entry point refuses bad sizes and pointers before any
    launch (no GPU needed)."""
    L = _measure.lib()
    assert L.nf_mfma_probe(FAKE, -1, 1, 0, FAKE, None, None) == NF_ERR_ARG and "iters" in _err()
    assert L.nf_mfma_probe(FAKE, 2**30 + 1, 1, 0, FAKE, None, None) == NF_ERR_ARG
    assert L.nf_mfma_probe(FAKE, 1, 0, 0, FAKE, None, None) == NF_ERR_ARG and "blocks" in _err()
    assert L.nf_mfma_probe(FAKE, 1, 2**20 + 1, 0, FAKE, None, None) == NF_ERR_ARG
    assert L.nf_mfma_probe(FAKE, 1, 1, 2, FAKE, None, None) == NF_ERR_ARG and "form" in _err()
    assert L.nf_mfma_probe(FAKE, 1, 1, 0, None, None, None) == NF_ERR_ARG and "out" in _err()
    assert L.nf_mfma_probe(FAKE + 8, 1, 1, 0, FAKE, None, None) == NF_ERR_ARG
    assert "aligned" in _err()


def test_mainloop_probe_argument_validation():
    """The mainloop-ingredients probe refuses bad modes, sizes and pointers,
    and a source too small for its mode, before any launch (no GPU needed)."""
    L = _measure.lib()
    mib = 1 << 20
    for mode in (0, 6):
        assert L.nf_mainloop_probe(mode, FAKE, FAKE, 64 * mib, 1, 1, FAKE, None, None) == NF_ERR_ARG
        assert "mode" in _err()
    assert L.nf_mainloop_probe(1, FAKE, None, 0, -1, 1, FAKE, None, None) == NF_ERR_ARG
    assert "iters" in _err()
    assert L.nf_mainloop_probe(1, FAKE, None, 0, 1, 0, FAKE, None, None) == NF_ERR_ARG
    assert "blocks" in _err()
    assert L.nf_mainloop_probe(1, FAKE, None, 0, 1, 2**20 + 1, FAKE, None, None) == NF_ERR_ARG
    assert L.nf_mainloop_probe(1, None, None, 0, 1, 1, FAKE, None, None) == NF_ERR_ARG
    assert L.nf_mainloop_probe(1, FAKE, None, 0, 1, 1, None, None, None) == NF_ERR_ARG
    assert L.nf_mainloop_probe(1, FAKE + 8, None, 0, 1, 1, FAKE, None, None) == NF_ERR_ARG
    assert "aligned" in _err()
    assert L.nf_mainloop_probe(3, FAKE, None, 0, 1, 1, FAKE, None, None) == NF_ERR_ARG
    assert L.nf_mainloop_probe(4, FAKE, FAKE, mib - 16, 1, 1, FAKE, None, None) == NF_ERR_ARG
    assert L.nf_mainloop_probe(5, FAKE, FAKE, mib, 1, 1, FAKE, None, None) == NF_ERR_ARG
    assert "needs" in _err()


def test_chunk_rows_argument():
    assert chunked_ce.chunk_rows_for(1024) == 1024
    assert chunked_ce.chunk_rows_for(7) == 7
    with pytest.raises(ValueError):
        chunked_ce.chunk_rows_for(0)


# ---------------------------------------------------------------------------
# Python drop-in on the CPU
# ---------------------------------------------------------------------------
def test_launch_heuristics_of_the_utils_module():
    """kernels.utils keeps the reference's helpers (utils.py:23-44): the next
    power of two, and the per-row wavefront count of the adaLN forward plan
    (64-lane wavefronts, up to two 8-element chunks per lane, >= 2 from 1024)."""
    from nuvla_forge_amd.kernels import utils

    assert [utils.next_power_of_2(n) for n in (0, 1, 2, 3, 1000, 1024, 1025)] == \
        [1, 1, 2, 4, 1024, 1024, 2048]
    want = {1: 1, 256: 1, 1000: 1, 1023: 1, 1024: 2, 2048: 2, 2049: 4, 4096: 4, 8192: 8,
            16384: 16}
    assert {n: utils.warps_for_block(n) for n in want} == want
    assert utils.HAS_TRITON is utils.HAS_HIP


def test_force_reference_adaln_matches_oracle():
    gen = torch.Generator().manual_seed(0)
    b, t, n = 2, 4, 32
    x, y = (torch.randn(b * t, n, generator=gen, dtype=torch.float64, requires_grad=True)
            for _ in range(2))
    cond = [torch.randn(b, n, generator=gen, dtype=torch.float64, requires_grad=True)
            for _ in range(3)]
    w = torch.randn(n, generator=gen, dtype=torch.float64, requires_grad=True)
    h, out = K.fused_adaln_residual_rmsnorm(x, y, cond[0], w, cond[1], cond[2], t,
                                            force_reference=True)
    dh, do = torch.randn_like(h), torch.randn_like(out)
    torch.autograd.backward([h, out], [dh, do])
    args = dict(x=x, y=y, gate=cond[0], weight=w, scale=cond[1], shift=cond[2])
    npa = {k: v.detach().numpy() for k, v in args.items()}
    hh, oo, _ = on.adaln_forward(**npa, t=t)
    grads = on.adaln_backward(**npa, t=t, dh_up=dh.numpy(), dout=do.numpy())
    assert on.rel_err(h.detach().numpy(), hh) < 1e-14
    assert on.rel_err(out.detach().numpy(), oo) < 1e-6  # the eager path norms in fp32
    for k, v in args.items():
        assert on.rel_err(v.grad.numpy(), grads[k]) < 1e-6, k


def test_force_reference_swiglu_and_ce():
    gen = torch.Generator().manual_seed(1)
    a = torch.randn(17, 33, generator=gen, requires_grad=True)
    b = torch.randn(17, 33, generator=gen, requires_grad=True)
    out = K.fused_swiglu(a, b, force_reference=True)
    assert on.rel_err(out.detach().numpy(), on.swiglu_forward(a.detach().double().numpy(),
                                                               b.detach().double().numpy())) < 1e-6
    m, d, v = 64, 32, 200
    hid = torch.randn(m, d, generator=gen, requires_grad=True)
    w = (torch.randn(v, d, generator=gen) * 0.02).requires_grad_(True)
    tgt = torch.randint(0, v, (m,), generator=gen)
    tgt[::3] = -100
    loss = K.chunked_cross_entropy(hid, w, tgt, chunk_size=16, force_reference=True)
    loss.backward()
    lo, dho, dwo = on.ce_forward_backward(hid.detach().double().numpy(),
                                          w.detach().double().numpy(), tgt.numpy())
    assert float(loss.detach()) == pytest.approx(lo, rel=1e-5)
    assert on.rel_err(hid.grad.numpy(), dho) < 1e-5
    assert on.rel_err(w.grad.numpy(), dwo) < 1e-5
    assert torch.all(hid.grad[::3] == 0)
    allign = torch.full((m,), -100)
    z = K.chunked_cross_entropy(hid, w, allign, chunk_size=16, force_reference=True)
    assert float(z.detach()) == 0.0


def test_eager_reference_module_matches_textbook_ce():
    gen = torch.Generator().manual_seed(2)
    hid = torch.randn(32, 8, generator=gen)
    w = torch.randn(40, 8, generator=gen)
    tgt = torch.randint(0, 40, (32,), generator=gen)
    lo, _, _ = on.ce_forward_backward(hid.double().numpy(), w.double().numpy(), tgt.numpy())
    assert float(reference.chunked_cross_entropy_ref(hid, w, tgt)) == pytest.approx(lo, rel=1e-5)
    assert np.isfinite(lo)
