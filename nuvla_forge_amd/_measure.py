"""ctypes binding of libnf_measure.so (include/nuvla_forge_measure.h).

The measurement aids the benchmark sets the product kernels against
(``nf_stream_probe``, ``nf_mfma_probe``, ``nf_mainloop_probe``) and the GEMM test hooks
(``nf_gemm_nt``, ``nf_gemm_nt_acc``, ``nf_gemm_nn``).  None of them is part of the product ABI and no op calls
them; they sit in their own library so that libnf_hip.so exports only the
product's entry points.  Failures are reported through the product library's
``nf_last_error`` (libnf_measure.so links libnf_hip.so), so ``_lib.check``
reads them.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

from . import _lib

LIB_PATH = Path(__file__).resolve().with_name("libnf_measure.so")

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int

# name -> (restype, argtypes); the order follows the C declarations
SIGNATURES = {
    "nf_gemm_nt": (_I32, [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _I32, _P]),
    "nf_gemm_nt_acc": (_I32, [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P]),
    "nf_gemm_nn": (_I32, [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _I32, _P]),
    "nf_stream_probe": (_I32, [_I32, _I32, _P, _P, _P, _P, _P, _P, _I64, _P]),
    "nf_mfma_probe": (_I32, [_P, _I64, _I64, _I32, _P, _P, _P]),
    "nf_mainloop_probe": (_I32, [_I32, _P, _P, ctypes.c_size_t, _I64, _I64, _P, _P, _P]),
}

_lib_m: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded measurement library (after the product library, whose
    already-loaded copy it binds to by soname); raises RuntimeError if
    either cannot be loaded."""
    global _lib_m
    if _lib_m is None:
        _lib.lib()
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH.name} is not built; run `python -m "
                               "nuvla_forge_amd.build`")
        try:
            m = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(m, name)
                fn.restype = res
                fn.argtypes = args
        except (OSError, AttributeError) as e:
            raise RuntimeError(f"{LIB_PATH.name} unavailable: {e}") from e
        _lib_m = m
    return _lib_m
