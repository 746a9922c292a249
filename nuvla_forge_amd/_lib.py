"""ctypes binding of libnf_hip.so (the C ABI declared in include/nuvla_forge_hip.h).

The library is loaded after ``import torch`` so that its ``libamdhip64.so.7``
dependency resolves (by soname) to the HIP runtime torch already loaded: one
runtime, one set of streams.  Nothing here falls back to another backend; a
missing or stale library raises.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("libnf_hip.so")
ABI_VERSION = 3

DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_F32 = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); the order follows the C declarations
SIGNATURES = {
    "nf_abi_version": (_I32, []),
    "nf_last_error": (ctypes.c_char_p, []),
    "nf_swiglu_fwd": (_I32, [_P, _P, _P, _I64, _I32, _P]),
    "nf_swiglu_bwd": (_I32, [_P, _P, _P, _P, _P, _I64, _I32, _P]),
    "nf_adaln_fwd": (
        _I32,
        [_P, _I64, _P, _I64, _P, _I64, _P, _P, _I64, _P, _I64, _P, _P, _P,
         _I64, _I64, _I64, _F32, _I32, _I32, _I32, _I32, _I32, _I32, _P],
    ),
    "nf_adaln_bwd_workspace": (_SZ, [_I64, _I64, _I64]),
    "nf_adaln_bwd": (
        _I32,
        [_P, _P, _P, _I64, _P, _I64, _P, _I64, _P, _P, _I64, _P, _P, _P,
         _P, _SZ, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _I32, _P],
    ),
    "nf_adaln_bwd_reduce": (
        _I32,
        [_P, _SZ, _P, _P, _I64, _P, _P, _P, _P, _I64, _I64, _I64,
         _I32, _I32, _I32, _I32, _P],
    ),
    "nf_adaln_bwd_noalloc": (
        _I32,
        [_P, _P, _P, _I64, _P, _I64, _P, _I64, _P, _P, _I64, _P, _P, _P,
         _P, _P, _P, _P, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _I32, _I32, _P],
    ),
    "nf_ce_state_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I32]),
    "nf_ce_fwd_workspace": (_SZ, [_I64, _I64, _I64, _I64, _I32]),
    "nf_ce_fwd": (
        _I32,
        [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _P, _SZ, _P, _SZ, _P],
    ),
    "nf_ce_bwd_workspace": (_SZ, [_I64, _I64, _I64, _I64, _I32]),
    "nf_ce_bwd": (
        _I32,
        [_I64, _I64, _I64, _I64, _I32, _P, _SZ, _P, _P, _I32, _P, _I32, _P, _SZ, _P],
    ),
    "nf_ce_workspace": (_SZ, [_I64, _I64, _I64, _I64, _I32]),
    "nf_ce_fwd_bwd": (
        _I32,
        [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _P, _P, _P,
         _SZ, _P],
    ),
    "nf_gemm_swiglu": (
        _I32, [_P, _I64, _P, _I64, _P, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _I32, _P],
    ),
    "nf_gemm_swiglu_wgrad_workspace": (_SZ, [_I64, _I64, _I64]),
    "nf_gemm_swiglu_wgrad": (
        _I32,
        [_P, _P, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _I32, _P, _SZ, _P],
    ),
}

_lib: ctypes.CDLL | None = None
_load_error: str | None = None


def _open() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH.name} is not built; run `python -m nuvla_forge_amd.build` "
            "(hipcc, gfx950)"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.nf_abi_version()
    if ver != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH.name} ABI {ver} != expected {ABI_VERSION}; rebuild")
    return lib


def lib() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError if it cannot be loaded."""
    global _lib, _load_error
    if _lib is None:
        try:
            _lib = _open()
        except (OSError, RuntimeError, AttributeError) as e:
            _load_error = str(e)
            raise RuntimeError(f"nuvla_forge_amd HIP library unavailable: {e}") from e
    return _lib


def available() -> bool:
    """True if libnf_hip.so loads (it may still lack a GPU to run on)."""
    try:
        lib()
        return True
    except RuntimeError:
        return False


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().nf_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")


def dtype_code(t: torch.Tensor | torch.dtype) -> int:
    dt = t if isinstance(t, torch.dtype) else t.dtype
    try:
        return DTYPE_CODE[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}; expected float32, bfloat16 or float16") from None


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    """Raw hipStream_t of torch's current stream on t's device.

    torch's own accessor for the handle (what ``current_stream().cuda_stream``
    reads, without building a Stream object per launch: at the model's small
    shapes the fused ops are host-bound and this is on every call)."""
    return torch._C._cuda_getCurrentRawStream(t.get_device())
