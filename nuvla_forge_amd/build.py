"""Build libnf_hip.so (the gfx950 kernels + C ABI) in-tree with hipcc.

Usage: ``python -m nuvla_forge_amd.build [-v]``.  Every ``csrc/*.hip`` file is
compiled to an object in ``_build/`` (in parallel), then linked into
``nuvla_forge_amd/libnf_hip.so`` (the product: include/nuvla_forge_hip.h).
The measurement aids and the GEMM test hook (``csrc/measure/*.hip``,
include/nuvla_forge_measure.h) go into ``nuvla_forge_amd/libnf_measure.so``,
which links the product library for its error reporting; only the benchmark
and the tests load it.  Both link ``libamdhip64.so.7`` by soname, so inside a
process that imported torch first they bind to the HIP runtime torch already
loaded.  Last, ``tests/c/abi_smoke`` (a C program using the product library
through its C ABI alone) is compiled with gcc.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG.parent / "_build"
LIB = PKG / "libnf_hip.so"
MEASURE_LIB = PKG / "libnf_measure.so"
INCLUDE = PKG.parent / "include"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: the compiler emits no packed fp32 add/mul/fma (v_pk_*_f32);
# some forms of those instructions have given wrong results on these GPUs
# without any error, so all fp32 math stays scalar.
CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def _hipcc() -> str:
    if shutil.which(HIPCC) or Path(HIPCC).exists():
        return HIPCC
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set HIPCC)")
    return found


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD / (("measure_" if src.parent.name == "measure" else "") + src.stem + ".o")
    cmd = [_hipcc(), *CFLAGS, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns about the device-only target feature; drop that
    noise = "'-packed-fp32-ops' is not a recognized feature"
    msg = "\n".join(ln for ln in (res.stdout + res.stderr).splitlines() if noise not in ln)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{msg}")
    if msg.strip() and verbose:
        print(msg, flush=True)
    return obj


def _link(objs: list[Path], out: Path, extra: list[str], verbose: bool) -> None:
    tmp = out.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs), *extra]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of {out.name} failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, out)


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every csrc/*.hip and csrc/measure/*.hip for gfx950 and link
    libnf_hip.so and libnf_measure.so.  Always rebuilds."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    measure = sorted((CSRC / "measure").glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no sources under {CSRC}")
    jobs = jobs or min(len(sources) + len(measure), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), sources + measure))
    _link(objs[:len(sources)], LIB, ["-Wl,-soname,libnf_hip.so"], verbose)
    _link(objs[len(sources):], MEASURE_LIB,
          [f"-L{PKG}", "-lnf_hip", "-Wl,-rpath,$ORIGIN"], verbose)
    build_c_smoke(verbose)
    return LIB


def build_c_smoke(verbose: bool = False) -> Path:
    """Compile tests/c/abi_smoke.c, a C program that drives libnf_hip.so
    through the C ABI alone (run by tests/test_gpu_c_abi.py), with gcc; it
    finds the library next to the package through its rpath."""
    src = PKG.parent / "tests" / "c" / "abi_smoke.c"
    exe = src.with_suffix("")
    rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
    cmd = [os.environ.get("CC", "gcc"), "-std=c99", "-O2", "-Wall", "-Wextra",
           "-D__HIP_PLATFORM_AMD__", f"-I{INCLUDE}", f"-I{rocm / 'include'}", str(src),
           "-o", str(exe), f"-L{LIB.parent}", "-lnf_hip", f"-L{rocm / 'lib'}", "-lamdhip64",
           "-lm", "-Wl,-rpath,$ORIGIN/../../nuvla_forge_amd", f"-Wl,-rpath,{rocm / 'lib'}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"C ABI smoke program failed to build:\n{res.stdout}{res.stderr}")
    return exe


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
