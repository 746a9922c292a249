"""Kernel microbenchmarks in the reference's report format.

Counterpart of ``nuvla_forge/bench/bench_kernels.py`` (217 lines): the same
command line (``--out``, ``--peak-bw``, ``--dtype``), the same shapes, the
same timing protocol (events around ``iters`` calls after ``warmup`` calls,
mean; forward + harness ops + backward, bench_kernels.py:48-58,70-76,104-107)
and the same ``reports/kernels.json`` schema (``device``, ``peak_bw_gb_s``,
``dtype``, and ``adaln`` / ``swiglu`` / ``cross_entropy`` row lists with the
keys bench/report.py:45-80 reads), so an MI355X run renders into the
reference's RESULTS.md tables unchanged.  The byte counts are the
reference's (11 * M * N * e for the seam, 8 * M * N * e for SwiGLU,
bench_kernels.py:84,120); "eager" is the reference formulation
(``force_reference=True``) on the same device.

    python -m nuvla_forge_amd.bench_kernels [--out reports/kernels.json]
"""

from __future__ import annotations

import argparse
import json
from pathlib import Path

import torch

from .kernels import chunked_cross_entropy, fused_adaln_residual_rmsnorm, fused_swiglu
from .kernels.reference import (
    adaln_residual_rmsnorm_ref,
    chunked_cross_entropy_ref,
    swiglu_ref,
)

# Spec-sheet peak HBM bandwidth by gfx architecture (the device name the HIP
# runtime reports can be generic, e.g. "AMD Radeon Graphics"); --peak-bw
# overrides.  Used only to put a measurement in context.
PEAK_BW_GB_S = {
    "gfx950": 8000.0,   # MI355X / MI350X: HBM3E
    "gfx942": 5300.0,   # MI300X
}

ADALN_SHAPES = [(8, 32, 384), (8, 128, 384), (16, 256, 768), (8, 512, 1024), (4, 1024, 1536)]
SWIGLU_SHAPES = [(8192, 1536), (16384, 1536), (32768, 3072)]
CE_SHAPES = [(4096, 384, 32000), (8192, 384, 32000), (16384, 384, 32000)]


def arch_name(device: int = 0) -> str:
    return torch.cuda.get_device_properties(device).gcnArchName.split(":")[0]


def peak_bw_for(arch: str, override: float | None = None) -> float:
    if override:
        return float(override)
    if arch not in PEAK_BW_GB_S:
        raise SystemExit(f"no peak bandwidth known for {arch}; pass --peak-bw")
    return PEAK_BW_GB_S[arch]


def bandwidth_gb_s(bytes_moved: int, ms: float) -> float:
    return bytes_moved / (ms * 1e-3) / 1e9


def roofline_note(achieved: float, peak: float) -> str:
    """The reference's verdict bands (profiling.py:125-142): >80% saturated,
    >50% healthy, >25% underutilised, else poor."""
    pct = 100.0 * achieved / peak
    if pct > 80:
        verdict = "bandwidth-saturated; no headroom left in this kernel"
    elif pct > 50:
        verdict = "healthy; remaining gap is launch overhead and tails"
    elif pct > 25:
        verdict = "underutilised; check occupancy and coalescing"
    else:
        verdict = "poor; likely uncoalesced or occupancy-starved"
    return f"{achieved:.0f} GB/s = {pct:.0f}% of {peak:.0f} GB/s peak -- {verdict}"


def timeit(fn, iters: int = 50, warmup: int = 10) -> float:
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


def _dtype_name(dtype: torch.dtype) -> str:
    return str(dtype).split(".")[-1]


def bench_adaln(b, t, n, dtype, dev, peak, iters=50, warmup=10):
    mk = lambda *s: torch.randn(*s, device=dev, dtype=dtype, requires_grad=True)  # noqa: E731
    args = {"x": mk(b * t, n), "y": mk(b * t, n), "gate": mk(b, n), "weight": mk(n),
            "scale": mk(b, n), "shift": mk(b, n)}
    dh = torch.randn(b * t, n, device=dev, dtype=dtype)
    dout = torch.randn(b * t, n, device=dev, dtype=dtype)

    def run(fn):
        def inner():
            for v in args.values():
                v.grad = None
            h, o = fn(**args, tokens_per_sample=t)
            (h * dh + o * dout).sum().backward()
        return inner

    eager_ms = timeit(run(adaln_residual_rmsnorm_ref), iters, warmup)
    fused_ms = timeit(run(fused_adaln_residual_rmsnorm), iters, warmup)
    bw = bandwidth_gb_s(11 * b * t * n * dtype.itemsize, fused_ms)
    return {"shape": f"B{b}xT{t}xN{n}", "dtype": _dtype_name(dtype), "eager_ms": eager_ms,
            "fused_ms": fused_ms, "speedup": eager_ms / fused_ms, "achieved_gb_s": bw,
            "roofline": roofline_note(bw, peak)}


def bench_swiglu(m, n, dtype, dev, peak, iters=50, warmup=10):
    a = torch.randn(m, n, device=dev, dtype=dtype, requires_grad=True)
    b = torch.randn(m, n, device=dev, dtype=dtype, requires_grad=True)
    dout = torch.randn(m, n, device=dev, dtype=dtype)

    def run(fn):
        def inner():
            a.grad = b.grad = None
            fn(a, b).backward(dout)
        return inner

    eager_ms = timeit(run(swiglu_ref), iters, warmup)
    fused_ms = timeit(run(fused_swiglu), iters, warmup)
    bw = bandwidth_gb_s(8 * m * n * dtype.itemsize, fused_ms)
    return {"shape": f"{m}x{n}", "dtype": _dtype_name(dtype), "eager_ms": eager_ms,
            "fused_ms": fused_ms, "speedup": eager_ms / fused_ms, "achieved_gb_s": bw,
            "roofline": roofline_note(bw, peak)}


def bench_ce(m, h, v, dtype, dev, iters=10, warmup=3):
    """Judged on peak memory, as in the reference (bench_kernels.py:134-163)."""
    hid = torch.randn(m, h, device=dev, dtype=dtype, requires_grad=True)
    w = torch.randn(v, h, device=dev, dtype=dtype, requires_grad=True)
    tgt = torch.randint(0, v, (m,), device=dev)
    row = {"shape": f"M{m}xH{h}xV{v}", "dtype": _dtype_name(dtype)}
    for name, fn in (("naive", lambda: chunked_cross_entropy_ref(hid, w, tgt)),
                     ("chunked", lambda: chunked_cross_entropy(hid, w, tgt, chunk_size=1024))):
        hid.grad = w.grad = None
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats()
        try:
            row[f"{name}_ms"] = timeit(lambda: fn().backward(), iters, warmup)  # noqa: B023
            row[f"{name}_peak_mib"] = torch.cuda.max_memory_allocated() / 2**20
        except torch.cuda.OutOfMemoryError:
            row[f"{name}_ms"] = row[f"{name}_peak_mib"] = None
            row[f"{name}_oom"] = True
    if row.get("naive_peak_mib") and row.get("chunked_peak_mib"):
        row["memory_reduction"] = row["naive_peak_mib"] / row["chunked_peak_mib"]
    return row


def run_all(dtype=torch.bfloat16, peak=None, adaln=ADALN_SHAPES, swiglu=SWIGLU_SHAPES,
            ce=CE_SHAPES, iters=50, warmup=10, log=print):
    """Measure every shape list; returns the kernels.json report dict."""
    dev = torch.device("cuda", 0)
    arch = arch_name()
    peak = peak_bw_for(arch, peak)
    report = {"device": f"{torch.cuda.get_device_name(0)} ({arch})", "peak_bw_gb_s": peak,
              "dtype": _dtype_name(dtype), "adaln": [], "swiglu": [], "cross_entropy": []}
    for b, t, n in adaln:
        r = bench_adaln(b, t, n, dtype, dev, peak, iters, warmup)
        report["adaln"].append(r)
        log(f"  adaLN  {r['shape']:<16} eager {r['eager_ms']:.3f} ms | fused {r['fused_ms']:.3f} "
            f"ms | {r['speedup']:.2f}x | {r['roofline']}")
    for m, n in swiglu:
        r = bench_swiglu(m, n, dtype, dev, peak, iters, warmup)
        report["swiglu"].append(r)
        log(f"  SwiGLU {r['shape']:<16} eager {r['eager_ms']:.3f} ms | fused {r['fused_ms']:.3f} "
            f"ms | {r['speedup']:.2f}x | {r['roofline']}")
    for m, h, v in ce:
        r = bench_ce(m, h, v, dtype, dev, max(2, iters // 5), max(1, warmup // 3))
        report["cross_entropy"].append(r)
        log(f"  CE     {r['shape']:<16} naive {r.get('naive_peak_mib') or 0:.0f} MiB "
            f"{r.get('naive_ms') or 0:.3f} ms | chunked {r.get('chunked_peak_mib') or 0:.0f} MiB "
            f"{r.get('chunked_ms') or 0:.3f} ms")
    return report


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--out", default="reports/kernels.json")
    ap.add_argument("--peak-bw", type=float, default=None)
    ap.add_argument("--dtype", default="bfloat16", choices=["bfloat16", "float16", "float32"])
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("needs a GPU")
    report = run_all(getattr(torch, args.dtype), args.peak_bw)
    out = Path(args.out)
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text(json.dumps(report, indent=2))
    print(f"wrote {out}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
