"""Write reports/kernels.json for the reference's RESULTS.md renderer.

The reference renders its kernel tables from ``reports/kernels.json``
(``section_kernels``, nuvla_forge/bench/report.py:45-80).  This module writes
that file from an MI355X run of this build, so the same renderer puts these
numbers beside the reference's published H100 NVL tables.  What is shared
with the reference is only what the renderer and the comparison need: the
file's keys, the shapes of the reference's report, and its byte counts
(11 * M * N * e for the adaLN seam, 8 * M * N * e for SwiGLU; the reference's
bench_kernels.py:84,120), so the GB/s columns compare one to one.

Measurement (this build's own protocol):
  * a seam or SwiGLU case is one forward plus one autograd backward over fresh
    leaves with pre-drawn upstream gradients, nothing else in the step; the
    fused op and its eager formulation (``force_reference=True``) are both
    captured in a HIP graph and timed by replay (``timing.time_graph``), so
    neither side carries launch or Python costs the other does not;
  * a cross-entropy case records the peak device memory of loss + backward,
    fused (``chunk_size`` 1024) against the unchunked eager loss, each from a
    fresh allocator peak, and both step times (eager launches, events);
  * every bandwidth row also carries ``hbm_frac`` (GB/s over the peak).

    python -m nuvla_forge_amd.bench_kernels [--out reports/kernels.json]
        [--peak-bw GB_PER_S] [--dtype bfloat16|float16|float32] [--steps K]
"""

from __future__ import annotations

import argparse
import json
from pathlib import Path

import torch

from .kernels import chunked_cross_entropy, fused_adaln_residual_rmsnorm, fused_swiglu
from .kernels.reference import chunked_cross_entropy_ref
from .timing import time_eager, time_graph

# Shapes of the reference's report (bench_kernels.py:187,195,203), so each row
# has a published counterpart: adaLN (B, T, N), SwiGLU (M, N), CE (M, H, V).
ADALN_SHAPES = [(8, 32, 384), (8, 128, 384), (16, 256, 768), (8, 512, 1024), (4, 1024, 1536)]
SWIGLU_SHAPES = [(8192, 1536), (16384, 1536), (32768, 3072)]
CE_SHAPES = [(4096, 384, 32000), (8192, 384, 32000), (16384, 384, 32000)]

# HBM3E bandwidth of the parts this build targets, by gfx architecture (the
# runtime's marketing name can be generic, e.g. "AMD Radeon Graphics").
HBM_GB_S = {"gfx950": 8000.0}


def device_peak_gb_s(arch: str, override: float | None = None) -> float:
    """The peak the fractions are taken against: `override` if given, else
    the spec figure for `arch` (SystemExit for an architecture not listed)."""
    if override:
        return float(override)
    try:
        return HBM_GB_S[arch]
    except KeyError:
        raise SystemExit(f"{arch}: not an MI355X-class part; pass --peak-bw") from None


def gb_per_s(nbytes: int, ms: float) -> float:
    return nbytes / ms / 1e6


def _draw(gen: torch.Generator, dtype, dev):
    def draw(*shape, std=1.0, mean=0.0):
        return (torch.randn(*shape, generator=gen) * std + mean).to(dtype).to(dev)
    return draw


def _bandwidth_row(label, dtype, nbytes, make_for, peak, steps, warmup):
    """Time make_for(force_reference) -> step-factory for both formulations."""
    fused = time_graph(make_for(False), steps, warmup)[0]
    eager = time_graph(make_for(True), steps, warmup)[0]
    rate = gb_per_s(nbytes, fused)
    return {"shape": label, "dtype": str(dtype).removeprefix("torch."), "eager_ms": eager,
            "fused_ms": fused, "speedup": eager / fused, "achieved_gb_s": rate,
            "hbm_frac": rate / peak, "bytes": nbytes}


def seam_row(b, t, n, dtype, dev, peak, steps, warmup):
    draw = _draw(torch.Generator().manual_seed(b * 7 + t * 5 + n), dtype, dev)
    tensors = [draw(b * t, n), draw(b * t, n), draw(b, n, std=0.1),
               draw(n, std=0.02, mean=1.0), draw(b, n, std=0.1), draw(b, n, std=0.1)]
    upstream = [draw(b * t, n), draw(b * t, n)]

    def make_for(force):
        def make():
            leaves = [v.detach().requires_grad_(True) for v in tensors]

            def step():
                h, out = fused_adaln_residual_rmsnorm(*leaves, tokens_per_sample=t,
                                                      force_reference=force)
                return torch.autograd.grad([h, out], leaves, upstream)
            return step
        return make

    nbytes = 11 * b * t * n * tensors[0].element_size()
    return _bandwidth_row(f"B{b}xT{t}xN{n}", dtype, nbytes, make_for, peak, steps, warmup)


def swiglu_row(m, n, dtype, dev, peak, steps, warmup):
    draw = _draw(torch.Generator().manual_seed(m + n), dtype, dev)
    a, b, grad = draw(m, n), draw(m, n), draw(m, n)

    def make_for(force):
        def make():
            leaves = [a.detach().requires_grad_(True), b.detach().requires_grad_(True)]

            def step():
                out = fused_swiglu(*leaves, force_reference=force)
                return torch.autograd.grad(out, leaves, grad)
            return step
        return make

    nbytes = 8 * m * n * a.element_size()
    return _bandwidth_row(f"{m}x{n}", dtype, nbytes, make_for, peak, steps, warmup)


def ce_row(m, h, v, dtype, dev, steps, warmup):
    draw = _draw(torch.Generator().manual_seed(m + h + v), dtype, dev)
    hidden, weight = draw(m, h), draw(v, h, std=0.02)
    targets = torch.randint(0, v, (m,), generator=torch.Generator().manual_seed(v)).to(dev)

    def loss_and_grads(fn):
        lh, lw = hidden.detach().requires_grad_(True), weight.detach().requires_grad_(True)
        loss = fn(lh, lw)
        return (loss, *torch.autograd.grad(loss, [lh, lw]))

    fused = lambda lh, lw: chunked_cross_entropy(lh, lw, targets, chunk_size=1024)  # noqa: E731
    eager = lambda lh, lw: chunked_cross_entropy_ref(lh, lw, targets)  # noqa: E731

    def peak_mib(fn):
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats()
        out = loss_and_grads(fn)
        torch.cuda.synchronize()
        del out
        return torch.cuda.max_memory_allocated() / 2 ** 20

    row = {"shape": f"M{m}xH{h}xV{v}", "dtype": str(dtype).removeprefix("torch.")}
    row["chunked_peak_mib"] = peak_mib(fused)
    row["fused_ms"] = time_eager(lambda: loss_and_grads(fused), steps, warmup)
    try:
        row["naive_peak_mib"] = peak_mib(eager)
        row["eager_ms"] = time_eager(lambda: loss_and_grads(eager), steps, warmup)
        row["memory_reduction"] = row["naive_peak_mib"] / row["chunked_peak_mib"]
    except torch.cuda.OutOfMemoryError:
        torch.cuda.empty_cache()
        row["naive_oom"] = True
    return row


def run_all(dtype=torch.bfloat16, peak_override=None, adaln=ADALN_SHAPES,
            swiglu=SWIGLU_SHAPES, ce=CE_SHAPES, steps=50, warmup=10, log=print) -> dict:
    """The whole report as a dict in the schema bench/report.py reads."""
    dev = torch.device("cuda", 0)
    arch = torch.cuda.get_device_properties(dev).gcnArchName.split(":")[0]
    peak = device_peak_gb_s(arch, peak_override)
    report = {"device": f"{torch.cuda.get_device_name(dev)} ({arch})", "peak_bw_gb_s": peak,
              "dtype": str(dtype).removeprefix("torch."),
              "adaln": [], "swiglu": [], "cross_entropy": []}
    for b, t, n in adaln:
        report["adaln"].append(seam_row(b, t, n, dtype, dev, peak, steps, warmup))
        log(report["adaln"][-1])
    for m, n in swiglu:
        report["swiglu"].append(swiglu_row(m, n, dtype, dev, peak, steps, warmup))
        log(report["swiglu"][-1])
    for m, h, v in ce:
        report["cross_entropy"].append(ce_row(m, h, v, dtype, dev, max(3, steps // 5),
                                              max(1, warmup // 5)))
        log(report["cross_entropy"][-1])
    return report


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--out", default="reports/kernels.json")
    ap.add_argument("--peak-bw", type=float, default=None)
    ap.add_argument("--dtype", default="bfloat16", choices=["bfloat16", "float16", "float32"])
    ap.add_argument("--steps", type=int, default=50)
    args = ap.parse_args()
    if not torch.cuda.is_available():
        raise SystemExit("bench_kernels: no ROCm GPU visible")
    report = run_all(getattr(torch, args.dtype), args.peak_bw, steps=args.steps)
    out = Path(args.out)
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text(json.dumps(report, indent=2) + "\n")
    print(f"wrote {out}")


if __name__ == "__main__":
    main()
