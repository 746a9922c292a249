#!/usr/bin/env python3
"""Benchmark of the fused adaLN-RMSNorm / SwiGLU / chunked-CE path on one MI355X.

    python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--no-extra] [--no-cpu]

Prints ONE JSON line (the driver's contract).  The headline workload is
fused_adaln_residual_rmsnorm forward + backward in bf16 at
the DiT-block shape B=8, T=1024, N=1024 (synthetic N(0,1) activations, N(0,0.1)
conditioning, weight 1+N(0,0.02)).  A "step" is one forward plus one autograd
backward through the drop-in Function, all inputs resident in HBM.

Timing:
  * value / ms_per_step: K steps as K/10 replays of a HIP graph holding 10
    consecutive steps (fresh leaves; warmup and capture on one side stream),
    bracketed by events + synchronize -- one graph launch per 10 steps, as a
    training loop's graph amortises it; the one-step-per-graph time is
    reported beside it;
    value = algorithmic bytes (10*M*N + 6*B*N + 2*N) * 2 / ms_per_step.
    The graph's outputs are compared bitwise with an eager step.
  * roofline: the dominant kernel (the backward row kernel, nf_adaln_bwd) on
    the step's inputs: 20 back-to-back launches captured in a HIP graph,
    replayed K times between two events on its launch stream; achieved = its
    algorithmic bytes (6*M*N + 2*B*N + N) * 2 per launch / mean launch time;
    peak = 8 TB/s HBM.
  * cpu_baseline: oracle/torch_cpu.py (the reference's eager PyTorch path,
    forward + autograd backward) on the host cores for the same workload.
  * extra: SwiGLU bf16 [8192, 4096], chunked CE bf16 M4096 D2048
    V32000 with 409 ignored rows (configs[3], tokens/s and MFMA fraction of
    2.5 PFLOP/s on 6*M_valid*V*D), the cfg5 stress chain, their CPU baselines;
    the two callers at the reference's model shape: the DiT seam (B8 T6 N384,
    autocast dtypes, chunk(6) views) and the reasoning-head CE (M512 D384
    V32000, bf16 hidden, fp32 lm_head), each beside its eager formulation;
    SwiGLU in the gate/up GEMM epilogue at the encoder MLP shape;
    nf_mfma_probe's MFMA rate with no memory traffic (random and zero bf16
    operands, with the shader clock), the CE's rate as a fraction of it.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
STEPS_PER_GRAPH = 10            # consecutive steps captured in one HIP graph
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-extra", action="store_true", help="headline workload only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--only", choices=("swiglu", "ce", "stress", "traffic", "dit", "head",
                                       "gateup", "copy", "adaln", "adaln_cold", "ce_gemm_ceiling",
                                       "mfma", "mainloop"),
                    default=None,
                    help="run one secondary workload alone (for profiling) and print its "
                         "record instead of the headline line")
    ap.add_argument("--json-out", default=None, help="also write the JSON record here")
    return ap.parse_args()


# ---------------------------------------------------------------------------
# timing helpers
# ---------------------------------------------------------------------------
def _timing():
    """nuvla_forge_amd.timing, imported on first use (after the --gpus check)."""
    from nuvla_forge_amd import timing

    return timing


def _sync():
    _timing().sync()


def time_eager(step, steps: int, warmup: int) -> float:
    return _timing().time_eager(step, steps, warmup)


def time_graph(make_step, steps: int, warmup: int, per_graph: int = 1):
    return _timing().time_graph(make_step, steps, warmup, per_graph)


def per_launch_ms(launch, steps: int, reps: int = 20) -> float:
    return _timing().per_launch_ms(launch, steps, reps)


def same(a, b) -> bool:
    import torch

    return all(torch.equal(x, y) for x, y in zip(a, b))


def cpu_threads() -> int:
    # the GPU box's CPU share is 16 cores per GPU, whatever the affinity mask says
    return max(1, min(16, len(os.sched_getaffinity(0))))


def time_cpu(fn, budget_s: float = 20.0, min_reps: int = 1, max_reps: int = 3) -> float:
    """1 warmup, then up to max_reps timed reps within budget; median seconds."""
    t0 = time.perf_counter()
    fn()
    first = time.perf_counter() - t0
    reps = []
    while len(reps) < max_reps and (len(reps) < min_reps or sum(reps) + first < budget_s):
        t0 = time.perf_counter()
        fn()
        reps.append(time.perf_counter() - t0)
    return statistics.median(reps)


# ---------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------
def adaln_inputs(b, t, n, dev, seed=0):
    import torch

    g = torch.Generator().manual_seed(seed)
    bf = torch.bfloat16

    def r(*shape, std=1.0, mean=0.0):
        return (torch.randn(*shape, generator=g) * std + mean).to(bf).to(dev)

    inp = {"x": r(b * t, n), "y": r(b * t, n), "gate": r(b, n, std=0.1),
           "weight": r(n, std=0.02, mean=1.0), "scale": r(b, n, std=0.1),
           "shift": r(b, n, std=0.1)}
    g1 = torch.Generator().manual_seed(seed + 1)
    dh = torch.randn(b * t, n, generator=g1).to(bf).to(dev)
    dout = torch.randn(b * t, n, generator=g1).to(bf).to(dev)
    return inp, dh, dout


def adaln_step_fn(inp, t, dh, dout):
    """A fwd + autograd-bwd step over fresh leaves sharing `inp`'s storage."""
    import torch

    from nuvla_forge_amd.kernels import fused_adaln_residual_rmsnorm

    leaves = [v.detach().requires_grad_(True) for v in inp.values()]

    def step():
        h, out = fused_adaln_residual_rmsnorm(*leaves, tokens_per_sample=t)
        grads = torch.autograd.grad([h, out], leaves, [dh, dout])
        return (h, out, *grads)

    return step


def adaln_alg_bytes(b, t, n, e=2):
    m = b * t
    return (10 * m * n + 6 * b * n + 2 * n) * e


def adaln_launchers(inp, t, dh, dout):
    """Closures that launch nf_adaln_fwd / nf_adaln_bwd / nf_adaln_bwd_reduce
    directly through the C ABI on the step's own inputs."""
    import torch

    from nuvla_forge_amd import _lib

    L, dc = _lib.lib(), _lib.dtype_code
    x, y, gate, w, scale, shift = (inp[k] for k in ("x", "y", "gate", "weight", "scale", "shift"))
    m, n = x.shape
    b = m // t
    h, out, dx, dy = (torch.empty_like(x) for _ in range(4))
    rstd = torch.empty(m, dtype=torch.float32, device=x.device)
    dgate, dscale, dshift = (torch.empty_like(gate) for _ in range(3))
    dweight = torch.empty_like(w)
    ws_bytes = L.nf_adaln_bwd_workspace(m, n, t)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)

    def fwd():
        _lib.check(L.nf_adaln_fwd(
            x.data_ptr(), n, y.data_ptr(), n, gate.data_ptr(), n, w.data_ptr(), scale.data_ptr(),
            n, shift.data_ptr(), n, h.data_ptr(), out.data_ptr(), rstd.data_ptr(), m, n, t, 1e-6,
            dc(x), dc(y), dc(gate), dc(w), dc(scale), dc(shift), _lib.stream_of(x)), "fwd")

    def bwd():
        _lib.check(L.nf_adaln_bwd(
            dh.data_ptr(), dout.data_ptr(), x.data_ptr(), n, y.data_ptr(), n, gate.data_ptr(), n,
            w.data_ptr(), scale.data_ptr(), n, rstd.data_ptr(), dx.data_ptr(), dy.data_ptr(),
            ws.data_ptr(), ws_bytes, m, n, t, dc(x), dc(y), dc(gate), dc(w), dc(scale),
            _lib.stream_of(x)), "bwd")

    def red():
        _lib.check(L.nf_adaln_bwd_reduce(
            ws.data_ptr(), ws_bytes, w.data_ptr(), scale.data_ptr(), n, dgate.data_ptr(),
            dweight.data_ptr(), dscale.data_ptr(), dshift.data_ptr(), m, n, t, dc(gate), dc(w),
            dc(scale), dc(shift), _lib.stream_of(x)), "reduce")

    assert b * t == m
    return fwd, bwd, red


def adaln_kernel_ms(inp, t, dh, dout, steps):
    """Per-launch time of nf_adaln_fwd / nf_adaln_bwd / nf_adaln_bwd_reduce on
    the step's own inputs."""
    fwd, bwd, red = adaln_launchers(inp, t, dh, dout)
    fwd()
    bwd()
    _sync()
    return {"nf_adaln_fwd": per_launch_ms(fwd, steps), "nf_adaln_bwd": per_launch_ms(bwd, steps),
            "nf_adaln_bwd_reduce": per_launch_ms(red, steps)}


TRAFFIC_FILE = "profiles/adaln_cfg2_pmc_traffic.json"


def pmc_traffic(kernel):
    """HBM bytes per launch of an adaLN kernel at cfg2, from the committed
    summary of the two rocprofv3 PMC passes (FETCH_SIZE, WRITE_SIZE) over
    `bench.py --only traffic`, each scaled by the counter's reading for a
    plain copy of known size; None when the summary is absent."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), TRAFFIC_FILE)
    try:
        with open(path) as f:
            return round(json.load(f)["kernels"][kernel]["traffic_bytes"])
    except (OSError, KeyError, ValueError):
        return None


COPY_BYTES = 64 << 20  # the reference copy of the traffic run: 64 MiB read + 64 MiB written


def bench_traffic(args, dev):
    """Workload for the PMC runs (rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE):
    a plain device copy of COPY_BYTES (torch's copy kernel), whose counters give
    the scale between counter and bytes, then the three adaLN kernels at cfg2,
    five launches each, eager."""
    import torch

    src = torch.randn(COPY_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    _sync()
    b, t, n = 8, 1024, 1024
    inp, dh, dout = adaln_inputs(b, t, n, dev)
    fwd, bwd, red = adaln_launchers(inp, t, dh, dout)
    for f in (fwd, bwd, red):
        for _ in range(5):
            f()
    _sync()
    return {"copy_bytes_each_way": COPY_BYTES, "launches": 5,
            "adaln_fwd_alg_bytes": (4 * b * t * n + 3 * b * n + n) * 2,
            "adaln_bwd_alg_bytes": (6 * b * t * n + 2 * b * n + n) * 2}


def bench_adaln(args, dev):
    b, t, n = 8, 1024, 1024
    m = b * t
    inp, dh, dout = adaln_inputs(b, t, n, dev)
    make = lambda: adaln_step_fn(inp, t, dh, dout)  # noqa: E731
    eager_step = make()
    eager_ms = time_eager(eager_step, args.steps, args.warmup)
    ref = [x.clone() for x in eager_step()]
    graph_ms, outs, graph = time_graph(make, args.steps, args.warmup, STEPS_PER_GRAPH)
    graph_ok = same(ref, outs)
    graph.replay()
    _sync()
    graph_ok = graph_ok and same(ref, outs)
    del graph, outs
    graph1_ms, _, graph1 = time_graph(make, args.steps, args.warmup, 1)
    cold_1r_ms = cold_replay_ms(graph1, dev, max(5, args.steps // 2))
    cold_dirty_ms = cold_replay_ms(graph1, dev, max(5, args.steps // 2), dirty=True)
    del graph1
    floor_ms = single_replay_floor_ms(dev, max(5, args.steps // 2))
    cold_ms, flush_ms = cold_graph_ms(make, dev)

    # per-kernel durations: back-to-back launches of each C-ABI entry point
    kern_ms = adaln_kernel_ms(inp, t, dh, dout, args.steps)
    instep_ms = adaln_in_step_ms(inp, t, dh, dout, args.steps)
    # the streaming probe on the same bytes, same box, same run: forward
    # 2 reads + 2 writes, backward 4 + 2 of [8192, 1024] bf16 arrays
    probe = stream_ceilings(args, dev, (("cfg2", m * n * 2),))

    alg = adaln_alg_bytes(b, t, n)
    bwd_alg = (6 * m * n + 2 * b * n + n) * 2
    fwd_alg = (4 * m * n + 3 * b * n + n) * 2
    bwd_gbs = bwd_alg / (kern_ms["nf_adaln_bwd"] * 1e-3) / 1e9
    fwd_gbs = fwd_alg / (kern_ms["nf_adaln_fwd"] * 1e-3) / 1e9
    return {
        "b": b, "t": t, "n": n, "alg_bytes": alg, "graph_ms": graph_ms, "eager_ms": eager_ms,
        "graph1_ms": graph1_ms, "cold_ms": cold_ms, "cold_1r_ms": cold_1r_ms,
        "cold_dirty_ms": cold_dirty_ms, "single_replay_floor_ms": floor_ms, "flush_ms": flush_ms,
        "graph_matches_eager": graph_ok, "kernel_ms": kern_ms, "in_step_ms": instep_ms,
        "bwd_alg_bytes": bwd_alg, "bwd_gbs": bwd_gbs, "fwd_alg_bytes": fwd_alg, "fwd_gbs": fwd_gbs,
        "bwd_gbs_in_step": bwd_alg / (instep_ms["nf_adaln_bwd"] * 1e-3) / 1e9,
        "gbs": alg / (graph_ms * 1e-3) / 1e9, "gbs_eager": alg / (eager_ms * 1e-3) / 1e9,
        "ref_style_gbs_11MNe": 11 * m * n * 2 / (graph_ms * 1e-3) / 1e9,
        "stream_probe": probe,
    }


def bench_ce_gemm_ceiling(args, dev):
    """The vendor GEMM library on the products of the CE at cfg4 (bf16 in,
    fp32 accumulate; torch.mm -> hipBLASLt), for context: the logits
    S = H_valid W^T ([3687, 2048] x [2048, 32000]), dH = P W ([3687, 32000] x
    [32000, 2048]) and dW = P^T H_valid ([32000, 3687] x [3687, 2048]) --
    6 M_valid V D flops in all, each timed as 20 back-to-back launches in a
    HIP graph, with fp32 outputs as this build's fp32 accumulators where the
    product is accumulated, bf16 where it is final; beside them 8192^3 on
    the library and this build's GEMM core (nf_gemm_nt, fp32 C) on the
    logits product and on 8192^3."""
    import torch

    g = torch.Generator().manual_seed(50)
    mv, d, v = 3687, 2048, 32000
    h = torch.randn(mv, d, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(v, d, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    p = (torch.randn(mv, v, generator=g) * 1e-4).to(torch.bfloat16).to(dev)
    pt = p.t().contiguous()
    out = {}
    cases = {"logits_S": (lambda: torch.mm(h, w.t()), 2 * mv * v * d),
             "dH": (lambda: torch.mm(p, w), 2 * mv * v * d),
             "dW": (lambda: torch.mm(pt, h), 2 * mv * v * d)}
    total = 0.0
    for name, (fn, flops) in cases.items():
        ms = per_launch_ms(fn, max(5, args.steps // 5))
        total += ms
        out[name] = {"us": ms * 1e3, "tflops": flops / (ms * 1e-3) / 1e12}
    out["sum_us"] = total * 1e3
    out["tflops_6MvVD"] = 6 * mv * v * d / (total * 1e-3) / 1e12
    # this build's GEMM core on the logits product and on 8192^3, beside the
    # library (the core stores fp32 C: twice the library's bf16 output bytes)
    from nuvla_forge_amd import _lib, _measure

    L = _measure.lib()
    sq = torch.randn(8192, 8192, generator=g).to(torch.bfloat16).to(dev)
    sq2 = torch.randn(8192, 8192, generator=g).to(torch.bfloat16).to(dev)
    core = {}
    for name, (a_, b_, flops) in {"logits_S": (h, w, 2 * mv * v * d),
                                  "square_8192": (sq, sq2, 2 * 8192 ** 3)}.items():
        m_, k_ = a_.shape
        n_ = b_.shape[0]
        c32 = torch.empty(m_, n_, device=dev)

        def launch(a_=a_, b_=b_, c32=c32, m_=m_, n_=n_, k_=k_):
            _lib.check(L.nf_gemm_nt(a_.data_ptr(), k_, b_.data_ptr(), k_, c32.data_ptr(), n_,
                                    m_, n_, k_, _lib.dtype_code(torch.bfloat16),
                                    _lib.stream_of(c32)), "nf_gemm_nt")

        ms = per_launch_ms(launch, max(5, args.steps // 5))
        core[name] = {"us": ms * 1e3, "tflops": flops / (ms * 1e-3) / 1e12}
        del c32
    ms = per_launch_ms(lambda: torch.mm(sq, sq2.t()), max(5, args.steps // 5))
    out["square_8192"] = {"us": ms * 1e3, "tflops": 2 * 8192 ** 3 / (ms * 1e-3) / 1e12}
    out["this_build_fp32_out"] = core
    return out


def bench_mfma_ceiling(args, dev, blocks=2048, iters=300):
    """`nf_mfma_probe` for context (never the roofline denominator): bf16
    MFMAs on operands held in registers, with no memory access in the loop --
    2048 blocks of 256 threads (one block per CU at a time: a block holds the
    register file of its CU's four SIMDs), each 300 rounds of 1 MFLOP per
    wavefront -- timed as 20 back-to-back launches in a HIP graph, on random
    N(0,1) bf16 operands and on zeros; v_mfma_f32_16x16x32 (the GEMM core's
    form) at the top level, v_mfma_f32_32x32x16 under `form_32x32x16`.  The
    shader clock comes from the stamps of the graph's last launch (shader
    cycles over the 100 MHz real-time counter, summed over blocks).  On
    random data the chip's power limit lowers the clock (a real product's
    operands toggle the multipliers; zeros do not), so the random-operand
    rate is the most a bf16 product of this build's data can reach."""
    import torch

    from nuvla_forge_amd import _lib, _measure

    L = _measure.lib()
    g = torch.Generator().manual_seed(60)
    ops = torch.randn(16, 256, 8, generator=g).to(torch.bfloat16).to(dev)
    out = torch.empty(blocks, 256, device=dev)
    stamps = torch.zeros(blocks, 4, dtype=torch.int64, device=dev)
    flops = blocks * 4 * iters * 64 * (2 * 16 * 16 * 32)  # = 32 * (2 * 32 * 32 * 16) per round
    res = {"blocks": blocks, "iters": iters, "flops_per_launch": flops,
           "form": "v_mfma_f32_16x16x32_bf16", "form_32x32x16": {}}
    for form, dst in ((0, res), (1, res["form_32x32x16"])):
        for name, ptr in (("random", ops.data_ptr()), ("zero", None)):
            def launch(ptr=ptr, form=form):
                _lib.check(L.nf_mfma_probe(ptr, iters, blocks, form, out.data_ptr(),
                                           stamps.data_ptr(), _lib.stream_of(out)),
                           "nf_mfma_probe")

            ms = per_launch_ms(launch, max(5, args.steps // 5))
            st = stamps.cpu().double()
            ghz = float((st[:, 1] - st[:, 0]).sum() / ((st[:, 3] - st[:, 2]).sum() / 100e6) / 1e9)
            tflops = flops / (ms * 1e-3) / 1e12
            dst[name] = {"us": ms * 1e3, "tflops": tflops,
                         "frac_of_spec": tflops / MFMA_BF16_PEAK_TFLOPS, "clock_ghz": ghz}
    return res


def bench_mainloop_probe(args, dev, blocks=2048, iters=300):
    """`nf_mainloop_probe` for context (never the roofline denominator): the
    GEMM core's mainloop instruction mix one ingredient at a time -- two
    wavefronts per SIMD, 128 accumulators each, 64 v_mfma_f32_16x16x32 per
    iteration on random bf16 operands; mode 1 registers only, 2 + the LDS
    operand reads, 3 + the direct-to-LDS copies (L2-resident source), 4 +
    the per-iteration barrier, 5 the copies over a 64 MiB footprint shared
    by the blocks of one XCD -- each timed as 20 back-to-back launches in a
    HIP graph, with the shader clock from the last launch's stamps.  Under
    the power limit each ingredient also lowers the clock."""
    import torch

    from nuvla_forge_amd import _lib, _measure

    L = _measure.lib()
    g = torch.Generator().manual_seed(61)
    ops = torch.randn(12, 512, 8, generator=g).to(torch.bfloat16).to(dev)
    src_bytes = 64 << 20
    src = torch.randn(src_bytes // 2, generator=g).to(torch.bfloat16).to(dev)
    out = torch.empty(blocks, 512, device=dev)
    stamps = torch.zeros(blocks, 4, dtype=torch.int64, device=dev)
    flops = blocks * 8 * iters * 64 * (2 * 16 * 16 * 32)
    names = {1: "registers", 2: "lds_reads", 3: "lds_reads_copies_l2", 4: "lds_reads_copies_barrier",
             5: "copies_64MiB_shared_streams"}
    res = {"blocks": blocks, "iters": iters, "flops_per_launch": flops}
    for mode, name in names.items():
        def launch(mode=mode):
            _lib.check(L.nf_mainloop_probe(mode, ops.data_ptr(), src.data_ptr(), src_bytes, iters,
                                           blocks, out.data_ptr(), stamps.data_ptr(),
                                           _lib.stream_of(out)), "nf_mainloop_probe")

        ms = per_launch_ms(launch, max(5, args.steps // 5))
        st = stamps.cpu().double()
        ghz = float((st[:, 1] - st[:, 0]).sum() / ((st[:, 3] - st[:, 2]).sum() / 100e6) / 1e9)
        tflops = flops / (ms * 1e-3) / 1e12
        # MFMA busy fraction at that clock: 1024 flops per SIMD per cycle
        busy = tflops * 1e12 / (1024 * 4 * 256 * ghz * 1e9)
        res[f"mode{mode}_{name}"] = {"us": ms * 1e3, "tflops": tflops,
                                     "frac_of_spec": tflops / MFMA_BF16_PEAK_TFLOPS,
                                     "clock_ghz": ghz, "mfma_busy_at_clock": busy}
    return res


def bench_copy(args, dev):
    """Streaming ceilings for context (never the roofline denominator): torch's
    own element-wise kernels -- copy (1 read + 1 write), add (2 + 1),
    addcmul (3 + 1) -- on bf16 tensors of the cfg2 activation size (16 MiB,
    [8192, 1024]: the working set stays in the 256 MB Infinity Cache) and of
    1 GiB ([32768, 16384]: beyond it), each as the mean of 20 back-to-back
    launches in a HIP graph."""
    import torch

    out = {}
    for label, shape in (("cfg2_16MiB", (8192, 1024)), ("beyond_cache_1GiB", (32768, 16384))):
        a, b, c, d = (torch.randn(*shape, device=dev).to(torch.bfloat16) for _ in range(4))
        nb = a.numel() * a.element_size()
        cases = {"copy_1r1w": (lambda: d.copy_(a), 2 * nb),
                 "add_2r1w": (lambda: torch.add(a, b, out=d), 3 * nb),
                 "addcmul_3r1w": (lambda: torch.addcmul(a, b, c, out=d), 4 * nb)}
        out[label] = {}
        for name, (fn, nbytes) in cases.items():
            ms = per_launch_ms(fn, max(5, args.steps // 5))
            out[label][name] = {"us": ms * 1e3, "gbs": nbytes / (ms * 1e-3) / 1e9,
                                "frac_of_8tbs": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
        del a, b, c, d
    out["stream_probe"] = stream_ceilings(args, dev)
    return out


def stream_ceilings(args, dev, sizes=(("cfg2_16MiB", 16 << 20), ("cfg5_256MiB", 256 << 20))):
    """`nf_stream_probe` (a grid-stride streaming kernel with no dependency
    between its accesses, non-temporal stores) on the adaLN step's traffic
    shapes -- forward 2 reads + 2 writes, backward 4 reads + 2 writes -- with
    arrays of the cfg2 activation size (16 MiB) and of the cfg5 adaLN size
    (256 MiB): microseconds per launch back to back on one set of arrays
    (`same`: inputs partly warm in the L2s) and alternating between two sets
    (`alt`: each launch finds the other set's data in the L2s, the cache state
    the row kernels meet inside a step).  Context, never the denominator."""
    import torch

    from nuvla_forge_amd import _lib, _measure

    L = _measure.lib()
    out = {}
    for label, nbytes in sizes:
        for r, w in ((2, 2), (4, 2)):
            sets = [[torch.empty(nbytes, dtype=torch.uint8, device=dev) for _ in range(r + w)]
                    for _ in range(2)]
            for t in sets[0] + sets[1]:
                t.random_(0, 256)

            def launch(k):
                ins, outs = sets[k][:r], sets[k][r:]
                ptrs = [t.data_ptr() for t in ins] + [None] * (4 - r)
                ptrs += [t.data_ptr() for t in outs] + [None] * (2 - w)
                _lib.check(L.nf_stream_probe(r, w, *ptrs, nbytes // 16, _lib.stream_of(ins[0])),
                           "nf_stream_probe")

            steps = max(5, args.steps // 5)
            same = per_launch_ms(lambda: launch(0), steps)
            alt = per_launch_ms(lambda: (launch(0), launch(1)), steps, 10) / 2
            moved = (r + w) * nbytes
            out[f"{label}_{r}r{w}w"] = {
                "bytes": moved, "same_us": same * 1e3, "same_gbs": moved / (same * 1e-3) / 1e9,
                "alt_us": alt * 1e3, "alt_gbs": moved / (alt * 1e-3) / 1e9}
            del sets
    return out


def cold_replay_ms(graph, dev, reps, dirty=False, flush_bytes=1 << 30):
    """Milliseconds per replay of a one-step graph with the caches cold: before
    each replay a read pass over `flush_bytes` (4x the 256 MB Infinity Cache)
    evicts the step's operands from the L2s and the Infinity Cache, so they
    come from HBM (with `dirty`, a read-modify-write pass, whose dirty lines
    the step then has to write back as well); only the replay lies between
    the events."""
    import torch

    flush = torch.ones(flush_bytes // 4, dtype=torch.int32, device=dev)
    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(reps)]
    for e0, e1 in pairs:
        if dirty:
            flush.add_(1)
        else:
            flush.sum(dtype=torch.int64)
        e0.record()
        graph.replay()
        e1.record()
    _sync()
    del flush
    return statistics.median(e0.elapsed_time(e1) for e0, e1 in pairs)


def cold_graph_ms(make_step, dev, per_graph=5, replays=6, flush_bytes=1 << 30):
    """Milliseconds per step with the caches cold, timed inside HIP graphs:
    one graph holds `per_graph` x [a read-only pass over `flush_bytes` (4x the
    256 MB Infinity Cache; nf_stream_probe's (1, 0) form), one step], a
    second graph the same passes alone, and the difference per step is the
    step after its operands left the L2s and the Infinity Cache.  Unlike
    events around a one-step replay (cold_replay_ms) it carries no per-replay
    launch or event cost; the step's own launches are in it, as in the
    headline."""
    import torch

    from nuvla_forge_amd import _lib, _measure

    M = _measure.lib()
    buf = torch.ones(flush_bytes // 4, dtype=torch.int32, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)

    def flush():
        _lib.check(M.nf_stream_probe(1, 0, buf.data_ptr(), None, None, None, sink.data_ptr(),
                                     None, flush_bytes // 16, _lib.stream_of(buf)),
                   "nf_stream_probe")

    def make_with():
        step = make_step()

        def run():
            flush()
            return step()
        return run

    total = per_graph * replays
    with_ms, _, g1 = time_graph(make_with, total, 2, per_graph)
    del g1
    flush_ms, _, g2 = time_graph(lambda: flush, total, 2, per_graph)
    del g2, buf
    return with_ms - flush_ms, flush_ms


def bench_adaln_cold(args, dev):
    """The adaLN cfg2 kernels one by one with their operands in HBM (the
    per-kernel view of `config.cold_ms_per_step`): cold_graph_ms of each C
    call, of the backward with its reduction, of the three, and of the
    streaming probe moving the forward's and the backward's arrays (2 reads +
    2 writes, 4 + 2, no dependency between accesses); beside each, the warm
    time of 10 back-to-back launches in one graph.  Microseconds."""
    import torch

    from nuvla_forge_amd import _lib, _measure

    b, t, n = 8, 1024, 1024
    inp, dh, dout = adaln_inputs(b, t, n, dev)
    fwd, bwd, red = adaln_launchers(inp, t, dh, dout)
    M = _measure.lib()
    x, y = inp["x"], inp["y"]
    h, o, dx, dy = (torch.empty_like(x) for _ in range(4))
    n16 = x.numel() * x.element_size() // 16

    def probe(reads, writes, ins, outs):
        ptrs = [a.data_ptr() for a in ins] + [None] * (4 - len(ins))
        optr = [a.data_ptr() for a in outs] + [None] * (2 - len(outs))
        _lib.check(M.nf_stream_probe(reads, writes, *ptrs, *optr, n16, _lib.stream_of(x)),
                   "nf_stream_probe")

    cases = {"nf_adaln_fwd": [fwd], "nf_adaln_bwd": [bwd], "nf_adaln_bwd_reduce": [red],
             "bwd_and_reduce": [bwd, red], "step_kernels": [fwd, bwd, red],
             "probe_2r2w_fwd_arrays": [lambda: probe(2, 2, [x, y], [h, o])],
             "probe_4r2w_bwd_arrays": [lambda: probe(4, 2, [x, y, dh, dout], [dx, dy])]}
    out = {}
    for name, fns in cases.items():
        def make(fns=fns):
            def run():
                for f in fns:
                    f()
            return run

        cold_ms, flush_ms = cold_graph_ms(make, dev)
        warm = per_launch_ms(make(), max(5, args.steps // 5), 10)
        out[name] = {"cold_us": cold_ms * 1e3, "warm_us": warm * 1e3}
    out["read_pass_1gib_us"] = flush_ms * 1e3
    return out


def single_replay_floor_ms(dev, reps):
    """What cold_replay_ms reads for a one-kernel graph that moves nothing (a
    64-element fill): the method's own cost of events around one replay."""
    import torch

    tiny = torch.zeros(64, device=dev)
    _, _, graph = time_graph(lambda: (lambda: tiny.fill_(1.0)), 2, 2, 1)
    ms = cold_replay_ms(graph, dev, reps)
    del graph
    return ms


def adaln_in_step_ms(inp, t, dh, dout, steps, reps=10):
    """Each adaLN kernel's share of the step as it runs inside the step:
    `reps` repetitions of forward -> backward -> reduction launched through
    the C ABI in one HIP graph, minus the same graph with that one launch
    left out (the others' inputs and outputs are unchanged, so their cache
    state is the step's).  Milliseconds per launch; 'sequence' is the whole
    three-launch sequence."""
    fwd, bwd, red = adaln_launchers(inp, t, dh, dout)
    seq = {"nf_adaln_fwd": fwd, "nf_adaln_bwd": bwd, "nf_adaln_bwd_reduce": red}

    def timed(names):
        def launch():
            for k in names:
                seq[k]()
        return per_launch_ms(launch, steps, reps)

    full = timed(list(seq))
    out = {k: full - timed([j for j in seq if j != k]) for k in seq}
    out["sequence"] = full
    return out


def bench_swiglu(args, dev, m=8192, h=4096):
    import torch

    from nuvla_forge_amd.kernels import fused_swiglu

    g = torch.Generator().manual_seed(10)
    a, b, dout = (torch.randn(m, h, generator=g).to(torch.bfloat16).to(dev) for _ in range(3))

    def make():
        la, lb = a.detach().requires_grad_(True), b.detach().requires_grad_(True)

        def step():
            out = fused_swiglu(la, lb)
            return (out, *torch.autograd.grad(out, [la, lb], dout))

        return step

    eager_step = make()
    eager_ms = time_eager(eager_step, args.steps, args.warmup)
    ref = [x.clone() for x in eager_step()]
    ms, outs, _ = time_graph(make, args.steps, args.warmup, STEPS_PER_GRAPH)
    alg = 8 * m * h * 2
    return {"m": m, "h": h, "alg_bytes": alg, "graph_ms": ms, "eager_ms": eager_ms,
            "graph_matches_eager": same(ref, outs), "gbs": alg / (ms * 1e-3) / 1e9,
            "hbm_frac": alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}


def ce_inputs(dev, m=4096, d=2048, v=32000, n_ignore=409):
    import torch

    g = torch.Generator().manual_seed(20)
    hid = torch.randn(m, d, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(v, d, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    tgt = torch.randint(0, v, (m,), generator=g)
    tgt[torch.randperm(m, generator=g)[:n_ignore]] = -100
    return hid, w, tgt.to(dev)


def ce_call_times(hid, w, tgt, chunk, steps):
    """nf_ce_fwd and nf_ce_bwd apart, through the C ABI: a HIP graph of 5
    (forward, backward) pairs and one of 5 forwards, each replayed `steps`
    times; the forward's time is the second's, the backward's the
    difference, so the two add up to the pair.  The forward holds the logits
    GEMM with its statistics and E store (and the small compaction, gather,
    lse and scaling kernels), the backward the gradient GEMM launch (dW and
    dH) and the dH scatter."""
    import torch

    from nuvla_forge_amd import _lib

    L = _lib.lib()
    m, d = hid.shape
    v = w.shape[0]
    code = _lib.dtype_code(torch.bfloat16)
    shape = (m, d, v, chunk, code)
    sb, fw, bw = L.nf_ce_state_bytes(*shape), L.nf_ce_fwd_workspace(*shape), L.nf_ce_bwd_workspace(*shape)
    state = torch.empty(sb, dtype=torch.uint8, device=hid.device)
    wsf = torch.empty(fw, dtype=torch.uint8, device=hid.device)
    wsb = torch.empty(bw, dtype=torch.uint8, device=hid.device)
    loss = torch.empty((), device=hid.device)
    g = torch.ones((), device=hid.device)
    dh, dw = torch.empty_like(hid), torch.empty_like(w)

    def fwd():
        _lib.check(L.nf_ce_fwd(hid.data_ptr(), w.data_ptr(), tgt.data_ptr(), m, d, v, -100, chunk,
                               code, loss.data_ptr(), None, state.data_ptr(), sb, wsf.data_ptr(),
                               fw, _lib.stream_of(hid)), "nf_ce_fwd")

    def bwd():
        _lib.check(L.nf_ce_bwd(m, d, v, chunk, code, state.data_ptr(), sb, g.data_ptr(),
                               dh.data_ptr(), code, dw.data_ptr(), code, wsb.data_ptr(), bw,
                               _lib.stream_of(hid)), "nf_ce_bwd")

    def pair():
        fwd()
        bwd()

    fwd()
    torch.cuda.synchronize()
    both = per_launch_ms(pair, steps, reps=5)
    f = per_launch_ms(fwd, steps, reps=5)
    return f, both - f


def bench_ce(args, dev):
    import torch

    from nuvla_forge_amd.kernels import chunked_cross_entropy

    m, d, v = 4096, 2048, 32000
    hid, w, tgt = ce_inputs(dev, m, d, v)
    m_valid = int((tgt != -100).sum())
    flops = 6 * m_valid * v * d
    # eager steps only feed the graph-vs-eager check; the graph is replayed
    # `args.steps` times, long enough (~75 ms) for the clock to settle at its
    # sustained level: 10 replays read 1.59-1.65 ms per step where 50, 200
    # and 500 read 1.505-1.510 ms on the same box
    steps = max(5, args.steps // 5)

    def run(chunk, weight=w):
        def make():
            lh, lw = hid.detach().requires_grad_(True), weight.detach().requires_grad_(True)

            def step():
                loss = chunked_cross_entropy(lh, lw, tgt, chunk_size=chunk)
                return (loss, *torch.autograd.grad(loss, [lh, lw]))

            return step

        eager_step = make()
        eager_ms = time_eager(eager_step, steps, max(2, args.warmup // 5))
        ref = [x.clone() for x in eager_step()]
        ms, outs, _ = time_graph(make, max(steps, args.steps), max(2, args.warmup))
        tflops = flops / (ms * 1e-3) / 1e12
        return {"chunk_size": chunk, "graph_ms": ms, "eager_ms": eager_ms,
                "graph_matches_eager": same(ref, outs), "tokens_per_s": m / (ms * 1e-3),
                "tflops": tflops, "mfma_frac": tflops / MFMA_BF16_PEAK_TFLOPS}

    # The figure of record is the reference's default chunk_size 1024
    # (chunked_ce.py:189).  chunk_size bounds E and the dW accumulator by the
    # bytes the reference's loop holds for them (its fp32 [1024, V] tile and
    # fp32 [V, D] accumulator, 393 MB): E held once in bf16 for all 3687
    # valid rows takes 262 MB with no accumulator, so one chunk.  Beside it
    # 4096: one chunk in both layouts (E and E^T, 2 x 262 MB, inside the
    # reference's 786 MB at that setting).
    main = run(1024)
    # the two calls apart: logits (2 M_valid V D credited) and gradients (4 M_valid V D)
    fms, bms = ce_call_times(hid, w, tgt, 1024, max(5, args.steps // 5))
    calls = {"nf_ce_fwd_ms": fms, "nf_ce_bwd_ms": bms,
             "fwd_tflops": flops / 3 / (fms * 1e-3) / 1e12,
             "bwd_tflops": 2 * flops / 3 / (bms * 1e-3) / 1e12}
    calls["fwd_mfma_frac"] = calls["fwd_tflops"] / MFMA_BF16_PEAK_TFLOPS
    calls["bwd_mfma_frac"] = calls["bwd_tflops"] / MFMA_BF16_PEAK_TFLOPS
    # robustness, not a figure of record: lm_head N(0, 1) instead of N(0, 0.02)
    # puts nearly every row's largest logit far above its target logit, so
    # every such row takes the statistics pass's rescale to its maximum
    far = run(1024, weight=w * 50.0)
    far = {"graph_ms": far["graph_ms"], "graph_matches_eager": far["graph_matches_eager"],
           "vs_normal_weights": far["graph_ms"] / main["graph_ms"],
           "weights": "lm_head N(0, 1): nearly every row far from its target logit"}
    return {"m": m, "d": d, "v": v, "m_valid": m_valid, "alg_flops": flops, **main,
            "calls_chunk_1024": calls,
            "holds": "E of every valid row, once",
            "chunk_4096": {**run(4096), "holds": "E and E^T of every valid row"},
            "every_row_far_chunk_1024": far}


def bench_stress(args, dev):
    import torch

    from nuvla_forge_amd.kernels import fused_swiglu

    b, t, n = 32, 2048, 2048
    sm, sh = 65536, 5632
    inp, dh, dout = adaln_inputs(b, t, n, dev, seed=30)
    g = torch.Generator().manual_seed(31)
    a, bb, gout = (torch.randn(sm, sh, generator=g).to(torch.bfloat16).to(dev) for _ in range(3))

    def make():
        ad_step = adaln_step_fn(inp, t, dh, dout)
        la, lb = a.detach().requires_grad_(True), bb.detach().requires_grad_(True)

        def step():
            r1 = ad_step()
            out = fused_swiglu(la, lb)
            return (*r1, out, *torch.autograd.grad(out, [la, lb], gout))

        return step

    # as many replays as the headline (~75 ms at 1.5 ms a step), so the
    # clock has settled
    ms, _, _ = time_graph(make, max(5, args.steps), max(2, args.warmup))
    alg = adaln_alg_bytes(b, t, n) + 8 * sm * sh * 2
    return {"alg_bytes": alg, "graph_ms": ms, "gbs": alg / (ms * 1e-3) / 1e9,
            "hbm_frac": alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}


def bench_dit_seam(args, dev, b=8, t=6, n=384):
    """The adaLN seam at the reference's DiT shape (model/dit.py:144-175,
    NuVLAConfig: width 384, horizon 6, batch 8) with the autocast mix the
    block passes: fp32 residual x, bf16 branch output y, bf16 conditioning as
    chunk(6) views of one [B, 6N] projection, fp32 norm weight.  Launch-bound:
    reported as microseconds per fwd+bwd, fused vs the eager formulation."""
    import torch

    from nuvla_forge_amd.kernels import fused_adaln_residual_rmsnorm

    g = torch.Generator().manual_seed(40)
    x = torch.randn(b * t, n, generator=g).to(dev)
    y = torch.randn(b * t, n, generator=g).to(torch.bfloat16).to(dev)
    cond = (torch.randn(b, 6 * n, generator=g) * 0.1).to(torch.bfloat16).to(dev)
    w = (1 + 0.02 * torch.randn(n, generator=g)).to(dev)
    dh = torch.randn(b * t, n, generator=g).to(dev)
    dout = torch.randn(b * t, n, generator=g).to(dev)

    def make(force):
        leaves = [x.detach().requires_grad_(True), y.detach().requires_grad_(True),
                  cond.detach().requires_grad_(True), w.detach().requires_grad_(True)]

        def step():
            lx, ly, lc, lw = leaves
            _, scale, gate, _, _, shift = lc.chunk(6, dim=-1)
            h, out = fused_adaln_residual_rmsnorm(lx, ly, gate, lw, scale, shift,
                                                  tokens_per_sample=t, force_reference=force)
            return (h, out, *torch.autograd.grad([h, out], leaves, [dh, dout]))

        return step

    fused_ms, _, _ = time_graph(lambda: make(False), args.steps, args.warmup)
    eager_ms, _, _ = time_graph(lambda: make(True), args.steps, args.warmup)
    return {"b": b, "t": t, "n": n, "fused_us": fused_ms * 1e3, "eager_us": eager_ms * 1e3,
            "speedup": eager_ms / fused_ms}


def bench_ce_reasoning_head(args, dev, m=512, d=384, v=32000):
    """The reasoning head at the reference's model shape (model/nuvla.py:150-164:
    batch 8 x 64 text tokens, width 384, vocabulary 32000, chunk_size 1024):
    fp32 lm_head under bf16 autocast, with bf16 hidden and, as the model feeds
    it (the fp32 residual stream out of the text blocks), fp32 hidden; fused vs
    the reference's eager chunk loop, tokens/s of forward + backward."""
    import torch

    g = torch.Generator().manual_seed(41)
    hid = torch.randn(m, d, generator=g)
    w = (torch.randn(v, d, generator=g) * 0.02).to(dev)
    tgt = torch.randint(0, v, (m,), generator=g)
    tgt[::7] = -100
    tgt = tgt.to(dev)
    out = {"m": m, "d": d, "v": v}
    out.update(_head_case(args, hid.to(torch.bfloat16).to(dev), w, tgt))
    out["hidden_fp32"] = _head_case(args, hid.to(dev), w, tgt)
    return out


def _head_case(args, hid, w, tgt):
    import torch

    from nuvla_forge_amd.kernels import chunked_cross_entropy

    m = hid.shape[0]

    def make(force):
        lh, lw = hid.detach().requires_grad_(True), w.detach().requires_grad_(True)

        def step():
            with torch.autocast("cuda", dtype=torch.bfloat16):
                loss = chunked_cross_entropy(lh, lw, tgt, chunk_size=1024, force_reference=force)
            return (loss, *torch.autograd.grad(loss, [lh, lw]))

        return step

    steps, warm = max(5, args.steps // 5), max(2, args.warmup // 5)
    # both formulations as eager launches (the eager loop reads n_valid back to
    # the host, so it cannot be graph-captured); the fused step's graph replay
    # time is reported beside them, not compared
    fused_ms = time_eager(make(False), steps, warm)
    eager_ms = time_eager(make(True), steps, warm)
    fused_graph_ms, _, _ = time_graph(lambda: make(False), steps, warm)
    return {"hidden_dtype": str(hid.dtype).replace("torch.", ""), "lm_head_dtype": "float32",
            "fused_ms": fused_ms, "eager_ms": eager_ms,
            "fused_graph_ms": fused_graph_ms, "timing": "both eager launches, events",
            "tokens_per_s": m / (fused_ms * 1e-3), "eager_tokens_per_s": m / (eager_ms * 1e-3),
            "speedup": eager_ms / fused_ms}


def bench_gate_up(args, dev, m=8 * 6 * 196, d=384, h=1536):
    """SwiGLU in the gate/up GEMM epilogue at the reference's encoder MLP
    shape (TransformerBlock's SwiGLUMLP(384, 1536), model/nuvla.py:47-59,
    over batch 8 x 6 views x 196 patches): fused_gate_up_swiglu vs the
    reference's composition (two Linears + fused SwiGLU) and the eager one,
    bf16, forward alone and forward + backward."""
    import torch
    import torch.nn.functional as F

    from nuvla_forge_amd.kernels import fused_gate_up_swiglu, fused_swiglu

    g = torch.Generator().manual_seed(42)
    x = torch.randn(m, d, generator=g).to(torch.bfloat16).to(dev)
    wg = (torch.randn(h, d, generator=g) * d ** -0.5).to(torch.bfloat16).to(dev)
    wu = (torch.randn(h, d, generator=g) * d ** -0.5).to(torch.bfloat16).to(dev)
    dact = torch.randn(m, h, generator=g).to(torch.bfloat16).to(dev)
    paths = {
        "fused_gemm_epilogue": lambda a, b, c: fused_gate_up_swiglu(a, b, c),
        "linears_plus_fused_swiglu": lambda a, b, c: fused_swiglu(F.linear(a, b), F.linear(a, c)),
        "eager": lambda a, b, c: F.silu(F.linear(a, b)) * F.linear(a, c),
    }
    out = {"m": m, "d": d, "h": h}
    for name, fn in paths.items():
        def make_fwd(fn=fn):
            return lambda: (fn(x, wg, wu),)

        def make_step(fn=fn):
            leaves = [t.detach().requires_grad_(True) for t in (x, wg, wu)]

            def step():
                act = fn(*leaves)
                return (act, *torch.autograd.grad(act, leaves, dact))

            return step

        out[name + "_fwd_us"] = time_graph(make_fwd, args.steps, args.warmup)[0] * 1e3
        out[name + "_fwdbwd_us"] = time_graph(make_step, args.steps, args.warmup)[0] * 1e3
    out["gemm_tflops_fused_fwd"] = 4 * m * d * h / (out["fused_gemm_epilogue_fwd_us"] * 1e-6) / 1e12
    return out


# ---------------------------------------------------------------------------
# CPU baselines (the reference's eager PyTorch path, oracle/torch_cpu.py)
# ---------------------------------------------------------------------------
def cpu_baselines(extra: bool):
    import torch

    from oracle import torch_cpu as tc

    threads = cpu_threads()
    torch.set_num_threads(threads)
    out = {}
    b, t, n = 8, 1024, 1024
    inp, dh, dout = adaln_inputs(b, t, n, "cpu")
    s = time_cpu(lambda: tc.adaln_fwd_bwd(**inp, t=t, dh_up=dh, dout=dout))
    out["adaln"] = {"value": adaln_alg_bytes(b, t, n) / s / 1e9, "unit": "GB/s", "cores": threads,
                    "kind": "port", "seconds_per_step": s,
                    "sample": "full cfg2 workload (bf16 [8,1024,1024] fwd + autograd bwd), "
                              "median of timed reps after 1 warmup"}
    if extra:
        g = torch.Generator().manual_seed(10)
        m, h = 8192, 4096
        a, bb, gd = (torch.randn(m, h, generator=g).to(torch.bfloat16) for _ in range(3))
        s = time_cpu(lambda: tc.swiglu_fwd_bwd(a, bb, gd))
        out["swiglu"] = {"value": 8 * m * h * 2 / s / 1e9, "unit": "GB/s", "cores": threads,
                         "kind": "port", "seconds_per_step": s,
                         "sample": "full cfg3 workload (bf16 [8192,4096])"}
        hid, w, tgt = ce_inputs("cpu")
        rows = 1024
        s = time_cpu(lambda: tc.chunked_ce_fwd_bwd(hid[:rows], w, tgt[:rows], chunk_size=1024),
                     max_reps=2)
        out["ce"] = {"value": rows / s, "unit": "tokens/s", "cores": threads, "kind": "port",
                     "seconds_per_step": s,
                     "sample": "first 1024 of the 4096 cfg4 rows (one 1024-row chunk of the "
                               "reference's CPU loop, fp32 GEMMs), tokens/s of that sample"}
    out["torch"] = torch.__version__
    try:
        with open("/proc/cpuinfo") as f:
            out["cpu_model"] = next(ln.split(":", 1)[1].strip() for ln in f
                                    if ln.startswith("model name"))
    except (OSError, StopIteration):
        out["cpu_model"] = "unknown"
    return out


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); the path "
              "has no multi-GPU leg. Run with --gpus 1.", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    log(f"device: {torch.cuda.get_device_name(0)}  torch {torch.__version__}")
    if args.only:
        fn = {"swiglu": bench_swiglu, "ce": bench_ce, "stress": bench_stress,
              "traffic": bench_traffic, "dit": bench_dit_seam,
              "head": bench_ce_reasoning_head, "gateup": bench_gate_up, "copy": bench_copy,
              "adaln": bench_adaln, "adaln_cold": bench_adaln_cold,
              "ce_gemm_ceiling": bench_ce_gemm_ceiling,
              "mfma": bench_mfma_ceiling, "mainloop": bench_mainloop_probe}[args.only]
        print(json.dumps({"workload": args.only, **fn(args, dev)}), flush=True)
        return 0

    log("adaLN cfg2 ...")
    ad = bench_adaln(args, dev)
    log(f"  graph {ad['graph_ms'] * 1e3:.1f} us ({ad['gbs']:.0f} GB/s), eager "
        f"{ad['eager_ms'] * 1e3:.1f} us; kernels {ad['kernel_ms']}")
    extra = {}
    if not args.no_extra:
        log("SwiGLU cfg3 ...")
        extra["swiglu_cfg3"] = bench_swiglu(args, dev)
        log(f"  {extra['swiglu_cfg3']}")
        log("chunked CE cfg4 ...")
        extra["ce_cfg4"] = bench_ce(args, dev)
        log(f"  {extra['ce_cfg4']}")
        log("MFMA ceiling probe ...")
        mp = bench_mfma_ceiling(args, dev)
        extra["mfma_probe"] = mp
        # context, not the roofline: the CE's rate on 6 n V D against what the
        # MFMA pipes reach with no memory traffic on random bf16 operands
        extra["ce_cfg4"]["frac_of_mfma_probe"] = extra["ce_cfg4"]["tflops"] / mp["random"]["tflops"]
        log(f"  {mp}")
        log("stress chain cfg5 ...")
        extra["stress_cfg5"] = bench_stress(args, dev)
        log(f"  {extra['stress_cfg5']}")
        log("DiT seam at model shape ...")
        extra["dit_seam_model_shape"] = bench_dit_seam(args, dev)
        log(f"  {extra['dit_seam_model_shape']}")
        log("reasoning-head CE at model shape ...")
        extra["ce_reasoning_head"] = bench_ce_reasoning_head(args, dev)
        log(f"  {extra['ce_reasoning_head']}")
        log("SwiGLU in the gate/up GEMM epilogue ...")
        extra["swiglu_gate_up_gemm"] = bench_gate_up(args, dev)
        log(f"  {extra['swiglu_gate_up_gemm']}")

    cpu = None
    if not args.no_cpu:
        log("CPU baselines ...")
        cpu = cpu_baselines(not args.no_extra)
        log(f"  {cpu}")
        for k in ("swiglu", "ce"):
            if k in cpu:
                extra.setdefault("cpu_baselines", {})[k] = cpu[k]

    bwd_ms = ad["kernel_ms"]["nf_adaln_bwd"]
    record = {
        "metric": "adaLN-RMSNorm fwd+bwd HBM GB/s & % of peak; chunked-CE tokens/s",
        "value": round(ad["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ad["graph_ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.1) conditioning)",
        "config": {
            "workload": "fused_adaln_residual_rmsnorm fwd+bwd bf16 B=8 T=1024 N=1024 "
                        "(BASELINE configs[1]); forward + autograd backward through the "
                        f"Function, {STEPS_PER_GRAPH} steps per HIP graph replay",
            "alg_bytes_per_step": ad["alg_bytes"],
            "hbm_frac_whole_step": round(ad["gbs"] / HBM_PEAK_GBS, 4),
            "eager_ms_per_step": round(ad["eager_ms"], 5),
            "graph1_ms_per_step": round(ad["graph1_ms"], 5),
            # the step with HBM-resident operands: inside HIP graphs, each
            # step after a 1 GiB read-only pass that evicts its operands
            # from the L2s and the Infinity Cache, minus the passes alone
            "cold_ms_per_step": round(ad["cold_ms"], 5),
            "hbm_frac_cold_step": round(ad["alg_bytes"] / (ad["cold_ms"] * 1e-3) / 1e9
                                        / HBM_PEAK_GBS, 4),
            # the same as events around single one-step replays after the
            # pass (a 1 GiB read, or read-modify-write whose dirty lines the
            # step writes back); single_replay_floor_ms is what that method
            # reads for a 64-element fill kernel, its own fixed cost
            "cold_single_replay_ms_per_step": round(ad["cold_1r_ms"], 5),
            "cold_dirty_single_replay_ms_per_step": round(ad["cold_dirty_ms"], 5),
            "single_replay_floor_ms": round(ad["single_replay_floor_ms"], 5),
            "graph_matches_eager": ad["graph_matches_eager"],
            "kernel_ms": {k: round(v, 5) for k, v in ad["kernel_ms"].items()},
            "in_step_kernel_ms": {k: round(v, 5) for k, v in ad["in_step_ms"].items()},
            "fwd_kernel_gbs": round(ad["fwd_gbs"], 1),
            "ref_style_gbs_11MNe": round(ad["ref_style_gbs_11MNe"], 1),
            # context, not the roofline: each row kernel against nf_stream_probe
            # moving the same array shapes with no dependencies, back to back
            # ('same') and with the L2s holding other data ('alt', as inside
            # the step); fractions are probe time / kernel time
            "stream_probe_ms": {
                "fwd_2r2w": {"same": round(ad["stream_probe"]["cfg2_2r2w"]["same_us"] / 1e3, 5),
                             "alt": round(ad["stream_probe"]["cfg2_2r2w"]["alt_us"] / 1e3, 5)},
                "bwd_4r2w": {"same": round(ad["stream_probe"]["cfg2_4r2w"]["same_us"] / 1e3, 5),
                             "alt": round(ad["stream_probe"]["cfg2_4r2w"]["alt_us"] / 1e3, 5)}},
            "frac_of_stream_probe": {
                "fwd_back_to_back": round(ad["stream_probe"]["cfg2_2r2w"]["same_us"] / 1e3
                                          / ad["kernel_ms"]["nf_adaln_fwd"], 3),
                "fwd_in_step": round(ad["stream_probe"]["cfg2_2r2w"]["alt_us"] / 1e3
                                     / ad["in_step_ms"]["nf_adaln_fwd"], 3),
                "bwd_back_to_back": round(ad["stream_probe"]["cfg2_4r2w"]["same_us"] / 1e3
                                          / ad["kernel_ms"]["nf_adaln_bwd"], 3),
                "bwd_in_step": round(ad["stream_probe"]["cfg2_4r2w"]["alt_us"] / 1e3
                                     / ad["in_step_ms"]["nf_adaln_bwd"], 3)},
        },
        "roofline": {
            "kernel": "adaln_bwd_pipe_kernel (nf_adaln_bwd)",
            "bound": "hbm",
            "achieved": round(ad["bwd_gbs"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(ad["bwd_gbs"] / HBM_PEAK_GBS, 4),
            "traffic": pmc_traffic("bwd"),
            "traffic_source": TRAFFIC_FILE,
            "alg_bytes_per_launch": ad["bwd_alg_bytes"],
            "mean_launch_ms": round(bwd_ms, 5),
            # the same kernel inside the fwd -> bwd -> reduce sequence (graph
            # of the sequence minus the graph without it), beside the
            # back-to-back launches above
            "in_step_ms": round(ad["in_step_ms"]["nf_adaln_bwd"], 5),
            "frac_in_step": round(ad["bwd_gbs_in_step"] / HBM_PEAK_GBS, 4),
        },
        "cpu_baseline": None if cpu is None else {
            k: cpu["adaln"][k] for k in ("value", "unit", "cores", "kind", "sample")
        } | {"cpu_model": cpu["cpu_model"], "torch": cpu["torch"]},
        "extra": extra,
    }
    line = json.dumps(record)
    if args.json_out:
        with open(args.json_out, "w") as f:
            f.write(line + "\n")
    print(line, flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
