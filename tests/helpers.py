"""Shared helpers for the GPU parity tests."""

from __future__ import annotations

import sys

import numpy as np
import torch

# BASELINE tolerances: norm-wise relative error against the fp64 oracle
# evaluated on the same (rounded) inputs.
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def note(msg: str) -> None:
    """Name the case before a GPU step (flushed, so it survives a crash)."""
    print(msg, flush=True)
    sys.stdout.flush()


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def randn(shape, seed_gen, dtype, device, std=1.0, mean=0.0):
    """CPU-seeded normal samples, rounded to `dtype`, moved to `device`."""
    t = torch.randn(*shape, generator=seed_gen, dtype=torch.float32) * std + mean
    return t.to(dtype).to(device)


def np64(t: torch.Tensor) -> np.ndarray:
    return t.detach().to("cpu", torch.float64).numpy()


def swiglu_rel_errs(a, b, dout, out, da, db, rows: int = 4096) -> dict:
    """Norm-wise relative errors of a SwiGLU forward/backward against the
    oracle evaluated in fp32 on the host, a block of rows at a time (the
    BASELINE stress shape has 369 M elements per tensor)."""
    from oracle import numerics as on

    num = {"out": 0.0, "da": 0.0, "db": 0.0}
    den = dict(num)
    m = a.shape[0]
    for r0 in range(0, m, rows):
        sl = slice(r0, min(r0 + rows, m))
        A, B, G = (t[sl].detach().to("cpu", torch.float32).numpy() for t in (a, b, dout))
        want = {"out": on.swiglu_forward(A, B)}
        want["da"], want["db"] = on.swiglu_backward(A, B, G)
        for k, got in (("out", out), ("da", da), ("db", db)):
            g = got[sl].detach().to("cpu", torch.float32).numpy()
            num[k] = max(num[k], float(np.abs(g - want[k]).max()))
            den[k] = max(den[k], float(np.abs(want[k]).max()))
    return {k: num[k] / den[k] if den[k] else num[k] for k in num}


def assert_graph_replays_match(make, replays: int = 3) -> None:
    """Capture ``make()()`` (a step returning tensors) into a HIP graph and
    check that every replay, with eager work and synchronisations between
    replays, reproduces the eager step bit for bit."""
    eager = [t.clone() for t in make()()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step = make()
        step()  # warm-up outside the capture (allocator, autograd state)
    side.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        outs = step()
    torch.cuda.current_stream().wait_stream(side)
    for i in range(replays):
        graph.replay()
        torch.cuda.synchronize()
        bad = [k for k, (a, b) in enumerate(zip(outs, eager)) if not torch.equal(a, b)]
        assert not bad, f"replay {i}: outputs {bad} differ from the eager step"
        make()()  # eager work between replays
        torch.cuda.synchronize()
