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
