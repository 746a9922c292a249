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
