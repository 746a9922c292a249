"""Device timing helpers shared by bench.py and the kernels report.

All three time work on torch's streams with HIP events read after a device
synchronisation:
  * time_eager     -- a step launched eagerly, mean over `steps` calls;
  * time_graph     -- a step captured in a HIP graph (optionally several
                      consecutive steps per graph), mean over replays;
  * per_launch_ms  -- one launch's mean duration: `reps` back-to-back
                      launches in a graph, replayed, with the events on the
                      stream the kernels run on.
"""

from __future__ import annotations

import torch


def sync() -> None:
    torch.cuda.synchronize()


def time_eager(step, steps: int, warmup: int) -> float:
    """Mean milliseconds per call of `step()` over `steps` eager calls."""
    for _ in range(warmup):
        step()
    sync()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    sync()
    return e0.elapsed_time(e1) / max(steps, 1)


def time_graph(make_step, steps: int, warmup: int, per_graph: int = 1):
    """Capture `per_graph` consecutive steps in one HIP graph and time
    `steps` steps (steps / per_graph replays).

    `make_step()` must build the step around fresh leaf tensors: their
    AccumulateGrad nodes are then created on the side stream that both warms
    up and captures the step, so autograd never has to synchronise the
    (non-capturing) default stream with the capture.  Returns (ms per step,
    outputs of the last captured step, graph).
    """
    per_graph = max(1, min(per_graph, steps))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step = make_step()
        for _ in range(max(warmup, 2)):
            step()
    side.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for _ in range(per_graph):
            outs = step()
    torch.cuda.current_stream().wait_stream(side)
    for _ in range(max(1, warmup // per_graph)):
        graph.replay()
    sync()
    replays = max(1, steps // per_graph)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        graph.replay()
    e1.record()
    sync()
    return e0.elapsed_time(e1) / (replays * per_graph), outs, graph


def per_launch_ms(launch, steps: int, reps: int = 20) -> float:
    """Mean duration of one launch: `reps` back-to-back launches captured in a
    HIP graph (on a side stream), replayed `steps` times between two events on
    the stream the kernels run on."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launch()
    side.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for _ in range(reps):
            launch()
    torch.cuda.current_stream().wait_stream(side)
    graph.replay()
    sync()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        graph.replay()
    e1.record()
    sync()
    return e0.elapsed_time(e1) / (steps * reps)
