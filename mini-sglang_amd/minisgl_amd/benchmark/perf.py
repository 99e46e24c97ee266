"""Kernel timing with HIP events and graph replay.

Same method as the reference's perf_cuda (python/minisgl/benchmark/perf.py:10-51):
capture ``f`` N times into a graph, replay it ``repetitions`` times between
events, report milliseconds per call. ``torch.cuda`` is HIP on ROCm.
"""

from __future__ import annotations

from typing import Any, Callable


def perf_hip(f: Callable[[], Any], *, repetitions: int = 10, graph_repetitions: int | None = 10) -> float:
    import torch

    tic = torch.cuda.Event(enable_timing=True)
    toc = torch.cuda.Event(enable_timing=True)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        f()
        if n := graph_repetitions:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for _ in range(n):
                    f()
            replay = g.replay
        else:
            replay, n = f, 1
        torch.cuda.synchronize()
        replay()
        tic.record(stream)
        for _ in range(repetitions):
            replay()
        toc.record(stream)
        toc.synchronize()
    return tic.elapsed_time(toc) / (n * repetitions)
