"""Static-shape forward/backward capture and replay on HIP graphs.

Mirrors the reference `GradientGraph` (src/gpa/training_graph.py:10-39): warm
up on a side stream without touching parameters, capture one loss forward and
backward, then `replay(*inputs)` copies new inputs into the captured buffers
and replays.  The optimizer step stays outside the graph.  Parameters and the
input buffers keep their addresses; replay overwrites the captured gradient
buffers, so `.grad` must not be reset to None while the graph is in use.

The HIP library is capture-safe: it never allocates, synchronises or writes
memory with hipMemset, and it enqueues on the current (capturing) stream.
While capturing, the schedule issues its independent scans in order on the
capturing stream instead of on side streams, so the graph is single-stream.
"""
from __future__ import annotations

import torch


class GradientGraph:
    def __init__(self, model, inputs, loss_fn, warmups: int = 3):
        self.inputs = tuple(x.detach().clone().requires_grad_(x.requires_grad) for x in inputs)
        current = torch.cuda.current_stream()
        stream = torch.cuda.Stream()
        stream.wait_stream(current)
        with torch.cuda.stream(stream):
            for _ in range(warmups):
                model.zero_grad(set_to_none=True)
                for x in self.inputs:
                    x.grad = None
                loss, _ = loss_fn(*self.inputs)
                loss.backward()
        current.wait_stream(stream)
        model.zero_grad(set_to_none=True)
        for x in self.inputs:
            x.grad = None
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.loss, self.output = loss_fn(*self.inputs)
            self.loss.backward()

    def replay(self, *inputs):
        with torch.no_grad():
            for static, value in zip(self.inputs, inputs):
                if static.shape != value.shape or static.dtype != value.dtype:
                    raise ValueError("a HIP graph replays only the captured input shapes/dtypes")
                static.copy_(value)
        self.graph.replay()
        return self.loss, self.output
