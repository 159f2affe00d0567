"""Static-shape forward/backward capture and replay on HIP graphs.

Mirrors the reference `GradientGraph` (src/gpa/training_graph.py:10-39): warm
up on a side stream without touching parameters, capture one loss forward and
backward, then `replay(*inputs)` copies new inputs into the captured buffers
and replays.  The optimizer step stays outside the graph.  Parameters and the
input buffers keep their addresses; replay overwrites the captured gradient
buffers, so `.grad` must not be reset to None while the graph is in use.

Steps over `MAX_CAPTURE_ROWS` rows or more are refused (see there).

The HIP library is capture-safe: it never allocates, synchronises or writes
memory with hipMemset, and it enqueues on the current (capturing) stream.
While capturing, the schedule issues its independent scans in order on the
capturing stream instead of on side streams, so the graph is single-stream.
"""
from __future__ import annotations

import gc

import torch

from . import glue, params, schedule


# Captures of steps over this many rows (batch x tokens) or more are refused:
# the capture of a B=1, T=8192 training step of the Qwen3-0.6B-shaped layer
# ended in a host segfault on ROCm 7.2 (whose cause is not known), and no
# capture at or above this size has passed.  Steps this large are launch-light
# anyway (a few hundred launches over tens of milliseconds).
MAX_CAPTURE_ROWS = 1024


class GradientGraph:
    def __init__(self, model, inputs, loss_fn, warmups: int = 3):
        rows = max((x.shape[0] * x.shape[1] for x in inputs if x.dim() >= 2), default=0)
        if rows >= MAX_CAPTURE_ROWS:
            raise NotImplementedError(
                f"GradientGraph: capture of steps over {rows} rows (batch x tokens) is switched off "
                f"(limit {MAX_CAPTURE_ROWS}); run such steps eagerly")
        self.inputs = tuple(x.detach().clone().requires_grad_(x.requires_grad) for x in inputs)
        current = torch.cuda.current_stream()
        stream = torch.cuda.Stream()
        stream.wait_stream(current)
        # Autograd graphs of earlier steps must be gone before the warm-up and
        # before the capture: a parameter's gradient-accumulation node is
        # reused while any graph holding it is alive, and it keeps the stream
        # it was created on, so the captured backward would accumulate on a
        # stream outside the capture (a cross-stream capture).
        gc.collect()
        with torch.cuda.stream(stream):
            for _ in range(warmups):
                model.zero_grad(set_to_none=True)
                for x in self.inputs:
                    x.grad = None
                loss, out = loss_fn(*self.inputs)
                loss.backward()
                del loss, out
                gc.collect()
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


class DecodeGraph:
    """One-token decode of a fixed batch on HIP graphs (inference, no autograd).

    A one-token call of the chunk model depends on its position in the block
    (which snapshots it reads, the offset it carries), so there is one graph
    per position: `chunk_size` graphs, captured in the order they replay and
    sharing one memory pool.  Each graph's output state lives in pool memory
    that a later graph of the same block reuses once the state has been read,
    so the graphs hold about two states, not one per position.

    The cache must start at a block boundary (chunk_offset 0).  Its tensors
    are copied into static buffers that the first graph reads and that every
    later graph of the block reads as the block snapshots; after the last
    position of a block the new cache is copied back into them (one state
    copy per block).

    Tensors derived from the parameters alone (packed weight layouts, gate
    constants) are computed once, kept by this object and read by the graphs
    (`params.frozen`), so the parameters must not change while the graphs are
    in use: `step` raises if one has been replaced, moved or updated in place
    through the parameter itself.

    `step(q, k, v)` ([B,1,H,D] like the captured token) copies the token into
    the static inputs, replays the graph of the current position and returns
    that position's output buffer.  The buffers are allocated outside the
    graphs' pool (each graph ends by copying its output into its own buffer),
    because the pool memory of one graph's output is free space to the graphs
    captured before it and is overwritten when they replay.  An output buffer
    holds until the same position replays `chunk_size` steps later.  `state`
    is the cache after the last step, at a block boundary (its tensors are the
    static buffers: clone to keep them).
    """

    def __init__(self, model, state, q, k, v, warmups: int = 2):
        if state.chunk_offset != 0:
            raise ValueError("DecodeGraph: the cache must start at a block boundary (chunk_offset 0)")
        if q.shape[1] != 1:
            raise ValueError("DecodeGraph: one token per call")
        if model.config.positional_mode == "moments":
            # the rotary embedding reads the absolute position, which a
            # replayed graph would keep at its captured value
            raise ValueError("DecodeGraph: positional_mode='moments' depends on the position; decode eagerly")
        from .state import _apply, tensors
        self._tensors = tensors
        self.chunk = state.chunk_size
        self.position = state.position
        self.offset = 0
        self.inputs = tuple(x.detach().clone() for x in (q, k, v))
        self.start = _apply(state, lambda t: t.detach().clone(memory_format=torch.contiguous_format))
        current = torch.cuda.current_stream()
        side = torch.cuda.Stream()
        side.wait_stream(current)
        self._params = params.fingerprints(list(model.parameters()))
        # The derived tensors live as long as the graphs that read them.
        self._derived = params.Store()
        with torch.no_grad(), torch.cuda.stream(side), params.frozen(self._derived):
            s = self.start
            for _ in range(warmups):
                _, s = model(*self.inputs, s)
        current.wait_stream(side)
        del s
        self.pool = torch.cuda.graph_pool_handle()
        self.graphs = []
        # One output buffer per position, from the ordinary allocator.
        self.outputs = [torch.empty_like(self.inputs[2]) for _ in range(self.chunk)]
        s = self.start
        with torch.no_grad(), params.frozen(self._derived):
            for o in range(self.chunk):
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, pool=self.pool):
                    with schedule.output_into(self.outputs[o]):
                        out, s = model(*self.inputs, s)
                    if out.data_ptr() != self.outputs[o].data_ptr():
                        self.outputs[o].copy_(out)
                del out
                self.graphs.append(graph)
        self.last = s  # the cache after a whole block
        pairs = list(zip(tensors(self.start), tensors(self.last)))
        if s.chunk_offset != 0 or len(pairs) != len(list(tensors(self.start))) or any(
                a.shape != b.shape for a, b in pairs):
            raise RuntimeError("DecodeGraph: the cache after a block does not match the cache it started from")

    def step(self, q, k, v):
        if not params.unchanged(self._params):
            raise RuntimeError("DecodeGraph: a parameter changed after capture; build a new DecodeGraph")
        for static, value in zip(self.inputs, (q, k, v)):
            if static.shape != value.shape or static.dtype != value.dtype:
                raise ValueError("DecodeGraph replays only the captured token shape/dtype")
        pairs = list(zip(self.inputs, (q, k, v)))
        if not (all(x.device == self.inputs[0].device for x in (q, k, v)) and glue.copy_many(pairs)):
            for static, value in pairs:
                static.copy_(value)
        o = self.offset
        self.graphs[o].replay()
        self.offset = (o + 1) % self.chunk
        self.position += 1
        if self.offset == 0:
            with torch.no_grad():
                for dst, src in zip(self._tensors(self.start), self._tensors(self.last)):
                    dst.copy_(src)
        return self.outputs[o]

    @property
    def state(self):
        if self.offset != 0:
            raise RuntimeError("DecodeGraph.state is available at block boundaries")
        import dataclasses
        return dataclasses.replace(self.start, position=self.position)
