"""Tensors derived from parameters alone (packed weight layouts, gate
nonlinearities of per-head parameters, edge softmaxes), cached between calls.

An entry is reused while every parameter it was computed from is the same
tensor object at the same version (`Tensor._version` counts in-place updates,
so an optimizer step invalidates it).  Values that autograd must see are
recomputed whenever grad mode is on and a source requires grad.  Inside a HIP
graph capture nothing is taken from the cache (a replay must see later
parameter updates), unless the capture runs under `frozen()`: `DecodeGraph`
captures that way and refuses to replay once a parameter has changed.
"""
from __future__ import annotations

import contextlib
import weakref

import torch

_CACHE: dict = {}
_FROZEN = [False]


@contextlib.contextmanager
def frozen():
    """Let graph captures inside the block use (and fill) the cache: the caller
    guarantees the parameters do not change while the graphs are replayed."""
    before = _FROZEN[0]
    _FROZEN[0] = True
    try:
        yield
    finally:
        _FROZEN[0] = before


def _signature(sources):
    return tuple((weakref.ref(t), t._version) for t in sources)


def _matches(sig, sources) -> bool:
    return len(sig) == len(sources) and all(ref() is t and ver == t._version
                                             for (ref, ver), t in zip(sig, sources))


def derived(key, sources, fn, *, differentiable: bool = False):
    """fn(), computed from the parameters `sources` only, cached under `key`.
    differentiable: the result carries autograd history to the sources."""
    if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing() and not _FROZEN[0]:
        return fn()
    if differentiable and torch.is_grad_enabled() and any(t.requires_grad for t in sources):
        return fn()
    hit = _CACHE.get(key)
    if hit is not None and _matches(hit[0], sources):
        return hit[1]
    value = fn()
    _CACHE[key] = (_signature(sources), value)
    return value


def clear() -> None:
    _CACHE.clear()
