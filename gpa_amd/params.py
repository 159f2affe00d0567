"""Tensors derived from parameters alone (packed weight layouts, gate
nonlinearities of per-head parameters, edge softmaxes).

Nothing is cached by default: `derived(key, sources, fn)` simply returns
`fn()`, as the reference recomputes these every call.  A caller that
guarantees the parameters do not change for a while opts in with
`frozen(store)`: inside the block, derived tensors are computed once per key
and kept in `store`, which the caller owns (so the tensors live exactly as
long as the caller needs them, e.g. as long as the HIP graphs that read them).
An entry is reused only while every source is the same tensor object with the
same version counter, storage address, dtype, device and shape; in-place
updates through `.data` are invisible to those checks, which is why caching
needs the caller's promise.  Values that autograd must see are recomputed
whenever grad mode is on and a source requires grad.
"""
from __future__ import annotations

import contextlib
import weakref

import torch


class Store:
    """Derived tensors of one frozen scope, keyed by the caller's key."""

    def __init__(self):
        self.entries: dict = {}

    def clear(self) -> None:
        self.entries.clear()

    def __len__(self) -> int:
        return len(self.entries)


_SCOPES: list[Store] = []


@contextlib.contextmanager
def frozen(store: Store | None = None):
    """Cache derived tensors inside the block in `store` (a fresh one if None;
    it is yielded).  The caller guarantees the parameters do not change while
    it uses what was computed here."""
    store = Store() if store is None else store
    _SCOPES.append(store)
    try:
        yield store
    finally:
        _SCOPES.pop()


def _fingerprint(t: torch.Tensor):
    return (t._version, t.data_ptr(), t.dtype, t.device, tuple(t.shape))


def _signature(sources):
    return tuple((weakref.ref(t), _fingerprint(t)) for t in sources)


def _matches(sig, sources) -> bool:
    return len(sig) == len(sources) and all(ref() is t and fp == _fingerprint(t)
                                             for (ref, fp), t in zip(sig, sources))


def derived(key, sources, fn, *, differentiable: bool = False):
    """fn(), computed from the tensors `sources` only; cached under `key` in
    the innermost `frozen()` store, if any.  differentiable: the result
    carries autograd history to the sources."""
    if not _SCOPES:
        return fn()
    if differentiable and torch.is_grad_enabled() and any(t.requires_grad for t in sources):
        return fn()
    store = _SCOPES[-1].entries
    hit = store.get(key)
    if hit is not None and _matches(hit[0], sources):
        return hit[1]
    value = fn()
    store[key] = (_signature(sources), value)
    return value


def fingerprints(tensors) -> list:
    """The identity of each tensor's current contents as far as `derived` can
    see it (object, version counter, storage address, dtype, device, shape)."""
    return [(t, _fingerprint(t)) for t in tensors]


def unchanged(prints) -> bool:
    return all(_fingerprint(t) == fp for t, fp in prints)
