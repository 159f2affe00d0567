"""Recurrent cache of a DenseGPA core.

The layout is the reference's (src/gpa/state.py:30-72), field for field, so a
cache produced by either package is readable by the other:

* `LevelState.inner`  A_j  [B,H,Dk,M_j]  key-major inner GDN state
* `LevelState.outer`  B_j  [B,H,M_j,Dv]  outer GDN state
* `LevelState.count`  n_j  [B,H,M_j]     soft write counts
* `RelationState.memory` R_ij [B,H,M_i,M_j] for every ordered edge i != j
* `GPAState.frozen`   block-start (A_j, B_j) snapshots, kept only while a
  chunk is incomplete (chunk_offset != 0)

State tensors are float32 (float64 for float64 inputs).  The cache is
immutable; `detach()` is explicit and never implied.
"""
from __future__ import annotations

from dataclasses import dataclass, fields, is_dataclass
from typing import Any, Callable, Iterator

import torch
from torch import Tensor


def _apply(value: Any, fn: Callable[[Tensor], Tensor]) -> Any:
    if isinstance(value, Tensor):
        return fn(value)
    if isinstance(value, tuple):
        return tuple(_apply(x, fn) for x in value)
    if is_dataclass(value):
        return type(value)(**{f.name: _apply(getattr(value, f.name), fn) for f in fields(value)})
    return value


def tensors(value: Any) -> Iterator[Tensor]:
    """Every tensor of a cache, in field order (depth first)."""
    if isinstance(value, Tensor):
        yield value
    elif isinstance(value, tuple):
        for item in value:
            yield from tensors(item)
    elif is_dataclass(value):
        for f in fields(value):
            yield from tensors(getattr(value, f.name))


@dataclass(frozen=True)
class LevelState:
    inner: Tensor
    outer: Tensor
    count: Tensor
    position: Tensor | None = None


@dataclass(frozen=True)
class RelationState:
    source: int
    target: int
    memory: Tensor


@dataclass(frozen=True)
class ResidualSnapshot:
    inner: Tensor
    outer: Tensor


@dataclass(frozen=True)
class GPAState:
    levels: tuple[LevelState, ...]
    relations: tuple[RelationState, ...]
    position: int = 0
    chunk_size: int = 1
    chunk_offset: int = 0
    frozen: tuple[ResidualSnapshot, ...] | None = None

    def detach(self) -> "GPAState":
        return _apply(self, lambda x: x.detach())

    def to(self, *args, **kwargs) -> "GPAState":
        return _apply(self, lambda x: x.to(*args, **kwargs))

    def numel(self) -> int:
        """Logical element count of every tensor, snapshots included."""
        return sum(x.numel() for x in tensors(self))


def state_dtype(x: Tensor) -> torch.dtype:
    """Recurrent-state arithmetic type: float64 for float64 inputs, else float32."""
    return torch.float64 if x.dtype == torch.float64 else torch.float32
