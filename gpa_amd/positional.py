"""Positional moments (`positional_mode="moments"`): the adjacent-pair rotary
embedding and the additive moment scan of the reference
(src/gpa/ops.py:88-137), used by the block segment at attention.py:305,
:318-323 and the token step at :265, :276-281.

The moment scan `S += k v^T; out = q^T S` runs in the gated moment-scan
kernel (`gpa_amd.moment`, no decay) for key and value widths up to 256, with
its three-scan backward.  Wider scans take the chunked form as device tensor
operations: per 64-token chunk the state at the chunk start is the initial
state plus the exclusive prefix sum of the earlier chunks' K^T V, and a token
reads `q^T S_chunk_start + sum_{s <= t in the chunk} (q_t . k_s) v_s` (batched
float32 matmuls).  The rotary embedding is a float32 (float64 for float64
inputs) device tensor operation with autograd.
"""
from __future__ import annotations

import torch
from torch import Tensor

from . import _lib, moment

CHUNK = 64  # tokens per chunk of the moment scan


def _work(x: Tensor) -> torch.dtype:
    return torch.float64 if x.dtype == torch.float64 else torch.float32


def rope(x: Tensor, positions, base: float = 10000.) -> Tensor:
    """Adjacent-pair rotary embedding of the last axis (reference ops.py:121-137):
    x [..., D] or [B,T,H,D]; positions a scalar, [T] or [B,T] (for [B,T,H,D]
    inputs) or broadcastable to x's leading axes.  Computed in float32 (float64
    for float64 x) and returned in x's dtype."""
    d = x.shape[-1]
    if d % 2:
        raise ValueError("RoPE needs an even head dimension")
    work = x.to(_work(x))
    pos = torch.as_tensor(positions, device=x.device, dtype=work.dtype)
    if x.ndim == 4:
        if pos.ndim == 1:
            pos = pos[None, :, None]
        elif pos.ndim == 2:
            pos = pos[:, :, None]
    freq = base ** (-torch.arange(0, d, 2, device=x.device, dtype=work.dtype) / d)
    angle = pos[..., None] * freq
    even, odd = work[..., 0::2], work[..., 1::2]
    cos, sin = angle.cos(), angle.sin()
    return torch.stack((even * cos - odd * sin, even * sin + odd * cos), -1).flatten(-2).to(x.dtype)


def additive_scan(q: Tensor, k: Tensor, v: Tensor, initial: Tensor) -> tuple[Tensor, Tensor]:
    """The reference's `linear_scan` (ops.py:88-118, backend="torch"): q, k
    [B,T,H,K], v [B,T,H,V], initial [B,H,K,V]; S_t = S_{t-1} + k_t v_t^T and
    out_t = q_t^T S_t (no normalisation).  Returns (out [B,T,H,V] in q's
    dtype, final state [B,H,K,V] in the work dtype).  Empty T returns
    (empty, initial)."""
    if q.shape != k.shape or q.shape[:3] != v.shape[:3]:
        raise ValueError("expected matching [B,T,H,K] Q/K and [B,T,H,V] V")
    bsz, tokens, heads, kd = q.shape
    vd = v.shape[-1]
    if tokens == 0:
        return v.new_empty(v.shape), initial
    if q.dtype != torch.float64 and q.is_cuda and moment.supported(q, v):
        return moment.moment_scan(q, k, v.to(q.dtype), None, initial)
    work = _work(q)
    n = -(-tokens // CHUNK)
    pad = n * CHUNK - tokens

    def chunks(x):  # [B,T,H,D] -> [B,H,N,C,D] in the work dtype, zero tail
        x = x.to(work)
        if pad:
            x = torch.nn.functional.pad(x, (0, 0, 0, 0, 0, pad))
        return x.view(bsz, n, CHUNK, heads, -1).permute(0, 3, 1, 2, 4).contiguous()

    qc, kc, vc = chunks(q), chunks(k), chunks(v)
    kt = kc.transpose(-1, -2).contiguous()                       # [B,H,N,K,C]
    kv = torch.matmul(kt, vc)                                    # [B,H,N,K,V] per-chunk K^T V
    s0 = initial.to(work).unsqueeze(2)                           # [B,H,1,K,V]
    before = torch.cumsum(kv[:, :, :-1], 2)                      # sum of the earlier chunks
    starts = torch.cat((s0, s0 + before), 2)                     # state at every chunk start
    scores = torch.matmul(qc, kt)                                # [B,H,N,C,C] q_t . k_s
    causal = torch.ones(CHUNK, CHUNK, device=q.device, dtype=torch.bool).tril()
    scores = scores.masked_fill(~causal, 0.)
    out = torch.matmul(qc, starts) + torch.matmul(scores, vc)    # [B,H,N,C,V]
    out = out.permute(0, 2, 3, 1, 4).reshape(bsz, n * CHUNK, heads, vd)[:, :tokens]
    final = initial.to(work) + kv.sum(2)
    return out.to(q.dtype), final


def linear_scan(q: Tensor, k: Tensor, v: Tensor, initial_state: Tensor, *,
                backend: str = "hip") -> tuple[Tensor, Tensor]:
    """Drop-in for the reference `linear_scan` (src/gpa/ops.py:88-118) on the
    GPU: additive positional moments, S += k v^T, no normalisation of inputs."""
    if q.shape != k.shape or q.shape[:3] != v.shape[:3]:
        raise ValueError("expected matching [B,T,H,K] Q/K and [B,T,H,V] V")
    if backend != "hip":
        raise ValueError(f"unknown backend: {backend}")
    _lib.require_device(q)
    return additive_scan(q, k, v, initial_state)
