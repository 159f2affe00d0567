"""Gated moment scans on the device (`gpa_moment_scan_many`).

The per-token recurrence S_t = a_t o S_{t-1} + k_t v_t^T, y_t = S_t^T q_t of
the reference's `moment_scan` (src/gpa/paper_dense.py:16-47), of its
`decayed_counts` (:50-58, the same recurrence with one key row) and of the
additive positional moments (`linear_scan`, src/gpa/ops.py:88-118, no decay).

Backward.  With D_t the gradient of S_t (D_t = a_{t+1} o D_{t+1} + q_t dy_t^T,
D_{T-1} = dfinal + q dy^T), the input gradients are
    dq_t = S_t dy_t          a forward scan of the transposed state (S^T takes
                             the updates v_t k_t^T and is read with dy_t),
    dv_t = D_t^T k_t         a reverse scan (updates q_t dy_t^T, read with k_t),
    dk_t = D_t v_t           a reverse scan of the transposed adjoint,
    dS_0 = a_0 o D_0         the reverse scan's final state,
all three in one launch.  The decay gradient uses the identity for the
cumulative log decay G_t = sum_{u<=t} g_u: dG_t = q_t o dq_t - k_t o dk_t per
key row (summed over rows for one decay per token), dy_t o y_t - v_t o dv_t
per value column, plus dfinal o S_T at the last token; dg is its reverse
cumulative sum over the call's tokens.
"""
from __future__ import annotations

import torch
from torch import Tensor

from . import _lib

_SWAP = {_lib.GATE_NONE: _lib.GATE_NONE, _lib.GATE_TOKEN: _lib.GATE_TOKEN,
         _lib.GATE_KEY: _lib.GATE_VALUE, _lib.GATE_VALUE: _lib.GATE_KEY}


def _last_contig(x: Tensor) -> Tensor:
    return x if x.stride(-1) == 1 else x.contiguous()


def _problem(q, k, v, g, gate, y, s0=None, final=None, reverse=False, y_f32=False) -> _lib.MomentProblem:
    bsz, tokens, heads, kd = q.shape
    p = _lib.MomentProblem()
    p.batch, p.heads, p.tokens, p.kdim, p.vdim = bsz, heads, tokens, kd, v.shape[-1]
    p.dtype = _lib.DTYPE_CODES[q.dtype]
    p.gate, p.reverse, p.y_f32 = gate, int(reverse), int(y_f32)
    p.q, p.k, p.v, p.y = (_lib.operand(x) for x in (q, k, v, y))
    p.g = _lib.operand(g) if g is not None else _lib.Operand(None, 0, 0, 0)
    if s0 is not None:
        p.s0, p.s0_sb, p.s0_sh = s0.data_ptr(), s0.stride(0), s0.stride(1)
    p.final = final.data_ptr() if final is not None else None
    return p


def _state_arg(s: Tensor | None) -> Tensor | None:
    """A float32 [B,H,K,V] state whose head slices are contiguous (batch and
    head strides free: an expanded prefix stays a view)."""
    if s is None:
        return None
    s = s.float()
    if s.stride(-1) != 1 or s.stride(-2) != s.shape[-1]:
        s = s.contiguous()
    return s


def _launch(problems, keep, device) -> None:
    lib = _lib.load()
    arr = (_lib.MomentProblem * len(problems))(*problems)
    _lib.check(lib.gpa_moment_scan_many(arr, len(problems), _lib.stream_handle(device)), "gpa_moment_scan_many")
    del keep


class _MomentScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, g, s0, gate: int, y_f32: bool):
        dev = q.device
        q, k, v = _last_contig(q), _last_contig(k), _last_contig(v)
        g = _last_contig(g.float()) if g is not None else None
        s0a = _state_arg(s0)
        bsz, tokens, heads, kd = q.shape
        vd = v.shape[-1]
        # the float32 read is kept when the decay gradient needs it (per-column decay)
        want32 = y_f32 or gate == _lib.GATE_VALUE
        y = torch.empty(bsz, tokens, heads, vd, device=dev, dtype=torch.float32 if want32 else q.dtype)
        final = torch.empty(bsz, heads, kd, vd, device=dev, dtype=torch.float32)
        _launch([_problem(q, k, v, g, gate, y, s0a, final, y_f32=want32)], (q, k, v, g, s0a, y, final), dev)
        ctx.gate, ctx.y_f32 = gate, y_f32
        ctx.s0_dtype = s0.dtype if s0 is not None else None
        ctx.save_for_backward(q, k, v, g, s0a, final, y if gate == _lib.GATE_VALUE else None)
        out = y if (y_f32 or not want32) else y.to(q.dtype)
        return out, final

    @staticmethod
    def backward(ctx, dy, dfinal):
        q, k, v, g, s0, final, y32 = ctx.saved_tensors
        gate = ctx.gate
        dev = q.device
        bsz, tokens, heads, kd = q.shape
        vd = v.shape[-1]
        work = q.dtype
        if dy is None:
            dy = torch.zeros(bsz, tokens, heads, vd, device=dev, dtype=work)
        if dy.dtype != work:  # a float32 read gradient: run the adjoint scans in float32 (exact for bf16 inputs)
            work = torch.float32
        qw, kw, vw = (x if x.dtype == work else x.to(work) for x in (q, k, v))
        dyw = _last_contig(dy.to(work))
        f32 = dict(device=dev, dtype=torch.float32)
        dq = torch.empty(bsz, tokens, heads, kd, **f32)
        dk = torch.empty(bsz, tokens, heads, kd, **f32)
        dv = torch.empty(bsz, tokens, heads, vd, **f32)
        ds0 = torch.empty(bsz, heads, kd, vd, **f32)
        s0t = s0.transpose(-1, -2).contiguous() if s0 is not None else None
        df = dfinal.float().contiguous() if dfinal is not None else None
        dft = df.transpose(-1, -2).contiguous() if df is not None else None
        swap = _SWAP[gate]
        problems = [
            _problem(dyw, vw, kw, g, swap, dq, s0t, None, reverse=False, y_f32=True),   # dq = S_t dy_t
            _problem(kw, qw, dyw, g, gate, dv, df, ds0, reverse=True, y_f32=True),      # dv = D_t^T k_t, dS0
            _problem(vw, dyw, qw, g, swap, dk, dft, None, reverse=True, y_f32=True),    # dk = D_t v_t
        ]
        _launch(problems, (qw, kw, vw, dyw, g, s0t, df, dft, dq, dk, dv, ds0), dev)
        dg = None
        if gate != _lib.GATE_NONE and ctx.needs_input_grad[3]:
            if gate == _lib.GATE_VALUE:
                dG = dy.float() * y32 - v.float() * dv
                last = (df * final).sum(-2) if df is not None else None
            else:
                dG = q.float() * dq - k.float() * dk
                last = (df * final).sum(-1) if df is not None else None
                if gate == _lib.GATE_TOKEN:
                    dG = dG.sum(-1)
                    last = last.sum(-1) if last is not None else None
            if last is not None:
                dG[:, -1] += last
            dg = dG.flip(1).cumsum(1).flip(1)
        ds0_out = ds0.to(ctx.s0_dtype) if (s0 is not None and ctx.needs_input_grad[4]) else None
        return (dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dg, ds0_out, None, None)


def _gate_form(g: Tensor | None, q: Tensor, v: Tensor, axis: str) -> int:
    if g is None:
        return _lib.GATE_NONE
    if g.ndim == 3:
        return _lib.GATE_TOKEN
    if axis == "value":
        if g.shape[-1] != v.shape[-1]:
            raise ValueError("a per-value decay needs g [B,T,H,V]")
        return _lib.GATE_VALUE
    if g.shape[-1] != q.shape[-1]:
        raise ValueError("a per-key decay needs g [B,T,H,K]")
    return _lib.GATE_KEY


def supported(q: Tensor, v: Tensor) -> bool:
    """Widths the kernel covers in both directions (the backward's transposed
    scans reduce over the value width)."""
    return (q.dtype in _lib.DTYPE_CODES and 1 <= q.shape[-1] <= _lib.MOMENT_MAX_KDIM
            and 1 <= v.shape[-1] <= _lib.MOMENT_MAX_KDIM)


def moment_scan(q: Tensor, k: Tensor, v: Tensor, g: Tensor | None, initial: Tensor,
                axis: str = "key", y_f32: bool = False) -> tuple[Tensor, Tensor]:
    """S = exp(g) o S + k v^T; y = q^T S per token (reference
    paper_dense.py:16-47, backend "torch").  q, k [B,T,H,K], v [B,T,H,V],
    g None (no decay), [B,T,H] (per token) or [B,T,H,K] / [B,T,H,V] (per key row
    or, with axis="value", per value column), initial [B,H,K,V].  Returns y in
    q's dtype (float32 with y_f32) and the final state in float32."""
    if q.shape != k.shape or q.shape[:3] != v.shape[:3]:
        raise ValueError("expected matching [B,T,H,K] Q/K and [B,T,H,V] V")
    _lib.require_device(q)
    if q.shape[1] == 0:
        return v.new_empty(v.shape), initial
    if not supported(q, v):
        raise _lib.HipBackendError("moment scan: float32/bfloat16 with key and value widths 1..256")
    dt = q.dtype
    k, v = k.to(dt), v.to(dt)
    gate = _gate_form(g, q, v, axis)
    return _MomentScan.apply(q, k, v, g, initial, gate, y_f32)


def decayed_counts(p: Tensor, g: Tensor, initial: Tensor) -> Tensor:
    """n_t = exp(g_t) o n_{t-1} + p_t for every token (reference
    paper_dense.py:50-58): p [B,T,H,M], g [B,T,H] or [B,T,H,M], initial
    [B,H,M]; float32 [B,T,H,M].  The moment scan with one key row."""
    bsz, tokens, heads, m = p.shape
    if tokens == 0:
        return initial.new_empty(bsz, 0, heads, m)
    ones = torch.ones(bsz, tokens, heads, 1, device=p.device, dtype=p.dtype)
    y, _ = moment_scan(ones, ones, p, g, initial[:, :, None, :], axis="value", y_f32=True)
    return y
