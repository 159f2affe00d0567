"""Autograd operators over libgpa_hip.

`gdn_scan_hip` is the HIP replacement of the reference `gdn_scan`
(src/gpa/ops.py:49-85) for a group of streams laid out as [B,T,H,D], extended
with what the block-lagged model needs from a chunked scan: the state at the
start of every chunk (the block boundaries of attention.py:397) and a token
offset that aligns chunks with blocks that began in an earlier call.
"""
from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from . import _lib, profiling


def _contig_last(x: Tensor) -> Tensor:
    return x if x.stride(-1) == 1 else x.contiguous()


def _f32_state(s: Tensor) -> Tensor:
    s = s.float() if s.dtype != torch.float32 else s
    return s if (s.stride(3) == 1 and s.stride(2) == s.shape[3]) else s.contiguous()


def _problem(q, k, v, g, beta, s0f, chunk, offset):
    bsz, tokens, heads, kd = k.shape
    return _lib.Problem(bsz, heads, tokens, offset, chunk, kd, v.shape[-1], _lib.DTYPE_CODES[k.dtype],
                        _lib.operand(q), _lib.operand(k), _lib.operand(v), _lib.operand(g), _lib.operand(beta),
                        s0f.data_ptr() if s0f is not None else None,
                        s0f.stride(0) if s0f is not None else 0, s0f.stride(1) if s0f is not None else 0)


def _ptr(t):
    return t.data_ptr() if t is not None else None


def _in_use_here(*tensors):
    """Mark tensors made on another stream as read by the current one, so the
    caching allocator keeps their memory until this stream's work is done."""
    if torch.cuda.is_current_stream_capturing():
        return  # a capture runs on one stream
    stream = torch.cuda.current_stream()
    for t in tensors:
        if t is not None:
            t.record_stream(stream)


class _Group:
    """One scan group's forward: its problem, saved intermediates (layouts of
    include/gpa_hip.h) and outputs."""

    def __init__(self, lib, q, k, v, g, beta, s0, chunk: int, offset: int, box=None):
        _in_use_here(q, k, v, g, beta, s0)
        bsz, tokens, heads, kd = k.shape
        vd = v.shape[-1]
        dev = k.device
        nch = lib.gpa_gdn_nchunks(tokens, offset, chunk)
        if nch <= 0:
            raise ValueError("gdn_scan_hip: invalid chunk geometry")
        s0f = _f32_state(s0) if s0 is not None else None
        self.prob = _problem(q, k, v, g, beta, s0f, chunk, offset)
        mfma = lib.gpa_gdn_path(self.prob) == 1
        chunks = bsz * heads * nch
        rows = chunks * _lib.CHUNK_ROWS
        f32 = dict(device=dev, dtype=torch.float32)
        b16 = dict(device=dev, dtype=torch.bfloat16)
        kn = torch.empty(rows * kd, **f32)
        qn = torch.empty(rows * kd, **f32) if q is not None else None
        w = torch.empty(rows * kd, **f32) if not mfma else None
        # U: value-major [S,N,V,64] on the FMA path; on the MFMA path fragment
        # order over ceil(V/32) whole 32-column strips (include/gpa_hip.h).
        u = torch.empty(rows * (-(-vd // 32) * 32 if mfma else vd), **f32)
        delta = torch.empty(rows * vd, **f32)
        tri = torch.empty(rows * _lib.CHUNK_ROWS, **f32)
        gam = torch.empty(rows, **f32)
        bet = torch.empty(rows, **f32)
        self.states = torch.empty(bsz, heads, nch, vd, kd, **f32)   # value-major chunk-start states
        self.final = torch.empty(bsz, heads, kd, vd, **f32)
        frags = [None] * 5
        if mfma:
            k16, rb = kd // 16, (kd + 31) // 32
            frags = [torch.empty(chunks * 2 * k16 * 64 * 16, **b16),   # wrow
                     torch.empty(chunks * rb * 4 * 64 * 16, **b16),    # wcol
                     torch.empty(chunks * 2 * k16 * 64 * 8, **b16),    # krow
                     torch.empty(chunks * rb * 4 * 64 * 8, **b16),     # kcol
                     torch.empty(chunks * rb * 4 * 64 * 8, **b16) if q is not None else None]  # qcol
        self.out = torch.empty(bsz, tokens, heads, vd, device=dev, dtype=k.dtype) if q is not None else None
        self.inter = (kn, qn, w, u, delta, tri, gam, bet, self.states, self.final, *frags)
        self.saved = _lib.Saved(*(_ptr(t) for t in self.inter))
        self.geom = (chunk, offset, nch, q is not None, s0 is not None, mfma)
        self.timing_args = (kd, vd, chunk, tokens * bsz * heads, k.dtype, q is not None)
        self.tensors = (q, k, v, g, beta, s0f) + self.inter
        self.token = None
        if box is not None:  # a late read will use these intermediates
            box.args = (k, v, g, beta, s0f, chunk, offset, nch)
            box.saved = (kn, w, u, delta, tri, gam, bet, self.states, self.final, *frags)
            self.token = torch.zeros(1, device=dev)

    def outputs(self):
        return self.out, self.states, self.final, self.token


_N_SAVED = 21  # tensors a group saves: q, k, v, g, beta, s0 and its 15 intermediates


class _GroupGrad:
    """One scan group's backward: gradient buffers and the library structs."""

    def __init__(self, saved_tensors, geom, box, dout, dstates, dfinal, needs_dq: bool):
        _in_use_here(dout, dstates, dfinal)
        chunk, offset, nch, has_q, has_s0, mfma = geom
        (q, k, v, g, beta, s0f, kn, qn, w, u, delta, tri, gam, bet, states, final, *frags) = saved_tensors
        self.box = box
        self.late = box is not None and box.dout is not None
        if self.late:  # the late read's gradient joins this backward as its read
            q, qn, dout = box.q, box.qn, box.dout
            frags[4] = box.qcol
            has_q = True
            _in_use_here(q, qn, dout, box.qcol)
        bsz, tokens, heads, kd = k.shape
        vd = v.shape[-1]
        dev = k.device
        rows = bsz * heads * nch * _lib.CHUNK_ROWS
        f32 = dict(device=dev, dtype=torch.float32)
        want_read = has_q and dout is not None
        if want_read:
            dout = _contig_last(dout.to(k.dtype))
        # dd0 and o: value-major on the FMA path, fragment order over whole
        # 32-column strips on the MFMA path (like u).
        vcols = -(-vd // 32) * 32 if mfma else vd
        dd0 = torch.empty(rows * vcols, **f32) if want_read else None
        obuf = torch.empty(rows * vcols, **f32) if want_read else None
        ddelta = torch.empty(rows * vd, **f32)
        dhend = torch.empty(bsz * heads * nch * kd * vd, **f32)
        dw = torch.empty(rows * kd, **f32)
        act = dict(device=dev, dtype=k.dtype)  # the kernels round dq, dk, dv to the activation type
        dq = torch.empty(bsz, tokens, heads, kd, **act) if has_q else None
        dk = torch.empty(bsz, tokens, heads, kd, **act)
        dv = torch.empty(bsz, tokens, heads, vd, **act)
        dg = torch.empty(bsz, tokens, heads, **f32)
        db = torch.empty(bsz, tokens, heads, **f32)
        ds0 = torch.empty(bsz, heads, kd, vd, **f32)
        dstates = dstates.float().contiguous() if dstates is not None else None
        dfinal = dfinal.float().contiguous() if dfinal is not None else None
        self.prob = _problem(q, k, v, g, beta, s0f, chunk, offset)
        self.saved = _lib.Saved(*(_ptr(t) for t in (kn, qn, w, u, delta, tri, gam, bet, states, final, *frags)))
        self.grads = _lib.Grads(_lib.operand(dout if want_read else None), _ptr(dstates), _ptr(dfinal),
                                _ptr(dd0), _ptr(obuf), ddelta.data_ptr(), dhend.data_ptr(), dw.data_ptr(),
                                _lib.operand(dq), _lib.operand(dk), _lib.operand(dv),
                                _lib.operand(dg), _lib.operand(db), ds0.data_ptr())
        # Every buffer the library reads or writes stays referenced until the
        # call is enqueued and the record is released: a gradient this group
        # does not return (ds0 without an initial state, dq of a late read) is
        # still written, and memory dropped early would be handed to the next
        # group's buffers of a packed call before the kernels run.
        self.keep = (dout, dstates, dfinal, dd0, obuf, ddelta, dhend, dw, q, qn, frags[4], dq, ds0)
        self.timing_args = (kd, vd, chunk, tokens * bsz * heads, k.dtype, want_read)
        self.inj = dstates is not None
        dq_out = dq if (has_q and not self.late and needs_dq) else None
        self.result = (dq_out, dk, dv, dg, db, ds0 if has_s0 else None)

    def done(self):
        """The gradients to return; the record (and so its buffers) must live
        until the library call that uses it has been enqueued."""
        if self.late:  # dq of the late read was returned by the read itself
            self.box.release()
        return self.result


class _GDNScan(torch.autograd.Function):
    """One group of GDN scans; saved intermediates per include/gpa_hip.h."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, s0, chunk: int, offset: int, box=None):
        lib = _lib.load()
        # Outputs nobody differentiates (often the chunk-start states) reach the
        # backward as None, so it neither fills nor streams zero gradients.
        ctx.set_materialize_grads(False)
        grp = _Group(lib, q, k, v, g, beta, s0, chunk, offset, box)
        timing = profiling.forward_timing(*grp.timing_args)
        _lib.check(lib.gpa_gdn_forward(grp.prob, grp.saved, _lib.operand(grp.out), timing,
                                       _lib.stream_handle(k.device)), "gpa_gdn_forward")
        ctx.geom, ctx.box = grp.geom, box
        ctx.save_for_backward(*grp.tensors)
        return grp.outputs()

    @staticmethod
    def backward(ctx, dout, dstates, dfinal, dtoken=None):
        lib = _lib.load()
        gg = _GroupGrad(ctx.saved_tensors, ctx.geom, ctx.box, dout, dstates, dfinal, ctx.needs_input_grad[0])
        timing = profiling.backward_timing(*gg.timing_args)
        _lib.check(lib.gpa_gdn_backward(gg.prob, gg.saved, gg.grads, timing,
                                        _lib.stream_handle(ctx.saved_tensors[1].device)), "gpa_gdn_backward")
        return gg.done() + (None, None, None)


class _GDNScanMany(torch.autograd.Function):
    """Several independent groups of GDN scans in one library call
    (gpa_gdn_forward_many / gpa_gdn_backward_many): their state recurrences
    advance together in packed launches.  Inputs: a spec of (chunk, offset,
    box) per group, then q, k, v, g, beta, s0 of every group; outputs: out,
    states, final, token of every group."""

    @staticmethod
    def forward(ctx, spec, *flat):
        lib = _lib.load()
        ctx.set_materialize_grads(False)
        groups = [_Group(lib, *flat[6 * i:6 * i + 6], chunk, offset, box)
                  for i, (chunk, offset, box) in enumerate(spec)]
        n = len(groups)
        probs, saved, outs = (_lib.Problem * n)(), (_lib.Saved * n)(), (_lib.Operand * n)()
        for i, grp in enumerate(groups):
            probs[i], saved[i], outs[i] = grp.prob, grp.saved, _lib.operand(grp.out)
        timing = profiling.forward_timing_many([grp.timing_args for grp in groups])
        _lib.check(lib.gpa_gdn_forward_many(probs, saved, outs, n, timing, _lib.stream_handle(flat[1].device)),
                   "gpa_gdn_forward_many")
        ctx.geoms = [grp.geom for grp in groups]
        ctx.boxes = [box for _, _, box in spec]
        ctx.save_for_backward(*(t for grp in groups for t in grp.tensors))
        # inputs that several groups read (a write is an edge's key and another's value)
        seen: dict[int, list[int]] = {}
        for pos, t in enumerate(flat):
            if isinstance(t, torch.Tensor):
                seen.setdefault(id(t), []).append(pos)
        ctx.shared = [ps for ps in seen.values() if len(ps) > 1]
        return tuple(x for grp in groups for x in grp.outputs())

    @staticmethod
    def backward(ctx, *douts):
        lib = _lib.load()
        saved_t = ctx.saved_tensors
        n = len(ctx.geoms)
        groups = [_GroupGrad(saved_t[_N_SAVED * i:_N_SAVED * (i + 1)], ctx.geoms[i], ctx.boxes[i],
                             douts[4 * i], douts[4 * i + 1], douts[4 * i + 2], ctx.needs_input_grad[1 + 6 * i])
                  for i in range(n)]
        probs, saved, grads = (_lib.Problem * n)(), (_lib.Saved * n)(), (_lib.Grads * n)()
        for i, gg in enumerate(groups):
            probs[i], saved[i], grads[i] = gg.prob, gg.saved, gg.grads
        timing = profiling.backward_timing_many([gg.timing_args + (gg.inj,) for gg in groups])
        _lib.check(lib.gpa_gdn_backward_many(probs, saved, grads, n, timing,
                                             _lib.stream_handle(saved_t[1].device)), "gpa_gdn_backward_many")
        flat = [x for gg in groups for x in gg.done()]
        for ps in ctx.shared:  # one gradient per shared input, summed in one pass
            live = [p for p in ps if flat[p] is not None]
            if len(live) > 1:
                flat[live[0]] = _sum_many([flat[p] for p in live])
                for p in live[1:]:
                    flat[p] = None
        return (None,) + tuple(flat)


def _sum_many(xs: list[Tensor]) -> Tensor:
    """Elementwise sum of equally shaped tensors (gpa_sum_many: float32
    accumulation, one rounding); pairwise device adds where the kernel's
    alignment rules do not hold."""
    x0 = xs[0]
    per = 16 // x0.element_size()
    ok = (x0.dtype in _lib.DTYPE_CODES and x0.numel() % per == 0
          and all(x.shape == x0.shape and x.dtype == x0.dtype and x.is_contiguous() and x.data_ptr() % 16 == 0
                  for x in xs))
    if not ok:
        out = xs[0]
        for x in xs[1:]:
            out = out + x
        return out
    lib = _lib.load()
    out = torch.empty_like(x0)
    rest = list(xs)
    first = True
    while rest:
        take = rest[:_lib.SUM_MAX - (0 if first else 1)]
        rest = rest[len(take):]
        srcs = take if first else [out] + take
        arr = (ctypes.c_void_p * len(srcs))(*(x.data_ptr() for x in srcs))
        _lib.check(lib.gpa_sum_many(out.data_ptr(), arr, len(srcs), x0.numel(), _lib.DTYPE_CODES[x0.dtype],
                                    _lib.stream_handle(x0.device)), "gpa_sum_many")
        first = False
    return out


class _ReadBox:
    """What a scan forward without a query hands to its late read, and what
    the read's backward hands back to the scan's backward.

    The box never holds a tensor across a forward/backward gap: the scan's
    forward leaves its inputs and intermediates here (args, saved), the
    read's forward takes them into its own saved tensors and empties the box,
    and the read's backward leaves the query, its normalised forms and dO
    here for the scan's backward, which releases them.  So activation
    checkpointing, which drops and recomputes saved tensors, frees all of it."""

    def __init__(self):
        self.args = self.saved = None
        self.q = self.qn = self.qcol = self.dout = None

    def release(self):
        self.q = self.qn = self.qcol = self.dout = None


class _GDNRead(torch.autograd.Function):
    """u(q)^T S of a scan that ran without a query (gpa_gdn_read).  Its
    backward computes dq alone (gpa_gdn_read_backward) and leaves dO for the
    scan's backward, which autograd runs after it: the read consumes the
    scan's `token` output."""

    @staticmethod
    def forward(ctx, q, token, box):
        lib = _lib.load()
        if box.args is None:
            raise ValueError("gdn_scan_deferred: the read of a scan can be taken once")
        k, v, g, beta, s0f, chunk, offset, nch = box.args
        inter = box.saved
        kn, w, u, delta, tri, gam, bet, states, final, *frags = inter
        _in_use_here(q, k, v, g, beta, s0f, kn, delta, gam, states, frags[3])
        bsz, tokens, heads, kd = k.shape
        vd = v.shape[-1]
        dev = k.device
        chunks = bsz * heads * nch
        qn = torch.empty(chunks * _lib.CHUNK_ROWS * kd, device=dev, dtype=torch.float32)
        qcol = torch.empty(chunks * ((kd + 31) // 32) * 4 * 64 * 8, device=dev, dtype=torch.bfloat16)
        out = torch.empty(bsz, tokens, heads, vd, device=dev, dtype=k.dtype)
        prob = _problem(q, k, v, g, beta, s0f, chunk, offset)
        saved = _read_saved(inter, qn, qcol)
        _lib.check(lib.gpa_gdn_read(prob, saved, _lib.operand(out), _lib.stream_handle(dev)), "gpa_gdn_read")
        ctx.box, ctx.geom = box, (chunk, offset)
        ctx.save_for_backward(q, qn, qcol, k, v, g, beta, s0f, *inter)
        box.args = box.saved = None
        return out

    @staticmethod
    def backward(ctx, dout):
        lib = _lib.load()
        box = ctx.box
        q, qn, qcol, k, v, g, beta, s0f, *inter = ctx.saved_tensors
        chunk, offset = ctx.geom
        dout = dout.to(k.dtype).contiguous()
        dq = torch.empty(q.shape, device=q.device, dtype=torch.float32)
        prob = _problem(q, k, v, g, beta, s0f, chunk, offset)
        saved = _read_saved(inter, qn, qcol)
        _lib.check(lib.gpa_gdn_read_backward(prob, saved, _lib.operand(dout), _lib.operand(dq),
                                             _lib.stream_handle(q.device)), "gpa_gdn_read_backward")
        # the scan's backward takes the read's gradient as its own read
        box.q, box.qn, box.qcol, box.dout = q, qn, qcol, dout
        return dq.to(q.dtype), torch.zeros(1, device=q.device), None


def _read_saved(inter, qn, qcol):
    """The scan's saved intermediates (kn, w, u, delta, tri, gam, bet,
    states, final, wrow, wcol, krow, kcol, qcol) with the read's qn and qcol."""
    kn, w, u, delta, tri, gam, bet, states, final, *frags = inter
    frags = list(frags)
    frags[4] = qcol
    return _lib.Saved(*(_ptr(t) for t in (kn, qn, w, u, delta, tri, gam, bet, states, final, *frags)))


def gdn_scan_hip(q: Tensor | None, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, s0: Tensor | None,
                 *, chunk: int, offset: int = 0):
    """Chunked GDN scan of B*H streams on the GPU.

    q, k [B,T,H,K] (q may be None), v [B,T,H,V] in float32 or bfloat16 with a
    contiguous last axis; g, beta [B,T,H] float32 (any strides, e.g. expanded
    constants); s0 [B,H,K,V] (None = zeros).  Returns
    (out [B,T,H,V] or None, states [B,H,N,K,V], final [B,H,K,V]) where
    states[:, :, n] is the state at the start of chunk n and chunk 0 begins
    `offset` positions before token 0.
    """
    _lib.require_device(k)
    if k.dtype not in _lib.DTYPE_CODES or v.dtype != k.dtype or (q is not None and q.dtype != k.dtype):
        raise ValueError("gdn_scan_hip: q/k/v must share float32 or bfloat16")
    if k.ndim != 4 or v.ndim != 4 or v.shape[:3] != k.shape[:3] or (q is not None and q.shape != k.shape):
        raise ValueError("gdn_scan_hip: expected q,k [B,T,H,K] and v [B,T,H,V]")
    if g.shape != k.shape[:3] or beta.shape != k.shape[:3]:
        raise ValueError("gdn_scan_hip: g and beta must be [B,T,H]")
    if k.shape[-1] > _lib.MAX_KDIM or v.shape[-1] > _lib.MAX_VDIM:
        raise ValueError(f"gdn_scan_hip: widths above K={_lib.MAX_KDIM}, V={_lib.MAX_VDIM} are not built")
    if s0 is not None and s0.shape != (k.shape[0], k.shape[2], k.shape[3], v.shape[3]):
        raise ValueError("gdn_scan_hip: s0 must be [B,H,K,V]")
    if not 1 <= chunk <= _lib.CHUNK_ROWS or not 0 <= offset < chunk:
        raise ValueError("gdn_scan_hip: need 1 <= chunk <= 64 and 0 <= offset < chunk")
    q = _contig_last(q) if q is not None else None
    k, v = _contig_last(k), _contig_last(v)
    g, beta = g.float(), beta.float()
    out, states_vk, final, _ = _GDNScan.apply(q, k, v, g, beta, s0, chunk, offset)
    return out, states_vk.transpose(-1, -2), final


def gdn_scan_noalloc(q: Tensor | None, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, s0: Tensor | None,
                     *, chunk: int, offset: int = 0, out: Tensor | None = None,
                     final: Tensor | None = None) -> tuple[Tensor | None, Tensor]:
    """Inference forward of `gdn_scan_hip` through the library's allocation-free
    entry point (gpa_gdn_scan_noalloc): the library allocates nothing; its
    intermediates live in a fixed per-device scratch array (64 MiB), and
    problems that need more are rejected.  Pass `out` ([B,T,H,V], the input
    dtype) and `final` ([B,H,K,V] float32, contiguous) to allocate nothing
    here either (e.g. under graph capture).  No autograd.  Calls overlapping
    on one device share the scratch array and must not run concurrently."""
    _lib.require_device(k)
    if k.dtype not in _lib.DTYPE_CODES or v.dtype != k.dtype or (q is not None and q.dtype != k.dtype):
        raise ValueError("gdn_scan_noalloc: q/k/v must share float32 or bfloat16")
    if k.ndim != 4 or v.ndim != 4 or v.shape[:3] != k.shape[:3] or (q is not None and q.shape != k.shape):
        raise ValueError("gdn_scan_noalloc: expected q,k [B,T,H,K] and v [B,T,H,V]")
    if g.shape != k.shape[:3] or beta.shape != k.shape[:3]:
        raise ValueError("gdn_scan_noalloc: g and beta must be [B,T,H]")
    if not 1 <= chunk <= _lib.CHUNK_ROWS or not 0 <= offset < chunk:
        raise ValueError("gdn_scan_noalloc: need 1 <= chunk <= 64 and 0 <= offset < chunk")
    _no_autograd("gdn_scan_noalloc", q, k, v, g, beta, s0)
    bsz, tokens, heads, kd = k.shape
    vd = v.shape[-1]
    if s0 is not None and s0.shape != (bsz, heads, kd, vd):
        raise ValueError("gdn_scan_noalloc: s0 must be [B,H,K,V]")
    q = _contig_last(q) if q is not None else None
    k, v = _contig_last(k), _contig_last(v)
    g, beta = g.float(), beta.float()
    s0f = _f32_state(s0) if s0 is not None else None
    if final is None:
        final = torch.empty(bsz, heads, kd, vd, device=k.device, dtype=torch.float32)
    elif final.shape != (bsz, heads, kd, vd) or final.dtype != torch.float32 or not final.is_contiguous():
        raise ValueError("gdn_scan_noalloc: final must be a contiguous float32 [B,H,K,V] tensor")
    if q is not None and out is None:
        out = torch.empty(bsz, tokens, heads, vd, device=k.device, dtype=k.dtype)
    elif q is not None and (out.shape != (bsz, tokens, heads, vd) or out.dtype != k.dtype or out.stride(-1) != 1):
        raise ValueError("gdn_scan_noalloc: out must be [B,T,H,V] in the input dtype with a contiguous last axis")
    prob = _problem(q, k, v, g, beta, s0f, chunk, offset)
    _lib.check(_lib.load().gpa_gdn_scan_noalloc(prob, _lib.operand(out if q is not None else None), final.data_ptr(),
                             _lib.stream_handle(k.device)), "gpa_gdn_scan_noalloc")
    return (out if q is not None else None), final


def read_supported(k: Tensor, v: Tensor) -> bool:
    """Whether gdn_scan_deferred can take a late read of these keys/values
    (bf16, K a multiple of 16 up to 256, V a multiple of 8 up to 256)."""
    kd, vd = k.shape[-1], v.shape[-1]
    return k.dtype == torch.bfloat16 and kd % 16 == 0 and kd <= 256 and vd % 8 == 0 and vd <= 256


def gdn_scan_deferred(k: Tensor, v: Tensor, g: Tensor, beta: Tensor, s0: Tensor | None, *, chunk: int,
                      offset: int = 0):
    """`gdn_scan_hip(None, ...)` whose read comes later: returns (states,
    final, read), where read(q) [B,T,H,K] gives the out that
    `gdn_scan_hip(q, k, v, g, beta, s0, ...)` would, without running the state
    recurrence again.  The gradients of the read and of the scan's own outputs
    are taken by one scan backward.  Keys/values must pass `read_supported`."""
    if not read_supported(k, v):
        raise ValueError("gdn_scan_deferred: needs bf16, K % 16 == 0 <= 256 and V % 8 == 0 <= 256")
    box = _ReadBox()
    _, states_vk, final, token = _GDNScan.apply(None, _contig_last(k), _contig_last(v), g.float(), beta.float(),
                                                s0, chunk, offset, box)

    def read(q: Tensor) -> Tensor:
        if q.shape != k.shape or q.dtype != k.dtype:
            raise ValueError("gdn_scan_deferred: the query must match the keys' shape and dtype")
        return _GDNRead.apply(_contig_last(q), token, box)

    return states_vk.transpose(-1, -2), final, read


def _check_group(q, k, v, g, beta, s0, chunk, offset, name):
    _lib.require_device(k)
    if k.dtype not in _lib.DTYPE_CODES or v.dtype != k.dtype or (q is not None and q.dtype != k.dtype):
        raise ValueError(f"{name}: q/k/v must share float32 or bfloat16")
    if k.ndim != 4 or v.ndim != 4 or v.shape[:3] != k.shape[:3] or (q is not None and q.shape != k.shape):
        raise ValueError(f"{name}: expected q,k [B,T,H,K] and v [B,T,H,V]")
    if g.shape != k.shape[:3] or beta.shape != k.shape[:3]:
        raise ValueError(f"{name}: g and beta must be [B,T,H]")
    if k.shape[-1] > _lib.MAX_KDIM or v.shape[-1] > _lib.MAX_VDIM:
        raise ValueError(f"{name}: widths above K={_lib.MAX_KDIM}, V={_lib.MAX_VDIM} are not built")
    if s0 is not None and s0.shape != (k.shape[0], k.shape[2], k.shape[3], v.shape[3]):
        raise ValueError(f"{name}: s0 must be [B,H,K,V]")
    if not 1 <= chunk <= _lib.CHUNK_ROWS or not 0 <= offset < chunk:
        raise ValueError(f"{name}: need 1 <= chunk <= 64 and 0 <= offset < chunk")


def gdn_scan_many(groups):
    """Several independent groups of `gdn_scan_hip` / `gdn_scan_deferred` in
    one library call whose state recurrences advance together (the packed
    level and edge scans of the reference, packed.py:77, 121, 155, and the
    paired A/B scans of a level, staged.py:14-35).  `groups` holds dicts with
    q (None for a deferred group), k, v, g, beta, s0, chunk, offset and
    optionally deferred=True (then q must be None); at most
    `_lib.GDN_MAX_PACK` groups on one device.  Returns, in order, (out, states
    [B,H,N,K,V], final) of each plain group and (states, final, read) of each
    deferred group, exactly as the one-group functions."""
    if not groups:
        return []
    if len(groups) > _lib.GDN_MAX_PACK:
        raise ValueError(f"gdn_scan_many: at most {_lib.GDN_MAX_PACK} groups per call")
    spec, flat, deferred = [], [], []
    for grp in groups:
        q, k, v, g, beta, s0 = (grp.get(x) for x in ("q", "k", "v", "g", "beta", "s0"))
        chunk, offset, late = grp["chunk"], grp.get("offset", 0), grp.get("deferred", False)
        _check_group(q, k, v, g, beta, s0, chunk, offset, "gdn_scan_many")
        if late and (q is not None or not read_supported(k, v)):
            raise ValueError("gdn_scan_many: a deferred group takes no query and needs read_supported keys/values")
        box = _ReadBox() if late else None
        spec.append((chunk, offset, box))
        deferred.append(late)
        flat += [_contig_last(q) if q is not None else None, _contig_last(k), _contig_last(v), g.float(),
                 beta.float(), s0]
    res = _GDNScanMany.apply(tuple(spec), *flat)
    outs = []
    for i, late in enumerate(deferred):
        out, states_vk, final, token = res[4 * i:4 * i + 4]
        if not late:
            outs.append((out, states_vk.transpose(-1, -2), final))
            continue
        k = flat[6 * i + 1]
        box = spec[i][2]

        def read(q: Tensor, k=k, token=token, box=box) -> Tensor:
            if q.shape != k.shape or q.dtype != k.dtype:
                raise ValueError("gdn_scan_deferred: the query must match the keys' shape and dtype")
            return _GDNRead.apply(_contig_last(q), token, box)
        outs.append((states_vk.transpose(-1, -2), final, read))
    return outs


def token_step_supported(k: Tensor, v: Tensor) -> bool:
    """Whether `gdn_token_hip` takes these keys/values: one token, float32 or
    bfloat16, K and V up to 256, V a multiple of 4."""
    return (k.dtype in _lib.DTYPE_CODES and k.ndim == 4 and k.shape[1] == 1 and k.shape[-1] <= 256
            and v.shape[-1] <= 256 and v.shape[-1] % 4 == 0)


def _token_state(s: Tensor) -> Tensor:
    """A float32 [B,H,K,V] state the token kernel reads in 16-byte vectors."""
    s = _f32_state(s)
    if s.data_ptr() % 16 or s.stride(0) % 4 or s.stride(1) % 4:
        s = s.contiguous()
    return s


def _no_autograd(name: str, *tensors) -> None:
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors):
        raise RuntimeError(f"{name} has no backward: call it under torch.no_grad() or inference_mode()")


def _token_call(q, k, v, g, beta, s0):
    """Checked arguments of one token step: (problem, final, out, tensors kept alive)."""
    _lib.require_device(k)
    if not token_step_supported(k, v) or v.dtype != k.dtype or (q is not None and q.dtype != k.dtype):
        raise ValueError("gdn_token_hip: needs one float32/bfloat16 token, K, V <= 256 and V % 4 == 0")
    if v.shape[:3] != k.shape[:3] or (q is not None and q.shape != k.shape):
        raise ValueError("gdn_token_hip: expected q,k [B,1,H,K] and v [B,1,H,V]")
    if g.shape != k.shape[:3] or beta.shape != k.shape[:3]:
        raise ValueError("gdn_token_hip: g and beta must be [B,1,H]")
    bsz, _, heads, kd = k.shape
    vd = v.shape[-1]
    if s0 is not None and s0.shape != (bsz, heads, kd, vd):
        raise ValueError("gdn_token_hip: s0 must be [B,H,K,V]")
    _no_autograd("gdn_token_hip", q, k, v, g, beta, s0)
    q = _contig_last(q) if q is not None else None
    k, v = _contig_last(k), _contig_last(v)
    g, beta = g.float(), beta.float()
    s0f = _token_state(s0) if s0 is not None else None
    final = torch.empty(bsz, heads, kd, vd, device=k.device, dtype=torch.float32)
    out = torch.empty(bsz, 1, heads, vd, device=k.device, dtype=k.dtype) if q is not None else None
    return _problem(q, k, v, g, beta, s0f, 1, 0), final, out, (q, k, v, g, beta, s0f)


def gdn_token_many(calls) -> list[tuple[Tensor | None, Tensor]]:
    """`gdn_token_hip` of several independent groups, for inference: one
    launch per element type, every key width in it (`gpa_gdn_token_step_many`),
    instead of one per group.  `calls` holds gdn_token_hip's argument tuples
    (q, k, v, g, beta, s0), at most `_lib.TOKEN_MAX_PACK` of them, on one
    device; returns [(out, final)] in the same order."""
    if not calls:
        return []
    if len(calls) > _lib.TOKEN_MAX_PACK:
        raise ValueError(f"gdn_token_many: at most {_lib.TOKEN_MAX_PACK} groups per call")
    lib = _lib.load()
    n = len(calls)
    probs, finals, outs = (_lib.Problem * n)(), (ctypes.c_void_p * n)(), (_lib.Operand * n)()
    keep, results = [], []
    for i, call in enumerate(calls):
        prob, final, out, alive = _token_call(*call)
        probs[i], finals[i], outs[i] = prob, final.data_ptr(), _lib.operand(out)
        keep.append(alive)
        results.append((out, final))
    _lib.check(lib.gpa_gdn_token_step_many(probs, finals, outs, n, _lib.stream_handle(calls[0][1].device)),
               "gpa_gdn_token_step_many")
    return results


def gdn_token_hip(q: Tensor | None, k: Tensor, v: Tensor, g: Tensor, beta: Tensor,
                  s0: Tensor | None) -> tuple[Tensor | None, Tensor]:
    """One token of B*H GDN streams without autograd (inference decode):
    `gdn_update` then `memory_read` of the reference (src/gpa/ops.py:29-46),
    i.e. `gdn_scan_hip` at T = 1 without the intermediates a backward needs.
    q (may be None), k [B,1,H,K], v [B,1,H,V], g/beta [B,1,H] (any strides),
    s0 [B,H,K,V] or None = zeros.  Returns (out [B,1,H,V] or None, final
    [B,H,K,V] float32).  Keys/values must pass `token_step_supported`."""
    lib = _lib.load()
    prob, final, out, alive = _token_call(q, k, v, g, beta, s0)
    _lib.check(lib.gpa_gdn_token_step(prob, final.data_ptr(), _lib.operand(out), _lib.stream_handle(k.device)),
               "gpa_gdn_token_step")
    return out, final


def gdn_token_read(q: Tensor, state: Tensor) -> Tensor:
    """u(q)^T S of one token per stream (reference ops.py:45-46): q [B,1,H,K],
    S [B,H,K,V] float32 -> [B,1,H,V] in q's dtype; no autograd."""
    _lib.require_device(q)
    bsz, tokens, heads, kd = q.shape
    if tokens != 1 or state.shape != (bsz, heads, kd, state.shape[-1]):
        raise ValueError("gdn_token_read: expected q [B,1,H,K] and S [B,H,K,V]")
    if q.dtype not in _lib.DTYPE_CODES or kd > 256 or state.shape[-1] > 256 or state.shape[-1] % 4:
        raise ValueError("gdn_token_read: needs float32/bfloat16, K, V <= 256 and V % 4 == 0")
    _no_autograd("gdn_token_read", q, state)
    lib = _lib.load()
    q = _contig_last(q)
    sf = _token_state(state)
    vd = sf.shape[-1]
    out = torch.empty(bsz, 1, heads, vd, device=q.device, dtype=q.dtype)
    prob = _lib.Problem(bsz, heads, 1, 0, 1, kd, vd, _lib.DTYPE_CODES[q.dtype], _lib.operand(q), _lib.operand(None),
                        _lib.operand(None), _lib.operand(None), _lib.operand(None), sf.data_ptr(), sf.stride(0),
                        sf.stride(1))
    _lib.check(lib.gpa_gdn_token_step(prob, None, _lib.operand(out), _lib.stream_handle(q.device)),
               "gpa_gdn_token_step")
    return out


# --------------------------------------------------------------------------- reference-signature operators
def _check_scan_args(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor) -> None:
    """The reference's argument checks and messages (src/gpa/ops.py:52-55)."""
    if q.shape != k.shape or q.shape[:3] != v.shape[:3]:
        raise ValueError("q/k must share [B,T,H,K], v must share [B,T,H]")
    if g.shape != q.shape[:3] or beta.shape != q.shape[:3]:
        raise ValueError("g and beta must be scalar per token/head: [B,T,H]")


def gdn_scan(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, initial_state: Tensor, *,
             backend: str = "hip", chunk_size: int = 64) -> tuple[Tensor, Tensor]:
    """Drop-in for the reference `gdn_scan` (src/gpa/ops.py:49-85): q,k [B,T,H,K],
    v [B,T,H,V], scalar g/beta [B,T,H], initial_state [B,H,K,V] key-major.
    Returns (out [B,T,H,V] in q's dtype, final state [B,H,K,V] float32).  Empty
    T returns (empty, initial_state) unchanged, as the reference does."""
    _check_scan_args(q, k, v, g, beta)
    if q.shape[1] == 0:
        return v.new_empty(*v.shape), initial_state
    if backend != "hip":
        raise ValueError(f"unknown backend: {backend}")
    out, _, final = gdn_scan_hip(q, k, v, g, beta, initial_state, chunk=chunk_size)
    return out, final


def gdn_update(state: Tensor, key: Tensor, value: Tensor, log_gate: Tensor, beta: Tensor) -> Tensor:
    """One GDN step of every stream (src/gpa/ops.py:29-42): S [B,H,K,V], k [B,H,K],
    v [B,H,V], scalar g/beta [B,H]; the HIP scan over a single token."""
    if log_gate.shape != key.shape[:-1] or beta.shape != key.shape[:-1]:
        raise ValueError("GDN scalar gates/beta must be [B,H], not vector gates")
    _, _, final = gdn_scan_hip(None, key[:, None], value[:, None], log_gate[:, None], beta[:, None], state,
                               chunk=1)
    return final.to(state.dtype)


def memory_read(query: Tensor, state: Tensor) -> Tensor:
    """u(q)^T S per stream (src/gpa/ops.py:45-46): q [B,H,K], S [B,H,K,V] -> [B,H,V]."""
    _lib.require_device(query)
    qn = torch.nn.functional.normalize(query.float(), p=2, dim=-1, eps=1e-6).to(query.dtype)
    return torch.matmul(qn.to(state.dtype)[..., None, :], state)[..., 0, :].to(query.dtype)


class TwoStageState:
    """Carried state of `two_stage_gdn` (src/gpa/ops.py:140-143): inner [B,H,Dk,M],
    outer [B,H,M,Dv], key-major."""
    __slots__ = ("inner", "outer")

    def __init__(self, inner: Tensor, outer: Tensor):
        self.inner, self.outer = inner, outer


def two_stage_gdn(q: Tensor, k: Tensor, slots: Tensor, v: Tensor, gi: Tensor, bi: Tensor, go: Tensor,
                  bo: Tensor, state: TwoStageState, *, route_weight: Tensor | None = None,
                  query_weight: Tensor | None = None, query_scale: float = 1 / 16,
                  backend: str = "hip") -> tuple[Tensor, TwoStageState]:
    """GDN(softmax(GDN(q,k,slots)) W_rs + q W_qs/16, slots, v) (src/gpa/ops.py:146-163)."""
    inner, a = gdn_scan(q, k, slots, gi, bi, state.inner, backend=backend)
    route = inner.float().softmax(-1).to(q.dtype)
    if route_weight is not None:
        route = torch.nn.functional.linear(route, route_weight.to(route.dtype))
    if query_weight is not None:
        route = route + query_scale * torch.nn.functional.linear(q, query_weight.to(q.dtype))
    out, b = gdn_scan(route, slots, v, go, bo, state.outer, backend=backend)
    return out, TwoStageState(a, b)
