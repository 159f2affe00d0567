"""Fused route reader of one target level (`gpa_route_forward/backward`).

The default read of the reference's `_bridge` (src/gpa/attention.py:225-262,
legacy branch :236-240), for every token of every head of one target level j:

    inc = sum_e w_e m_e;  z = centre(inc) / rms;  r0 = softmax(base + gain tanh z)
    r1  = r0 + mlp_gain gelu(r0 U) D;   qo = r1 W_rs + query_scale q W_qs

`route_reader` returns (qo, r1) in the activation dtype and is differentiable
in every input: the base logits, the messages, q, the edge weights, both gains
and the four weight matrices.  With `paper_product_read` (and
`relation_marginal`) the relation read is the product form of
attention.py:231-236 instead: `product_read` (gpa_product_read_forward /
_backward) forms the base logits from the messages, and `route_reader` then
runs with no incoming messages.  With shared_query_center the query weight is
W_qs + center^T / query_scale (attention.py:254-256), formed by the caller.
`rsa_update` rescales r1 by its clamped L1 norm before the query product
(attention.py:251-253) and `balanced_bridge` mixes the unit rows of the two
query halves with mix = .1 + .8 sigmoid(bridge_mix_raw) (attention.py:256-259),
both inside the kernels, with gradients to mix.  Only non-linear slot
features keep the device glue.
"""
from __future__ import annotations

import torch
from torch import Tensor

from . import _lib, params


def supported(cfg, dtype: torch.dtype, slots: int) -> bool:
    return (dtype in _lib.DTYPE_CODES and cfg.slot_feature == "linear"
            and slots <= _lib.ROUTE_MAX_WIDTH and cfg.key_dim <= _lib.ROUTE_MAX_WIDTH
            and cfg.levels - 1 <= _lib.ROUTE_MAX_INCOMING)


def _pad(x: int, m: int) -> int:
    return (x + m - 1) // m * m


def _pack(w: Tensor, dtype: torch.dtype, transpose: bool) -> Tensor:
    """[H,K,N] weight -> [H,N32,K16] rows of the contraction for each output
    column (transpose=True), or [H,K,N] -> [H,K32,N16] (transpose=False:
    output column = K, contraction = N); rounded to `dtype`, zero padded.
    Inside params.frozen() a leaf weight (a parameter) is packed once per
    scope; otherwise, and for a weight computed in the call, it is packed
    afresh."""
    if not w.is_leaf:
        return _pack_now(w, dtype, transpose)
    return params.derived(("route_pack", id(w), dtype, transpose), (w,), lambda: _pack_now(w, dtype, transpose))


def _pack_now(w: Tensor, dtype: torch.dtype, transpose: bool) -> Tensor:
    w = w.detach()
    if transpose:
        w = w.transpose(1, 2)
    h, n, k = w.shape
    pn, pk = _pad(n, 32), _pad(k, 16)
    if (pn, pk) == (n, k):  # no padding: the rounding and the transpose are one copy
        out = torch.empty(h, n, k, device=w.device, dtype=dtype)
        out.copy_(w)
        return out
    out = torch.zeros(h, pn, pk, device=w.device, dtype=dtype)
    out[:, :n, :k] = w
    return out


def _operand(t: Tensor | None) -> _lib.Operand:
    return _lib.operand(t)


def _rows_operand(t: Tensor, tokens: int) -> _lib.Operand:
    """A [H][R][M] row buffer addressed as [B,T,H,M] (r = b*T + t)."""
    heads, rows, m = t.shape
    return _lib.Operand(t.data_ptr(), tokens * m, m, rows * m)


def _problem(base, q, edge_w, gain, mlp_gain, msgs, query_scale, weights, outs, saved, flags=(0, 0),
             mix=None, halves=(None, None)):
    bsz, tokens, heads, dk = q.shape
    p = _lib.RouteProblem()
    p.batch, p.tokens, p.heads, p.slots, p.key_dim = bsz, tokens, heads, base.shape[-1], dk
    p.incoming, p.dtype, p.query_scale = len(msgs), _lib.DTYPE_CODES[q.dtype], float(query_scale)
    p.base, p.q = _operand(base), _operand(q)
    for e, m in enumerate(msgs):
        p.msg[e] = _operand(m)
    p.edge_weight = edge_w.data_ptr() if msgs else None
    p.gain, p.mlp_gain = gain.data_ptr(), mlp_gain.data_ptr()
    for name, w in weights.items():
        setattr(p, name, w.data_ptr())
    p.qo, p.route = _operand(outs[0]), _operand(outs[1])
    p.r0, p.h1, p.hd = (t.data_ptr() for t in saved)
    p.rsa, p.balanced = flags
    if flags[1]:
        p.mix, p.qr, p.qdir = mix.data_ptr(), halves[0].data_ptr(), halves[1].data_ptr()
    return p


def _forward_problem(base, q, edge_w, gain, mlp_gain, up, down, rs, qs, query_scale, msgs, flags=(0, 0),
                     mix=None):
    """The forward problem of one target level and every tensor it points
    into: (problem, (base, q, edge_w, g, mg, msgs, packed weights, mix), (qo,
    route), saved rows (r0, h1, hd[, qr, qdir])).  The caller keeps these
    alive until the launch."""
    dtype = q.dtype
    bsz, tokens, heads, _ = q.shape
    m = base.shape[-1]
    rows = bsz * tokens
    base = base.float().contiguous()
    q = q.contiguous()
    msgs = tuple(x.to(dtype).contiguous() for x in msgs)
    edge_w = edge_w.detach().float().contiguous() if msgs else None
    g, mg = gain.detach().float().contiguous(), mlp_gain.detach().float().contiguous()
    weights = {"up_t": _pack(up, dtype, True), "down_t": _pack(down, dtype, True),
               "rs_t": _pack(rs, dtype, True), "qs_t": _pack(qs, dtype, True)}
    qo = torch.empty(bsz, tokens, heads, m, device=q.device, dtype=dtype)
    route = torch.empty_like(qo)
    saved = (torch.empty(heads, rows, m, device=q.device, dtype=dtype),
             torch.empty(heads, rows, 2 * m, device=q.device, dtype=dtype),
             torch.empty(heads, rows, m, device=q.device, dtype=dtype))
    halves = (None, None)
    if flags[1]:
        mix = mix.detach().float().contiguous()
        halves = tuple(torch.empty(heads, rows, m, device=q.device, dtype=dtype) for _ in range(2))
    prob = _problem(base, q, edge_w, g, mg, msgs, query_scale, weights, (qo, route), saved, flags, mix, halves)
    if flags[1]:
        saved = saved + halves
    return prob, (base, q, edge_w, g, mg, msgs, weights, mix), (qo, route), saved


class _RouteReader(torch.autograd.Function):
    @staticmethod
    def forward(ctx, base, q, edge_w, gain, mlp_gain, up, down, rs, qs, query_scale, flags, mix, *msgs):
        _lib.require_device(q)
        ctx.set_materialize_grads(False)
        lib = _lib.load()
        prob, (base, q, edge_w, g, mg, msgs, packed, mix_f), (qo, route), saved = _forward_problem(
            base, q, edge_w, gain, mlp_gain, up, down, rs, qs, query_scale, msgs, flags, mix)
        _lib.check(lib.gpa_route_forward(prob, _lib.stream_handle(q.device)), "gpa_route_forward")
        del packed
        ctx.query_scale = query_scale
        ctx.flags = flags
        ctx.n_in = len(msgs)
        ctx.param_dtypes = (edge_w.dtype if msgs else None, gain.dtype, mlp_gain.dtype,
                            up.dtype, down.dtype, rs.dtype, qs.dtype, mix.dtype if flags[1] else None)
        halves = saved[3:] if flags[1] else (None, None)
        ctx.save_for_backward(base, q, edge_w if msgs else None, g, mg, up, down, rs, qs, route, *saved[:3],
                              mix_f, *halves, *msgs)
        return qo, route

    @staticmethod
    def backward(ctx, dqo, droute):
        lib = _lib.load()
        (base, q, edge_w, g, mg, up, down, rs, qs, route, r0, h1, hd, mix, qr, qdir,
         *msgs) = ctx.saved_tensors
        flags = ctx.flags
        dtype = q.dtype
        bsz, tokens, heads, dk = q.shape
        m = base.shape[-1]
        rows = bsz * tokens
        dev = q.device
        if dqo is None:
            dqo = torch.zeros_like(route)
        dqo = dqo.to(dtype).contiguous()
        droute = droute.to(dtype).contiguous() if droute is not None else None
        weights = {"up_t": None, "down_t": None, "rs_t": None, "qs_t": None,
                   "up": _pack(up, dtype, False), "down": _pack(down, dtype, False),
                   "rs": _pack(rs, dtype, False), "qs": _pack(qs, dtype, False)}
        prob = _problem(base, q, edge_w, g, mg, msgs, ctx.query_scale,
                        {k: v for k, v in weights.items() if v is not None},
                        (route, route), (r0, h1, hd), flags, mix, (qr, qdir))
        dbase = torch.empty_like(base)
        dmsgs = [torch.empty_like(x) for x in msgs]
        dq = torch.empty_like(q)
        dh1 = torch.empty(heads, rows, 2 * m, device=dev, dtype=dtype)
        dhd = torch.empty(heads, rows, m, device=dev, dtype=dtype)
        dqs = torch.empty(heads, rows, m, device=dev, dtype=dtype)
        hg = torch.empty(heads, rows, 2 * m, device=dev, dtype=dtype)
        blocks = (rows + _lib.ROUTE_ROWS - 1) // _lib.ROUTE_ROWS
        partials = torch.empty(blocks, heads, 2 + len(msgs), device=dev, dtype=torch.float32)
        gr = _lib.RouteGrads()
        gr.dqo, gr.droute, gr.dbase, gr.dq = (_operand(dqo), _operand(droute), _operand(dbase), _operand(dq))
        for e, x in enumerate(dmsgs):
            gr.dmsg[e] = _operand(x)
        gr.dh1, gr.dhd, gr.dqs, gr.partials = dh1.data_ptr(), dhd.data_ptr(), dqs.data_ptr(), partials.data_ptr()
        gr.hg = hg.data_ptr()
        if flags[1]:
            dqr, ddir = torch.empty_like(qr), torch.empty_like(qdir)
            mix_parts = torch.empty(blocks, heads, device=dev, dtype=torch.float32)
            gr.dqr, gr.ddir = _rows_operand(dqr, tokens), _rows_operand(ddir, tokens)
            gr.mix_partials = mix_parts.data_ptr()
        stream = _lib.stream_handle(dev)
        _lib.check(lib.gpa_route_backward(prob, gr, stream), "gpa_route_backward")
        d_up = torch.empty(heads, m, 2 * m, device=dev, dtype=torch.float32)
        d_down = torch.empty(heads, 2 * m, m, device=dev, dtype=torch.float32)
        d_rs = torch.empty(heads, m, m, device=dev, dtype=torch.float32)
        d_qs = torch.empty(heads, dk, m, device=dev, dtype=torch.float32)
        _lib.check(lib.gpa_route_weight_grads(prob, gr, d_up.data_ptr(), d_down.data_ptr(), d_rs.data_ptr(),
                                              d_qs.data_ptr(), stream), "gpa_route_weight_grads")
        sums = partials.sum(0)
        dt = ctx.param_dtypes
        d_edge = sums[:, 2:].t().contiguous().to(dt[0]) if msgs else None
        d_mix = mix_parts.sum(0).to(dt[7]) if flags[1] else None
        return (dbase, dq, d_edge, sums[:, 1].to(dt[1]), sums[:, 0].to(dt[2]), d_up.to(dt[3]), d_down.to(dt[4]),
                d_rs.to(dt[5]), d_qs.to(dt[6]), None, None, d_mix, *dmsgs)


def route_reader_many(reads) -> list[tuple[Tensor, Tensor]]:
    """`route_reader` of several target levels, for inference (no autograd):
    one launch where the library can pack them (`gpa_route_forward_many`:
    bf16 one-token calls), else one per level.  `reads` holds route_reader's
    argument tuples; returns [(qo, route)] in the same order."""
    if not reads:
        return []
    if torch.is_grad_enabled():
        raise RuntimeError("route_reader_many is for inference: call it under torch.no_grad()")
    if len(reads) > _lib.ROUTE_MAX_PACK:
        raise ValueError(f"route_reader_many: at most {_lib.ROUTE_MAX_PACK} levels")
    lib = _lib.load()
    probs = (_lib.RouteProblem * len(reads))()
    keep, outs = [], []
    for i, read in enumerate(reads):
        base, q, edge_w, gain, mlp_gain, up, down, rs, qs, query_scale, msgs = read[:11]
        rsa, mix = (read[11], read[12]) if len(read) > 11 else (False, None)
        _lib.require_device(q)
        if not msgs:
            edge_w = gain.new_zeros(0, gain.shape[0])
        prob, inputs, out, saved = _forward_problem(base, q, edge_w, gain, mlp_gain, up, down, rs, qs,
                                                    query_scale, msgs, (int(rsa), int(mix is not None)), mix)
        probs[i] = prob
        keep.append((inputs, saved))
        outs.append(out)
    _lib.check(lib.gpa_route_forward_many(probs, len(reads), _lib.stream_handle(reads[0][1].device)),
               "gpa_route_forward_many")
    return outs


def route_reader(base: Tensor, q: Tensor, edge_w: Tensor | None, gain: Tensor, mlp_gain: Tensor, up: Tensor,
                 down: Tensor, rs: Tensor, qs: Tensor, query_scale: float, msgs, rsa: bool = False,
                 mix: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """(qo, route) of one target level; base [B,T,H,M] float32 logits, q
    [B,T,H,Dk], msgs the incoming messages [B,T,H,M] in edge order with their
    softmax weights edge_w [n_in,H]; gain, mlp_gain [H]; U [H,M,2M],
    D [H,2M,M], W_rs [H,M,M], W_qs [H,Dk,M].  rsa: rsa_update's L1 rescale of
    the route; mix [H] (.1 + .8 sigmoid(bridge_mix_raw)): balanced_bridge."""
    if not msgs:
        # no incoming edges: the relation gain and edge weights are unused (no gradient)
        gain, edge_w = gain.detach(), gain.new_zeros(0, gain.shape[0])
    flags = (int(rsa), int(mix is not None))
    return _RouteReader.apply(base, q, edge_w, gain, mlp_gain, up, down, rs, qs, query_scale, flags, mix, *msgs)


class _ProductRead(torch.autograd.Function):
    """gpa_product_read_forward / _backward (see product_read)."""

    @staticmethod
    def forward(ctx, base, gexp, edge_w, counts, *pairs):
        ni = len(pairs) // 2
        msgs, norms = pairs[:ni], pairs[ni:]
        _lib.require_device(base)
        lib = _lib.load()
        b, t, h, m = base.shape
        gexp_f = gexp.detach().float().contiguous()
        w = edge_w.detach().float().contiguous()
        out = torch.empty(b, t, h, m, device=base.device, dtype=torch.float32)
        p = _product_problem(base, gexp_f, w, counts, msgs, norms, out)
        _lib.check(lib.gpa_product_read_forward(p, _lib.stream_handle(base.device)), "gpa_product_read_forward")
        ctx.save_for_backward(base, gexp_f, w, counts if counts is not None else base.new_zeros(0), *msgs, *norms)
        ctx.marginal = counts is not None
        ctx.ni = ni
        return out

    @staticmethod
    def backward(ctx, dout):
        base, gexp, w, counts, *rest = ctx.saved_tensors
        ni = ctx.ni
        msgs, norms = rest[:ni], rest[ni:]
        counts = counts if ctx.marginal else None
        lib = _lib.load()
        b, t, h, m = base.shape
        dout = dout.float().contiguous()
        dmsgs = [torch.empty_like(x) for x in msgs]
        dnorms = [torch.empty(b, t, h, device=base.device, dtype=torch.float32) for _ in range(ni)]
        dcounts = torch.empty(b, t, h, m, device=base.device, dtype=torch.float32) if ctx.marginal else None
        nblk = -(-b * t // _lib.PRODUCT_ROWS)
        partials = torch.empty(nblk, h, 2 + ni, device=base.device, dtype=torch.float32)
        p = _product_problem(base, gexp, w, counts, msgs, norms, None)
        g = _lib.ProductGrads()
        g.dout = dout.data_ptr()
        for e in range(ni):
            g.dmsg[e], g.dnorm[e] = _lib.operand(dmsgs[e]), dnorms[e].data_ptr()
        g.dcounts = dcounts.data_ptr() if dcounts is not None else None
        g.partials = partials.data_ptr()
        _lib.check(lib.gpa_product_read_backward(p, g, _lib.stream_handle(base.device)), "gpa_product_read_backward")
        sums = partials.sum(0)  # [H, 2 + ni]
        dgexp = m * sums[:, 0] - (sums[:, 1] if ctx.marginal else 0.)
        dw = sums[:, 2:].transpose(0, 1)  # [ni, H]
        dnorms = [x[..., None] if n.dim() == 4 else x for x, n in zip(dnorms, norms)]
        return (dout, dgexp, dw, dcounts, *dmsgs, *dnorms)


def _product_problem(base, gexp, w, counts, msgs, norms, out) -> _lib.ProductProblem:
    b, t, h, m = base.shape
    p = _lib.ProductProblem()
    p.batch, p.tokens, p.heads, p.slots, p.incoming = b, t, h, m, len(msgs)
    p.dtype, p.marginal = _lib.DTYPE_CODES[msgs[0].dtype], int(counts is not None)
    p.base = _lib.operand(base)
    for e, (msg, n) in enumerate(zip(msgs, norms)):
        p.msg[e] = _lib.operand(msg)
        p.norm[e] = _lib.Operand(n.data_ptr(), n.stride(0), n.stride(1), n.stride(2))
    if counts is not None:
        p.counts = _lib.operand(counts)
    p.edge_weight, p.gexp = w.data_ptr(), gexp.data_ptr()
    p.out = out.data_ptr() if out is not None else None
    return p


def product_read(base: Tensor, gexp: Tensor, edge_w: Tensor, msgs, norms, counts: Tensor | None) -> Tensor:
    """The product relation read of one target level (attention.py:231-236):
    base [B,T,H,M] float32 + (M gexp) sum_e (w_e msg_e) n_e, minus gexp
    log1p(counts) when `counts` [B,T,H,M] float32 is given (relation_marginal);
    gexp = e^{clamp(gain, -4, 4)} [H], edge_w [n_in,H] the edge softmax, msgs
    [B,T,H,M] (one activation dtype) and norms [B,T,H] or [B,T,H,1] float32,
    |softmax(source logits)| per row.  Returns float32 [B,T,H,M], with autograd
    to every input."""
    msgs = [x if x.stride(-1) == 1 else x.contiguous() for x in msgs]
    if not 1 <= len(msgs) <= _lib.ROUTE_MAX_INCOMING or len(norms) != len(msgs):
        raise ValueError("product_read: one norm per message, 1 to 3 messages")
    if any(x.dtype != msgs[0].dtype for x in msgs) or msgs[0].dtype not in _lib.DTYPE_CODES:
        raise ValueError("product_read: messages of one float32 or bfloat16 dtype")
    if base.dtype != torch.float32 or base.stride(-1) != 1:
        raise ValueError("product_read: float32 base logits with contiguous slots")
    if counts is not None and (counts.dtype != torch.float32 or counts.stride(-1) != 1):
        raise ValueError("product_read: float32 counts with contiguous slots")
    norms = [n.float() for n in norms]
    return _ProductRead.apply(base, gexp, edge_w, counts, *msgs, *norms)
