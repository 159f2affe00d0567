"""CPU restatement of the reference DenseGPA ``backend="torch"`` path.

TEST INFRASTRUCTURE ONLY: imported by tests/, `__graft_entry__.smoke()` and
the CPU-baseline leg of bench.py.  Never shipped in, or called by, the
`gpa_amd` product.

Every function restates one piece of the reference (file:line cited) from its
equations, keeping the reference's dtype flow (bf16 activations rounded where
the reference rounds them, fp32/fp64 recurrent state) so that it reproduces
the reference's numbers, not merely its mathematics.  The recurrences here are
the literal per-token definitions -- no chunked algebra -- which is what makes
this an independent check of the chunked HIP kernels.

Parameters come from any object with the reference's parameter names (the
`gpa_amd.DenseGPA` module is one); cache objects are `gpa_amd.state` classes,
whose layout equals the reference's.
"""
from __future__ import annotations

import math
from dataclasses import fields
from types import SimpleNamespace

import torch
import torch.nn.functional as F
from torch import Tensor

from gpa_amd.state import GPAState, LevelState, RelationState, ResidualSnapshot


def _work(x: Tensor) -> torch.dtype:
    # ops.py:10-11: float64 stays float64, everything else runs in float32.
    return torch.float64 if x.dtype == torch.float64 else torch.float32


def unit(x: Tensor) -> Tensor:
    """x / max(||x||_2, 1e-6) on the last axis, in the work type (ops.py:14-17)."""
    return F.normalize(x.to(_work(x)), p=2, dim=-1, eps=1e-6).to(x.dtype)


def gdn_step(state: Tensor, key: Tensor, value: Tensor, log_gate: Tensor, beta: Tensor) -> Tensor:
    """One gated delta-rule update, S:[B,H,K,V] (ops.py:29-42).

    S' = a*S + beta * u(k) (v - u(k)^T a*S)^T with a = exp(g).
    """
    if log_gate.shape != key.shape[:-1] or beta.shape != key.shape[:-1]:
        raise ValueError("GDN scalar gates/beta must be [B,H], not vector gates")
    kh = unit(key).to(state.dtype)
    scaled = state * torch.exp(log_gate.to(state.dtype))[..., None, None]
    predicted = (kh.unsqueeze(-2) @ scaled).squeeze(-2)
    residual = value.to(state.dtype) - predicted
    return scaled + beta.to(state.dtype)[..., None, None] * (kh.unsqueeze(-1) * residual.unsqueeze(-2))


def gdn_read(query: Tensor, state: Tensor) -> Tensor:
    """u(q)^T S, returned in the query dtype (ops.py:45-46)."""
    qh = unit(query).to(state.dtype)
    return (qh.unsqueeze(-2) @ state).squeeze(-2).to(query.dtype)


def gdn_scan(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, initial: Tensor):
    """Causal scan of `gdn_step` then `gdn_read` per token (ops.py:49-57, 78-85)."""
    if q.shape != k.shape or q.shape[:3] != v.shape[:3]:
        raise ValueError("q/k must share [B,T,H,K], v must share [B,T,H]")
    if g.shape != q.shape[:3] or beta.shape != q.shape[:3]:
        raise ValueError("g and beta must be scalar per token/head: [B,T,H]")
    if q.shape[1] == 0:
        return v.new_empty(*v.shape), initial
    state, reads = initial, []
    for t in range(q.shape[1]):
        state = gdn_step(state, k[:, t], v[:, t], g[:, t], beta[:, t])
        reads.append(gdn_read(q[:, t], state))
    return torch.stack(reads, 1), state


def additive_scan(q: Tensor, k: Tensor, v: Tensor, initial: Tensor):
    """S += k v^T, read q^T S, no normalisation (ops.py:88-91, 110-118)."""
    if q.shape[1] == 0:
        return v.new_empty(v.shape), initial
    state, reads = initial, []
    for t in range(q.shape[1]):
        state = state + k[:, t].to(state.dtype).unsqueeze(-1) * v[:, t].to(state.dtype).unsqueeze(-2)
        reads.append((q[:, t].to(state.dtype).unsqueeze(-2) @ state).squeeze(-2).to(q.dtype))
    return torch.stack(reads, 1), state


def rope(x: Tensor, positions, base: float = 10000.) -> Tensor:
    """Adjacent-pair rotary embedding (ops.py:121-137)."""
    d = x.shape[-1]
    if d % 2:
        raise ValueError("RoPE needs an even head dimension")
    work = x.to(_work(x))
    pos = torch.as_tensor(positions, device=x.device, dtype=work.dtype)
    if x.ndim == 4:
        pos = pos[None, :, None] if pos.ndim == 1 else (pos[:, :, None] if pos.ndim == 2 else pos)
    inv_freq = base ** (-torch.arange(0, d, 2, device=x.device, dtype=work.dtype) / d)
    angle = pos[..., None] * inv_freq
    cos, sin = angle.cos(), angle.sin()
    even, odd = work[..., 0::2], work[..., 1::2]
    rotated = torch.stack((even * cos - odd * sin, even * sin + odd * cos), dim=-1)
    return rotated.flatten(-2).to(x.dtype)


def two_stage(q, k, slots, v, gi, bi, go, bo, inner, outer, *, route_weight=None,
              query_weight=None, query_scale=1 / 16):
    """GDN(softmax(GDN(q,k,slots)) W_rs + q W_qs*scale, slots, v) (ops.py:146-163)."""
    read, a = gdn_scan(q, k, slots, gi, bi, inner)
    route = read.to(_work(read)).softmax(-1).to(q.dtype)
    if route_weight is not None:
        route = F.linear(route, route_weight.to(route.dtype))
    if query_weight is not None:
        route = route + query_scale * F.linear(q, query_weight.to(q.dtype))
    out, b = gdn_scan(route, slots, v, go, bo, outer)
    return out, a, b


def quadratic_features(fm, x: Tensor) -> Tensor:
    """The quadratic Q/K feature map (features.py:17-25) with the parameters of
    `fm` (left, right [H,D,D], gain_raw [H]): u = unit(x); z = u +
    2 sigmoid(gain_raw) sqrt(D) (u L)(u R); out = unit(z) sqrt(sum x^2 + 1e-12)."""
    work = _work(x)
    u = unit(x)
    a = _typed_product("...hd,hdf->...hf", u, fm.left, x.dtype).to(work)
    b = _typed_product("...hd,hdf->...hf", u, fm.right, x.dtype).to(work)
    gain = 2 * fm.gain_raw.sigmoid()[..., None]
    z = u.to(work) + gain * math.sqrt(x.shape[-1]) * a * b
    norm = (x.to(work).square().sum(-1, keepdim=True) + 1e-12).sqrt()
    return (F.normalize(z, p=2, dim=-1, eps=1e-6) * norm).to(x.dtype)


def _typed_product(eq: str, x: Tensor, w: Tensor, dtype) -> Tensor:
    """einsum of two `dtype` operands as the reference's typed einsum (bf16
    operands multiplied in float32 and rounded once)."""
    if dtype == torch.bfloat16:
        return torch.einsum(eq, x.to(dtype).float(), w.to(dtype).float()).to(dtype)
    return torch.einsum(eq, x.to(dtype), w.to(dtype))


def _softplus_inverse(x: float) -> float:
    return math.log(math.expm1(x))


def initial_state(model, batch: int, *, device=None, dtype=None, chunk_size=None) -> GPAState:
    """Prefixes expanded over the batch, zero counts (attention.py:146-159)."""
    cfg = model.config
    ref = model.center[0]
    device = ref.device if device is None else device
    dtype = ref.dtype if dtype is None else dtype
    work = torch.float64 if dtype == torch.float64 else torch.float32
    grow = lambda p: p.to(device=device, dtype=work).unsqueeze(0).expand(batch, *p.shape)  # noqa: E731
    levels = []
    for m, a, b in zip(cfg.slots, model.inner_prefix, model.outer_prefix):
        pos = (torch.zeros(batch, cfg.heads, cfg.key_dim, m, device=device, dtype=work)
               if cfg.positional_mode == "moments" else None)
        levels.append(LevelState(grow(a), grow(b), torch.zeros(batch, cfg.heads, m, device=device, dtype=work), pos))
    relations = tuple(RelationState(i, j, grow(p)) for (i, j), p in zip(cfg_edges(cfg), model.relation_prefix))
    return GPAState(tuple(levels), relations, chunk_size=cfg.chunk_size if chunk_size is None else chunk_size)


def cfg_edges(cfg):
    n = len(cfg.slots)
    return tuple((i, j) for i in range(n) for j in range(n) if i != j)


class OracleRun:
    """The reference forward (attention.py:161-413) bound to one parameter set."""

    def __init__(self, model, chunk_size: int | None = None):
        base = model.config
        values = {f.name: getattr(base, f.name) for f in fields(base)}
        if chunk_size is not None:
            values["chunk_size"] = chunk_size
        self.cfg = SimpleNamespace(**values)
        self.p = model
        self.edges = cfg_edges(self.cfg)

    # -- level glue ---------------------------------------------------------
    def gate_inputs(self, key, j, control):
        """The gate product before its bias, [B,T,H,4] in the activation type
        (attention.py:162-165)."""
        cfg, w = self.cfg, self.p.gate_weight[j]
        if cfg.control_dim:
            return torch.einsum("...d,hdc->...hc", control, w.to(control.dtype))
        src = key if cfg.rsa_update else unit(key)
        return torch.einsum("...hd,hdc->...hc", src, w.to(key.dtype))

    def gates(self, key, j, control):
        """(g_in, beta_in, g_out, beta_out), each [B,T,H] (attention.py:161-174)."""
        cfg = self.cfg
        raw = self.gate_inputs(key, j, control).to(_work(key)) + self.p.gate_bias[j]
        g_in, b_in, g_out, b_out = raw.unbind(-1)
        g_in = -F.softplus(g_in).clamp(max=10.)
        g_out = -F.softplus(g_out).clamp(max=10.)
        if cfg.rsa_update:
            tier = (1., .1, .01, .001)[j] if len(cfg.slots) == 4 else .1 ** j
            g_in, g_out = g_in * tier, g_out * tier
        if cfg.positional_mode == "none":
            g_in, g_out = g_in * 0, g_out * 0
        return g_in, cfg.beta_max * b_in.sigmoid(), g_out, cfg.beta_max * b_out.sigmoid()

    def feature(self, x):
        """Symmetric slot feature map (attention.py:179-184)."""
        cfg = self.cfg
        if cfg.slot_feature == "softmax":
            return (cfg.slot_scale * x.to(_work(x))).softmax(-1).to(x.dtype)
        if cfg.slot_feature == "tanh":
            return (cfg.slot_scale * x.to(_work(x))).tanh().to(x.dtype)
        return x

    def slot(self, key, j):
        """s_j = feature(key C_j^T) (attention.py:176-177)."""
        return self.feature(torch.einsum("...hd,hmd->...hm", key, self.p.center[j].to(key.dtype)))

    def assignment(self, slot):
        """Write assignment that does not need a state read (attention.py:186-188)."""
        if self.cfg.slot_feature == "softmax":
            return slot
        return (slot / .25).softmax(-1) if self.cfg.rsa_update else None

    def residual(self, key, value, rk, rv, j):
        """k - eta_k*rk, v - eta_v*rv, eta = 1 + tanh(raw)/4 (attention.py:190-194)."""
        eta = 1 + .25 * self.p.residual_raw[j].tanh()
        new_key = (key - eta[:, 0, None] * rk.to(key.dtype)).to(key.dtype)
        new_value = (value - eta[:, 1, None] * rv.to(value.dtype)).to(value.dtype)
        return new_key, new_value

    @staticmethod
    def counts(count0, write):
        """Soft slot counts after every token, n0 + cumsum_t(write) (attention.py:316)."""
        return count0[:, None] + write.to(count0.dtype).cumsum(1)

    def base_logits(self, raw, count, moment, j):
        """read_scale*raw + softplus(c_j) log1p(n) [+ moment term] (attention.py:196-204)."""
        cfg = self.cfg
        gain = F.softplus(self.p.count_gain_raw[j])[..., None]
        if cfg.learn_read_scale:
            scale = self.p.read_log_scale[j].clamp(math.log(.25), math.log(64.)).exp()[..., None]
        else:
            scale = cfg.read_scale
        out = scale * raw.to(count.dtype) + gain * count.log1p()
        if moment is not None:
            out = out + self.p.moment_gain[j][..., None] * torch.tanh(moment / (1 + count))
        return out

    # -- relations and route --------------------------------------------------
    def relations(self, local, writes, rel_states):
        """R_ij GDN scans over every ordered edge (attention.py:206-223)."""
        cfg, p = self.cfg, self.p
        incoming = [[] for _ in local]
        finals = []
        for e, ((i, j), old) in enumerate(zip(self.edges, rel_states)):
            lead = writes[i].shape[:-1]
            g = (-F.softplus(p.relation_decay_raw[e])).expand(lead)
            if cfg.positional_mode == "none":
                g = g * 0
            beta = p.relation_beta_raw[e].sigmoid().expand(lead)
            target = writes[j]
            if cfg.rsa_update:
                norm = (writes[i].to(_work(writes[i])).square().sum(-1) + 1e-6).sqrt()
                target = (target / norm[..., None]).to(target.dtype)
                beta = (beta * norm.square()).clamp_max(.9)
            msg, memory = gdn_scan(local[i], writes[i], target, g, beta, old.memory)
            incoming[j].append((e, msg))
            finals.append(RelationState(i, j, memory))
        return incoming, tuple(finals)

    def bridge(self, q, logits, incoming, counts):
        """Edge softmax -> aggregate -> route -> MLP -> query (attention.py:225-262)."""
        cfg, p = self.cfg, self.p
        routes, queries = [], []
        for j, base in enumerate(logits):
            if incoming[j]:
                ids = [e for e, _ in incoming[j]]
                w = p.edge_logits[ids].softmax(0)
                if cfg.paper_product_read:
                    total = 0
                    for wt, (e, msg) in zip(w, incoming[j]):
                        src_norm = logits[self.edges[e][0]].softmax(-1).norm(dim=-1, keepdim=True)
                        total = total + wt[..., None] * msg * src_norm
                    gain = p.relation_gain[j].clamp(-4, 4).exp()[..., None]
                    base = base + base.shape[-1] * gain * total
                    if cfg.relation_marginal:
                        base = base - gain * counts[j].log1p()
                else:
                    total = 0
                    for wt, (_, msg) in zip(w, incoming[j]):
                        total = total + wt[..., None] * msg
                    centred = total - total.mean(-1, keepdim=True)
                    z = centred / (centred.square().mean(-1, keepdim=True) + 1e-5).sqrt()
                    base = base + p.relation_gain[j][..., None] * z.tanh()
            route = base.softmax(-1).to(q.dtype)
            hidden = F.gelu(torch.einsum("...hm,hmr->...hr", route, p.route_up[j].to(q.dtype)))
            route = route + p.route_mlp_gain[j][..., None] * torch.einsum(
                "...hr,hrm->...hm", hidden, p.route_down[j].to(q.dtype))
            route = route.to(q.dtype)
            if cfg.rsa_update:
                wide = route.to(_work(route))
                route = (wide / wide.abs().sum(-1, keepdim=True).clamp(.25, 4.)).to(q.dtype)
            qo = torch.einsum("...hm,hmn->...hn", route, p.route_weight[j].to(q.dtype))
            qw = p.query_weight[j]
            if cfg.shared_query_center:
                qw = qw + p.center[j].transpose(-1, -2) / cfg.query_scale
            direct = self.feature(cfg.query_scale * torch.einsum("...hd,hdm->...hm", q, qw.to(q.dtype)))
            if cfg.balanced_bridge:
                mix = .1 + .8 * p.bridge_mix_raw[j].sigmoid()[..., None]
                qo = mix * unit(qo) + (1 - mix) * unit(direct)
            else:
                qo = qo + direct
            routes.append(route)
            queries.append(qo.to(q.dtype))
        return routes, queries

    def mix_outputs(self, reads):
        w = self.p.output_logits.softmax(0)
        total = 0
        for j, y in enumerate(reads):
            total = total + w[j][..., None] * y
        return total

    # -- one token, recurrent post-update semantics (chunk_size == 1) ----------
    def token(self, q, k, v, state, position, control):
        """attention.py:264-297."""
        cfg = self.cfg
        qr = rope(q, position) if cfg.positional_mode == "moments" else q
        key, value = k, v
        new_levels, writes, logits = [], [], []
        for j, old in enumerate(state.levels):
            slot = self.slot(key, j)
            g_in, b_in, g_out, b_out = self.gates(key, j, control)
            a = gdn_step(old.inner, key, slot, g_in, b_in)
            b = gdn_step(old.outer, slot, value, g_out, b_out)
            write = self.assignment(slot)
            if write is None:
                write = gdn_read(key, a).softmax(-1)
            count = old.count + write.to(old.count.dtype)
            moment, correction = old.position, None
            if moment is not None:
                kh = unit(key)
                delta = (rope(kh, position) - kh).to(moment.dtype)
                moment = moment + delta.unsqueeze(-1) * write.to(delta.dtype).unsqueeze(-2)
                correction = gdn_read(qr, moment)
            logits.append(self.base_logits(gdn_read(qr, a), count, correction, j))
            writes.append(write)
            new_levels.append(LevelState(a, b, count, moment))
            rk = (a @ write.to(a.dtype).unsqueeze(-1)).squeeze(-1)
            rv = (write.to(b.dtype).unsqueeze(-2) @ b).squeeze(-2)
            key, value = self.residual(key, value, rk, rv, j)
        local = [x.softmax(-1).to(q.dtype).unsqueeze(1) for x in logits]
        incoming, relations = self.relations(local, [w.unsqueeze(1) for w in writes], state.relations)
        incoming = [[(e, m[:, 0]) for e, m in group] for group in incoming]
        routes, queries = self.bridge(qr, logits, incoming, [lv.count for lv in new_levels])
        out = self.mix_outputs([gdn_read(qo, lv.outer) for qo, lv in zip(queries, new_levels)])
        new = GPAState(tuple(new_levels), relations, state.position + 1, cfg.chunk_size)
        return out.to(v.dtype), new, routes

    # -- one block segment, block-lagged residuals (chunk_size > 1) ------------
    def block(self, q, k, v, state, positions, control):
        """attention.py:299-345 (reference execution; packed/staged are identical)."""
        cfg = self.cfg
        snaps = state.frozen or tuple(ResidualSnapshot(lv.inner, lv.outer) for lv in state.levels)
        qr = rope(q, positions) if cfg.positional_mode == "moments" else q
        key, value = k, v
        carried, writes, logits, outer_in, history = [], [], [], [], []
        for j, (old, snap) in enumerate(zip(state.levels, snaps)):
            slot = self.slot(key, j)
            g_in, b_in, g_out, b_out = self.gates(key, j, control)
            raw, a = gdn_scan(qr, key, slot, g_in, b_in, old.inner)
            write = self.assignment(slot)
            if write is None:
                write = torch.einsum("bthd,bhdm->bthm", unit(key).to(snap.inner.dtype), snap.inner).softmax(-1)
            write = write.to(q.dtype)
            counts = self.counts(old.count, write)
            history.append(counts)
            moment, correction = old.position, None
            if moment is not None:
                kh = unit(key)
                correction, moment = additive_scan(unit(qr), rope(kh, positions) - kh, write, moment)
            logits.append(self.base_logits(raw, counts, correction, j))
            writes.append(write)
            carried.append((a, counts[:, -1], moment))
            outer_in.append((slot, value, g_out, b_out))
            rk = torch.einsum("bhdm,bthm->bthd", snap.inner, write.to(snap.inner.dtype))
            rv = torch.einsum("bthm,bhmv->bthv", write.to(snap.outer.dtype), snap.outer)
            key, value = self.residual(key, value, rk, rv, j)
        local = [x.softmax(-1).to(q.dtype) for x in logits]
        incoming, relations = self.relations(local, writes, state.relations)
        routes, queries = self.bridge(qr, logits, incoming, history)
        reads, levels = [], []
        for j, qo in enumerate(queries):
            slot, value_j, g_out, b_out = outer_in[j]
            y, b = gdn_scan(qo, slot, value_j, g_out, b_out, state.levels[j].outer)
            a, count, moment = carried[j]
            levels.append(LevelState(a, b, count, moment))
            reads.append(y)
        out = self.mix_outputs(reads)
        offset = (state.chunk_offset + q.shape[1]) % cfg.chunk_size
        new = GPAState(tuple(levels), relations, state.position + q.shape[1], cfg.chunk_size,
                       offset, snaps if offset else None)
        return out.to(v.dtype), new, routes

    # -- the public forward ------------------------------------------------------
    def __call__(self, q, k, v, state=None, *, position_ids=None, control_input=None,
                 return_diagnostics=False):
        """attention.py:347-413."""
        cfg, p = self.cfg, self.p
        if q.ndim != 4 or q.shape != k.shape or q.shape[:3] != v.shape[:3]:
            raise ValueError("expected Q,K [B,T,H,Dk], V [B,T,H,Dv]")
        if q.shape[2:] != (cfg.heads, cfg.key_dim) or v.shape[-1] != cfg.value_dim:
            raise ValueError("input heads/dimensions do not match GPAConfig")
        if cfg.control_dim and (control_input is None
                                or control_input.shape != q.shape[:2] + (cfg.control_dim,)):
            raise ValueError("full hidden controls [B,T,control_dim] required")
        if cfg.quadratic_features:
            q, k = quadratic_features(p.feature_map, torch.stack((q, k))).unbind(0)
        if state is None:
            state = initial_state(p, q.shape[0], device=q.device, dtype=q.dtype, chunk_size=cfg.chunk_size)
        if state.chunk_size != cfg.chunk_size:
            raise ValueError("cannot switch cache between recurrent and lagged chunk semantics")
        if position_ids is None:
            position_ids = torch.arange(state.position, state.position + q.shape[1], device=q.device)
        outs, history = [], [[] for _ in cfg.slots]
        start, total = 0, q.shape[1]
        while start < total:
            if cfg.chunk_size == 1:
                pos = position_ids[start] if position_ids.ndim == 1 else position_ids[:, start, None]
                ctl = control_input[:, start] if control_input is not None else None
                y, state, routes = self.token(q[:, start], k[:, start], v[:, start], state, pos, ctl)
                outs.append(y.unsqueeze(1))
                routes = [r.unsqueeze(1) for r in routes]
                stop = start + 1
            else:
                stop = min(total, start + cfg.chunk_size - state.chunk_offset)
                pos = position_ids[start:stop] if position_ids.ndim == 1 else position_ids[:, start:stop]
                ctl = control_input[:, start:stop] if control_input is not None else None
                y, state, routes = self.block(q[:, start:stop], k[:, start:stop], v[:, start:stop], state, pos, ctl)
                outs.append(y)
            for h, r in zip(history, routes):
                h.append(r)
            start = stop
        output = torch.cat(outs, 1) if outs else v.new_empty(v.shape)
        if return_diagnostics:
            routes = tuple(torch.cat(h, 1) if h else q.new_empty(q.shape[:3] + (m,))
                           for h, m in zip(history, cfg.slots))
            return output, state, {"routes": routes, "edges": self.edges,
                                   "state_elements": state.numel(),
                                   "position": state.position}
        return output, state


def forward(model, q, k, v, state=None, *, chunk_size=None, **kwargs):
    """Run the reference forward with `model`'s parameters (optionally another chunk size)."""
    return OracleRun(model, chunk_size)(q, k, v, state, **kwargs)
