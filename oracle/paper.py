"""CPU restatement of the reference's counted dense core (`PaperDenseGPA`,
``backend="torch"``) and of its moment recurrences.

TEST INFRASTRUCTURE ONLY: imported by tests/ (never by the `gpa_amd`
product).  Each function restates one piece of src/gpa/paper_dense.py (lines
cited) with the reference's dtype flow: activations in their own type,
recurrent state and gate arithmetic in float32 (float64 for float64 inputs),
rounding to the activation type where the reference rounds.  The recurrences
are the literal per-token definitions.  Parameters come from any object with
the reference's parameter names and buffers (the `gpa_amd.paper_dense`
module is one).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import Tensor

from gpa_amd.paper_dense import PaperState
from gpa_amd.state import LevelState, RelationState, ResidualSnapshot

from .reference import gdn_scan, unit


def moment_scan(q: Tensor, k: Tensor, v: Tensor, g: Tensor | None, initial: Tensor, axis: str = "key"):
    """S = exp(g) o S + k v^T, y_t = q_t^T S per token (paper_dense.py:38-47);
    g None means no decay (ops.py:111-118, `linear_scan`).  g [B,T,H] decays
    the whole state, [B,T,H,D] one key row (axis "key") or one value column
    (axis "value") per element."""
    s, ys = initial, []
    for t in range(q.shape[1]):
        if g is not None:
            a = g[:, t].exp().to(s.dtype)
            a = a[..., None, None] if g.ndim == 3 else a[..., None, :] if axis == "value" else a[..., :, None]
            s = a * s
        s = s + k[:, t].to(s.dtype)[..., :, None] * v[:, t].to(s.dtype)[..., None, :]
        ys.append((q[:, t].to(s.dtype).unsqueeze(-2) @ s).squeeze(-2).to(q.dtype))
    return torch.stack(ys, 1), s


def decayed_counts(p: Tensor, g: Tensor, initial: Tensor) -> Tensor:
    """n_t = exp(g_t) o n_{t-1} + p_t for every token (paper_dense.py:50-58,
    whose closed forms compute this recurrence); g [B,T,H] or [B,T,H,M]."""
    n, out = initial, []
    for t in range(p.shape[1]):
        a = g[:, t].exp()
        n = (a[..., None] if g.ndim == 3 else a) * n + p[:, t].to(initial.dtype)
        out.append(n)
    return torch.stack(out, 1)


def initial_state(model, batch: int, device=None, dtype=torch.float32) -> PaperState:
    """paper_dense.py:136-145: prefixes scaled by softplus(count_raw)."""
    work = torch.float64 if dtype == torch.float64 else torch.float32
    n = F.softplus(model.count_raw).to(device, work)
    a = model.key_prefix.to(device, work) * n[..., None, :]
    b = model.value_prefix.to(device, work) * n[..., :, None]
    nl = len(model.config.slots)
    levels = tuple(LevelState(a[i][None].expand(batch, -1, -1, -1), b[i][None].expand(batch, -1, -1, -1),
                              n[i][None].expand(batch, -1, -1)) for i in range(nl))
    r = model.relation_prefix.to(device, work)
    relations = tuple(RelationState(i, j, r[e][None].expand(batch, -1, -1, -1))
                      for e, (i, j) in enumerate(model.edges))
    return PaperState(levels, relations, chunk_size=model.config.chunk_size)


def _dot(eq: str, x: Tensor, w: Tensor, dtype) -> Tensor:
    """The reference's einsum of two `dtype` operands (float32 accumulation)."""
    if dtype == torch.bfloat16:
        return torch.einsum(eq, x.to(dtype).float(), w.to(dtype).float()).to(dtype)
    return torch.einsum(eq, x.to(dtype), w.to(dtype))


def segment(model, q: Tensor, k: Tensor, v: Tensor, state: PaperState, control: Tensor | None):
    """One block segment (paper_dense.py:147-258)."""
    c = model.config
    b, t, h, d = q.shape
    nl, m, dv = len(c.slots), c.slots[0], c.value_dim
    dtype = q.dtype
    work = state.levels[0].count.dtype
    feat = unit if c.normalize_features else (lambda x: x)
    frozen = state.frozen or tuple(ResidualSnapshot(s.inner / s.count.clamp_min(1e-5)[..., None, :],
                                                    s.outer / s.count.clamp_min(1e-5)[..., :, None])
                                   for s in state.levels)
    keys, values, probs, writes, gates, counts = [], [], [], [], [], []
    for i, snap in enumerate(frozen):
        keys.append(k)
        values.append(v)
        scale = model.feature_log_scale[i].clamp(math.log(.25), math.log(64.)).exp()
        p = (_dot("bthd,hmd->bthm", feat(k), model.center[i], k.dtype).to(work)
             * scale[None, None, :, None]).softmax(-1).to(k.dtype)
        if c.control_dim:
            ctrl = _dot("btc,hcf->bthf", control, model.control_weight[i], control.dtype)
        else:
            ctrl = _dot("bthd,hdc->bthc", feat(k), model.control_weight[i], k.dtype)
        ctrl = ctrl.to(work) + model.control_bias[i]
        g = -(model.decay_log_rate[i].exp() * F.softplus(ctrl[..., 0])).clamp(max=.02) * model.time_scales[i]
        w = ctrl[..., 1].sigmoid()
        pwrite = (p * w[..., None]).to(dtype)
        if c.slot_decay:
            g = g[..., None] + torch.log1p(-(model.forget_raw[i].sigmoid()[None, None, :, None]
                                             * pwrite.to(work)).clamp_max(.95))
        probs.append(p)
        writes.append(pwrite)
        gates.append(g)
        counts.append(decayed_counts(pwrite, g, state.levels[i].count))
        rk = torch.einsum("bthm,bhdm->bthd", p.to(snap.inner.dtype), snap.inner)
        rv = torch.einsum("bthm,bhmv->bthv", p.to(snap.outer.dtype), snap.outer)
        eta = 1 + .25 * model.residual_raw[i].tanh()
        k = (k - eta[:, 0, None] * rk.to(k.dtype)).to(k.dtype)
        v = (v - eta[:, 1, None] * rv.to(v.dtype)).to(v.dtype)

    def pack(xs):
        return torch.stack(xs, 2).reshape(b, t, nl * h, *xs[0].shape[3:])

    def pack_state(xs):
        return torch.stack(xs, 1).reshape(b, nl * h, *xs[0].shape[2:])

    qp = feat(q)[:, :, None].expand(b, t, nl, h, d).reshape(b, t, nl * h, d)
    raw, af = moment_scan(qp, pack(keys), pack(writes), pack(gates), pack_state([s.inner for s in state.levels]),
                          axis="value")
    raw = raw.reshape(b, t, nl, h, m)
    n = torch.stack(counts, 2).clamp_min(1e-5)
    fl = _dot("bthd,lhmd->btlhm", feat(q), model.center, dtype).to(n.dtype)
    fl = fl * model.feature_log_scale.clamp(math.log(.25), math.log(64.)).exp()[None, None, :, :, None]
    gain = model.count_gain.clamp(0, 1)[None, None, :, :, None]
    logits = model.content_log_scale.clamp(0, math.log(64.)).exp()[None, None, :, :, None] * raw.to(n.dtype) / n + fl
    if c.dense_read == "local":
        logits = logits + gain * n.log()
    local = logits.softmax(-1).to(dtype)
    relations = state.relations
    if model.edges and c.use_relations:
        ne = len(model.edges)
        ep = torch.stack(probs, 2)
        source, target = ep.index_select(2, model.source), ep.index_select(2, model.target)
        norm = (source.to(work).square().sum(-1) + 1e-6).sqrt()
        val = target / norm.to(dtype)[..., None]
        rb = (model.relation_beta_raw.sigmoid()[None, None] * norm.square()).clamp_max(.9)
        if c.strong_relations:
            act = torch.stack(writes, 2).to(work).sum(-1)
            rb = rb * (act.index_select(2, model.source) * act.index_select(2, model.target)).clamp_min(1e-12).sqrt()
        rg = -F.softplus(model.relation_decay_raw)[None, None].expand(b, t, -1, -1)
        r0 = torch.stack([s.memory for s in state.relations], 1).reshape(b, ne * h, m, m)
        rq = local.index_select(2, model.source)
        args = (source.reshape(b, t, ne * h, m), val.to(dtype).reshape(b, t, ne * h, m),
                rg.reshape(b, t, ne * h), rb.reshape(b, t, ne * h), r0)
        msg, rf = gdn_scan(rq.reshape(b, t, ne * h, m), *args)
        msg = msg.reshape(b, t, ne, h, m) * rq.to(work).norm(dim=-1, keepdim=True)
        messages = (m * msg.to(work)).log_softmax(-1)
        rmix = (model.relation_mix_raw.clamp(-6, math.log(16.)).exp() if c.strong_relations
                else model.relation_mix_raw.sigmoid())
        routed = []
        if c.dense_read == "transport":
            total = torch.stack([messages.index_select(2, model.incoming[j]).sum(2)
                                 + local[:, :, j].to(work).clamp_min(1e-8).log() for j in range(nl)], 2)
            comp = total.index_select(2, model.source) - messages.index_select(2, model.reverse_edge)
            consensus = comp.softmax(-1)
            strength = rmix[model.source][None, None, :, :, None]
            root = ((local.index_select(2, model.source).to(work) + strength * consensus) / (1 + strength)).to(dtype)
            moved, _ = gdn_scan(root.reshape(b, t, ne * h, m), *args)
            moved = moved.reshape(b, t, ne, h, m) * root.to(work).norm(dim=-1, keepdim=True)
            tl = (m * moved.to(work)).log_softmax(-1)
            local_mass = local.to(work).clamp_min(1e-8).log() + gain * n.log()
            local_route = local_mass.softmax(-1)
            cross_mass = local_mass
            if c.strong_relations:
                cross_mass = (model.read_local_raw.sigmoid()[None, None, :, :, None]
                              * local.to(work).clamp_min(1e-8).log() + gain * n.log())
            cross = (tl + cross_mass.index_select(2, model.target)).softmax(-1)
            for j in range(nl):
                inc = cross.index_select(2, model.incoming[j])
                if c.strong_relations:
                    wts = model.read_edge_logits.index_select(0, model.incoming[j]).softmax(0)
                    proposal = (inc * wts[None, None, :, :, None]).sum(2)
                else:
                    proposal = inc.mean(2)
                mix = rmix[j][None, None, :, None]
                routed.append((local_route[:, :, j] + mix * proposal) / (1 + mix))
        else:
            for j in range(nl):
                product = messages.index_select(2, model.incoming[j]).sum(2).softmax(-1)
                mix = rmix[j][None, None, :, None]
                routed.append((local[:, :, j].to(work) + mix * product) / (1 + mix))
        route = torch.stack(routed, 2)
        rf = rf.reshape(b, ne, h, m, m)
        relations = tuple(RelationState(i, j, rf[:, e]) for e, (i, j) in enumerate(model.edges))
    elif c.dense_read == "local":
        route = local.to(work)
    else:
        route = (local.to(work).clamp_min(1e-8).log() + gain * n.log()).softmax(-1)
    delta = _dot("btlhr,lhrm->btlhm", F.gelu(_dot("btlhm,lhmr->btlhr", route, model.mlp_up, dtype)),
                 model.mlp_down, dtype)
    route = (route.clamp_min(1e-8).log() + .1 * delta.to(work)).softmax(-1)
    route = route / route.abs().sum(-1, keepdim=True).clamp(.25, 4.)
    oq = (route / n).to(dtype).reshape(b, t, nl * h, m)
    out, bf = moment_scan(oq, pack(writes), pack(values), pack(gates), pack_state([s.outer for s in state.levels]))
    out = out.reshape(b, t, nl, h, dv)
    output = (out * model.level_logits.softmax(0)[None, None, :, :, None] * nl).sum(2).to(dtype)
    af, bf = af.reshape(b, nl, h, d, m), bf.reshape(b, nl, h, m, dv)
    levels = tuple(LevelState(af[:, i], bf[:, i], counts[i][:, -1]) for i in range(nl))
    offset = (state.chunk_offset + t) % c.chunk_size
    return output, PaperState(levels, relations, state.position + t, c.chunk_size, offset,
                              frozen if offset else None), route


def forward(model, q: Tensor, k: Tensor, v: Tensor, state: PaperState | None = None, *, control_input=None):
    """paper_dense.py:260-278: the call split at block boundaries."""
    c = model.config
    if state is None:
        state = initial_state(model, q.shape[0], q.device, q.dtype)
    outs, start = [], 0
    while start < q.shape[1]:
        end = min(q.shape[1], start + c.chunk_size - state.chunk_offset)
        ctrl = control_input[:, start:end] if control_input is not None else None
        y, state, _ = segment(model, q[:, start:end], k[:, start:end], v[:, start:end], state, ctrl)
        outs.append(y)
        start = end
    return (torch.cat(outs, 1) if outs else v.new_empty(v.shape)), state
