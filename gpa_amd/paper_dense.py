"""`PaperDenseGPA`: the counted dense core on the HIP backend.

Drop-in for the reference's `PaperDenseGPA`, `PaperConfig` and `PaperState`
(src/gpa/paper_dense.py:61-278): decayed counted key/value moments per level,
full paired relations between levels and a dense product read.  Parameter
names, shapes, registration order and initialisation (and so the order in
which the global RNG is consumed) are the reference's, so `state_dict`s load
strictly both ways and a seeded construction gives identical parameters.

Compute.  Every recurrence runs in a HIP kernel: the inner and outer moment
scans of all levels (packed as L*H heads, as the reference packs them) and the
decayed counts in `gpa_moment_scan_many` (`gpa_amd.moment`), the relation
memories in the GDN scan (`gpa_amd.ops.gdn_scan`, the reference's
`gdn_scan`).  The per-token glue between them (slot products, gates, softmaxes,
the route MLP) runs as device tensor operations with the reference's rounding
points; products of activation-typed operands are taken in float32 and rounded
to the activation type, as a bf16 matrix product with float32 accumulation.
Calls are split at block boundaries like the reference's (residuals read the
block-start snapshots).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from . import _lib
from .moment import decayed_counts, moment_scan
from .ops import gdn_scan
from .state import GPAState, LevelState, RelationState, ResidualSnapshot


def _unit(x: Tensor) -> Tensor:
    """u(x) in float32, rounded back to x's dtype (reference ops.py:14-17)."""
    work = torch.float64 if x.dtype == torch.float64 else torch.float32
    return F.normalize(x.to(work), p=2, dim=-1, eps=1e-6).to(x.dtype)


def _mm(eq: str, x: Tensor, w: Tensor, dtype: torch.dtype) -> Tensor:
    """einsum of operands rounded to `dtype`, result in `dtype`; bf16 operands
    are multiplied in float32 (float32 accumulation, one rounding at the end)."""
    if dtype == torch.bfloat16:
        return torch.einsum(eq, x.to(dtype).float(), w.to(dtype).float()).to(dtype)
    return torch.einsum(eq, x.to(dtype), w.to(dtype))


@dataclass(frozen=True)
class PaperConfig:
    """Reference `PaperConfig` (paper_dense.py:61-79); `backend` is "hip"."""
    heads: int = 4
    key_dim: int = 32
    value_dim: int = 32
    slots: tuple = (16, 16, 16, 16)
    chunk_size: int = 64
    backend: str = "hip"
    read_scale: float = 8.
    decay_init: float = .0001
    write_init: float = .6
    relation_beta: float = .6
    use_relations: bool = True
    decay_tiers: tuple | None = None
    normalize_features: bool = True
    dense_read: str = "local"  # local | transport
    control_dim: int = 0
    slot_decay: bool = False
    strong_relations: bool = False


@dataclass(frozen=True)
class PaperState(GPAState):
    pass


class PaperDenseGPA(nn.Module):
    """q, k [B,T,H,Dk], v [B,T,H,Dv] -> output [B,T,H,Dv] and a `PaperState`
    (reference paper_dense.py:87-278, same call signature)."""

    def __init__(self, config: PaperConfig):
        super().__init__()
        self.config = c = config
        if len(set(c.slots)) != 1 or c.chunk_size < 1 or c.backend != "hip":
            raise ValueError("uniform positive slots/chunk and backend='hip' required")
        h, d, dv, m, lv = c.heads, c.key_dim, c.value_dim, c.slots[0], len(c.slots)
        # registration order = the reference's (the RNG is drawn by center,
        # key_prefix, value_prefix, mlp_up in this order)
        self.center = nn.Parameter(torch.randn(lv, h, m, d) / math.sqrt(d))
        self.key_prefix = nn.Parameter(torch.randn(lv, h, d, m) * .002)
        self.value_prefix = nn.Parameter(torch.randn(lv, h, m, dv) * .002)
        self.count_raw = nn.Parameter(torch.full((lv, h, m), math.log(math.expm1(.001))))
        self.control_weight = nn.Parameter(torch.zeros(lv, h, c.control_dim or d, 2))
        bias = torch.tensor([math.log(math.expm1(c.decay_init)), math.log(c.write_init / (1 - c.write_init))])
        self.control_bias = nn.Parameter(bias.repeat(lv, h, 1))
        self.decay_log_rate = nn.Parameter(torch.zeros(lv, h))
        if c.slot_decay:
            self.forget_raw = nn.Parameter(torch.full((lv, h), math.log(.9 / .1)))
        self.feature_log_scale = nn.Parameter(torch.full((lv, h), math.log(4.)))
        self.content_log_scale = nn.Parameter(torch.full((lv, h), math.log(c.read_scale)))
        self.count_gain = nn.Parameter(torch.ones(lv, h))
        self.residual_raw = nn.Parameter(torch.zeros(lv, h, 2))
        self.mlp_up = nn.Parameter(torch.randn(lv, h, m, 2 * m) / math.sqrt(m))
        self.mlp_down = nn.Parameter(torch.zeros(lv, h, 2 * m, m))
        self.edges = tuple((i, j) for i in range(lv) for j in range(lv) if i != j)
        ne = len(self.edges)
        self.relation_prefix = nn.Parameter(torch.zeros(ne, h, m, m))
        self.relation_beta_raw = nn.Parameter(torch.full((ne, h), math.log(c.relation_beta / (1 - c.relation_beta))))
        self.relation_decay_raw = nn.Parameter(torch.full((ne, h), math.log(math.expm1(.0001))))
        self.relation_mix_raw = nn.Parameter(torch.full((lv, h), math.log(.1 / .9)))
        if c.strong_relations:
            self.read_edge_logits = nn.Parameter(torch.zeros(ne, h))
            self.read_local_raw = nn.Parameter(torch.zeros(lv, h))
        self.level_logits = nn.Parameter(torch.zeros(lv, h))
        long = dict(dtype=torch.long)
        self.register_buffer("source", torch.tensor([i for i, _ in self.edges], **long), persistent=False)
        self.register_buffer("target", torch.tensor([j for _, j in self.edges], **long), persistent=False)
        self.register_buffer("incoming", torch.tensor([[e for e, (_, t) in enumerate(self.edges) if t == j]
                                                       for j in range(lv)], **long), persistent=False)
        self.register_buffer("reverse_edge", torch.tensor([self.edges.index((j, i)) for i, j in self.edges], **long),
                             persistent=False)
        tiers = c.decay_tiers or ((1., .1, .01, .001) if lv == 4 else
                                  (1., .3, .1, .03, .01, .003, .001, .0003) if lv == 8 else
                                  tuple(.1 ** i for i in range(lv)))
        if len(tiers) != lv or any(s <= 0 for s in tiers):
            raise ValueError("one positive decay tier per level required")
        self.register_buffer("time_scales", torch.tensor(tiers).float(), persistent=False)

    def initial_state(self, batch: int, device, dtype) -> PaperState:
        """Prefix moments scaled by the initial counts (paper_dense.py:136-145);
        every tensor a batch broadcast of the parameters."""
        work = torch.float64 if dtype == torch.float64 else torch.float32
        n = F.softplus(self.count_raw).to(device, work)
        a = self.key_prefix.to(device, work) * n[..., None, :]
        b = self.value_prefix.to(device, work) * n[..., :, None]
        levels = tuple(LevelState(a[i][None].expand(batch, -1, -1, -1), b[i][None].expand(batch, -1, -1, -1),
                                  n[i][None].expand(batch, -1, -1)) for i in range(len(self.config.slots)))
        r = self.relation_prefix.to(device, work)
        relations = tuple(RelationState(i, j, r[e][None].expand(batch, -1, -1, -1))
                          for e, (i, j) in enumerate(self.edges))
        return PaperState(levels, relations, chunk_size=self.config.chunk_size)

    # ---- one block segment (paper_dense.py:147-258)
    def _level_inputs(self, i: int, k: Tensor, control: Tensor | None, feature, work, dtype):
        """Slot probabilities, write, decay and count of level i (paper_dense.py:156-172)."""
        c = self.config
        scale = self.feature_log_scale[i].clamp(math.log(.25), math.log(64.)).exp()
        fk = feature(k)
        logits = _mm("bthd,hmd->bthm", fk, self.center[i], k.dtype).to(work) * scale[None, None, :, None]
        p = logits.softmax(-1).to(k.dtype)
        if c.control_dim:
            ctrl = _mm("btc,hcf->bthf", control, self.control_weight[i], control.dtype)
        else:
            ctrl = _mm("bthd,hdc->bthc", fk, self.control_weight[i], k.dtype)
        ctrl = ctrl.to(work) + self.control_bias[i]
        g = -(self.decay_log_rate[i].exp() * F.softplus(ctrl[..., 0])).clamp(max=.02) * self.time_scales[i]
        w = ctrl[..., 1].sigmoid()
        pwrite = (p * w[..., None]).to(dtype)
        if c.slot_decay:
            forget = self.forget_raw[i].sigmoid()[None, None, :, None] * pwrite.to(work)
            g = g[..., None] + torch.log1p(-forget.clamp_max(.95))
        return p, pwrite, g

    def _segment(self, q: Tensor, k: Tensor, v: Tensor, state: PaperState, control: Tensor | None):
        c = self.config
        b, t, h, d = q.shape
        nl, m, dv = len(c.slots), c.slots[0], c.value_dim
        dtype = q.dtype
        work = state.levels[0].count.dtype
        feature = _unit if c.normalize_features else (lambda x: x)
        frozen = state.frozen or tuple(
            ResidualSnapshot(s.inner / s.count.clamp_min(1e-5)[..., None, :],
                             s.outer / s.count.clamp_min(1e-5)[..., :, None]) for s in state.levels)
        keys, values, probs, writes, gates, counts = [], [], [], [], [], []
        for i, snap in enumerate(frozen):
            keys.append(k)
            values.append(v)
            p, pwrite, g = self._level_inputs(i, k, control, feature, work, dtype)
            probs.append(p)
            writes.append(pwrite)
            gates.append(g)
            counts.append(decayed_counts(pwrite, g, state.levels[i].count))
            rk = torch.einsum("bthm,bhdm->bthd", p.to(snap.inner.dtype), snap.inner)
            rv = torch.einsum("bthm,bhmv->bthv", p.to(snap.outer.dtype), snap.outer)
            eta = 1 + .25 * self.residual_raw[i].tanh()
            k = (k - eta[:, 0, None] * rk.to(k.dtype)).to(k.dtype)
            v = (v - eta[:, 1, None] * rv.to(v.dtype)).to(v.dtype)

        def pack(xs):  # per-level [B,T,H,...] -> level-major heads [B,T,L*H,...]
            return torch.stack(xs, 2).reshape(b, t, nl * h, *xs[0].shape[3:])

        def pack_state(xs):
            return torch.stack(xs, 1).reshape(b, nl * h, *xs[0].shape[2:])

        qf = feature(q)
        qp = qf[:, :, None].expand(b, t, nl, h, d).reshape(b, t, nl * h, d)
        gp = pack(gates)
        raw, af = moment_scan(qp, pack(keys), pack(writes), gp, pack_state([s.inner for s in state.levels]),
                              axis="value")
        raw = raw.reshape(b, t, nl, h, m)
        n = torch.stack(counts, 2).clamp_min(1e-5)
        feature_logits = _mm("bthd,lhmd->btlhm", qf, self.center, dtype).to(n.dtype)
        feature_logits = feature_logits * self.feature_log_scale.clamp(math.log(.25), math.log(64.)).exp()[
            None, None, :, :, None]
        gain = self.count_gain.clamp(0, 1)[None, None, :, :, None]
        logits = (self.content_log_scale.clamp(0, math.log(64.)).exp()[None, None, :, :, None] * raw.to(n.dtype) / n
                  + feature_logits)
        if c.dense_read == "local":
            logits = logits + gain * n.log()
        local = logits.softmax(-1).to(dtype)
        relations = state.relations
        if self.edges and c.use_relations:
            route, relations = self._relations(probs, writes, local, n, state, work, dtype)
        elif c.dense_read == "local":
            route = local.to(work)
        else:
            route = (local.to(work).clamp_min(1e-8).log() + gain * n.log()).softmax(-1)
        hidden = F.gelu(_mm("btlhm,lhmr->btlhr", route, self.mlp_up, dtype))
        delta = _mm("btlhr,lhrm->btlhm", hidden, self.mlp_down, dtype)
        route = (route.clamp_min(1e-8).log() + .1 * delta.to(work)).softmax(-1)
        route = route / route.abs().sum(-1, keepdim=True).clamp(.25, 4.)
        oq = (route / n).to(dtype).reshape(b, t, nl * h, m)
        out, bf = moment_scan(oq, pack(writes), pack(values), gp, pack_state([s.outer for s in state.levels]))
        out = out.reshape(b, t, nl, h, dv)
        output = (out * self.level_logits.softmax(0)[None, None, :, :, None] * nl).sum(2).to(dtype)
        af, bf = af.reshape(b, nl, h, d, m), bf.reshape(b, nl, h, m, dv)
        levels = tuple(LevelState(af[:, i], bf[:, i], counts[i][:, -1]) for i in range(nl))
        offset = (state.chunk_offset + t) % c.chunk_size
        new = PaperState(levels, relations, state.position + t, c.chunk_size, offset, frozen if offset else None)
        return output, new, route

    def _relations(self, probs, writes, local, n, state, work, dtype):
        """Relation memories and the relation-routed read (paper_dense.py:185-252)."""
        c = self.config
        b, t, nl, h, m = local.shape
        ne = len(self.edges)
        ep = torch.stack(probs, 2)
        source, target = ep.index_select(2, self.source), ep.index_select(2, self.target)
        norm = (source.to(work).square().sum(-1) + 1e-6).sqrt()
        val = (target / norm.to(dtype)[..., None]).to(dtype)
        rb = (self.relation_beta_raw.sigmoid()[None, None] * norm.square()).clamp_max(.9)
        if c.strong_relations:
            activity = torch.stack(writes, 2).to(work).sum(-1)
            rb = rb * (activity.index_select(2, self.source) * activity.index_select(2, self.target)).clamp_min(
                1e-12).sqrt()
        rg = -F.softplus(self.relation_decay_raw)[None, None].expand(b, t, -1, -1)
        r0 = torch.stack([s.memory for s in state.relations], 1).reshape(b, ne * h, m, m)
        rq = local.index_select(2, self.source)
        flat = dict(k=source.reshape(b, t, ne * h, m), v=val.reshape(b, t, ne * h, m),
                    g=rg.reshape(b, t, ne * h), beta=rb.reshape(b, t, ne * h))
        msg, rf = gdn_scan(rq.reshape(b, t, ne * h, m), flat["k"], flat["v"], flat["g"], flat["beta"], r0)
        msg = msg.reshape(b, t, ne, h, m) * rq.to(work).norm(dim=-1, keepdim=True)
        messages = (m * msg.to(work)).log_softmax(-1)
        mix_all = (self.relation_mix_raw.clamp(-6, math.log(16.)).exp() if c.strong_relations
                   else self.relation_mix_raw.sigmoid())
        gain = self.count_gain.clamp(0, 1)[None, None, :, :, None]
        routed = []
        if c.dense_read == "transport":
            total = torch.stack([messages.index_select(2, self.incoming[j]).sum(2)
                                 + local[:, :, j].to(work).clamp_min(1e-8).log() for j in range(nl)], 2)
            complements = total.index_select(2, self.source) - messages.index_select(2, self.reverse_edge)
            consensus = complements.softmax(-1)
            root_local = local.index_select(2, self.source).to(work)
            strength = mix_all[self.source][None, None, :, :, None]
            root_query = ((root_local + strength * consensus) / (1 + strength)).to(dtype)
            # the same memories read a second time with another query (one more scan of the same writes)
            moved, _ = gdn_scan(root_query.reshape(b, t, ne * h, m), flat["k"], flat["v"], flat["g"], flat["beta"], r0)
            moved = moved.reshape(b, t, ne, h, m) * root_query.to(work).norm(dim=-1, keepdim=True)
            transport_logits = (m * moved.to(work)).log_softmax(-1)
            local_mass = local.to(work).clamp_min(1e-8).log() + gain * n.log()
            local_route = local_mass.softmax(-1)
            cross_mass = local_mass
            if c.strong_relations:
                cross_mass = (self.read_local_raw.sigmoid()[None, None, :, :, None]
                              * local.to(work).clamp_min(1e-8).log() + gain * n.log())
            cross = (transport_logits + cross_mass.index_select(2, self.target)).softmax(-1)
            for j in range(nl):
                inc = cross.index_select(2, self.incoming[j])
                if c.strong_relations:
                    weights = self.read_edge_logits.index_select(0, self.incoming[j]).softmax(0)
                    proposal = (inc * weights[None, None, :, :, None]).sum(2)
                else:
                    proposal = inc.mean(2)
                mix = mix_all[j][None, None, :, None]
                routed.append((local_route[:, :, j] + mix * proposal) / (1 + mix))
        else:
            for j in range(nl):
                product = messages.index_select(2, self.incoming[j]).sum(2).softmax(-1)
                mix = mix_all[j][None, None, :, None]
                routed.append((local[:, :, j].to(work) + mix * product) / (1 + mix))
        route = torch.stack(routed, 2)
        rf = rf.reshape(b, ne, h, m, m)
        relations = tuple(RelationState(i, j, rf[:, e]) for e, (i, j) in enumerate(self.edges))
        return route, relations

    def forward(self, q: Tensor, k: Tensor, v: Tensor, state: PaperState | None = None, *,
                return_diagnostics: bool = False, control_input: Tensor | None = None):
        c = self.config
        if (q.ndim != 4 or q.shape != k.shape or q.shape[:3] != v.shape[:3] or q.shape[2:] != (c.heads, c.key_dim)
                or v.shape[-1] != c.value_dim):
            raise ValueError("Q/K [B,T,H,Dk], V [B,T,H,Dv] must match config")
        _lib.require_device(q)
        if q.dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("backend='hip' computes in float32 or bfloat16 activations")
        if state is None:
            state = self.initial_state(q.shape[0], q.device, q.dtype)
        if c.control_dim and (control_input is None or control_input.shape != q.shape[:2] + (c.control_dim,)):
            raise ValueError("full hidden controls [B,T,control_dim] required")
        if not isinstance(state, PaperState) or state.chunk_size != c.chunk_size:
            raise ValueError("PaperDenseGPA requires its own matching cache")
        outputs, routes = [], []
        start = 0
        while start < q.shape[1]:
            end = min(q.shape[1], start + c.chunk_size - state.chunk_offset)
            ctrl = control_input[:, start:end] if control_input is not None else None
            y, state, r = self._segment(q[:, start:end], k[:, start:end], v[:, start:end], state, ctrl)
            outputs.append(y)
            if return_diagnostics:
                routes.append(r)
            start = end
        y = torch.cat(outputs, 1) if outputs else v.new_empty(v.shape)
        if return_diagnostics:
            empty = q.new_empty(q.shape[:2] + (len(c.slots), c.heads, c.slots[0]))
            return y, state, {"routes": torch.cat(routes, 1) if routes else empty, "state_elements": state.numel()}
        return y, state
