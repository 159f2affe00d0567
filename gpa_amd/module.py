"""`DenseGPA`: parameters, initial cache and the forward entry of the HIP backend.

Parameter names, shapes, registration order and default initialisation
(including the order in which the global RNG is consumed) follow the reference
module (src/gpa/attention.py:91-144), so `state_dict`s load strictly in both
directions and a seeded construction yields bit-identical parameters.  The
forward pass validates exactly what the reference validates
(attention.py:347-369) and then runs the level-major HIP schedule in
`gpa_amd.schedule`.
"""
from __future__ import annotations

import math

import torch
from torch import Tensor, nn

from .config import GPAConfig
from .state import GPAState, LevelState, RelationState


def _softplus_inverse(x: float) -> float:
    return math.log(math.expm1(x))


class QuadraticFeatures(nn.Module):
    """Norm-preserving quadratic Q/K sketch (reference src/gpa/features.py:8-25).

    z = u(x) + 2*sigmoid(gain_raw)*sqrt(D)*(u(x)L)*(u(x)R);  out = u(z)*||x||.
    Parameters and initialisation are the reference's; the map runs in the HIP
    kernels of gpa_amd.features.
    """

    def __init__(self, heads: int, dim: int):
        super().__init__()
        self.left = nn.Parameter(torch.empty(heads, dim, dim))
        self.right = nn.Parameter(torch.empty(heads, dim, dim))
        for matrix in (*self.left, *self.right):
            nn.init.orthogonal_(matrix)
        self.gain_raw = nn.Parameter(torch.full((heads,), math.log(.25 / 1.75)))
        self.dim = dim

    def forward(self, x: Tensor) -> Tensor:
        """x [..., H, D] on the GPU: one HIP launch forward, one backward (plus
        the weight gradients' batched product), gpa_amd.features."""
        from .features import quadratic_features
        return quadratic_features(x, self.left, self.right, self.gain_raw)


class DenseGPA(nn.Module):
    """Projected Q,K [B,T,H,Dk], V [B,T,H,Dv] -> output [B,T,H,Dv] and a cache.

    Same call signature and return convention as the reference
    (attention.py:347-413): ``forward(q, k, v, state=None, *, position_ids=None,
    return_diagnostics=False, control_input=None)``.
    """

    def __init__(self, config: GPAConfig):
        super().__init__()
        self.config = config
        h, dk, dv = config.heads, config.key_dim, config.value_dim
        names = ("center", "inner_prefix", "outer_prefix", "route_weight", "query_weight",
                 "route_up", "route_down", "gate_weight", "gate_bias")
        for name in names:
            setattr(self, name, nn.ParameterList())
        gate_in = config.control_dim or dk
        bias_row = [_softplus_inverse(config.decay_init),
                    math.log(config.beta_init / (config.beta_max - config.beta_init))] * 2
        for m in config.slots:
            # One level's parameters; the randn calls run in this exact order.
            self.center.append(nn.Parameter(torch.randn(h, m, dk) / math.sqrt(dk)))
            self.inner_prefix.append(nn.Parameter(torch.randn(h, dk, m) * .002))
            self.outer_prefix.append(nn.Parameter(torch.randn(h, m, dv) * .002))
            self.route_weight.append(nn.Parameter(torch.eye(m).repeat(h, 1, 1)))
            self.query_weight.append(nn.Parameter(torch.randn(h, dk, m) / math.sqrt(dk)))
            self.route_up.append(nn.Parameter(torch.randn(h, m, 2 * m) / math.sqrt(m)))
            self.route_down.append(nn.Parameter(torch.randn(h, 2 * m, m) * .002))
            self.gate_weight.append(nn.Parameter(torch.zeros(h, gate_in, 4)))
            self.gate_bias.append(nn.Parameter(torch.tensor(bias_row).repeat(h, 1)))
        n_levels = config.levels
        self.residual_raw = nn.Parameter(torch.zeros(n_levels, h, 2))
        self.count_gain_raw = nn.Parameter(torch.full((n_levels, h), _softplus_inverse(.1)))
        self.moment_gain = nn.Parameter(torch.full((n_levels, h), .1))
        self.route_mlp_gain = nn.Parameter(torch.full((n_levels, h), .1))
        self.output_logits = nn.Parameter(torch.zeros(n_levels, h))
        self.edges = config.edges
        self.register_buffer("_edge_source", torch.tensor([i for i, _ in self.edges], dtype=torch.long),
                             persistent=False)
        self.register_buffer("_edge_target", torch.tensor([j for _, j in self.edges], dtype=torch.long),
                             persistent=False)
        self.relation_prefix = nn.ParameterList(
            [nn.Parameter(torch.zeros(h, config.slots[i], config.slots[j])) for i, j in self.edges])
        n_edges = len(self.edges)
        self.edge_logits = nn.Parameter(torch.zeros(n_edges, h))
        self.relation_gain = nn.Parameter(torch.full((n_levels, h), .1))
        self.relation_decay_raw = nn.Parameter(
            torch.full((n_edges, h), _softplus_inverse(config.relation_decay_init)))
        self.relation_beta_raw = nn.Parameter(
            torch.full((n_edges, h), math.log(config.relation_beta_init / (1 - config.relation_beta_init))))
        if config.balanced_bridge:
            self.bridge_mix_raw = nn.Parameter(torch.zeros(n_levels, h))
        if config.quadratic_features:
            self.feature_map = QuadraticFeatures(h, dk)
        if config.learn_read_scale:
            self.read_log_scale = nn.Parameter(torch.full((n_levels, h), math.log(config.read_scale)))

    # ------------------------------------------------------------------ cache
    def initial_state(self, batch: int, *, device=None, dtype=None) -> GPAState:
        """Learned prefixes broadcast over the batch, zero counts (attention.py:146-159).

        The prefixes are expanded, not copied, so gradients of a loss reach
        `inner_prefix`, `outer_prefix` and `relation_prefix`.
        """
        anchor = self.center[0]
        device = anchor.device if device is None else device
        dtype = anchor.dtype if dtype is None else dtype
        work = torch.float64 if dtype == torch.float64 else torch.float32

        def spread(p: Tensor) -> Tensor:
            return p.to(device=device, dtype=work).unsqueeze(0).expand(batch, *p.shape)

        moments = self.config.positional_mode == "moments"
        levels = []
        for m, a, b in zip(self.config.slots, self.inner_prefix, self.outer_prefix):
            count = torch.zeros(batch, self.config.heads, m, device=device, dtype=work)
            position = (torch.zeros(batch, self.config.heads, self.config.key_dim, m, device=device, dtype=work)
                        if moments else None)
            levels.append(LevelState(spread(a), spread(b), count, position))
        relations = tuple(RelationState(i, j, spread(p)) for (i, j), p in zip(self.edges, self.relation_prefix))
        return GPAState(tuple(levels), relations, chunk_size=self.config.chunk_size)

    # ---------------------------------------------------------------- forward
    def forward(self, q: Tensor, k: Tensor, v: Tensor, state: GPAState | None = None, *,
                position_ids: Tensor | None = None, return_diagnostics: bool = False,
                control_input: Tensor | None = None):
        cfg = self.config
        if q.ndim != 4 or q.shape != k.shape or q.shape[:3] != v.shape[:3]:
            raise ValueError("expected Q,K [B,T,H,Dk], V [B,T,H,Dv]")
        if q.shape[2:] != (cfg.heads, cfg.key_dim) or v.shape[-1] != cfg.value_dim:
            raise ValueError("input heads/dimensions do not match GPAConfig")
        if q.device != k.device or q.device != v.device or q.dtype != k.dtype or q.dtype != v.dtype:
            raise ValueError("Q,K,V must share device and floating dtype")
        if cfg.control_dim and (control_input is None
                                or control_input.shape != q.shape[:2] + (cfg.control_dim,)):
            raise ValueError("full hidden controls [B,T,control_dim] required")
        if cfg.quadratic_features:
            q, k = self.feature_map(torch.stack((q, k))).unbind(0)
        if state is None:
            state = self.initial_state(q.shape[0], device=q.device, dtype=q.dtype)
        if state.chunk_size != cfg.chunk_size:
            raise ValueError("cannot switch cache between recurrent and lagged chunk semantics")
        if (len(state.levels) != cfg.levels
                or tuple((r.source, r.target) for r in state.relations) != self.edges):
            raise ValueError("cache topology does not match this model")
        if position_ids is None and cfg.positional_mode == "moments":
            # only the positional moments read positions (attention.py:305, :318-323)
            position_ids = torch.arange(state.position, state.position + q.shape[1], device=q.device)
        if position_ids is not None and position_ids.shape not in ((q.shape[1],), (q.shape[0], q.shape[1])):
            raise ValueError("position_ids must be [T] or [B,T]")
        from .decode import decode_step, decode_supported
        from .schedule import run_segment, run_tokens
        if q.shape[1] == 0:
            out, new_state, routes = v.new_empty(v.shape), state, None
        elif cfg.chunk_size == 1:
            out, new_state, routes = run_tokens(self, q, k, v, state, control_input,
                                                want_routes=return_diagnostics, position_ids=position_ids)
        elif not return_diagnostics and decode_supported(self, q, k, v, state, control_input):
            (out, new_state), routes = decode_step(self, q, k, v, state), None
        else:
            out, new_state, routes = run_segment(self, q, k, v, state, position_ids, control_input,
                                                 want_routes=return_diagnostics)
        if return_diagnostics:
            if routes is None:
                routes = tuple(q.new_empty(q.shape[:3] + (m,)) for m in cfg.slots)
            return out, new_state, {"routes": routes, "edges": self.edges,
                                    "state_elements": new_state.numel(),
                                    "position": new_state.position}
        return out, new_state
