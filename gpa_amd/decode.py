"""Fused single-token decode of the DenseGPA core (`gpa_decode_step`).

The reference decodes in chunk mode by running its block segment on one token
(src/gpa/attention.py:396-405 with T = 1).  Here one HIP kernel does the whole
token for every (batch, head) stream.  It is used by `DenseGPA.forward` for a
one-token call when no gradient is needed and the configuration is one the
kernel covers (`decode_supported`); every other call takes the level-major
schedule.  The cache semantics are the reference's: new tensors are returned,
the block-start snapshots are the incoming states when the token starts a
block, and the returned cache keeps them while the block is open.
"""
from __future__ import annotations

import torch
from torch import Tensor

from . import _lib
from .state import GPAState, LevelState, RelationState, ResidualSnapshot

# The fused kernel is switched off: its first launch on an MI355X ended in a GPU
# memory fault whose cause has not been found (the host build of the same
# source, under AddressSanitizer, matches the oracle with every access in
# bounds: tests/test_decode_emulated.py).  While it is off, every one-token call
# takes the level-major schedule and `decode_step` refuses to launch.
FUSED_DECODE = False


def decode_supported(model, q: Tensor, k: Tensor, v: Tensor, state: GPAState, control) -> bool:
    cfg = model.config
    if not FUSED_DECODE:
        return False
    if q.shape[1] != 1 or control is not None or q.dtype not in _lib.DTYPE_CODES:
        return False
    if (cfg.positional_mode not in ("gated", "none") or cfg.slot_feature != "linear" or cfg.control_dim
            or cfg.rsa_update or cfg.paper_product_read or cfg.shared_query_center or cfg.balanced_bridge
            or cfg.quadratic_features or cfg.learn_read_scale):
        return False
    if (cfg.levels > _lib.DECODE_MAX_LEVELS or max(cfg.slots) > _lib.DECODE_MAX_WIDTH
            or cfg.key_dim > _lib.DECODE_MAX_WIDTH or cfg.value_dim > _lib.DECODE_MAX_WIDTH):
        return False
    if torch.is_grad_enabled():
        tracked = [q, k, v, *model.parameters()]
        tracked += [t for lv in state.levels for t in (lv.inner, lv.outer, lv.count)]
        tracked += [r.memory for r in state.relations]
        if any(t.requires_grad for t in tracked):
            return False
    return True


def _state_arg(t: Tensor) -> tuple[_lib.DecodeState, Tensor]:
    """A [B,H,rows,cols] (or [B,H,cols]) fp32 state whose head slices are
    contiguous; the batch stride may be anything (0 for a broadcast prefix)."""
    t = t.float()
    inner = t.shape[1:]
    want, step = [], 1
    for size in reversed(inner):
        want.append(step)
        step *= size
    if tuple(t.stride()[1:]) != tuple(reversed(want)):
        t = t.contiguous()
    return _lib.DecodeState(t.data_ptr(), t.stride(0)), t


def decode_step(model, q: Tensor, k: Tensor, v: Tensor, state: GPAState):
    """One token of every stream: q,k [B,1,H,Dk], v [B,1,H,Dv] -> (out, new state)."""
    if not FUSED_DECODE:
        raise _lib.HipBackendError("the fused decode kernel is switched off (unresolved GPU memory fault)")
    _lib.require_device(q)
    cfg = model.config
    lib = _lib.load()
    bsz, _, heads, dk = q.shape
    dv = v.shape[-1]
    dev = q.device
    f32 = dict(device=dev, dtype=torch.float32)
    q, k, v = (x if x.stride(-1) == 1 else x.contiguous() for x in (q, k, v))
    out = torch.empty(bsz, 1, heads, dv, device=dev, dtype=v.dtype)
    frozen = state.frozen or tuple(ResidualSnapshot(lv.inner, lv.outer) for lv in state.levels)
    keep = []  # tensors whose memory the launch reads
    prob = _lib.DecodeProblem()
    prob.batch, prob.heads, prob.key_dim, prob.value_dim = bsz, heads, dk, dv
    prob.levels, prob.dtype = cfg.levels, _lib.DTYPE_CODES[q.dtype]
    prob.positional_none = int(cfg.positional_mode == "none")
    prob.read_scale, prob.query_scale, prob.beta_max = cfg.read_scale, cfg.query_scale, cfg.beta_max
    prob.q, prob.k, prob.v, prob.out = (_lib.operand(x) for x in (q, k, v, out))

    def param(t: Tensor) -> int:
        t = t.detach().float().contiguous()
        keep.append(t)
        return t.data_ptr()

    prob.residual_raw = param(model.residual_raw)
    prob.count_gain_raw = param(model.count_gain_raw)
    prob.route_mlp_gain = param(model.route_mlp_gain)
    prob.output_logits = param(model.output_logits)
    prob.relation_gain = param(model.relation_gain)
    prob.edge_logits = param(model.edge_logits)
    prob.relation_decay_raw = param(model.relation_decay_raw)
    prob.relation_beta_raw = param(model.relation_beta_raw)
    new_levels = []
    for j, (m, lv, snap) in enumerate(zip(cfg.slots, state.levels, frozen)):
        d = prob.level[j]
        d.slots = m
        d.center, d.gate_weight, d.gate_bias = (param(p[j]) for p in (model.center, model.gate_weight,
                                                                      model.gate_bias))
        d.route_weight, d.query_weight = param(model.route_weight[j]), param(model.query_weight[j])
        d.route_up, d.route_down = param(model.route_up[j]), param(model.route_down[j])
        for name, t in (("inner", lv.inner), ("outer", lv.outer), ("count", lv.count),
                        ("snap_inner", snap.inner), ("snap_outer", snap.outer)):
            arg, t = _state_arg(t)
            keep.append(t)
            setattr(d, name, arg)
        a = torch.empty(bsz, heads, dk, m, **f32)
        b = torch.empty(bsz, heads, m, dv, **f32)
        n = torch.empty(bsz, heads, m, **f32)
        d.inner_out, d.outer_out, d.count_out = a.data_ptr(), b.data_ptr(), n.data_ptr()
        new_levels.append(LevelState(a, b, n, None))
    new_rel = []
    for e, ((i, j), r) in enumerate(zip(model.edges, state.relations)):
        arg, t = _state_arg(r.memory)
        keep.append(t)
        prob.relation[e] = arg
        mem = torch.empty(bsz, heads, cfg.slots[i], cfg.slots[j], **f32)
        prob.relation_out[e] = mem.data_ptr()
        new_rel.append(RelationState(i, j, mem))
    _lib.check(lib.gpa_decode_step(prob, _lib.stream_handle(dev)), "gpa_decode_step")
    offset = (state.chunk_offset + 1) % cfg.chunk_size
    new = GPAState(tuple(new_levels), tuple(new_rel), state.position + 1, cfg.chunk_size, offset,
                   frozen if offset else None)
    return out, new
