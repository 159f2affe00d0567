"""Slot products and gate inputs of one level (`gpa_slot_gates_forward/backward`).

The reference computes, per level j (src/gpa/attention.py:176-177 and :165),

    slot = einsum("...hd,hmd->...hm", k, center[j].to(k.dtype))
    raw  = einsum("...hd,hdc->...hc", unit(k), gate_weight[j].to(k.dtype))

as two typed products over the same key rows.  `slot_gates` runs both in one
pass over the keys (and their gradients in one pass over dslot, draw) with
the same rounding points; the slot feature and the gate nonlinearities stay
with the caller.
"""
from __future__ import annotations

import torch
from torch import Tensor

from . import _lib, params


def supported(cfg, key: Tensor, slots: int) -> bool:
    """bf16 keys whose rows are 16-byte aligned; gates from unit(k) (no
    control input, no rsa_update); key width a multiple of 16 up to 256,
    slots a multiple of 32 up to 256."""
    d = key.shape[-1]
    aligned = (key.stride(-1) == 1 and all(s % 8 == 0 for s in key.stride()[:-1])
               and key.data_ptr() % 16 == 0)
    return (key.dtype == torch.bfloat16 and not cfg.control_dim and not cfg.rsa_update and aligned
            and d % 16 == 0 and 16 <= d <= 256 and slots % 32 == 0 and 32 <= slots <= 256)


def _problem(key: Tensor, cb: Tensor, ct: Tensor | None, wg: Tensor, slot: Tensor | None,
             raw: Tensor | None) -> _lib.SlotProblem:
    b, t, h, d = key.shape
    p = _lib.SlotProblem()
    p.batch, p.tokens, p.heads, p.key_dim, p.slots = b, t, h, d, cb.shape[1]
    p.dtype = _lib.DTYPE_CODES[key.dtype]
    p.key = _lib.operand(key)
    p.center, p.gate_w = cb.data_ptr(), wg.data_ptr()
    p.center_t = ct.data_ptr() if ct is not None else None
    if slot is not None:
        p.slot, p.raw = _lib.operand(slot), _lib.operand(raw)
    return p


class _SlotGates(torch.autograd.Function):
    @staticmethod
    def forward(ctx, key, center, gate_w):
        _lib.require_device(key)
        ctx.set_materialize_grads(False)
        lib = _lib.load()
        b, t, h, _ = key.shape
        cb = params.derived(("slot_center", id(center), key.dtype), (center,),
                            lambda: center.detach().to(key.dtype).contiguous())
        wg = params.derived(("slot_gate_w", id(gate_w), key.dtype), (gate_w,),
                            lambda: gate_w.detach().to(key.dtype).contiguous())
        slot = key.new_empty(b, t, h, cb.shape[1])
        raw = key.new_empty(b, t, h, 4)
        prob = _problem(key, cb, None, wg, slot, raw)
        _lib.check(lib.gpa_slot_gates_forward(prob, _lib.stream_handle(key.device)), "gpa_slot_gates_forward")
        ctx.save_for_backward(key, cb, wg)
        ctx.param_dtypes = (center.dtype, gate_w.dtype)
        return slot, raw

    @staticmethod
    def backward(ctx, dslot, draw):
        lib = _lib.load()
        key, cb, wg = ctx.saved_tensors
        b, t, h, d = key.shape
        m = cb.shape[1]
        dslot = dslot.to(key.dtype).contiguous() if dslot is not None else key.new_zeros(b, t, h, m)
        draw = draw.to(key.dtype).contiguous() if draw is not None else key.new_zeros(b, t, h, 4)
        ct = cb.transpose(1, 2).contiguous()
        dkey = torch.empty(b, t, h, d, device=key.device, dtype=key.dtype)
        dcenter = torch.empty(h, m, d, device=key.device, dtype=torch.float32)
        dgate = torch.empty(h, d, 4, device=key.device, dtype=torch.float32)
        prob = _problem(key, cb, ct, wg, None, None)
        gr = _lib.SlotGrads()
        gr.dslot, gr.draw, gr.dkey = _lib.operand(dslot), _lib.operand(draw), _lib.operand(dkey)
        gr.dcenter, gr.dgate_w = dcenter.data_ptr(), dgate.data_ptr()
        _lib.check(lib.gpa_slot_gates_backward(prob, gr, _lib.stream_handle(key.device)), "gpa_slot_gates_backward")
        dt = ctx.param_dtypes
        return dkey, dcenter.to(dt[0]), dgate.to(dt[1])


def slot_gates(key: Tensor, center: Tensor, gate_w: Tensor) -> tuple[Tensor, Tensor]:
    """(slot [B,T,H,M], raw gate inputs [B,T,H,4]) in key's dtype, from key
    [B,T,H,Dk], center [H,M,Dk] and gate_w [H,Dk,4]."""
    return _SlotGates.apply(key, center, gate_w)


def slot_gates_act(key: Tensor, center: Tensor, gate_w: Tensor, bias: Tensor, beta_max: float,
                   decay_scale: float) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """`slot_gates` followed by the gate nonlinearities (`glue.gate_act`) in
    one launch, for inference (no autograd): (slot [B,T,H,M] in key's dtype,
    g_in, b_in, g_out, b_out each float32 [B,T,H]), the bits of the two calls."""
    _lib.require_device(key)
    if torch.is_grad_enabled() and any(x.requires_grad for x in (key, center, gate_w, bias)):
        raise RuntimeError("slot_gates_act has no backward: call it under torch.no_grad() or inference_mode()")
    lib = _lib.load()
    b, t, h, _ = key.shape
    cb = params.derived(("slot_center", id(center), key.dtype), (center,),
                        lambda: center.detach().to(key.dtype).contiguous())
    wg = params.derived(("slot_gate_w", id(gate_w), key.dtype), (gate_w,),
                        lambda: gate_w.detach().to(key.dtype).contiguous())
    slot = key.new_empty(b, t, h, cb.shape[1])
    raw = key.new_empty(b, t, h, 4)
    prob = _problem(key, cb, None, wg, slot, raw)
    outs = [torch.empty(b, t, h, device=key.device, dtype=torch.float32) for _ in range(4)]
    bias = bias.detach().float().contiguous()
    gates = _lib.GateProblem(b, t, h, _lib.DTYPE_CODES[key.dtype], _lib.operand(raw), bias.data_ptr(),
                             float(beta_max), float(decay_scale), *(o.data_ptr() for o in outs))
    _lib.check(lib.gpa_slot_gates_act_forward(prob, gates, _lib.stream_handle(key.device)),
               "gpa_slot_gates_act_forward")
    return (slot, *outs)
