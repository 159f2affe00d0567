"""Element-wise glue of the inference path in one launch each
(`gpa_gate_act_forward`, `gpa_token_logits_forward`, `gpa_output_mix_forward`,
csrc/token_glue.hip): the gate nonlinearities of a level (reference
attention.py:161-174), one token's counts, base logits and local read
distribution (:316-323, :196-204, :330) and the output mix (:340-341).  They
carry no autograd: the schedule uses them when no gradient is recorded."""
from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from . import _lib


def gate_act(raw: Tensor, bias: Tensor, beta_max: float, decay_scale: float):
    """(g_in, b_in, g_out, b_out), each float32 [B,T,H], from the gate inputs
    raw [B,T,H,4] and the bias [H,4]."""
    lib = _lib.load()
    b, t, h, _ = raw.shape
    outs = [torch.empty(b, t, h, device=raw.device, dtype=torch.float32) for _ in range(4)]
    bias = bias.detach().float().contiguous()
    p = _lib.GateProblem(b, t, h, _lib.DTYPE_CODES[raw.dtype], _lib.operand(raw), bias.data_ptr(),
                         float(beta_max), float(decay_scale), *(o.data_ptr() for o in outs))
    _lib.check(lib.gpa_gate_act_forward(p, _lib.stream_handle(raw.device)), "gpa_gate_act_forward")
    return tuple(outs)


class _GateAct(torch.autograd.Function):
    """The gate nonlinearities with their gradient (gpa_gate_act_forward /
    gpa_gate_act_backward): the gate inputs' gradient in their dtype and the
    bias gradient from per-workgroup partial sums."""

    @staticmethod
    def forward(ctx, raw, bias, beta_max, decay_scale):
        ctx.set_materialize_grads(False)
        raw = raw if raw.stride(-1) == 1 else raw.contiguous()
        outs = gate_act(raw, bias, beta_max, decay_scale)
        ctx.save_for_backward(raw, bias)
        ctx.consts = (float(beta_max), float(decay_scale))
        return outs

    @staticmethod
    def backward(ctx, dg_in, db_in, dg_out, db_out):
        lib = _lib.load()
        raw, bias = ctx.saved_tensors
        b, t, h, _ = raw.shape
        beta_max, decay_scale = ctx.consts
        grads = [None if d is None else d.float().contiguous() for d in (dg_in, db_in, dg_out, db_out)]
        draw = torch.empty_like(raw)
        part = torch.empty(-(-(b * t * h) // 256), h, 4, device=raw.device, dtype=torch.float32)
        bf = bias.detach().float().contiguous()
        p = _lib.GateProblem(b, t, h, _lib.DTYPE_CODES[raw.dtype], _lib.operand(raw), bf.data_ptr(),
                             beta_max, decay_scale, None, None, None, None)
        gg = _lib.GateGrads(*(d.data_ptr() if d is not None else None for d in grads), _lib.operand(draw),
                            part.data_ptr())
        _lib.check(lib.gpa_gate_act_backward(p, gg, _lib.stream_handle(raw.device)), "gpa_gate_act_backward")
        return draw, part.sum(0).to(bias.dtype), None, None


def gate_act_supported(raw: Tensor) -> bool:
    return raw.is_cuda and raw.dtype in _lib.DTYPE_CODES and raw.ndim == 4 and raw.shape[-1] == 4 \
        and raw.shape[2] <= _lib.GATE_MAX_HEADS and raw.numel() > 0


def gate_act_train(raw: Tensor, bias: Tensor, beta_max: float, decay_scale: float):
    """gate_act with autograd through the gate inputs and the bias [H,4]."""
    return _GateAct.apply(raw, bias, beta_max, decay_scale)


def token_logits(raw: Tensor, write: Tensor, count0: Tensor, gain: Tensor, scale: Tensor):
    """(logits [B,1,H,M] float32, counts [B,H,M] float32, local [B,1,H,M] in
    raw's dtype) of one token of one level."""
    lib = _lib.load()
    b, _, h, m = raw.shape
    c0 = count0.float()
    if c0.stride(2) != 1 or c0.stride(1) != m:
        c0 = c0.contiguous()
    gain, scale = gain.detach().float().contiguous(), scale.detach().float().contiguous()
    logits = torch.empty(b, 1, h, m, device=raw.device, dtype=torch.float32)
    count = torch.empty(b, h, m, device=raw.device, dtype=torch.float32)
    local = torch.empty(b, 1, h, m, device=raw.device, dtype=raw.dtype)
    p = _lib.TokenLogitsProblem(b, h, m, _lib.DTYPE_CODES[raw.dtype], _lib.operand(raw), _lib.operand(write),
                                c0.data_ptr(), c0.stride(0), gain.data_ptr(), scale.data_ptr(),
                                logits.data_ptr(), count.data_ptr(), local.data_ptr())
    _lib.check(lib.gpa_token_logits_forward(p, _lib.stream_handle(raw.device)), "gpa_token_logits_forward")
    return logits, count, local


def token_logits_many(calls) -> list[tuple[Tensor, Tensor, Tensor]]:
    """`token_logits` of several levels in one launch (gpa_token_logits_many);
    `calls` holds its (raw, write, count0, gain, scale) tuples, all of one
    dtype.  Returns [(logits, counts, local)] in order, the bits of one call
    per level."""
    if not calls:
        return []
    if len(calls) > _lib.TOKEN_LOGITS_MAX_PACK:
        raise ValueError(f"token_logits_many: at most {_lib.TOKEN_LOGITS_MAX_PACK} levels per call")
    lib = _lib.load()
    probs = (_lib.TokenLogitsProblem * len(calls))()
    keep, outs = [], []
    for i, (raw, write, count0, gain, scale) in enumerate(calls):
        b, _, h, m = raw.shape
        c0 = count0.float()
        if c0.stride(2) != 1 or c0.stride(1) != m:
            c0 = c0.contiguous()
        gain, scale = gain.detach().float().contiguous(), scale.detach().float().contiguous()
        logits = torch.empty(b, 1, h, m, device=raw.device, dtype=torch.float32)
        count = torch.empty(b, h, m, device=raw.device, dtype=torch.float32)
        local = torch.empty(b, 1, h, m, device=raw.device, dtype=raw.dtype)
        probs[i] = _lib.TokenLogitsProblem(b, h, m, _lib.DTYPE_CODES[raw.dtype], _lib.operand(raw),
                                           _lib.operand(write), c0.data_ptr(), c0.stride(0), gain.data_ptr(),
                                           scale.data_ptr(), logits.data_ptr(), count.data_ptr(), local.data_ptr())
        keep.append((c0, gain, scale))
        outs.append((logits, count, local))
    _lib.check(lib.gpa_token_logits_many(probs, len(calls), _lib.stream_handle(calls[0][0].device)),
               "gpa_token_logits_many")
    return outs


def output_mix(reads, weights: Tensor, out: Tensor | None = None) -> Tensor:
    """sum_j weights[j][h] reads[j], rounded to the reads' dtype; into `out`
    (a [B,T,H,Dv] tensor of that dtype) when given."""
    lib = _lib.load()
    b, t, h, dv = reads[0].shape
    if out is None:
        out = torch.empty_like(reads[0])
    elif out.shape != reads[0].shape or out.dtype != reads[0].dtype or out.device != reads[0].device:
        raise ValueError("output_mix: out must match the reads' shape, dtype and device")
    w = weights.detach().float().contiguous()
    p = _lib.MixProblem()
    p.batch, p.tokens, p.heads, p.value_dim, p.levels = b, t, h, dv, len(reads)
    p.dtype = _lib.DTYPE_CODES[reads[0].dtype]
    for j, r in enumerate(reads):
        p.read[j] = _lib.operand(r)
    p.weights, p.out = w.data_ptr(), _lib.operand(out)
    _lib.check(lib.gpa_output_mix_forward(p, _lib.stream_handle(out.device)), "gpa_output_mix_forward")
    return out


def _mix_problem(reads, weights: Tensor, out: Tensor | None) -> _lib.MixProblem:
    b, t, h, dv = reads[0].shape
    p = _lib.MixProblem()
    p.batch, p.tokens, p.heads, p.value_dim, p.levels = b, t, h, dv, len(reads)
    p.dtype = _lib.DTYPE_CODES[reads[0].dtype]
    for j, r in enumerate(reads):
        p.read[j] = _lib.operand(r)
    p.weights = weights.data_ptr()
    p.out = _lib.operand(out)
    return p


class _OutputMix(torch.autograd.Function):
    """The output mix with its gradient (attention.py:340-341):
    gpa_output_mix_forward, then gpa_output_mix_backward (the reads' gradients
    and per-tile partial sums of the weights' gradient)."""

    @staticmethod
    def forward(ctx, weights, *reads):
        reads = [r if r.stride(-1) == 1 else r.contiguous() for r in reads]
        w = weights.detach().float().contiguous()
        out = output_mix(reads, w)
        ctx.save_for_backward(w, *reads)
        return out

    @staticmethod
    def backward(ctx, dout):
        lib = _lib.load()
        w, *reads = ctx.saved_tensors
        b, t, h, dv = reads[0].shape
        dout = dout.to(reads[0].dtype).contiguous()
        dreads = [torch.empty_like(r) for r in reads]
        tiles = -(-(b * t) // 32)
        part = torch.empty(tiles, len(reads), h, device=dout.device, dtype=torch.float32)
        g = _lib.MixGrads()
        g.dout = _lib.operand(dout)
        for j, d in enumerate(dreads):
            g.dread[j] = _lib.operand(d)
        g.dweights = part.data_ptr()
        _lib.check(lib.gpa_output_mix_backward(_mix_problem(reads, w, None), g, _lib.stream_handle(dout.device)),
                   "gpa_output_mix_backward")
        return (part.sum(0), *dreads)


def output_mix_supported(reads) -> bool:
    """Shapes the backward kernel takes: 16-byte value vectors (V a multiple of
    8 in bf16, 4 in float32), at most 512 of them per token, contiguous reads."""
    r0 = reads[0]
    if not (1 <= len(reads) <= _lib.DECODE_MAX_LEVELS and r0.dtype in _lib.DTYPE_CODES and r0.ndim == 4):
        return False
    vec = 16 // r0.element_size()
    return (r0.shape[1] > 0 and r0.shape[2] <= _lib.MIX_MAX_HEADS and r0.shape[3] % vec == 0
            and r0.shape[2] * r0.shape[3] <= 512 * vec
            and all(r.shape == r0.shape and r.dtype == r0.dtype and r.is_contiguous() and r.data_ptr() % 16 == 0
                    for r in reads))


def output_mix_train(reads, weights: Tensor) -> Tensor:
    """sum_j weights[j][h] reads[j] rounded to the reads' dtype, differentiable
    in the reads and the weights [L,H]."""
    return _OutputMix.apply(weights, *reads)


class _RowSoftmax(torch.autograd.Function):
    """softmax(x, -1).to(dtype) of float32 logits with its gradient
    (gpa_row_softmax_forward / _backward: the backward recomputes the float32
    softmax from the logits)."""

    @staticmethod
    def forward(ctx, x, dtype):
        lib = _lib.load()
        x = x.contiguous()
        y = torch.empty(x.shape, device=x.device, dtype=dtype)
        _lib.check(lib.gpa_row_softmax_forward(x.data_ptr(), y.data_ptr(), x.numel() // x.shape[-1], x.shape[-1],
                                               _lib.DTYPE_CODES[dtype], _lib.stream_handle(x.device)),
                   "gpa_row_softmax_forward")
        ctx.save_for_backward(x)
        ctx.dtype = dtype
        return y

    @staticmethod
    def backward(ctx, dy):
        lib = _lib.load()
        (x,) = ctx.saved_tensors
        dy = dy.to(ctx.dtype).contiguous()
        dx = torch.empty_like(x)
        _lib.check(lib.gpa_row_softmax_backward(x.data_ptr(), dy.data_ptr(), dx.data_ptr(), x.numel() // x.shape[-1],
                                                x.shape[-1], _lib.DTYPE_CODES[ctx.dtype],
                                                _lib.stream_handle(x.device)), "gpa_row_softmax_backward")
        return dx, None


def softmax_rows(x: Tensor, dtype: torch.dtype) -> Tensor:
    """softmax(x, -1).to(dtype) for float32 logits on the device, rows of up to
    1024 values; the device ops otherwise."""
    if x.dtype != torch.float32 or dtype not in _lib.DTYPE_CODES or not 1 <= x.shape[-1] <= 1024 or not x.is_cuda:
        return x.softmax(-1).to(dtype)
    return _RowSoftmax.apply(x, dtype)


COPY_MAX = 4  # buffers per gpa_copy_many launch


def copy_many(pairs) -> bool:
    """dst.copy_(src) for up to COPY_MAX (dst, src) pairs of contiguous device
    tensors with equal shape and dtype, in one launch (`gpa_copy_many`).  Returns
    False, copying nothing, when a pair is not 16-byte aligned and sized."""
    if not 1 <= len(pairs) <= COPY_MAX:
        raise ValueError("copy_many: 1 to 4 pairs")
    for d, s in pairs:
        _lib.require_device(d)
        if d.shape != s.shape or d.dtype != s.dtype or d.device != s.device:
            raise ValueError("copy_many: each pair must match in shape, dtype and device")
        if (not d.is_contiguous() or not s.is_contiguous() or d.data_ptr() % 16 or s.data_ptr() % 16
                or (d.numel() * d.element_size()) % 16):
            return False
    lib = _lib.load()
    n = len(pairs)
    dst = (ctypes.c_void_p * n)(*(d.data_ptr() for d, _ in pairs))
    src = (ctypes.c_void_p * n)(*(s.data_ptr() for _, s in pairs))
    size = (ctypes.c_int64 * n)(*(d.numel() * d.element_size() for d, _ in pairs))
    _lib.check(lib.gpa_copy_many(dst, src, size, n, _lib.stream_handle(pairs[0][0].device)), "gpa_copy_many")
    return True
