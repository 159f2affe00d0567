"""Slot counts and base logits of one level (`gpa_count_logits_forward/backward`).

The reference builds, per level j (src/gpa/attention.py:196-204, counts of
:318-319),

    counts = count0 + cumsum_t(write)          # float32, [B,T,H,M]
    logits = read_scale * raw + softplus(count_gain) * log1p(counts)

`count_logits` returns (logits, final counts) without materialising the
counts; it is differentiable in raw, write, count0 and the two per-head
scalars.
"""
from __future__ import annotations

import torch
from torch import Tensor

from . import _lib

TILE = 64


def supported(cfg, dtype: torch.dtype, slots: int) -> bool:
    """The per-token counts are needed elsewhere only by the product read with
    relation marginals (attention.py:247-250)."""
    return (dtype in _lib.DTYPE_CODES and slots <= 256
            and not (cfg.paper_product_read and cfg.relation_marginal))


def _count0(c: Tensor) -> tuple[Tensor, int]:
    c = c.float()
    b, h, m = c.shape
    if c.stride(2) != 1 or c.stride(1) != m:
        c = c.contiguous()
    return c, c.stride(0)


def _problem(raw, write, c0, sb, gain, scale, logits, final, prefix):
    b, t, h, m = raw.shape
    p = _lib.CountProblem()
    p.batch, p.tokens, p.heads, p.slots, p.dtype = b, t, h, m, _lib.DTYPE_CODES[raw.dtype]
    p.raw, p.write = _lib.operand(raw), _lib.operand(write)
    p.count0, p.count0_sb = c0.data_ptr(), sb
    p.gain, p.scale = gain.data_ptr(), scale.data_ptr()
    p.logits = logits.data_ptr() if logits is not None else None
    p.final_count = final.data_ptr() if final is not None else None
    p.prefix = prefix.data_ptr()
    return p


class _CountLogits(torch.autograd.Function):
    @staticmethod
    def forward(ctx, raw, write, count0, gain, scale):
        _lib.require_device(raw)
        ctx.set_materialize_grads(False)
        lib = _lib.load()
        b, t, h, m = raw.shape
        n = (t + TILE - 1) // TILE
        f32 = dict(device=raw.device, dtype=torch.float32)
        c0, sb = _count0(count0)
        g, s = gain.detach().float().contiguous(), scale.detach().float().contiguous()
        logits = torch.empty(b, t, h, m, **f32)
        final = torch.empty(b, h, m, **f32)
        prefix = torch.empty(b, h, n, m, **f32)
        prob = _problem(raw, write, c0, sb, g, s, logits, final, prefix)
        _lib.check(lib.gpa_count_logits_forward(prob, _lib.stream_handle(raw.device)), "gpa_count_logits_forward")
        ctx.save_for_backward(raw, write, c0, g, s, prefix)
        ctx.sb = sb
        ctx.param_dtypes = (count0.dtype, gain.dtype, scale.dtype)
        return logits, final

    @staticmethod
    def backward(ctx, dlogits, dfinal):
        lib = _lib.load()
        raw, write, c0, g, s, prefix = ctx.saved_tensors
        b, t, h, m = raw.shape
        n = prefix.shape[2]
        dev = raw.device
        f32 = dict(device=dev, dtype=torch.float32)
        dlogits = dlogits.float().contiguous() if dlogits is not None else torch.zeros(b, t, h, m, **f32)
        dfinal = dfinal.float().contiguous() if dfinal is not None else None
        draw, dwrite = torch.empty_like(raw), torch.empty_like(write)
        dcount0 = torch.empty(b, h, m, **f32) if ctx.needs_input_grad[2] else None
        partials = torch.empty(b * h * n, 2, **f32)
        tsum = torch.empty(b, h, n, m, **f32)
        prob = _problem(raw, write, c0, ctx.sb, g, s, None, None, prefix)
        gr = _lib.CountGrads()
        gr.dlogits = dlogits.data_ptr()
        gr.dfinal = dfinal.data_ptr() if dfinal is not None else None
        gr.draw, gr.dwrite = _lib.operand(draw), _lib.operand(dwrite)
        gr.dcount0 = dcount0.data_ptr() if dcount0 is not None else None
        gr.partials, gr.tsum = partials.data_ptr(), tsum.data_ptr()
        _lib.check(lib.gpa_count_logits_backward(prob, gr, _lib.stream_handle(dev)), "gpa_count_logits_backward")
        sums = partials.view(b, h, n, 2).sum((0, 2))
        dt = ctx.param_dtypes
        return (draw, dwrite, dcount0.to(dt[0]) if dcount0 is not None else None,
                sums[:, 0].to(dt[1]) if ctx.needs_input_grad[3] else None,
                sums[:, 1].to(dt[2]) if ctx.needs_input_grad[4] else None)


def count_logits(raw: Tensor, write: Tensor, count0: Tensor, gain: Tensor, scale: Tensor) -> tuple[Tensor, Tensor]:
    """(logits [B,T,H,M] float32, final counts [B,H,M]) of one level: raw and
    write [B,T,H,M] in the activation dtype, count0 [B,H,M], gain and scale
    [H] (softplus of the count gain, and the read scale)."""
    if write.dtype != raw.dtype:
        write = write.to(raw.dtype)
    raw = raw if raw.stride(-1) == 1 else raw.contiguous()
    write = write if write.stride(-1) == 1 else write.contiguous()
    return _CountLogits.apply(raw, write, count0, gain, scale)
