"""Fused level write and residual of the chunk model (`gpa_level_forward/backward`).

For every token of block n (reference _block_segment, src/gpa/attention.py:
314-329, _residual :190-194), from the block's snapshots A^_n [Dk,M] and
B^_n [M,Dv]:

    w = softmax(u(key) A^_n);   key' = key - eta0 A^_n w;   value' = value - eta1 w^T B^_n

The snapshots are the scans' chunk-start states, read in place (value-major,
as `gdn_scan_hip` saves them), except block 0 when the call starts inside a
block: then it is the cached snapshot.  `level_mix` is differentiable in the
keys, values, both state tensors, the cached snapshots and eta; the state
gradients come back in the states' own layout.  `level_residual` is the same
step for a write that is given (rsa_update's softmax(slot / .25) or softmax
slot features, attention.py:186-188): only the reconstructions and the
residual run on the kernels, and the write gets its gradient through them.
"""
from __future__ import annotations

import torch
from torch import Tensor

from . import _lib, params


def supported(cfg, dtype: torch.dtype, key_dim: int, value_dim: int, slots: int) -> bool:
    """Whether the level kernels take these widths (either write mode)."""
    return (dtype in _lib.DTYPE_CODES and max(key_dim, value_dim, slots) <= _lib.LEVEL_MAX_WIDTH
            and cfg.chunk_size <= 64)


def _snapshot(t: Tensor | None) -> tuple[Tensor | None, int]:
    """A [B,H,R,C] float32 snapshot with contiguous heads; keeps a broadcast
    batch (stride 0) as it is."""
    if t is None:
        return None, 0
    t = t.detach().float()
    h, r, c = t.shape[1:]
    if t.stride()[1:] != (r * c, c, 1):
        t = t.contiguous()
    return t, t.stride(0)


def _problem(key, value, a_vm, b_vm, a_first, b_first, eta, chunk, offset, outs, saved):
    bsz, tokens, heads, dk = key.shape
    p = _lib.LevelProblem()
    p.batch, p.tokens, p.heads, p.key_dim, p.value_dim = bsz, tokens, heads, dk, value.shape[-1]
    p.slots, p.chunk, p.offset, p.dtype = a_vm.shape[-2], chunk, offset, _lib.DTYPE_CODES[key.dtype]
    p.key, p.value = _lib.operand(key), _lib.operand(value)
    p.a_states, p.b_states = a_vm.data_ptr(), b_vm.data_ptr()
    (af, asb), (bf, bsb) = a_first, b_first
    p.a_first, p.a_first_sb = (af.data_ptr() if af is not None else None), asb
    p.b_first, p.b_first_sb = (bf.data_ptr() if bf is not None else None), bsb
    p.eta = eta.data_ptr()
    p.write, p.key_out, p.value_out = (_lib.operand(t) for t in outs)
    p.rk, p.rv, p.stats = (t.data_ptr() if t is not None else None for t in saved)
    return p


def _inputs(key, value, a_vm, b_vm, a_first, b_first, eta):
    """The kernels' operand layouts: contiguous activations, float32
    contiguous states, [B,H,R,C] snapshots (with their batch strides) and eta."""
    key, value = key.contiguous(), value.contiguous()
    a_vm, b_vm = a_vm.detach().float().contiguous(), b_vm.detach().float().contiguous()
    return key, value, a_vm, b_vm, (_snapshot(a_first), _snapshot(b_first)), eta.detach().float().contiguous()


def _state_grads(key, a_vm, b_vm, af, bf):
    """Gradient buffers of the block states (block 0 zeroed where the cached
    snapshots stand in for it) and of the cached snapshots."""
    bsz, _, heads, dk = key.shape
    da, db = torch.empty_like(a_vm), torch.empty_like(b_vm)
    if af is not None:
        da[:, :, 0].zero_()
    if bf is not None:
        db[:, :, 0].zero_()
    da_first = torch.empty(bsz, heads, dk, a_vm.shape[-2], device=key.device) if af is not None else None
    m, dv = b_vm.shape[-1], b_vm.shape[-2]  # b_vm is value-major [B,H,N,Dv,M]
    db_first = torch.empty(bsz, heads, m, dv, device=key.device) if bf is not None else None
    return da, db, da_first, db_first


class _LevelMix(torch.autograd.Function):
    @staticmethod
    def forward(ctx, key, value, a_vm, b_vm, a_first, b_first, eta, chunk, offset):
        _lib.require_device(key)
        ctx.set_materialize_grads(False)
        lib = _lib.load()
        dtype = key.dtype
        bsz, tokens, heads, dk = key.shape
        dv, m = value.shape[-1], a_vm.shape[-2]
        key, value, a_vm, b_vm, firsts, eta = _inputs(key, value, a_vm, b_vm, a_first, b_first, eta)
        write = torch.empty(bsz, tokens, heads, m, device=key.device, dtype=dtype)
        key_out, value_out = torch.empty_like(key), torch.empty_like(value)
        rk = torch.empty(bsz, tokens, heads, dk, device=key.device, dtype=dtype)
        rv = torch.empty(bsz, tokens, heads, dv, device=key.device, dtype=dtype)
        stats = torch.empty(bsz, tokens, heads, 2, device=key.device, dtype=torch.float32)
        prob = _problem(key, value, a_vm, b_vm, *firsts, eta, chunk, offset, (write, key_out, value_out),
                        (rk, rv, stats))
        _lib.check(lib.gpa_level_forward(prob, _lib.stream_handle(key.device)), "gpa_level_forward")
        ctx.chunk, ctx.offset = chunk, offset
        ctx.has_first = (a_first is not None, b_first is not None)
        ctx.first_sb = (firsts[0][1], firsts[1][1])
        ctx.save_for_backward(key, value, a_vm, b_vm, firsts[0][0], firsts[1][0], eta, write, rk, rv, stats)
        return write, key_out, value_out

    @staticmethod
    def backward(ctx, dwrite, dkey_out, dvalue_out):
        lib = _lib.load()
        key, value, a_vm, b_vm, af, bf, eta, write, rk, rv, stats = ctx.saved_tensors
        dtype = key.dtype
        bsz, tokens, heads, dk = key.shape
        dv = value.shape[-1]
        value_used = dvalue_out is not None
        zeros = lambda t, like: torch.zeros_like(like) if t is None else t.to(dtype).contiguous()  # noqa: E731
        dwrite, dkey_out, dvalue_out = zeros(dwrite, write), zeros(dkey_out, key), zeros(dvalue_out, value)
        prob = _problem(key, value, a_vm, b_vm, (af, ctx.first_sb[0]), (bf, ctx.first_sb[1]), eta, ctx.chunk,
                        ctx.offset, (write, write, write), (rk, rv, stats))
        prob.key_out, prob.value_out = _lib.operand(key), _lib.operand(value)
        da, db, da_first, db_first = _state_grads(key, a_vm, b_vm, af, bf)
        nblocks = a_vm.shape[2]
        deta = torch.empty(bsz * heads * nblocks, 2, device=key.device)
        dkey = torch.empty_like(key)
        gr = _lib.LevelGrads()
        gr.dwrite, gr.dkey_out, gr.dvalue_out, gr.dkey = (_lib.operand(t) for t in (dwrite, dkey_out, dvalue_out,
                                                                                    dkey))
        gr.da_states, gr.db_states, gr.deta = da.data_ptr(), db.data_ptr(), deta.data_ptr()
        gr.da_first = da_first.data_ptr() if da_first is not None else None
        gr.db_first = db_first.data_ptr() if db_first is not None else None
        _lib.check(lib.gpa_level_backward(prob, gr, _lib.stream_handle(key.device)), "gpa_level_backward")
        deta = deta.view(bsz, heads, nblocks, 2).sum((0, 2))
        if not value_used:
            # value' unused (the last level): B^ and value get no gradient, so
            # the outer scan's state backward is not woken for nothing
            db, db_first, dvalue_out = None, None, None
        return dkey, dvalue_out, da, db, da_first, db_first, deta, None, None


class _LevelResidual(torch.autograd.Function):
    """(key', value') of one level whose write is an input: the kernels' given-
    write mode.  The backward returns the write's gradient through A^ w and
    w^T B^ (its other uses add theirs in autograd); key' depends on the key
    only through the subtraction, so d key = d key'."""

    @staticmethod
    def forward(ctx, key, value, write, a_vm, b_vm, a_first, b_first, eta, chunk, offset):
        _lib.require_device(key)
        ctx.set_materialize_grads(False)
        lib = _lib.load()
        key, value, a_vm, b_vm, firsts, eta = _inputs(key, value, a_vm, b_vm, a_first, b_first, eta)
        write = write.to(key.dtype).contiguous()
        key_out, value_out = torch.empty_like(key), torch.empty_like(value)
        rk, rv = torch.empty_like(key), torch.empty_like(value)
        prob = _problem(key, value, a_vm, b_vm, *firsts, eta, chunk, offset, (write, key_out, value_out),
                        (rk, rv, None))
        prob.given_write = 1
        _lib.check(lib.gpa_level_forward(prob, _lib.stream_handle(key.device)), "gpa_level_forward")
        ctx.chunk, ctx.offset = chunk, offset
        ctx.first_sb = (firsts[0][1], firsts[1][1])
        ctx.save_for_backward(key, value, a_vm, b_vm, firsts[0][0], firsts[1][0], eta, write, rk, rv)
        return key_out, value_out

    @staticmethod
    def backward(ctx, dkey_out, dvalue_out):
        if dkey_out is None and dvalue_out is None:
            return (None,) * 10
        lib = _lib.load()
        key, value, a_vm, b_vm, af, bf, eta, write, rk, rv = ctx.saved_tensors
        bsz, _, heads, _ = key.shape
        value_used = dvalue_out is not None
        zeros = lambda t, like: torch.zeros_like(like) if t is None else t.to(key.dtype).contiguous()  # noqa: E731
        dkey_out, dvalue_out = zeros(dkey_out, key), zeros(dvalue_out, value)
        prob = _problem(key, value, a_vm, b_vm, (af, ctx.first_sb[0]), (bf, ctx.first_sb[1]), eta, ctx.chunk,
                        ctx.offset, (write, key, value), (rk, rv, None))
        prob.given_write = 1
        da, db, da_first, db_first = _state_grads(key, a_vm, b_vm, af, bf)
        nblocks = a_vm.shape[2]
        deta = torch.empty(bsz * heads * nblocks, 2, device=key.device)
        dwrite = torch.empty_like(write)
        gr = _lib.LevelGrads()
        gr.dkey_out, gr.dvalue_out, gr.dwrite_given = (_lib.operand(t) for t in (dkey_out, dvalue_out, dwrite))
        gr.da_states, gr.db_states, gr.deta = da.data_ptr(), db.data_ptr(), deta.data_ptr()
        gr.da_first = da_first.data_ptr() if da_first is not None else None
        gr.db_first = db_first.data_ptr() if db_first is not None else None
        _lib.check(lib.gpa_level_backward(prob, gr, _lib.stream_handle(key.device)), "gpa_level_backward")
        deta = deta.view(bsz, heads, nblocks, 2).sum((0, 2))
        if not value_used:
            db, db_first, dvalue_out = None, None, None
        return dkey_out, dvalue_out, dwrite, da, db, da_first, db_first, deta, None, None


def _block_problem(key: Tensor, value: Tensor, a_first: Tensor, b_first: Tensor, eta: Tensor, chunk: int,
                   offset: int, residual: bool = True):
    """Checked arguments of a `level_mix_block` call: (problem, write, key',
    value', tensors kept alive); key' and value' are None (and not formed)
    without `residual`."""
    _lib.require_device(key)
    bsz, tokens, heads, dk = key.shape
    if offset + tokens > chunk:
        raise ValueError("level_mix_block: the call must stay inside one block")
    if torch.is_grad_enabled() and any(t.requires_grad for t in (key, value, a_first, b_first, eta)):
        raise RuntimeError("level_mix_block has no backward: call it under torch.no_grad() or inference_mode()")
    dtype, dv, m = key.dtype, value.shape[-1], a_first.shape[-1]
    key, value = key.contiguous(), value.contiguous()
    (af, asb), (bf, bsb) = _snapshot(a_first), _snapshot(b_first)
    eta = eta.detach().float().contiguous()
    write = torch.empty(bsz, tokens, heads, m, device=key.device, dtype=dtype)
    key_out, value_out = (torch.empty_like(key), torch.empty_like(value)) if residual else (None, None)
    rk, rv = torch.empty_like(key), torch.empty_like(value)
    stats = torch.empty(bsz, tokens, heads, 2, device=key.device, dtype=torch.float32)
    p = _lib.LevelProblem()
    p.batch, p.tokens, p.heads, p.key_dim, p.value_dim = bsz, tokens, heads, dk, dv
    p.slots, p.chunk, p.offset, p.dtype = m, chunk, offset, _lib.DTYPE_CODES[dtype]
    p.key, p.value = _lib.operand(key), _lib.operand(value)
    # One block, taken from the snapshots: the kernels read the start states
    # only for later blocks, so the snapshots stand in for the (unused) pointers.
    p.a_states, p.b_states = af.data_ptr(), bf.data_ptr()
    p.a_first, p.a_first_sb, p.b_first, p.b_first_sb = af.data_ptr(), asb, bf.data_ptr(), bsb
    p.eta = eta.data_ptr()
    p.write, p.key_out, p.value_out = (_lib.operand(t) for t in (write, key_out, value_out))
    p.rk, p.rv, p.stats = rk.data_ptr(), rv.data_ptr(), stats.data_ptr()
    return p, write, key_out, value_out, (key, value, af, bf, eta, rk, rv, stats)


def level_mix_block(key: Tensor, value: Tensor, a_first: Tensor, b_first: Tensor, eta: Tensor, chunk: int,
                    offset: int, residual: bool = True) -> tuple[Tensor, Tensor | None, Tensor | None]:
    """`level_mix` of a call that stays inside one block (offset + T <= chunk)
    whose snapshots A^ [B,H,Dk,M] and B^ [B,H,M,Dv] are given: the scans'
    chunk-start states are not needed (inference decode); no autograd.
    Without `residual` (one token: the last level, whose residual nothing
    reads) only the write is formed and key', value' are None."""
    lib = _lib.load()
    if not residual and key.shape[1] != 1:
        raise ValueError("level_mix_block: the write-only form takes one token")
    p, write, key_out, value_out, alive = _block_problem(key, value, a_first, b_first, eta, chunk, offset,
                                                         residual)
    if key.shape[1] == 1 and _TOKEN_KERNEL[0]:
        _lib.check(lib.gpa_level_token_forward(p, _lib.stream_handle(key.device)), "gpa_level_token_forward")
    else:
        _lib.check(lib.gpa_level_forward(p, _lib.stream_handle(key.device)), "gpa_level_forward")
    return write, key_out, value_out


def token_step_and_level(step, key: Tensor, value: Tensor, a_first: Tensor, b_first: Tensor, eta: Tensor,
                         chunk: int, offset: int, residual: bool = True):
    """A level's inner one-token step `ops.gdn_token_hip(*step)` and its
    one-token `level_mix_block(key, value, a_first, b_first, eta, chunk,
    offset, residual)` in one launch where the library has it
    (`gpa_token_level_forward`; inference decode, the two share no buffers).
    Returns (out, final, write, key', value') with the results of the two
    separate calls."""
    from .ops import _token_call, gdn_token_hip
    if key.shape[1] != 1:
        raise ValueError("token_step_and_level: needs one token")
    if not _TOKEN_KERNEL[0]:
        return gdn_token_hip(*step) + level_mix_block(key, value, a_first, b_first, eta, chunk, offset, residual)
    lib = _lib.load()
    sp, final, out, alive_s = _token_call(*step)
    lp, write, key_out, value_out, alive_l = _block_problem(key, value, a_first, b_first, eta, chunk, offset,
                                                            residual)
    _lib.check(lib.gpa_token_level_forward(sp, final.data_ptr(), _lib.operand(out), lp,
                                           _lib.stream_handle(key.device)), "gpa_token_level_forward")
    return out, final, write, key_out, value_out


def slot_step_supported(key: Tensor, slots: int) -> bool:
    """Whether `token_slot_step` takes these widths: bf16 keys of one token,
    K a multiple of 32 up to 128 (of 64 up to 256), slots a multiple of 4 up
    to 256 (the slot products and gates themselves as `slots.supported`)."""
    k = key.shape[-1]
    return (key.dtype == torch.bfloat16 and key.ndim == 4 and key.shape[1] == 1 and k <= 256
            and k % (64 if k > 128 else 32) == 0 and slots <= 256 and slots % 4 == 0)


def token_slot_step(q: Tensor, key: Tensor, s0: Tensor, center: Tensor, gate_w: Tensor, bias: Tensor,
                    beta_max: float, decay_scale: float, level=None):
    """A level's one-token inner step `ops.gdn_token_hip(q, key, slot, g_in,
    b_in, s0)` with its value slot = key C^T and its gates formed inside the
    step (`gpa_token_slot_step`; the results of `slots.slot_gates_act`), and,
    with `level` = (key, value, a_first, b_first, eta, chunk, offset,
    residual), the level's one-token write in the same launch where the
    library has it (as `token_step_and_level`).  Inference only.  Returns
    (out, final, slot, g_in, b_in, g_out, b_out) + (write, key', value') with
    a level."""
    from .ops import _token_call
    lib = _lib.load()
    if torch.is_grad_enabled() and any(x.requires_grad for x in (q, key, center, gate_w, bias)):
        raise RuntimeError("token_slot_step has no backward: call it under torch.no_grad() or inference_mode()")
    b, _, h, _ = key.shape
    cb = params.derived(("slot_center", id(center), key.dtype), (center,),
                        lambda: center.detach().to(key.dtype).contiguous())
    wg = params.derived(("slot_gate_w", id(gate_w), key.dtype), (gate_w,),
                        lambda: gate_w.detach().to(key.dtype).contiguous())
    slot = key.new_empty(b, 1, h, cb.shape[1])
    gates = [torch.empty(b, 1, h, device=key.device, dtype=torch.float32) for _ in range(4)]
    # the step's value and gates are the outputs: the kernel does not read them
    sp, final, out, alive = _token_call(q, key, slot, gates[0], gates[1], s0)
    bias = bias.detach().float().contiguous()
    ts = _lib.TokenSlot()
    ts.center, ts.gate_w, ts.slot = cb.data_ptr(), wg.data_ptr(), _lib.operand(slot)
    ts.gates = _lib.GateProblem(b, 1, h, _lib.DTYPE_CODES[key.dtype], _lib.Operand(), bias.data_ptr(),
                                float(beta_max), float(decay_scale), *(g.data_ptr() for g in gates))
    lp, rest = None, ()
    if level is not None:
        lp, write, key_out, value_out, alive_l = _block_problem(*level)
        rest = (write, key_out, value_out)
    _lib.check(lib.gpa_token_slot_step(sp, ts, final.data_ptr(), _lib.operand(out), lp,
                                       _lib.stream_handle(key.device)), "gpa_token_slot_step")
    return (out, final, slot, *gates) + rest


_TOKEN_KERNEL = [True]  # one-token calls of level_mix_block on gpa_level_token_forward

_REG_PIECES = 8  # float4 pieces of each snapshot per thread in the register level kernel


def write_only_supported(key_dim: int, value_dim: int, slots: int) -> bool:
    """Whether gpa_level_token_forward takes the write-only form for these
    widths: its register kernel covers them (widths multiples of 4, a thread
    count of 256, 512 or 1024 that the float4 column groups of A^ and B^
    divide, and at most 8 float4 pieces of each snapshot per thread)."""
    if slots % 4 or value_dim % 4:
        return False
    for nt in (256, 512, 1024):
        if nt % (slots // 4) or nt % (value_dim // 4):
            continue
        if key_dim * slots // 4 <= _REG_PIECES * nt and slots * value_dim // 4 <= _REG_PIECES * nt:
            return True
    return False


def level_mix(key: Tensor, value: Tensor, a_vm: Tensor, b_vm: Tensor, a_first: Tensor | None,
              b_first: Tensor | None, eta: Tensor, chunk: int, offset: int):
    """(write, key', value') of one level.  key [B,T,H,Dk], value [B,T,H,Dv];
    a_vm [B,H,N,M,Dk] and b_vm [B,H,N,Dv,M]: the scans' value-major chunk-start
    states; a_first [B,H,Dk,M] / b_first [B,H,M,Dv]: cached block-0 snapshots
    (None: block 0 is the scans' initial state); eta [H,2]."""
    return _LevelMix.apply(key, value, a_vm, b_vm, a_first, b_first, eta, chunk, offset)


def level_residual(key: Tensor, value: Tensor, write: Tensor, a_vm: Tensor, b_vm: Tensor, a_first: Tensor | None,
                   b_first: Tensor | None, eta: Tensor, chunk: int, offset: int):
    """(key', value') of one level whose write [B,T,H,M] is given (arguments
    otherwise as `level_mix`): key' = key - eta0 round(A^ w), value' = value -
    eta1 round(w^T B^), differentiable in the write as in everything else."""
    return _LevelResidual.apply(key, value, write, a_vm, b_vm, a_first, b_first, eta, chunk, offset)
