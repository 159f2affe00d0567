"""Level-major block-lagged schedule of the DenseGPA core on the HIP backend.

The reference walks the sequence block by block (attention.py:376-405) and,
inside each block, level by level (attention.py:309-329).  Block n of level
j+1 only needs level j's *block-start* states, and the level-j recurrences
never depend on the query (docs/EQUATIONS.md:57-60).  So this schedule runs
each level once over the whole call:

  for level j:   A_j scan (reads raw_j = u(q)^T A_t, keeps A at every block start)
                 B_j scan (state only, keeps B at every block start)
                 writes a_j = softmax(u(key) A_hat), counts, logits and the
                 residual key/value of level j+1 from those block-start states
  all edges:     R_ij scans (messages u(p_i)^T R_t)
  route reader:  edge softmax -> aggregate -> normalise/tanh -> route MLP -> q_out
  outer reads:   o_j = u(q_out_j)^T B_t, mixed over levels

Every GDN recurrence is the HIP chunked scan (`ops.gdn_scan_hip`, chunks
aligned with the model's blocks, including a block begun in an earlier call).
The per-token glue between scans runs as float32 device tensor ops, rounding
to the activation dtype where the reference rounds.  There is no CPU path.
"""
from __future__ import annotations

import contextlib
import math

import torch
import torch.nn.functional as F
from torch import Tensor

from . import _lib, glue, params
from .ops import gdn_scan_deferred, gdn_scan_hip, gdn_scan_many, gdn_token_hip, gdn_token_many
from .ops import gdn_token_read
from .ops import token_step_supported
from .ops import read_supported as late_read_supported
from .counts import count_logits
from .slots import slot_gates, slot_gates_act
from .slots import supported as slot_gates_supported
from .counts import supported as fused_counts_supported
from .level import (level_mix, level_mix_block, level_residual, slot_step_supported, token_slot_step,
                    token_step_and_level, write_only_supported)
from .level import supported as fused_level_supported
from .route import route_reader, route_reader_many
from .route import product_read
from .route import supported as fused_route_supported
from .positional import additive_scan, rope
from .state import GPAState, LevelState, RelationState, ResidualSnapshot

_F32 = torch.float32
_LANES = 4          # side streams for independent scans (the device has 4 hardware queues per process)
_STREAMS: dict = {}
_SERIAL = [False]   # set by `one_stream()`


_OUT_BUFFER = [None]  # set by `output_into()`


@contextlib.contextmanager
def output_into(buffer: Tensor):
    """Calls of the chunk model inside the block write their output into
    `buffer` where the output-mix kernel produces it (one-token inference);
    the caller compares data pointers to know whether it did."""
    before = _OUT_BUFFER[0]
    _OUT_BUFFER[0] = buffer
    try:
        yield
    finally:
        _OUT_BUFFER[0] = before


@contextlib.contextmanager
def one_stream():
    """Run every job of the schedule in order on the current stream, so that no
    two kernels overlap (used to time kernels one at a time)."""
    before = _SERIAL[0]
    _SERIAL[0] = True
    try:
        yield
    finally:
        _SERIAL[0] = before


def _side_streams(device) -> list:
    """The device's side streams (default priority), created once."""
    pool = _STREAMS.get(device)
    if pool is None:
        pool = _STREAMS[device] = [torch.cuda.Stream(device=device) for _ in range(_LANES)]
    return pool


def _tensors(x):
    if isinstance(x, Tensor):
        yield x
    elif isinstance(x, (tuple, list)):
        for y in x:
            yield from _tensors(y)
    elif hasattr(x, "tensors"):
        yield from x.tensors()


def _concurrent(jobs):
    """Run independent jobs (fn, input tensors) on the side streams, job i on
    stream i % 4, and return their results in order.  Every side stream first
    waits for the current stream; the current stream then waits for all of
    them.  Inputs are recorded as used on their side stream and results as
    used on the current stream, so the caching allocator does not hand their
    memory to another stream early.  Autograd runs each job's backward on the
    job's stream, so the backward scans overlap the same way.  During a graph
    capture the jobs run in order on the capturing stream."""
    if _SERIAL[0] or torch.cuda.is_current_stream_capturing():
        # Inside a HIP graph capture everything stays on the capturing stream
        # (no cross-stream fork/join, no allocator stream records).
        return [fn() for fn, _ in jobs]
    main = torch.cuda.current_stream()
    streams = _side_streams(main.device)[:len(jobs)]
    for stream in streams:
        stream.wait_stream(main)
    results = []
    for i, (fn, inputs) in enumerate(jobs):
        stream = streams[i % len(streams)]
        for t in _tensors(inputs):
            t.record_stream(stream)
        with torch.cuda.stream(stream):
            results.append(fn())
    for stream in streams:
        main.wait_stream(stream)
    for t in _tensors(results):
        t.record_stream(main)
    return results


def _unit(x: Tensor) -> Tensor:
    """u(x) computed in float32, rounded back to x's dtype (ops.py:14-17)."""
    return F.normalize(x.float(), p=2, dim=-1, eps=1e-6).to(x.dtype)


def _mm(x: Tensor, w: Tensor, eq: str, dtype: torch.dtype) -> Tensor:
    """A dtype-typed einsum: operands rounded to `dtype`, float32 accumulate,
    result rounded to `dtype` (what a bf16 einsum with fp32 accumulation does)."""
    return torch.einsum(eq, x.to(dtype).float(), w.to(dtype).float()).to(dtype)


class _Blocks:
    """Token <-> (block, row) views for a call that starts `offset` rows into a block."""

    def __init__(self, tokens: int, offset: int, chunk: int):
        self.t, self.o, self.c = tokens, offset, chunk
        self.n = (offset + tokens + chunk - 1) // chunk
        self.tail = self.n * chunk - offset - tokens

    def split(self, x: Tensor) -> Tensor:
        """[B,T,H,D] -> [B,N,C,H,D] with void rows zero."""
        y = F.pad(x, (0, 0, 0, 0, self.o, self.tail))
        return y.view(x.shape[0], self.n, self.c, *x.shape[2:])

    def merge(self, y: Tensor) -> Tensor:
        return y.reshape(y.shape[0], self.n * self.c, *y.shape[3:])[:, self.o:self.o + self.t]


def _snapshots(starts: Tensor, first: Tensor) -> Tensor:
    """Frozen state of every block: the cached snapshot for block 0, the scan's
    block-start states after it (attention.py:304, 342-344)."""
    if starts.shape[2] == 1:
        return first.unsqueeze(2)
    return torch.cat((first.unsqueeze(2).to(starts.dtype), starts[:, :, 1:]), dim=2)


class _Level:
    __slots__ = ("slot", "value", "g_out", "b_out", "write", "counts", "final_count", "logits", "a_final",
                 "b_final", "a_starts", "b_starts", "b_read", "local", "b_token", "correction", "moment")

    def __init__(self):
        self.logits = None
        self.local = None  # the local read distribution, when the counts kernel gave it
        # positional moments: the read of the moment state and the new state
        self.correction = self.moment = None
        # A one-token outer step deferred to its read: (slot, value, g, beta, s0)
        # of the B_j step, which runs with the route query in one kernel.
        self.b_token = None


def _chunks(items, n):
    return [items[i:i + n] for i in range(0, len(items), n)]


def run_segment(model, q: Tensor, k: Tensor, v: Tensor, state: GPAState, position_ids: Tensor,
                control: Tensor | None, *, want_routes: bool = False):
    cfg = model.config
    _lib.require_device(q)
    if q.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("backend='hip' computes in float32 or bfloat16 activations")
    bsz, tokens, heads, dk = q.shape
    dtype = q.dtype
    chunk, offset = cfg.chunk_size, state.chunk_offset
    blocks = _Blocks(tokens, offset, chunk)
    frozen0 = state.frozen or tuple(ResidualSnapshot(lv.inner, lv.outer) for lv in state.levels)
    scan = dict(chunk=chunk, offset=offset)
    # Inference on one token (decode): each recurrence is a single token step
    # that reads and writes its state once, and the level mix reads the cached
    # block snapshots, so no chunk-start states are kept.
    token = _TOKEN_STEP[0] and tokens == 1 and not torch.is_grad_enabled()
    # positional moments: the inner reads and the route reader take the rotated
    # query (attention.py:305)
    qr = rope(q, position_ids) if cfg.positional_mode == "moments" else q

    # ---- level pass (storage + inner reads), attention.py:309-329
    key, value = k, v
    levels: list[_Level] = []
    token_logits = []  # (level, j, inner read, old state) whose one-token logits come after the pass
    etas = _etas(model).unbind(0)  # one unbind: its backward stacks the levels' gradients once
    for j, (old, snap) in enumerate(zip(state.levels, frozen0)):
        lv = _Level()
        act = (_FUSED_SLOTS[0] and slot_gates_supported(cfg, key, cfg.slots[j]) and _GLUE[0]
               and not torch.is_grad_enabled() and cfg.slot_feature == "linear")
        if (token and act and _SLOT_STEP[0] and _TOKEN_LEVEL[0] and _FUSED_LEVEL[0]
                and slot_step_supported(key, cfg.slots[j]) and value.shape[-1] % 4 == 0
                and fused_level_supported(cfg, dtype, key.shape[-1], value.shape[-1], cfg.slots[j])):
            # one token: the slot products and gates inside the A_j step, beside the
            # level write (the last level's alone, as below)
            eta = etas[j]
            residual = j + 1 < len(state.levels) or not write_only_supported(
                key.shape[-1], value.shape[-1], cfg.slots[j])
            raw, a_final, slot, _, _, g_out, b_out, write, key_next, value_next = token_slot_step(
                qr, key, old.inner, model.center[j], model.gate_weight[j], model.gate_bias[j], cfg.beta_max,
                _decay_scale(model, j), (key, value, snap.inner, snap.outer, eta, chunk, offset, residual))
            _token_level_done(model, lv, j, raw, a_final, slot, value, g_out, b_out, write, old, key, qr,
                              position_ids, levels, token_logits)
            key, value = key_next, value_next
            continue
        if act:
            # inference: slot products, gate inputs and gate nonlinearities in one launch
            slot, g_in, b_in, g_out, b_out = slot_gates_act(key, model.center[j], model.gate_weight[j],
                                                            model.gate_bias[j], cfg.beta_max, _decay_scale(model, j))
        elif _FUSED_SLOTS[0] and slot_gates_supported(cfg, key, cfg.slots[j]):
            proj, raw = slot_gates(key, model.center[j], model.gate_weight[j])
            slot = _slot_feature(cfg, proj)
            g_in, b_in, g_out, b_out = _gates(model, key, j, control, raw)
        else:
            slot = _slot_feature(cfg, _mm(key, model.center[j], "bthd,hmd->bthm", key.dtype))
            g_in, b_in, g_out, b_out = _gates(model, key, j, control)
        eta = etas[j]
        write = _assignment(cfg, slot)
        level_kernels = _FUSED_LEVEL[0] and fused_level_supported(
            cfg, dtype, key.shape[-1], value.shape[-1], slot.shape[-1])
        fused_level = write is None and level_kernels
        if token and fused_level and token_step_supported(key, slot) and token_step_supported(slot, value):
            step = (qr, key, slot, g_in, b_in, old.inner)
            # the last level's residual is never read (attention.py:327-329 after the
            # loop's last pass): its level kernel forms the write alone
            residual = j + 1 < len(state.levels) or not write_only_supported(
                key.shape[-1], value.shape[-1], slot.shape[-1])
            if _TOKEN_LEVEL[0]:
                # the A_j step and the level write in one launch (they share no buffers)
                raw, a_final, write, key_next, value_next = token_step_and_level(
                    step, key, value, snap.inner, snap.outer, eta, chunk, offset, residual)
            else:
                raw, a_final = gdn_token_hip(*step)
                write, key_next, value_next = level_mix_block(key, value, snap.inner, snap.outer, eta, chunk, offset,
                                                              residual)
            _token_level_done(model, lv, j, raw, a_final, slot, value, g_out, b_out, write, old, key, qr,
                              position_ids, levels, token_logits)
            key, value = key_next, value_next
            continue
        if token and write is not None and token_step_supported(key, slot) and token_step_supported(slot, value):
            # a write that does not read the snapshots (rsa_update's softmax(slot / .25), softmax
            # slot features): the A_j token step, then the residual from the cached block snapshots
            raw, a_final = gdn_token_hip(qr, key, slot, g_in, b_in, old.inner)
            write = write.to(dtype)
            key_next, value_next = (_token_residual(key, value, snap.inner, snap.outer, write, eta)
                                    if j + 1 < len(state.levels) else (None, None))  # the last is never read
            _token_level_done(model, lv, j, raw, a_final, slot, value, g_out, b_out, write, old, key, qr,
                              position_ids, levels, token_logits)
            key, value = key_next, value_next
            continue
        # The outer read of this level (below) runs the B recurrence with the
        # same keys, values, gates and initial state: where the kernels allow,
        # the B scan keeps its intermediates for that read instead.
        deferred = _DEFER_OUTER_READ[0] and late_read_supported(slot, value)
        if _PACKED[0]:
            # the A_j and B_j scans in one call: their state recurrences advance together
            (raw, a_starts, a_final), b = gdn_scan_many([
                dict(q=qr, k=key, v=slot, g=g_in, beta=b_in, s0=old.inner, **scan),
                dict(q=None, k=slot, v=value, g=g_out, beta=b_out, s0=old.outer, deferred=deferred, **scan)])
            b_starts, b_final, lv.b_read = b if deferred else b[1:] + (None,)
        else:
            b_scan = gdn_scan_deferred if deferred else (
                lambda *a, **kw: gdn_scan_hip(None, *a, **kw)[1:] + (None,))
            (raw, a_starts, a_final), (b_starts, b_final, lv.b_read) = _concurrent([
                (lambda: gdn_scan_hip(qr, key, slot, g_in, b_in, old.inner, **scan),
                 (qr, key, slot, g_in, b_in, old.inner)),
                (lambda: b_scan(slot, value, g_out, b_out, old.outer, **scan),
                 (slot, value, g_out, b_out, old.outer))])
        # Snapshots: block 0 uses the cached ones, which are the scans' own
        # initial states unless the call starts inside a block.
        first_a = None if snap.inner is old.inner else snap.inner
        first_b = None if snap.outer is old.outer else snap.outer
        if fused_level:
            write, key_next, value_next = level_mix(key, value, a_starts.transpose(-1, -2),
                                                    b_starts.transpose(-1, -2), first_a, first_b, eta, chunk, offset)
        elif write is not None and j + 1 == len(state.levels):
            # a given write at the last level: its residual is never read
            write, key_next, value_next = write.to(dtype), None, None
        elif level_kernels:
            write = write.to(dtype)
            key_next, value_next = level_residual(key, value, write, a_starts.transpose(-1, -2),
                                                  b_starts.transpose(-1, -2), first_a, first_b, eta, chunk, offset)
        else:
            write, key_next, value_next = _level_mix_torch(key, value, a_starts, b_starts, snap.inner, snap.outer,
                                                           eta, blocks, write)
        lv.slot, lv.value, lv.g_out, lv.b_out = slot, value, g_out, b_out
        lv.write = write
        _moments(lv, key, qr, position_ids, old)
        _level_logits(model, lv, j, raw, old)
        lv.a_final, lv.b_final, lv.a_starts, lv.b_starts = a_final, b_final, a_starts, b_starts
        levels.append(lv)
        key, value = key_next, value_next

    for part in _chunks(token_logits, _lib.TOKEN_LOGITS_MAX_PACK):
        done = glue.token_logits_many([(raw, lv.write, old.count) + _count_scalars(model, j, raw)
                                       for lv, j, raw, old in part])
        for (lv, _, _, _), (lv.logits, lv.final_count, lv.local) in zip(part, done):
            lv.counts = lv.final_count[:, None]

    # ---- relations, attention.py:206-223
    local = [lv.local if lv.local is not None else glue.softmax_rows(lv.logits, dtype) for lv in levels]
    incoming, relations = _relations(model, local, [lv.write for lv in levels], state.relations, scan, token)

    # ---- route reader, attention.py:225-262
    routes, queries = _bridge(model, qr, [lv.logits for lv in levels], incoming, [lv.counts for lv in levels])

    # ---- outer reads and level mix, attention.py:333-341
    ol = model.output_logits
    weights = params.derived(("out_w", id(ol)), (ol,), lambda: ol.softmax(0), differentiable=True)

    def outer_read(lv, qo, s0):
        if lv.b_read is not None:
            return lambda: lv.b_read(qo)
        return lambda: gdn_scan_hip(qo, lv.slot, lv.value, lv.g_out, lv.b_out, s0, **scan)[0]

    if all(lv.b_token is not None for lv in levels):
        # one-token outer steps of every level, packed into as few launches as the library takes
        reads = []
        for part in _chunks(list(zip(levels, queries)), _lib.TOKEN_MAX_PACK):
            done = gdn_token_many([(qo,) + lv.b_token for lv, qo in part])
            for (lv, _), (out_j, lv.b_final) in zip(part, done):
                reads.append(out_j)
    else:
        for lv in levels:
            if lv.b_token is not None:
                lv.b_read = _outer_token(lv)
        jobs = [(outer_read(lv, qo, state.levels[j].outer),
                 (qo, lv.slot, lv.value, lv.g_out, lv.b_out, state.levels[j].outer))
                for j, (lv, qo) in enumerate(zip(levels, queries))]
        # with packed scans everything runs in order on the current stream
        reads = [fn() for fn, _ in jobs] if _PACKED[0] else _concurrent(jobs)
    if not (_SERIAL[0] or torch.cuda.is_current_stream_capturing()):
        for lv in levels:  # states made by a one-token outer step on a side stream
            if lv.b_starts is None and lv.b_final is not None:
                lv.b_final.record_stream(torch.cuda.current_stream())
    if _GLUE[0] and not torch.is_grad_enabled() and all(r.dtype == v.dtype for r in reads) \
            and len(reads) <= _lib.DECODE_MAX_LEVELS:
        buf = _OUT_BUFFER[0]
        out = glue.output_mix(reads, weights, buf if buf is not None and buf.shape == reads[0].shape
                              and buf.dtype == reads[0].dtype else None)
    elif _GLUE[0] and all(r.dtype == v.dtype for r in reads) and glue.output_mix_supported(reads):
        out = glue.output_mix_train(reads, weights)
    else:
        out = 0
        for w_j, read in zip(weights.unbind(0), reads):
            out = out + w_j[..., None] * read
        out = out.to(v.dtype)

    # ---- new cache, attention.py:342-344
    new_offset = (offset + tokens) % chunk
    frozen = None
    if new_offset:
        last = blocks.n - 1
        frozen = frozen0 if last == 0 else tuple(
            ResidualSnapshot(lv.a_starts[:, :, last], lv.b_starts[:, :, last]) for lv in levels)
    new_levels = tuple(LevelState(lv.a_final, lv.b_final, lv.final_count, lv.moment) for lv in levels)
    new_state = GPAState(new_levels, relations, state.position + tokens, chunk, new_offset, frozen)
    return out, new_state, (tuple(routes) if want_routes else None)


def _outer_token(lv):
    """The read of a level's deferred one-token outer step on its own; the new
    state goes to lv.b_final."""
    def read(qo):
        out, lv.b_final = gdn_token_hip(qo, *lv.b_token)
        return out
    return read


def run_tokens(model, q: Tensor, k: Tensor, v: Tensor, state: GPAState, control: Tensor | None, *,
               want_routes: bool = False, position_ids: Tensor | None = None):
    """The tokenwise model (`chunk_size == 1`, attention.py:264-297, the loop at
    :385-393).  Each token passes through every level with the updated states:
    the write reads the updated inner state, the residuals use the updated
    inner and outer states, the relation scans and the route reader follow,
    and each level's output reads its updated outer state.  Every GDN step is
    the HIP scan at chunk length 1; the glue is the device code of the chunk
    schedule on one-token views."""
    cfg = model.config
    _lib.require_device(q)
    if q.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("backend='hip' computes in float32 or bfloat16 activations")
    if position_ids is None and cfg.positional_mode == "moments":
        position_ids = torch.arange(state.position, state.position + q.shape[1], device=q.device)
    outs, routes = [], []
    for t in range(q.shape[1]):
        ctl = control[:, t:t + 1] if control is not None else None
        pos = None if position_ids is None else (
            position_ids[t] if position_ids.ndim == 1 else position_ids[:, t:t + 1])
        out, state, r = _token(model, q[:, t:t + 1], k[:, t:t + 1], v[:, t:t + 1], state, ctl, pos)
        outs.append(out)
        routes.append(r)
    routes = tuple(torch.cat(r, 1) for r in zip(*routes)) if want_routes else None
    return torch.cat(outs, 1), state, routes


def _read(x: Tensor, s: Tensor) -> Tensor:
    """u(x)^T S for one token: x [B,1,H,K], S [B,H,K,V] -> [B,1,H,V] in x's
    dtype (ops.py:44-46)."""
    return torch.einsum("bthk,bhkv->bthv", _unit(x).float(), s.float()).to(x.dtype)


def _token(model, q, k, v, state: GPAState, control, position=None):
    """One token of the tokenwise model (attention.py:264-297), on [B,1,H,.] views."""
    cfg = model.config
    dtype = q.dtype
    qr = rope(q, position) if cfg.positional_mode == "moments" else q
    step = dict(chunk=1, offset=0)
    infer = _TOKEN_STEP[0] and not torch.is_grad_enabled()
    key, value = k, v
    new_levels, writes, logits = [], [], []
    for j, old in enumerate(state.levels):
        slot = _slot_feature(cfg, _mm(key, model.center[j], "bthd,hmd->bthm", key.dtype))
        g_in, b_in, g_out, b_out = _gates(model, key, j, control)
        if infer and token_step_supported(key, slot) and token_step_supported(slot, value):
            # inference: both recurrences as one-token steps in one launch (no saved intermediates)
            (raw, a), (_, b) = gdn_token_many([(qr, key, slot, g_in, b_in, old.inner),
                                               (None, slot, value, g_out, b_out, old.outer)])
        else:
            (raw, _, a), (_, _, b) = _concurrent([
                (lambda: gdn_scan_hip(qr, key, slot, g_in, b_in, old.inner, **step),
                 (qr, key, slot, g_in, b_in, old.inner)),
                (lambda: gdn_scan_hip(None, slot, value, g_out, b_out, old.outer, **step),
                 (slot, value, g_out, b_out, old.outer))])
        write = _assignment(cfg, slot)
        if write is None:
            write = _read(key, a).softmax(-1)
        count = old.count + write[:, 0].to(old.count.dtype)
        moment, correction = old.position, None
        if moment is not None:  # attention.py:276-281
            kh = _unit(key)
            delta = (rope(kh, position) - kh).to(moment.dtype)
            moment = moment + delta[:, 0, :, :, None] * write[:, 0].to(delta.dtype)[..., None, :]
            correction = _read(qr, moment)
        logits.append(_base_logits(model, raw, count[:, None], j, correction))
        writes.append(write)
        new_levels.append(LevelState(a, b, count, moment))
        rk = torch.einsum("bhdm,bthm->bthd", a, write.float())
        rv = torch.einsum("bthm,bhmv->bthv", write.float(), b)
        key, value = _residual(model, key, value, rk, rv, j)
    local = [lg.softmax(-1).to(dtype) for lg in logits]
    incoming, relations = _relations(model, local, writes, state.relations, step, token=infer)
    routes, queries = _bridge(model, qr, logits, incoming, [lv.count[:, None] for lv in new_levels])
    weights = model.output_logits.softmax(0)
    out = 0
    for j, qo in enumerate(queries):
        out = out + weights[j][..., None] * _read(qo, new_levels[j].outer)
    new = GPAState(tuple(new_levels), relations, state.position + 1, cfg.chunk_size)
    return out.to(v.dtype), new, routes


# --------------------------------------------------------------------------- glue
def _cumsum_tokens(x: Tensor) -> Tensor:
    """Cumulative sum over tokens of a [B,T,H,M] tensor, scanned along the
    innermost axis (a scan over an outer axis is far slower on the GPU)."""
    return x.permute(0, 2, 3, 1).contiguous().cumsum(-1).permute(0, 3, 1, 2).contiguous()


def _slot_feature(cfg, x: Tensor) -> Tensor:
    """attention.py:179-184."""
    if cfg.slot_feature == "softmax":
        return (cfg.slot_scale * x.float()).softmax(-1).to(x.dtype)
    if cfg.slot_feature == "tanh":
        return (cfg.slot_scale * x.float()).tanh().to(x.dtype)
    return x


def _assignment(cfg, slot: Tensor):
    """attention.py:186-188."""
    if cfg.slot_feature == "softmax":
        return slot
    return (slot / .25).softmax(-1) if cfg.rsa_update else None


def _tier(cfg, j: int) -> float:
    """The rsa_update decay tier of level j (attention.py:170-171), else 1."""
    return ((1., .1, .01, .001)[j] if cfg.levels == 4 else .1 ** j) if cfg.rsa_update else 1.


def _decay_scale(model, j: int) -> float:
    """The factor on both decays of level j: 0 without positions, else the tier."""
    cfg = model.config
    return 0. if cfg.positional_mode == "none" else _tier(cfg, j)


def _token_logits_supported(raw: Tensor, write_like: Tensor) -> bool:
    """One-token counts / logits / local read by a glue kernel (inference)."""
    return (_GLUE[0] and not torch.is_grad_enabled() and raw.shape[1] == 1 and raw.dtype in _lib.DTYPE_CODES
            and write_like.dtype == raw.dtype and raw.shape[-1] <= _lib.TOKEN_LOGITS_MAX_SLOTS)


def _gates(model, key: Tensor, j: int, control: Tensor | None, raw: Tensor | None = None):
    """Scalar decay/strength gates per token and head (attention.py:161-174);
    `raw` is the gate input product when the caller has it already."""
    cfg = model.config
    w = model.gate_weight[j]
    if raw is not None:
        pass
    elif cfg.control_dim:
        raw = _mm(control, w, "btd,hdc->bthc", control.dtype)
    else:
        src = key if cfg.rsa_update else _unit(key)
        raw = _mm(src, w, "bthd,hdc->bthc", key.dtype)
    tier = _tier(cfg, j)
    if _GLUE[0] and not torch.is_grad_enabled() and raw.dtype in _lib.DTYPE_CODES:
        return glue.gate_act(raw, model.gate_bias[j], cfg.beta_max, _decay_scale(model, j))
    if _GLUE[0] and glue.gate_act_supported(raw):
        return glue.gate_act_train(raw, model.gate_bias[j], cfg.beta_max, _decay_scale(model, j))
    raw = raw.float() + model.gate_bias[j]
    g_in, b_in, g_out, b_out = raw.unbind(-1)
    g_in = -F.softplus(g_in).clamp(max=10.)
    g_out = -F.softplus(g_out).clamp(max=10.)
    if cfg.rsa_update:
        g_in, g_out = g_in * tier, g_out * tier
    if cfg.positional_mode == "none":
        g_in, g_out = g_in * 0, g_out * 0
    return g_in, cfg.beta_max * b_in.sigmoid(), g_out, cfg.beta_max * b_out.sigmoid()


def _base_logits(model, raw: Tensor, counts: Tensor, j: int, moment: Tensor | None = None) -> Tensor:
    """read_scale*raw + softplus(c_j) log1p(n) [+ moment_gain_j tanh(moment / (1 + n))]
    (attention.py:196-204)."""
    cfg = model.config
    gain = F.softplus(model.count_gain_raw[j])[..., None]
    if cfg.learn_read_scale:
        scale = model.read_log_scale[j].clamp(math.log(.25), math.log(64.)).exp()[..., None]
    else:
        scale = cfg.read_scale
    logits = scale * raw.float() + gain * counts.log1p()
    if moment is not None:
        logits = logits + model.moment_gain[j][..., None] * torch.tanh(moment / (1 + counts))
    return logits


def _moments(lv, key: Tensor, qr: Tensor, positions, old: LevelState) -> None:
    """The level's positional moments (attention.py:318-323): the additive scan
    of rope(u(key)) - u(key) against the write, read by u(rope(q)); sets
    lv.correction and lv.moment (both None without moments)."""
    if old.position is None:
        return
    kh = _unit(key)
    lv.correction, lv.moment = additive_scan(_unit(qr), rope(kh, positions) - kh, lv.write, old.position)


def _count_scalars(model, j: int, like: Tensor):
    """Per-head count gain and read scale of level j, as [H] tensors."""
    cfg = model.config
    raw = model.count_gain_raw
    gain = params.derived(("count_gain", id(raw)), (raw,), lambda: F.softplus(raw), differentiable=True)[j]
    if cfg.learn_read_scale:
        scale = model.read_log_scale[j].clamp(math.log(.25), math.log(64.)).exp()
    else:
        scale = params.derived(("read_scale", cfg.heads, float(cfg.read_scale), like.device), (),
                               lambda: torch.full((cfg.heads,), float(cfg.read_scale), device=like.device))
    return gain, scale


_FUSED_COUNTS = [True]  # counts and base logits in HIP (counts.py)
_GLUE = [True]  # one-launch gate, one-token logits and output-mix kernels without autograd (glue.py)
_FUSED_SLOTS = [True]  # slot products and gate inputs in HIP (slots.py)
_SLOT_STEP = [True]  # one-token calls: slot products and gates inside the A_j step (level.token_slot_step)


def _etas(model) -> Tensor:
    """1 + .25 tanh(residual_raw), [L,H,2] (attention.py:192)."""
    raw = model.residual_raw
    return params.derived(("eta", id(raw)), (raw,), lambda: 1 + .25 * raw.tanh(), differentiable=True)


def _residual(model, key, value, rk, rv, j):
    """attention.py:190-194."""
    return _residual_eta(key, value, rk, rv, _etas(model)[j])


def _residual_eta(key, value, rk, rv, eta):
    new_key = (key - eta[:, 0, None] * rk.to(key.dtype)).to(key.dtype)
    new_value = (value - eta[:, 1, None] * rv.to(value.dtype)).to(value.dtype)
    return new_key, new_value


_FUSED_LEVEL = [True]  # the fused level write and residual (level.py)
_DEFER_OUTER_READ = [True]  # outer reads as late reads of the B scans (ops.gdn_scan_deferred)
_TOKEN_STEP = [True]  # one-token inference calls as token steps (ops.gdn_token_hip)
_TOKEN_LEVEL = [True]  # a level's inner token step and its level write in one launch (level.token_step_and_level)
_PACKED = [True]  # a level's A/B scans and all edge scans as packed calls (ops.gdn_scan_many)


def _token_residual(key, value, snap_inner, snap_outer, write, eta):
    """The residual of one token per stream from a given write and the block
    snapshots A^ [B,H,Dk,M], B^ [B,H,M,Dv] (attention.py:327-329): key -
    eta0 A^ w, value - eta1 w^T B^, the products in float32."""
    w = write[:, 0].float()                                        # [B,H,M]
    rk = torch.matmul(snap_inner.float(), w.unsqueeze(-1))[..., 0]  # [B,H,Dk]
    rv = torch.matmul(w.unsqueeze(-2), snap_outer.float())[..., 0, :]  # [B,H,Dv]
    return _residual_eta(key, value, rk.unsqueeze(1), rv.unsqueeze(1), eta)


def _token_level_done(model, lv, j, raw, a_final, slot, value, g_out, b_out, write, old, key, qr, position_ids,
                      levels, token_logits):
    """Bookkeeping of a level whose A_j step ran as one token step.  The B_j
    step runs at its read, after the route reader (nothing before needs the
    new B_j): one pass over the state for both.  Nothing in the level pass
    reads the logits, so where the one-token logits kernel applies every
    level's run in one launch after the pass."""
    lv.b_read, lv.b_token = None, (slot, value, g_out, b_out, old.outer)
    lv.slot, lv.value, lv.g_out, lv.b_out, lv.write = slot, value, g_out, b_out, write
    lv.a_final, lv.b_final, lv.a_starts, lv.b_starts = a_final, None, None, None
    if old.position is None and _token_logits_supported(raw, write):
        token_logits.append((lv, j, raw, old))
    else:
        _moments(lv, key, qr, position_ids, old)
        _level_logits(model, lv, j, raw, old)
    levels.append(lv)


def _level_mix_torch(key, value, a_starts, b_starts, snap_inner, snap_outer, eta, blocks, write=None):
    """The level write and residual as device ops (attention.py:314-329): the
    write (unless given by the slot feature), A^ w, w^T B^ and the residual
    step, from the block snapshots ([B,H,N,Dk,M] / [B,H,N,M,Dv] views of the
    scans' states, block 0 from the cached snapshots)."""
    dtype = key.dtype
    a_hat = _snapshots(a_starts, snap_inner)       # [B,H,N,Dk,M]
    b_hat = _snapshots(b_starts, snap_outer)       # [B,H,N,M,Dv]
    if write is None:
        kb = blocks.split(_unit(key).float())       # [B,N,C,H,Dk]
        write = blocks.merge(torch.einsum("bnchd,bhndm->bnchm", kb, a_hat)).softmax(-1)
    write = write.to(dtype)
    wb = blocks.split(write.float())
    rk = blocks.merge(torch.einsum("bhndm,bnchm->bnchd", a_hat, wb))
    rv = blocks.merge(torch.einsum("bnchm,bhnmv->bnchv", wb, b_hat))
    return (write, *_residual_eta(key, value, rk, rv, eta))


def _level_logits(model, lv, j: int, raw: Tensor, old: LevelState) -> None:
    """Counts after every token and the level's base logits (attention.py:
    319-323 and :165-175) into lv."""
    cfg = model.config
    if lv.correction is not None:  # positional moments: the logits take the moment term
        lv.counts = old.count[:, None] + _cumsum_tokens(lv.write.float())
        lv.final_count = lv.counts[:, -1]
        lv.logits = _base_logits(model, raw, lv.counts, j, lv.correction)
        return
    if _token_logits_supported(raw, lv.write):
        gain, scale = _count_scalars(model, j, raw)
        lv.logits, lv.final_count, lv.local = glue.token_logits(raw, lv.write, old.count, gain, scale)
        lv.counts = lv.final_count[:, None]
        return
    if _FUSED_COUNTS[0] and fused_counts_supported(cfg, raw.dtype, lv.write.shape[-1]):
        gain, scale = _count_scalars(model, j, raw)
        lv.logits, lv.final_count = count_logits(raw, lv.write, old.count, gain, scale)
        lv.counts = None  # not needed past the logits on this path
    else:
        lv.counts = old.count[:, None] + _cumsum_tokens(lv.write.float())
        lv.final_count = lv.counts[:, -1]
        lv.logits = _base_logits(model, raw, lv.counts, j)


def _relations(model, local, writes, rel_states, scan, token=False):
    """Every ordered edge's R_ij scan (attention.py:206-223); one token step
    per edge when `token` (inference on one token)."""
    cfg = model.config
    # Every edge's decay and write strength [E,H].
    rd, rb = model.relation_decay_raw, model.relation_beta_raw
    decay = params.derived(("rel_decay", id(rd), cfg.positional_mode == "none"), (rd,),
                           lambda: -F.softplus(rd) * (0. if cfg.positional_mode == "none" else 1.),
                           differentiable=True)
    strength = params.derived(("rel_beta", id(rb)), (rb,), lambda: rb.sigmoid(), differentiable=True)
    # Per-edge [B,T,H] views of both, taken with one unbind: the backward then
    # stacks the edges' gradients once and reduces them in one sum, instead of
    # a reduction, a zero fill, a copy and an add per edge and tensor.
    lead = writes[0].shape[:-1]
    n_e = len(model.edges)
    g_edge = decay[:, None, None, :].expand(n_e, *lead).unbind(0)
    b_edge = strength[:, None, None, :].expand(n_e, *lead).unbind(0)

    def edge(e, i, j, old):
        def run():
            g, beta = g_edge[e], b_edge[e]
            target = writes[j]
            if cfg.rsa_update:
                target, beta = _rsa_target(writes[i], target, beta)
            if token and token_step_supported(writes[i], target):
                return gdn_token_hip(local[i], writes[i], target, g, beta, old.memory)
            msg, _, memory = gdn_scan_hip(local[i], writes[i], target, g, beta, old.memory, **scan)
            return msg, memory
        return run, (local[i], writes[i], writes[j], old.memory, decay, strength)

    if token and all(token_step_supported(writes[i], writes[j]) for i, j in model.edges):
        # every edge's one-token step, packed into as few launches as the library takes
        calls = []
        for e, ((i, j), old) in enumerate(zip(model.edges, rel_states)):
            g, beta, target = g_edge[e], b_edge[e], writes[j]
            if cfg.rsa_update:
                target, beta = _rsa_target(writes[i], target, beta)
            calls.append((local[i], writes[i], target, g, beta, old.memory))
        done = [r for part in _chunks(calls, _lib.TOKEN_MAX_PACK) for r in gdn_token_many(part)]
    elif _PACKED[0]:
        # every edge's scan in as few library calls as it takes: the state
        # recurrences of all edges advance together
        groups = []
        for e, ((i, j), old) in enumerate(zip(model.edges, rel_states)):
            g, beta, target = g_edge[e], b_edge[e], writes[j]
            if cfg.rsa_update:
                target, beta = _rsa_target(writes[i], target, beta)
            groups.append(dict(q=local[i], k=writes[i], v=target, g=g, beta=beta, s0=old.memory, **scan))
        done = [(msg, final) for part in _chunks(groups, _lib.GDN_MAX_PACK)
                for msg, _, final in gdn_scan_many(part)]
    else:
        done = _concurrent([edge(e, i, j, old) for e, ((i, j), old) in enumerate(zip(model.edges, rel_states))])
    incoming = [[] for _ in local]
    finals = []
    for e, ((i, j), (msg, memory)) in enumerate(zip(model.edges, done)):
        incoming[j].append((e, msg))
        finals.append(RelationState(i, j, memory))
    return incoming, tuple(finals)


def _rsa_target(source: Tensor, target: Tensor, beta: Tensor):
    """rsa_update's relation value and strength (attention.py:215-218): the
    target write over the source write's norm, beta * norm^2 capped at .9."""
    norm = (source.float().square().sum(-1) + 1e-6).sqrt()
    return (target / norm[..., None]).to(target.dtype), (beta * norm.square()).clamp_max(.9)


def _incoming_index(model, j: int) -> Tensor:
    """Device index of the edges into level j (i-major order), built from the
    module's edge-target buffer so that no host copy happens inside a graph
    capture."""
    target = model._edge_target
    return params.derived(("edge_in", id(target), j), (target,),
                          lambda: (target == j).nonzero_static(size=model.config.levels - 1)[:, 0])


def _product_base(model, j: int, logits, incoming, counts) -> Tensor:
    """Level j's base logits after the product relation read (attention.py:
    231-236) on the HIP kernel (route.product_read): the messages weighted by
    the edge softmax and by |softmax(source logits)| per row, scaled by
    M e^{clamp(gain)}, and the marginal term when relation_marginal."""
    cfg = model.config
    norms = [logits[model.edges[e][0]].softmax(-1).norm(dim=-1) for e, _ in incoming[j]]
    gexp = model.relation_gain[j].clamp(-4, 4).exp()
    return product_read(logits[j].float(), gexp, _incoming_weights(model, j), [msg for _, msg in incoming[j]],
                        norms, counts[j].float() if cfg.relation_marginal else None)


def _incoming_weights(model, j: int) -> Tensor:
    """Softmax of the logits of the edges into level j over those edges, [n_in,H]."""
    logits = model.edge_logits
    return params.derived(("edge_w", id(logits), j), (logits, model._edge_target),
                          lambda: logits.index_select(0, _incoming_index(model, j)).softmax(0), differentiable=True)


_FUSED_ROUTE = [True]  # the fused route reader for the default read (route.py)


def _bridge(model, q: Tensor, logits, incoming, counts):
    """Route reader and query projection per target level (attention.py:225-262)."""
    cfg = model.config
    dtype = q.dtype
    routes, queries = [], []

    def query_weight(j):
        # shared_query_center: W_qs + center^T / query_scale (attention.py:254-256)
        qw = model.query_weight[j]
        if not cfg.shared_query_center:
            return qw
        c = model.center[j]
        return params.derived(("query_center", id(qw), id(c), float(cfg.query_scale)), (qw, c),
                              lambda: qw + c.transpose(-1, -2) / cfg.query_scale, differentiable=True)

    def reader_args(j, base):
        # the route reader's base logits and incoming messages: the product read
        # folds the messages into the base logits first (product_read)
        if not incoming[j]:
            return base, None, []
        if cfg.paper_product_read:
            return _product_base(model, j, logits, incoming, counts), None, []
        return base, _incoming_weights(model, j), [msg for _, msg in incoming[j]]

    def mix(j):
        # balanced_bridge: .1 + .8 sigmoid(bridge_mix_raw_j), per head (attention.py:257)
        return .1 + .8 * model.bridge_mix_raw[j].sigmoid() if cfg.balanced_bridge else None

    if (_FUSED_ROUTE[0] and not torch.is_grad_enabled() and 1 < len(logits) <= _lib.ROUTE_MAX_PACK
            and all(fused_route_supported(cfg, dtype, base.shape[-1]) for base in logits)):
        # inference: every level's read in one launch where the library can pack them
        reads = []
        for j, base in enumerate(logits):
            base_j, w, msgs = reader_args(j, base)
            reads.append((base_j, q, w, model.relation_gain[j], model.route_mlp_gain[j], model.route_up[j],
                          model.route_down[j], model.route_weight[j], query_weight(j), cfg.query_scale, msgs,
                          cfg.rsa_update, mix(j)))
        done = route_reader_many(reads)
        return [route for _, route in done], [qo for qo, _ in done]
    for j, base in enumerate(logits):
        if _FUSED_ROUTE[0] and fused_route_supported(cfg, dtype, base.shape[-1]):
            base_j, w, msgs = reader_args(j, base)
            qo, route = route_reader(base_j, q, w, model.relation_gain[j], model.route_mlp_gain[j],
                                     model.route_up[j], model.route_down[j], model.route_weight[j],
                                     query_weight(j), cfg.query_scale, msgs, cfg.rsa_update, mix(j))
            routes.append(route)
            queries.append(qo)
            continue
        if incoming[j]:
            w = _incoming_weights(model, j)
            total = 0
            if cfg.paper_product_read:
                for wt, (e, msg) in zip(w, incoming[j]):
                    src_norm = logits[model.edges[e][0]].softmax(-1).norm(dim=-1, keepdim=True)
                    total = total + wt[..., None] * msg.float() * src_norm
                gain = model.relation_gain[j].clamp(-4, 4).exp()[..., None]
                base = base + base.shape[-1] * gain * total
                if cfg.relation_marginal:
                    base = base - gain * counts[j].log1p()
            else:
                for wt, (_, msg) in zip(w, incoming[j]):
                    total = total + wt[..., None] * msg.float()
                centred = total - total.mean(-1, keepdim=True)
                z = centred / (centred.square().mean(-1, keepdim=True) + 1e-5).sqrt()
                base = base + model.relation_gain[j][..., None] * z.tanh()
        route = base.softmax(-1).to(dtype)
        hidden = F.gelu(_mm(route, model.route_up[j], "bthm,hmr->bthr", dtype).float()).to(dtype)
        route = (route.float() + model.route_mlp_gain[j][..., None]
                 * _mm(hidden, model.route_down[j], "bthr,hrm->bthm", dtype).float()).to(dtype)
        if cfg.rsa_update:
            wide = route.float()
            route = (wide / wide.abs().sum(-1, keepdim=True).clamp(.25, 4.)).to(dtype)
        qo = _mm(route, model.route_weight[j], "bthm,hmn->bthn", dtype)
        qw = model.query_weight[j]
        if cfg.shared_query_center:
            qw = qw + model.center[j].transpose(-1, -2) / cfg.query_scale
        direct = (cfg.query_scale * _mm(q, qw, "bthd,hdm->bthm", dtype).float()).to(dtype)
        direct = _slot_feature(cfg, direct)
        if cfg.balanced_bridge:
            mix = .1 + .8 * model.bridge_mix_raw[j].sigmoid()[..., None]
            qo = (mix * _unit(qo).float() + (1 - mix) * _unit(direct).float()).to(dtype)
        else:
            qo = (qo.float() + direct.float()).to(dtype)
        routes.append(route)
        queries.append(qo)
    return routes, queries
