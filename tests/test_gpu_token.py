"""One-token inference steps (gpa_amd/ops.py gdn_token_hip / gdn_token_read,
csrc/gdn_token.hip) and the decode path of the schedule that uses them.

Operators: against the oracle's gdn_step then gdn_read (reference
src/gpa/ops.py:29-46) on the CPU, for float32 (relative L2 1e-5) and bfloat16
(2e-2), several widths (K not a multiple of 16, K = V = 256), no initial state,
a batch-broadcast initial state (stride 0) and calls without a query.
Module: DenseGPA one-token calls from a fresh cache across block boundaries
(offsets 0..3 of a 4-token block) at C3 widths, against the oracle (1e-4 in
float32, 2e-2 in bfloat16) and against the chunked-scan path of the same
schedule: output and every cache tensor.
"""
import copy

import pytest
import torch

import oracle
from oracle import reference as ref
from gpa_amd import DenseGPA, GPAConfig, schedule
from gpa_amd.ops import gdn_token_hip, gdn_token_many, gdn_token_read
from gpa_amd.state import tensors

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / max(b.norm().item(), 1e-30)).item()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("b,h,k,v,s0,query", [(3, 2, 128, 128, "full", True), (2, 3, 64, 96, "broadcast", True),
                                              (1, 2, 256, 256, "full", True), (2, 1, 20, 12, None, True),
                                              (2, 2, 128, 256, "full", False), (1, 1, 200, 4, "broadcast", True)])
def test_token_step_matches_reference_step_and_read(b, h, k, v, s0, query, dtype):
    g = torch.Generator().manual_seed(b * 100 + k + v)
    q = torch.randn(b, 1, h, k, generator=g).to(dtype)
    key = torch.randn(b, 1, h, k, generator=g).to(dtype)
    val = torch.randn(b, 1, h, v, generator=g).to(dtype)
    lg = -torch.rand(b, 1, h, generator=g)
    beta = torch.rand(b, 1, h, generator=g)
    if s0 == "full":
        state = torch.randn(b, h, k, v, generator=g) * .2
    elif s0 == "broadcast":
        state = (torch.randn(1, h, k, v, generator=g) * .2).expand(b, h, k, v)
    else:
        state = None
    with torch.no_grad():
        out, final = gdn_token_hip(q.to(DEV) if query else None, key.to(DEV), val.to(DEV), lg.to(DEV),
                                   beta.to(DEV), state.to(DEV) if state is not None else None)
    s_ref = ref.gdn_step(state if state is not None else torch.zeros(b, h, k, v), key[:, 0], val[:, 0],
                         lg[:, 0], beta[:, 0])
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert final.dtype == torch.float32 and final.shape == (b, h, k, v)
    assert _rel(final, s_ref) < tol
    if query:
        o_ref = ref.gdn_read(q[:, 0], s_ref)
        assert out.dtype == dtype and out.shape == (b, 1, h, v)
        assert _rel(out[:, 0], o_ref) < tol
    else:
        assert out is None


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_token_many_matches_one_call_per_group_and_reference(dtype):
    """gdn_token_many (one launch per key-width class) gives the bits of one
    gdn_token_hip per group, for groups of three key-width classes in mixed
    order, with and without a query and an initial state, and each matches the
    oracle's step and read."""
    g = torch.Generator().manual_seed(5)
    shapes = [(64, 1, 128, 128, True, "full"), (64, 1, 256, 128, True, "full"), (2, 3, 20, 12, False, None),
              (64, 1, 128, 256, True, "broadcast"), (2, 3, 256, 4, True, "full"), (64, 1, 128, 128, True, "full")]
    calls = []
    for b, h, k, v, query, s0 in shapes:
        q = torch.randn(b, 1, h, k, generator=g).to(dtype) if query else None
        key = torch.randn(b, 1, h, k, generator=g).to(dtype)
        val = torch.randn(b, 1, h, v, generator=g).to(dtype)
        lg, beta = -torch.rand(b, 1, h, generator=g), torch.rand(b, 1, h, generator=g)
        st = {"full": torch.randn(b, h, k, v, generator=g) * .2,
              "broadcast": (torch.randn(1, h, k, v, generator=g) * .2).expand(b, h, k, v), None: None}[s0]
        calls.append(tuple(x.to(DEV) if x is not None else None for x in (q, key, val, lg, beta, st)))
    with torch.no_grad():
        many = gdn_token_many(calls)
        one = [gdn_token_hip(*c) for c in calls]
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for (out_m, fin_m), (out_1, fin_1), (q, key, val, lg, beta, st) in zip(many, one, calls):
        assert torch.equal(fin_m, fin_1)
        assert (out_m is None) == (out_1 is None)
        b, _, h, k = key.shape
        s_ref = ref.gdn_step(st.cpu() if st is not None else torch.zeros(b, h, k, val.shape[-1]), key[:, 0].cpu(),
                             val[:, 0].cpu(), lg[:, 0].cpu(), beta[:, 0].cpu())
        assert _rel(fin_m, s_ref) < tol
        if out_m is not None:
            assert torch.equal(out_m, out_1)
            assert _rel(out_m[:, 0], ref.gdn_read(q[:, 0].cpu(), s_ref)) < tol


def test_token_many_refuses_too_many_groups():
    k = torch.randn(1, 1, 1, 8, device=DEV)
    g, beta = torch.zeros(1, 1, 1, device=DEV), torch.ones(1, 1, 1, device=DEV)
    with pytest.raises(ValueError):
        gdn_token_many([(None, k, k, g, beta, None)] * 13)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_token_read_matches_reference_read(dtype):
    g = torch.Generator().manual_seed(11)
    q = torch.randn(2, 1, 3, 96, generator=g).to(dtype)
    state = torch.randn(2, 3, 96, 64, generator=g)
    with torch.no_grad():
        out = gdn_token_read(q.to(DEV), state.to(DEV))
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert out.dtype == dtype and _rel(out[:, 0], ref.gdn_read(q[:, 0], state)) < tol


def test_token_step_refuses_autograd():
    k = torch.randn(1, 1, 1, 8, device=DEV, requires_grad=True)
    v = torch.randn(1, 1, 1, 8, device=DEV)
    g, beta = torch.zeros(1, 1, 1, device=DEV), torch.ones(1, 1, 1, device=DEV)
    with pytest.raises(RuntimeError, match="no backward"):
        gdn_token_hip(None, k, v, g, beta, None)


C3 = dict(heads=2, key_dim=128, value_dim=128, slots=(128, 128, 128, 256), chunk_size=4)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_decode_token_steps_match_oracle_and_chunk_path(dtype, monkeypatch):
    torch.manual_seed(21)
    model = DenseGPA(GPAConfig(**C3))
    oracle_run = oracle.OracleRun(copy.deepcopy(model))
    hip = model.to(DEV)
    b, steps = 2, 7
    g = torch.Generator().manual_seed(5)
    toks = []
    for _ in range(steps):
        q = torch.randn(b, 1, 2, 128, generator=g)
        k = torch.nn.functional.normalize(torch.randn(b, 1, 2, 128, generator=g), dim=-1)
        toks.append((q.to(dtype), k.to(dtype), torch.randn(b, 1, 2, 128, generator=g).to(dtype)))

    def decode(token_path):
        monkeypatch.setattr(schedule, "_TOKEN_STEP", [token_path])
        outs, state = [], None
        with torch.no_grad():
            for x in toks:
                y, state = hip(*(t.to(DEV) for t in x), state)
                outs.append(y)
        return torch.cat(outs, 1), state

    y_tok, s_tok = decode(True)
    y_chunk, s_chunk = decode(False)
    ref_outs, ref_state = [], None
    with torch.no_grad():
        for x in toks:
            y, ref_state = oracle_run(*x, ref_state)
            ref_outs.append(y)
    y_ref = torch.cat(ref_outs, 1)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    assert y_tok.dtype == dtype and _rel(y_tok, y_ref) < tol
    assert _rel(y_tok, y_chunk) < tol
    assert s_tok.chunk_offset == ref_state.chunk_offset == steps % 4
    for a, r, c in zip(tensors(s_tok), tensors(ref_state), tensors(s_chunk)):
        assert _rel(a, r) < tol and _rel(a, c) < tol


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("b,h,dk,dv,m,first", [(3, 2, 128, 128, 128, "full"), (2, 2, 128, 128, 256, "broadcast"),
                                               (2, 1, 20, 8, 12, "full"), (1, 3, 256, 96, 64, "broadcast"),
                                               (64, 16, 128, 128, 128, "full"), (64, 16, 128, 128, 256, "full")])
def test_level_token_kernel_matches_block_kernel(b, h, dk, dv, m, first, dtype, monkeypatch):
    """gpa_level_token_forward (one token from the block snapshots) against the
    block kernel gpa_level_forward on the same call: write, key', value'; the
    last two cases have the decode batch's 1024 streams."""
    from gpa_amd import level
    g = torch.Generator().manual_seed(b + dk + m)
    key = torch.randn(b, 1, h, dk, generator=g).to(dtype).to(DEV)
    value = torch.randn(b, 1, h, dv, generator=g).to(dtype).to(DEV)
    lead = b if first == "full" else 1
    fa = (torch.randn(lead, h, dk, m, generator=g) * .3).to(DEV).expand(b, h, dk, m)
    fb = (torch.randn(lead, h, m, dv, generator=g) * .3).to(DEV).expand(b, h, m, dv)
    eta = (1 + .25 * torch.randn(h, 2, generator=g).tanh()).to(DEV)
    outs = {}
    for token_kernel in (True, False):
        monkeypatch.setattr(level, "_TOKEN_KERNEL", [token_kernel])
        with torch.no_grad():
            outs[token_kernel] = level.level_mix_block(key, value, fa, fb, eta, 4, 2)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for name, a, r in zip(("write", "key'", "value'"), outs[True], outs[False]):
        assert a.dtype == r.dtype == dtype and a.shape == r.shape, name
        assert _rel(a, r) < tol, (name, _rel(a, r))


@pytest.mark.parametrize("b,h,dk,m", [(64, 16, 128, 128), (64, 16, 128, 256), (3, 2, 256, 128), (2, 3, 64, 96)])
def test_slot_gates_act_matches_slot_gates_then_gate_act(b, h, dk, m):
    """gpa_slot_gates_act_forward (slot products, gate inputs and gate
    nonlinearities in one launch) gives the bits of gpa_slot_gates_forward
    followed by gpa_gate_act_forward."""
    from gpa_amd import glue
    from gpa_amd.slots import slot_gates, slot_gates_act
    g = torch.Generator().manual_seed(b + dk + m)
    key = torch.randn(b, 1, h, dk, generator=g).bfloat16().to(DEV)
    center = (torch.randn(h, m, dk, generator=g) * .1).to(DEV)
    gate_w = (torch.randn(h, dk, 4, generator=g) * .3).to(DEV)
    bias = torch.randn(h, 4, generator=g).to(DEV)
    with torch.no_grad():
        slot, raw = slot_gates(key, center, gate_w)
        gates = glue.gate_act(raw, bias, .9, .5)
        fused = slot_gates_act(key, center, gate_w, bias, .9, .5)
    assert torch.equal(fused[0], slot)
    for a, r in zip(fused[1:], gates):
        assert a.dtype == torch.float32 and torch.equal(a, r)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_token_logits_many_matches_one_call_per_level(dtype):
    """gpa_token_logits_many (the one-token logits of several levels in one
    launch) gives the bits of one gpa_token_logits_forward per level: slot
    widths 128, 256, 12 and 96, full and batch-broadcast counts."""
    from gpa_amd import glue
    g = torch.Generator().manual_seed(9)
    calls = []
    for b, h, m, bcast in [(64, 16, 128, False), (64, 16, 256, True), (3, 2, 12, False), (5, 3, 96, True)]:
        raw = torch.randn(b, 1, h, m, generator=g).to(dtype).to(DEV)
        write = torch.rand(b, 1, h, m, generator=g).to(dtype).to(DEV)
        c0 = (torch.rand(1 if bcast else b, h, m, generator=g) * 5).to(DEV).expand(b, h, m)
        gain, scale = (torch.rand(h, generator=g) + .5).to(DEV), (torch.rand(h, generator=g) * 4).to(DEV)
        calls.append((raw, write, c0, gain, scale))
    with torch.no_grad():
        many = glue.token_logits_many(calls)
        one = [glue.token_logits(*c) for c in calls]
    for got, ref in zip(many, one):
        for name, a, r in zip(("logits", "counts", "local"), got, ref):
            assert a.dtype == r.dtype and a.shape == r.shape and torch.equal(a, r), name


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("step_shape,lvl", [((8, 16, 128, 128), (8, 16, 128, 128, 128)),
                                            ((8, 16, 128, 256), (8, 16, 128, 256, 128)),
                                            ((3, 4, 128, 64), (2, 4, 128, 128, 128)),
                                            ((4, 4, 100, 128), (1, 4, 128, 128, 128)),
                                            ((2, 3, 20, 12), (2, 3, 20, 12, 8))],
                         ids=["m128", "m256", "fewer_steps", "more_steps", "two_launches"])
def test_token_level_matches_separate_calls(step_shape, lvl, dtype):
    """A level's inner token step and its level write in one launch
    (gpa_token_level_forward) give the bits of the two separate calls."""
    from gpa_amd import level
    g = torch.Generator().manual_seed(sum(step_shape) + sum(lvl))
    b, h, k, v = step_shape
    q, key, val = (torch.randn(b, 1, h, d, generator=g).to(DEV, dtype) for d in (k, k, v))
    lg, beta = -torch.rand(b, 1, h, generator=g).to(DEV), torch.rand(b, 1, h, generator=g).to(DEV)
    step = (q, key, val, lg, beta, (torch.randn(b, h, k, v, generator=g) * .2).to(DEV))
    lb, lh, dk, m, dv = lvl
    lkey = torch.randn(lb, 1, lh, dk, generator=g).to(DEV, dtype)
    lval = torch.randn(lb, 1, lh, dv, generator=g).to(DEV, dtype)
    fa = (torch.randn(lb, lh, dk, m, generator=g) * .3).to(DEV)
    fb = (torch.randn(lb, lh, m, dv, generator=g) * .3).to(DEV)
    eta = (1 + .25 * torch.randn(lh, 2, generator=g).tanh()).to(DEV)
    with torch.no_grad():
        fused = level.token_step_and_level(step, lkey, lval, fa, fb, eta, 64, 5)
        apart = gdn_token_hip(*step) + level.level_mix_block(lkey, lval, fa, fb, eta, 64, 5)
    torch.cuda.synchronize()
    for name, a, r in zip(("out", "final", "write", "key'", "value'"), fused, apart):
        assert a.dtype == r.dtype and torch.equal(a, r), name


def test_copy_many_matches_copy():
    """One launch copies a decode token's q, k and v (gpa_copy_many) with the
    bytes of Tensor.copy_; an unaligned pair is refused without copying."""
    from gpa_amd import glue
    src = [torch.randn(64, 1, 16, 128, device=DEV).bfloat16(), torch.randn(3, 1, 2, 8, device=DEV),
           torch.randn(0, 4, device=DEV)]
    dst = [torch.zeros_like(x) for x in src]
    assert glue.copy_many(list(zip(dst, src)))
    torch.cuda.synchronize()
    assert all(torch.equal(d, s) for d, s in zip(dst, src))
    odd = torch.randn(7, device=DEV)
    keep = torch.zeros(7, device=DEV)
    assert not glue.copy_many([(keep, odd)])
    assert not glue.copy_many([(torch.zeros(8, device=DEV)[1:5], torch.randn(4, device=DEV))])
    torch.cuda.synchronize()
    assert torch.count_nonzero(keep) == 0
