"""The one-token inference kernels (gpa_amd/csrc/gdn_token.hip,
level_token.hip) built for the host under AddressSanitizer (tests/host_emu/)
and compared on the CPU:

- `gdn_token_hip` / `gdn_token_read` against the oracle's gdn_step and
  gdn_read (reference src/gpa/ops.py:29-46): float32 at 1e-5, bfloat16 at
  2e-2, for widths that are not multiples of 16 (K = 20, 200; V = 4, 12, 96),
  no initial state, a batch-broadcast initial state, and a read alone;
- `gdn_token_many` (the packed launch, workgroups found through the kernel
  arguments) against one call per group, bit for bit;
- `level_mix_block` at one token on the one-token level kernel against the
  block kernel of the same host build, for register and generic shapes
  (M = 12, Dv = 8) and batch-broadcast snapshots;
- `token_step_and_level` (a level's inner token step and its level write in
  one launch) against the two separate calls, bit for bit, with as many, fewer
  and more step workgroups than level streams, and a shape that takes the
  two launches.

Every access of these kernels is bounds-checked here before they run on a GPU.
"""
import pytest
import torch

from gpa_amd import level, ops
from oracle import reference as ref
from tests.host_emu import harness


@pytest.fixture
def runner(host_runner):
    return host_runner


@pytest.fixture
def host(runner, tmp_path, monkeypatch):
    lib = harness.HostLib(runner, str(tmp_path))
    harness.use_host(monkeypatch, lib)
    return lib


def _rel(a, b):
    a, b = a.detach().double(), b.detach().double()
    return ((a - b).norm() / max(b.norm().item(), 1e-30)).item()


def _call(g, b, h, k, v, dtype, s0, query):
    q = torch.randn(b, 1, h, k, generator=g).to(dtype) if query else None
    key = torch.randn(b, 1, h, k, generator=g).to(dtype)
    val = torch.randn(b, 1, h, v, generator=g).to(dtype)
    lg, beta = -torch.rand(b, 1, h, generator=g), torch.rand(b, 1, h, generator=g)
    state = {"full": torch.randn(b, h, k, v, generator=g) * .2,
             "broadcast": (torch.randn(1, h, k, v, generator=g) * .2).expand(b, h, k, v), None: None}[s0]
    return q, key, val, lg, beta, state


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("b,h,k,v,s0,query", [(2, 1, 20, 12, None, True), (1, 2, 200, 4, "broadcast", True),
                                              (2, 3, 64, 96, "full", False), (1, 1, 128, 128, "full", True),
                                              (1, 2, 256, 128, "full", True), (2, 1, 160, 36, None, True)])
def test_token_step_matches_oracle_step_and_read(host, b, h, k, v, s0, query, dtype):
    g = torch.Generator().manual_seed(b * 7 + k + v)
    q, key, val, lg, beta, state = _call(g, b, h, k, v, dtype, s0, query)
    with torch.no_grad():
        out, final = ops.gdn_token_hip(q, key, val, lg, beta, state)
    s_ref = ref.gdn_step(state if state is not None else torch.zeros(b, h, k, v), key[:, 0], val[:, 0], lg[:, 0],
                         beta[:, 0])
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert final.shape == (b, h, k, v) and _rel(final, s_ref) < tol
    if query:
        assert out.dtype == dtype and _rel(out[:, 0], ref.gdn_read(q[:, 0], s_ref)) < tol
    else:
        assert out is None


def test_token_read_alone_matches_oracle_read(host):
    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 1, 3, 36, generator=g)
    state = torch.randn(2, 3, 36, 20, generator=g)
    with torch.no_grad():
        out = ops.gdn_token_read(q, state)
    assert _rel(out[:, 0], ref.gdn_read(q[:, 0], state)) < 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_token_many_matches_one_call_per_group(host, dtype):
    g = torch.Generator().manual_seed(11)
    calls = [_call(g, *shape, dtype, s0, query) for shape, s0, query in
             [((2, 1, 128, 32), "full", True), ((1, 2, 256, 12), "broadcast", True), ((2, 1, 20, 8), None, False),
              ((1, 1, 64, 64), "full", True)]]
    with torch.no_grad():
        many = ops.gdn_token_many(calls)
        one = [ops.gdn_token_hip(*c) for c in calls]
    for (out_m, fin_m), (out_1, fin_1) in zip(many, one):
        assert torch.equal(fin_m, fin_1)
        assert (out_m is None) == (out_1 is None)
        if out_m is not None:
            assert torch.equal(out_m, out_1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("b,h,dk,dv,m,first", [(2, 2, 16, 8, 12, "full"), (3, 1, 20, 8, 12, "broadcast"),
                                               (2, 1, 64, 32, 64, "full"), (1, 2, 128, 128, 256, "broadcast")])
def test_level_token_kernel_matches_block_kernel(host, monkeypatch, b, h, dk, dv, m, first, dtype):
    g = torch.Generator().manual_seed(b + dk + m)
    key = torch.randn(b, 1, h, dk, generator=g).to(dtype)
    value = torch.randn(b, 1, h, dv, generator=g).to(dtype)
    lead = b if first == "full" else 1
    fa = (torch.randn(lead, h, dk, m, generator=g) * .3).expand(b, h, dk, m)
    fb = (torch.randn(lead, h, m, dv, generator=g) * .3).expand(b, h, m, dv)
    eta = 1 + .25 * torch.randn(h, 2, generator=g).tanh()
    outs = {}
    for token_kernel in (True, False):
        monkeypatch.setattr(level, "_TOKEN_KERNEL", [token_kernel])
        with torch.no_grad():
            outs[token_kernel] = level.level_mix_block(key, value, fa, fb, eta, 4, 2)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for name, a, r in zip(("write", "key'", "value'"), outs[True], outs[False]):
        assert a.dtype == r.dtype == dtype and a.shape == r.shape, name
        assert _rel(a, r) < tol, (name, _rel(a, r))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("step_shape,lvl", [((2, 2, 128, 128), (2, 2, 128, 128, 128)),
                                            ((1, 2, 128, 256), (1, 2, 128, 256, 128)),
                                            ((3, 2, 128, 64), (2, 2, 128, 128, 128)),
                                            ((4, 2, 100, 128), (1, 2, 128, 128, 128)),
                                            ((1, 2, 256, 128), (1, 2, 128, 128, 128)),
                                            ((2, 1, 20, 12), (2, 1, 20, 12, 8))],
                         ids=["m128", "m256", "fewer_steps", "more_steps", "k256", "two_launches"])
def test_token_level_matches_separate_calls(host, step_shape, lvl, dtype):
    g = torch.Generator().manual_seed(sum(step_shape) + sum(lvl))
    step = _call(g, *step_shape, dtype, "full", True)
    lb, lh, dk, m, dv = lvl
    key = torch.randn(lb, 1, lh, dk, generator=g).to(dtype)
    value = torch.randn(lb, 1, lh, dv, generator=g).to(dtype)
    fa, fb = torch.randn(lb, lh, dk, m, generator=g) * .3, torch.randn(lb, lh, m, dv, generator=g) * .3
    eta = 1 + .25 * torch.randn(lh, 2, generator=g).tanh()
    with torch.no_grad():
        fused = level.token_step_and_level(step, key, value, fa, fb, eta, 4, 2)
        apart = ops.gdn_token_hip(*step) + level.level_mix_block(key, value, fa, fb, eta, 4, 2)
    for name, a, r in zip(("out", "final", "write", "key'", "value'"), fused, apart):
        assert a.dtype == r.dtype and torch.equal(a, r), name


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("b,h,dk,dv,m", [(2, 2, 64, 32, 64), (1, 2, 128, 128, 256), (2, 1, 128, 128, 128)])
def test_write_only_level_token_gives_the_same_write(host, b, h, dk, dv, m, dtype):
    """The last level's write-only form (key_out / value_out null: B^ is not
    read, no residual product) gives the bits of the full form's write, alone
    and beside the inner token step."""
    assert level.write_only_supported(dk, dv, m)
    g = torch.Generator().manual_seed(b + dk + m + 1)
    key = torch.randn(b, 1, h, dk, generator=g).to(dtype)
    value = torch.randn(b, 1, h, dv, generator=g).to(dtype)
    fa, fb = torch.randn(b, h, dk, m, generator=g) * .3, torch.randn(b, h, m, dv, generator=g) * .3
    eta = 1 + .25 * torch.randn(h, 2, generator=g).tanh()
    step = _call(g, b, h, dk, m, dtype, "full", True)
    with torch.no_grad():
        full = level.level_mix_block(key, value, fa, fb, eta, 4, 2)
        only = level.level_mix_block(key, value, fa, fb, eta, 4, 2, residual=False)
        fused = level.token_step_and_level(step, key, value, fa, fb, eta, 4, 2, residual=False)
        apart = ops.gdn_token_hip(*step)
    assert only[1] is None and only[2] is None and fused[3] is None and fused[4] is None
    assert torch.equal(only[0], full[0]) and torch.equal(fused[2], full[0])
    assert torch.equal(fused[0], apart[0]) and torch.equal(fused[1], apart[1])


@pytest.mark.parametrize("b,h,k,m,dv,with_level", [(2, 2, 128, 128, 128, True), (3, 1, 64, 96, 32, True),
                                                   (1, 2, 128, 256, 128, False), (2, 1, 32, 160, 12, True)],
                         ids=["c3", "small", "m256_step_only", "narrow_keys"])
def test_slot_in_step_matches_slot_gates_then_step(host, b, h, k, m, dv, with_level):
    """gpa_token_slot_step (the slot products and gates inside the one-token
    inner step, with the level write where given) against
    gpa_slot_gates_act_forward followed by the step (and the level write):
    the slot, gates, new state, read and level outputs.  The slot dot
    products are summed in another order, so a slot may round to the
    neighbouring bf16 value; everything downstream follows."""
    from gpa_amd import slots
    g = torch.Generator().manual_seed(b + k + m)
    bf = torch.bfloat16
    q = torch.randn(b, 1, h, k, generator=g).to(bf)
    key = torch.randn(b, 1, h, k, generator=g).to(bf)
    center = torch.randn(h, m, k, generator=g) / k ** .5
    gate_w = torch.randn(h, k, 4, generator=g) * .3
    bias = torch.randn(h, 4, generator=g)
    s0 = torch.randn(b, h, k, m, generator=g) * .2
    args = (center, gate_w, bias, .9, .5)
    lvl = None
    if with_level:
        value = torch.randn(b, 1, h, dv, generator=g).to(bf)
        fa, fb = torch.randn(b, h, k, m, generator=g) * .3, torch.randn(b, h, m, dv, generator=g) * .3
        eta = 1 + .25 * torch.randn(h, 2, generator=g).tanh()
        lvl = (key, value, fa, fb, eta, 4, 1, True)
    with torch.no_grad():
        got = level.token_slot_step(q, key, s0, *args, lvl)
        slot, g_in, b_in, g_out, b_out = slots.slot_gates_act(key, *args)
        out, final = ops.gdn_token_hip(q, key, slot, g_in, b_in, s0)
        ref = (out, final, slot, g_in, b_in, g_out, b_out)
        if with_level:
            ref += level.level_mix_block(*lvl)
    names = ("out", "final", "slot", "g_in", "b_in", "g_out", "b_out", "write", "key'", "value'")
    assert len(got) == len(ref)
    ulp = (got[2].float() - ref[2].float()).abs() / ref[2].float().abs().clamp_min(1e-30)
    assert (ulp > 2 ** -8).sum() <= max(1, ref[2].numel() // 200), "slot: more than a rare 1-ulp difference"
    for name, a, r in zip(names, got, ref):
        assert a.dtype == r.dtype and a.shape == r.shape, name
        tol = {"slot": 1e-2, "out": 2e-2, "final": 1e-2}.get(name, 1e-6)
        assert _rel(a, r) <= tol, (name, _rel(a, r))
