"""HIP chunked GDN scan vs the oracle's per-token recurrence (reference ops.py:29-85).

The HIP operator returns the read, the state at the start of every chunk and
the final state; its backward takes gradients for all three.  The oracle runs
the literal recurrence in float64 on the CPU from the same inputs (bf16 inputs
are compared after their exact widening), segment by segment so that the
chunk-start states are observable.
"""
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _inputs(b, t, h, kd, vd, dtype, seed, q=True, s0=True, const_gates=False):
    g = torch.Generator().manual_seed(seed)
    qq = torch.randn(b, t, h, kd, generator=g) if q else None
    kk = torch.randn(b, t, h, kd, generator=g)
    vv = torch.randn(b, t, h, vd, generator=g)
    if const_gates:
        gate = -torch.rand(1, 1, h, generator=g).expand(b, t, h) * .5
        beta = torch.rand(1, 1, h, generator=g).expand(b, t, h)
    else:
        gate = -torch.rand(b, t, h, generator=g) * .5
        beta = torch.rand(b, t, h, generator=g)
    state = torch.randn(b, h, kd, vd, generator=g) * .3 if s0 else None
    cast = lambda x: None if x is None else x.to(dtype)  # noqa: E731
    return cast(qq), cast(kk), cast(vv), gate, beta, state


def _oracle_segments(q, k, v, g, beta, s0, chunk, offset):
    """Per-token oracle in float64; returns out, chunk-start states, final."""
    b, t, h, kd = k.shape
    vd = v.shape[-1]
    d = lambda x: None if x is None else x.detach().double()  # noqa: E731
    q, k, v, g, beta = d(q), d(k), d(v), d(g), d(beta)
    state = d(s0) if s0 is not None else torch.zeros(b, h, kd, vd, dtype=torch.float64)
    nch = (offset + t + chunk - 1) // chunk
    outs, starts = [], []
    for n in range(nch):
        lo, hi = max(0, n * chunk - offset), min(t, (n + 1) * chunk - offset)
        starts.append(state)
        qq = q[:, lo:hi] if q is not None else k[:, lo:hi]
        y, state = oracle.gdn_scan(qq, k[:, lo:hi], v[:, lo:hi], g[:, lo:hi], beta[:, lo:hi], state)
        outs.append(y)
    return torch.cat(outs, 1), torch.stack(starts, 2), state


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


CASES = [
    # (B, T, H, K, V, chunk, offset, dtype)
    (2, 9, 2, 4, 3, 3, 0, torch.float32),
    (2, 9, 2, 4, 3, 4, 2, torch.float32),
    (1, 1, 3, 32, 48, 64, 5, torch.float32),
    (1, 130, 2, 32, 48, 64, 0, torch.float32),
    (1, 70, 2, 64, 128, 64, 17, torch.float32),
    (1, 130, 1, 128, 128, 64, 0, torch.float32),
    (1, 96, 1, 128, 256, 64, 0, torch.float32),
    (1, 96, 1, 256, 128, 64, 30, torch.float32),
    (1, 130, 2, 128, 128, 64, 0, torch.bfloat16),
    (1, 64, 1, 256, 256, 64, 0, torch.bfloat16),
    # bf16 MFMA state path: K below its tile, partial 64-column tiles, offsets.
    (2, 70, 2, 32, 48, 64, 17, torch.bfloat16),
    (1, 100, 3, 64, 200, 64, 63, torch.bfloat16),
    (1, 129, 1, 256, 96, 64, 1, torch.bfloat16),
    (1, 20, 2, 48, 16, 8, 3, torch.bfloat16),
    (1, 100, 2, 64, 128, 64, 5, torch.bfloat16),
    # bf16 FMA path (K not a multiple of 16)
    (1, 40, 2, 40, 24, 16, 5, torch.bfloat16),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}T{c[1]}H{c[2]}K{c[3]}V{c[4]}C{c[5]}o{c[6]}{str(c[7])[6:]}")
def test_gdn_forward_matches_recurrence(case):
    from gpa_amd.ops import gdn_scan_hip
    b, t, h, kd, vd, chunk, offset, dtype = case
    q, k, v, g, beta, s0 = _inputs(b, t, h, kd, vd, dtype, seed=hash(case) % 1000)
    out, states, final = gdn_scan_hip(q.to(DEV), k.to(DEV), v.to(DEV), g.to(DEV), beta.to(DEV), s0.to(DEV),
                                      chunk=chunk, offset=offset)
    ref_out, ref_states, ref_final = _oracle_segments(q, k, v, g, beta, s0, chunk, offset)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    print(case, "out", _rel(out, ref_out), "states", _rel(states, ref_states), "final", _rel(final, ref_final))
    assert out.dtype == dtype
    assert _rel(out, ref_out) < tol
    assert _rel(states, ref_states) < tol
    assert _rel(final, ref_final) < tol


@pytest.mark.parametrize("case", CASES[:8] + CASES[8:], ids=lambda c: f"B{c[0]}T{c[1]}H{c[2]}K{c[3]}V{c[4]}C{c[5]}o{c[6]}{str(c[7])[6:]}")
@pytest.mark.parametrize("with_q", [True, False])
@pytest.mark.parametrize("inject", [True, False], ids=["states", "nostates"])
def test_gdn_backward_matches_autograd_of_recurrence(case, with_q, inject):
    from gpa_amd.ops import gdn_scan_hip
    b, t, h, kd, vd, chunk, offset, dtype = case
    if t > 96 and kd * vd > 128 * 128:
        pytest.skip("oracle autograd too slow at this size")
    if not inject and not (dtype == torch.bfloat16 and kd % 16 == 0):
        pytest.skip("only the MFMA state kernels have a separate no-injection build")
    q, k, v, g, beta, s0 = _inputs(b, t, h, kd, vd, dtype, seed=7 + hash(case) % 1000, q=with_q,
                                   const_gates=(kd == 32))
    gen = torch.Generator().manual_seed(3)
    nch = (offset + t + chunk - 1) // chunk
    w_out = torch.randn(b, t, h, vd, generator=gen, dtype=torch.float64)
    w_states = torch.randn(b, h, nch, kd, vd, generator=gen, dtype=torch.float64) * .1
    w_final = torch.randn(b, h, kd, vd, generator=gen, dtype=torch.float64)

    def loss(out, states, final):
        total = (final.double() * w_final.to(final.device)).sum()
        if inject:
            total = total + (states.double() * w_states.to(states.device)).sum()
        if out is not None:
            total = total + (out.double() * w_out.to(out.device)).sum()
        return total

    # HIP
    leaves = [x.to(DEV).requires_grad_() if x is not None else None for x in (q, k, v)]
    g_d = g.to(DEV).requires_grad_()
    b_d = beta.to(DEV).requires_grad_()
    s_d = s0.to(DEV).requires_grad_()
    out, states, final = gdn_scan_hip(leaves[0], leaves[1], leaves[2], g_d, b_d, s_d, chunk=chunk, offset=offset)
    loss(out, states, final).backward()
    # Oracle in float64 from the same (possibly bf16-valued) inputs.
    ref_leaves = [x.detach().double().requires_grad_() if x is not None else None for x in (q, k, v)]
    g_r = g.double().requires_grad_()
    b_r = beta.double().requires_grad_()
    s_r = s0.double().requires_grad_()
    ro, rs, rf = _oracle_segments_autograd(ref_leaves, g_r, b_r, s_r, chunk, offset)
    loss(ro if with_q else None, rs, rf).backward()
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    pairs = [("dk", leaves[1].grad, ref_leaves[1].grad), ("dv", leaves[2].grad, ref_leaves[2].grad),
             ("dg", g_d.grad, g_r.grad), ("dbeta", b_d.grad, b_r.grad), ("ds0", s_d.grad, s_r.grad)]
    if with_q:
        pairs.append(("dq", leaves[0].grad, ref_leaves[0].grad))
    errs = {name: _rel(a, r) for name, a, r in pairs}
    print(case, with_q, errs)
    assert all(e < tol for e in errs.values()), errs


def _oracle_segments_autograd(leaves, g, beta, s0, chunk, offset):
    q, k, v = leaves
    b, t, h, kd = k.shape
    vd = v.shape[-1]
    state = s0
    nch = (offset + t + chunk - 1) // chunk
    outs, starts = [], []
    for n in range(nch):
        lo, hi = max(0, n * chunk - offset), min(t, (n + 1) * chunk - offset)
        starts.append(state)
        qq = q[:, lo:hi] if q is not None else k[:, lo:hi]
        y, state = oracle.gdn_scan(qq, k[:, lo:hi], v[:, lo:hi], g[:, lo:hi], beta[:, lo:hi], state)
        outs.append(y)
    return torch.cat(outs, 1), torch.stack(starts, 2), state


# The forms of the 128-key strip state kernels, by the waves that share a
# 32-column strip: quarter (4 waves, 32-column workgroups) while its
# workgroups fit on the device's 256 CUs, split (2 waves, 64 columns) while
# those fit, else wide (1 wave, 128 columns).  The wide shapes put 288 and 576
# split workgroups in one launch; the split shapes 320 quarter and 160 split
# workgroups; the quarter shapes 128.
WIDE_FWD = [(9, 130, 16, 128, 128, 64, 0, torch.bfloat16), (3, 70, 48, 128, 256, 64, 17, torch.bfloat16)]
WIDE_BWD = [(9, 40, 16, 128, 128, 16, 5, torch.bfloat16), (1, 40, 72, 128, 256, 32, 0, torch.bfloat16)]
FORM_CASES = [("quarter", (1, 130, 32, 128, 128, 64, 0, torch.bfloat16)),
              ("quarter", (2, 40, 8, 128, 256, 16, 5, torch.bfloat16)),
              ("split", (5, 70, 16, 128, 128, 64, 17, torch.bfloat16))]


def _kernel_names(fn):
    """Names of the device kernels `fn` launches (torch profiler)."""
    from torch.profiler import ProfilerActivity, profile
    torch.cuda.synchronize()
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        fn()
        torch.cuda.synchronize()
    return {e.name for e in prof.events()}


def _form_ran(names, kind, nq):
    want = {"fwd": f"gdn_state_fwd_strip<128, true, {nq}>",
            "bwd_q": f"gdn_state_bwd_strip<128, true, true, false, {nq}>",
            "bwd_q_inj": f"gdn_state_bwd_strip<128, true, true, true, {nq}>",
            "bwd": f"gdn_state_bwd_strip<128, true, false, false, {nq}>"}[kind]
    return any(want in n for n in names)


def _wide_ran(names, kind):
    return _form_ran(names, kind, 1)


@pytest.mark.parametrize("case", WIDE_FWD, ids=lambda c: f"B{c[0]}T{c[1]}H{c[2]}V{c[4]}")
def test_wide_strip_forward_matches_recurrence(case):
    from gpa_amd.ops import gdn_scan_hip
    b, t, h, kd, vd, chunk, offset, dtype = case
    q, k, v, g, beta, s0 = _inputs(b, t, h, kd, vd, dtype, seed=11)
    res = {}

    def run():
        res["r"] = gdn_scan_hip(q.to(DEV), k.to(DEV), v.to(DEV), g.to(DEV), beta.to(DEV), s0.to(DEV), chunk=chunk,
                                offset=offset)
    names = _kernel_names(run)
    assert _wide_ran(names, "fwd"), sorted(n for n in names if "state" in n)
    out, states, final = res["r"]
    ref_out, ref_states, ref_final = _oracle_segments(q, k, v, g, beta, s0, chunk, offset)
    errs = [_rel(out, ref_out), _rel(states, ref_states), _rel(final, ref_final)]
    print(case, errs)
    assert max(errs) < 2e-2, errs


@pytest.mark.parametrize("with_q", [True, False])
@pytest.mark.parametrize("case", WIDE_BWD, ids=lambda c: f"B{c[0]}T{c[1]}H{c[2]}V{c[4]}")
def test_wide_strip_backward_matches_autograd_of_recurrence(case, with_q):
    from gpa_amd.ops import gdn_scan_hip
    b, t, h, kd, vd, chunk, offset, dtype = case
    q, k, v, g, beta, s0 = _inputs(b, t, h, kd, vd, dtype, seed=13, q=with_q)
    gen = torch.Generator().manual_seed(5)
    w_out = torch.randn(b, t, h, vd, generator=gen, dtype=torch.float64)
    w_final = torch.randn(b, h, kd, vd, generator=gen, dtype=torch.float64)

    def loss(out, final):  # no state injections: the wide backward is built without them
        total = (final.double() * w_final.to(final.device)).sum()
        return total + (out.double() * w_out.to(out.device)).sum() if out is not None else total

    leaves = [x.to(DEV).requires_grad_() if x is not None else None for x in (q, k, v)]
    g_d, b_d, s_d = (x.to(DEV).requires_grad_() for x in (g, beta, s0))
    out, states, final = gdn_scan_hip(leaves[0], leaves[1], leaves[2], g_d, b_d, s_d, chunk=chunk, offset=offset)
    names = _kernel_names(lambda: loss(out, final).backward())
    assert _wide_ran(names, "bwd_q" if with_q else "bwd"), sorted(n for n in names if "state" in n)
    ref_leaves = [x.detach().double().requires_grad_() if x is not None else None for x in (q, k, v)]
    g_r, b_r, s_r = (x.double().requires_grad_() for x in (g, beta, s0))
    ro, _, rf = _oracle_segments_autograd(ref_leaves, g_r, b_r, s_r, chunk, offset)
    loss(ro if with_q else None, rf).backward()
    pairs = [("dk", leaves[1].grad, ref_leaves[1].grad), ("dv", leaves[2].grad, ref_leaves[2].grad),
             ("dg", g_d.grad, g_r.grad), ("dbeta", b_d.grad, b_r.grad), ("ds0", s_d.grad, s_r.grad)]
    if with_q:
        pairs.append(("dq", leaves[0].grad, ref_leaves[0].grad))
    errs = {name: _rel(a, r) for name, a, r in pairs}
    print(case, with_q, errs)
    assert all(e < 2e-2 for e in errs.values()), errs


def test_wide_pack_matches_split_single_calls():
    """Nine 128-key groups in one packed call (the relation edges' shape at
    B=1, H=16: 288 split workgroups) take the wide form; one call per group
    takes the quarter form.  The two differ only in the order of the sums over
    the key rows."""
    from gpa_amd.ops import gdn_scan_hip, gdn_scan_many
    results = {}
    for packed in (True, False):
        groups = []
        for i in range(9):
            xs = _inputs(1, 130, 16, 128, 128, torch.bfloat16, 40 + i)
            groups.append([x.to(DEV).requires_grad_() if x is not None else None for x in xs])

        def fwd():
            if packed:
                return gdn_scan_many([dict(q=lv[0], k=lv[1], v=lv[2], g=lv[3], beta=lv[4], s0=lv[5], chunk=64,
                                           offset=0, deferred=False) for lv in groups])
            return [gdn_scan_hip(*lv, chunk=64, offset=0) for lv in groups]
        res = {}
        names = _kernel_names(lambda: res.setdefault("r", fwd()))
        assert _wide_ran(names, "fwd") == packed
        gen = torch.Generator().manual_seed(9)
        loss = 0.
        for out, states, final in res["r"]:
            for x in (out, final):
                if x is not None:
                    loss = loss + (x.float() * torch.randn(x.shape, generator=gen).to(DEV)).sum()
        names = _kernel_names(loss.backward)
        assert _wide_ran(names, "bwd_q") == packed
        fwd_t = [x.detach() for r in res["r"] for x in r if x is not None]
        grads = [x.grad for lv in groups for x in lv if x is not None]
        results[packed] = (fwd_t, grads)
    (fa, ga), (fb, gb) = results[True], results[False]
    for i, (a, b) in enumerate(zip(fa, fb)):
        tol = 1e-5 if a.dtype == torch.float32 else 2e-3
        assert _rel(a, b) < tol, ("forward", i, _rel(a, b))
    for i, (a, b) in enumerate(zip(ga, gb)):
        assert _rel(a, b) < 2e-3, ("grad", i, _rel(a, b))


@pytest.mark.parametrize("form,case", FORM_CASES, ids=lambda c: c if isinstance(c, str) else f"B{c[0]}H{c[2]}V{c[4]}")
def test_strip_forms_match_autograd_of_recurrence(form, case):
    """Forward and backward (read gradient and chunk-start state injections,
    as the level scans have) in the quarter and split forms, checked through
    the profiler for the form that ran."""
    from gpa_amd.ops import gdn_scan_hip
    nq = {"quarter": 4, "split": 2}[form]
    b, t, h, kd, vd, chunk, offset, dtype = case
    q, k, v, g, beta, s0 = _inputs(b, t, h, kd, vd, dtype, seed=17)
    gen = torch.Generator().manual_seed(6)
    nch = (offset + t + chunk - 1) // chunk
    w_out = torch.randn(b, t, h, vd, generator=gen, dtype=torch.float64)
    w_states = torch.randn(b, h, nch, kd, vd, generator=gen, dtype=torch.float64) * .1
    w_final = torch.randn(b, h, kd, vd, generator=gen, dtype=torch.float64)

    def loss(out, states, final):
        return ((final.double() * w_final.to(final.device)).sum() + (states.double() * w_states.to(states.device)).sum()
                + (out.double() * w_out.to(out.device)).sum())

    leaves = [x.to(DEV).requires_grad_() for x in (q, k, v)]
    g_d, b_d, s_d = (x.to(DEV).requires_grad_() for x in (g, beta, s0))
    res = {}
    names = _kernel_names(lambda: res.setdefault("r", gdn_scan_hip(*leaves, g_d, b_d, s_d, chunk=chunk,
                                                                    offset=offset)))
    assert _form_ran(names, "fwd", nq), sorted(n for n in names if "state" in n)
    out, states, final = res["r"]
    names = _kernel_names(lambda: loss(out, states, final).backward())
    assert _form_ran(names, "bwd_q_inj", nq), sorted(n for n in names if "state" in n)
    ref_leaves = [x.detach().double().requires_grad_() for x in (q, k, v)]
    g_r, b_r, s_r = (x.double().requires_grad_() for x in (g, beta, s0))
    ro, rs, rf = _oracle_segments_autograd(ref_leaves, g_r, b_r, s_r, chunk, offset)
    errs = {"out": _rel(out, ro), "states": _rel(states, rs), "final": _rel(final, rf)}
    loss(ro, rs, rf).backward()
    pairs = [("dq", leaves[0].grad, ref_leaves[0].grad), ("dk", leaves[1].grad, ref_leaves[1].grad),
             ("dv", leaves[2].grad, ref_leaves[2].grad), ("dg", g_d.grad, g_r.grad), ("dbeta", b_d.grad, b_r.grad),
             ("ds0", s_d.grad, s_r.grad)]
    errs.update({name: _rel(a, r) for name, a, r in pairs})
    print(form, case, errs)
    assert all(e < 2e-2 for e in errs.values()), errs


def test_gdn_rejects_bad_geometry_before_launch():
    from gpa_amd.ops import gdn_scan_hip
    q, k, v, g, beta, s0 = _inputs(1, 4, 1, 8, 8, torch.float32, seed=1)
    with pytest.raises(ValueError):
        gdn_scan_hip(q.to(DEV), k.to(DEV), v.to(DEV), g.to(DEV), beta.to(DEV), s0.to(DEV), chunk=65)
    with pytest.raises(ValueError):
        gdn_scan_hip(q.to(DEV), k.to(DEV), v.to(DEV), g.to(DEV), beta.to(DEV), s0.to(DEV), chunk=4, offset=4)
    big = torch.zeros(1, 4, 1, 300, device=DEV)
    with pytest.raises(ValueError):
        gdn_scan_hip(big, big, v.to(DEV), g.to(DEV), beta.to(DEV), None, chunk=4)


LATE_CASES = [
    # (B, T, H, K, V, chunk, offset)
    (1, 130, 2, 128, 128, 64, 0),
    (1, 96, 1, 256, 128, 64, 30),
    (2, 70, 2, 64, 48, 64, 17),
    (1, 20, 2, 32, 16, 8, 3),
    (1, 64, 1, 128, 256, 64, 0),
]


@pytest.mark.parametrize("case", LATE_CASES, ids=lambda c: f"B{c[0]}T{c[1]}H{c[2]}K{c[3]}V{c[4]}C{c[5]}o{c[6]}")
def test_late_read_matches_scan_with_query(case):
    """gdn_scan_deferred + read(q) against gdn_scan_hip(q, ...) and the float64
    recurrence: outputs, states and every input gradient (bf16 bar 2e-2; the
    two HIP paths agree far more closely)."""
    from gpa_amd.ops import gdn_scan_deferred, gdn_scan_hip
    b, t, h, kd, vd, chunk, offset = case
    q, k, v, g, beta, s0 = _inputs(b, t, h, kd, vd, torch.bfloat16, seed=31 + kd + vd)
    gen = torch.Generator().manual_seed(4)
    nch = (offset + t + chunk - 1) // chunk
    w_out = torch.randn(b, t, h, vd, generator=gen, dtype=torch.float64).to(DEV)
    w_states = (torch.randn(b, h, nch, kd, vd, generator=gen, dtype=torch.float64) * .1).to(DEV)
    w_final = torch.randn(b, h, kd, vd, generator=gen, dtype=torch.float64).to(DEV)

    def run(deferred):
        xs = [x.to(DEV).requires_grad_() for x in (q, k, v, g, beta, s0)]
        if deferred:
            states, final, read = gdn_scan_deferred(*xs[1:], chunk=chunk, offset=offset)
            out = read(xs[0])
        else:
            out, states, final = gdn_scan_hip(*xs, chunk=chunk, offset=offset)
        loss = ((out.double() * w_out).sum() + (states.double() * w_states).sum()
                + (final.double() * w_final).sum())
        loss.backward()
        return out, states, final, [x.grad for x in xs]

    out_d, st_d, fin_d, grads_d = run(True)
    out_p, st_p, fin_p, grads_p = run(False)
    assert torch.equal(st_d, st_p) and torch.equal(fin_d, fin_p)
    assert _rel(out_d, out_p) < 1e-6, _rel(out_d, out_p)
    names = ("dq", "dk", "dv", "dg", "dbeta", "ds0")
    close = {n: _rel(a, r) for n, a, r in zip(names, grads_d, grads_p)}
    print(case, "deferred vs plain", close)
    assert all(e < 5e-3 for e in close.values()), close
    # the float64 oracle
    ref_leaves = [x.detach().double().requires_grad_() for x in (q, k, v)]
    g_r, b_r, s_r = (x.double().requires_grad_() for x in (g, beta, s0))
    ro, rs, rf = _oracle_segments_autograd(ref_leaves, g_r, b_r, s_r, chunk, offset)
    ((ro * w_out.cpu()).sum() + (rs * w_states.cpu()).sum() + (rf * w_final.cpu()).sum()).backward()
    assert _rel(out_d, ro) < 2e-2
    refs = [ref_leaves[0].grad, ref_leaves[1].grad, ref_leaves[2].grad, g_r.grad, b_r.grad, s_r.grad]
    errs = {n: _rel(a, r) for n, a, r in zip(names, grads_d, refs)}
    print(case, "deferred vs oracle", errs)
    assert all(e < 2e-2 for e in errs.values()), errs


def test_late_read_taken_once():
    from gpa_amd.ops import gdn_scan_deferred
    q, k, v, g, beta, s0 = _inputs(1, 8, 1, 32, 16, torch.bfloat16, seed=2)
    _, _, read = gdn_scan_deferred(*(x.to(DEV) for x in (k, v, g, beta, s0)), chunk=4)
    read(q.to(DEV))
    with pytest.raises(ValueError):
        read(q.to(DEV))


# Packed groups (gpa_gdn_forward_many / gpa_gdn_backward_many): K <= 128 bf16
# groups share their strip state launches, the 256-key bf16 groups share the
# MFMA state launches, the fp32 and non-multiple-of-16 groups launch alone.
# Offsets and chunk lengths differ between groups; some groups have no
# initial state (their ds0 is written but not returned).
MANY = [
    # (B, T, H, K, V, chunk, offset, dtype, query, s0, deferred)
    (1, 130, 2, 128, 128, 64, 0, torch.bfloat16, True, True, False),
    (1, 130, 2, 128, 256, 64, 0, torch.bfloat16, False, True, True),
    (2, 70, 2, 64, 96, 64, 17, torch.bfloat16, True, False, False),
    (1, 129, 1, 256, 128, 64, 1, torch.bfloat16, True, True, False),
    (1, 100, 2, 128, 64, 32, 5, torch.bfloat16, True, True, False),
    (1, 96, 2, 256, 256, 64, 30, torch.bfloat16, True, False, False),
    (1, 130, 1, 256, 96, 64, 0, torch.bfloat16, True, True, False),
    (1, 40, 2, 40, 24, 16, 5, torch.bfloat16, True, True, False),
    (1, 70, 2, 32, 48, 64, 17, torch.float32, True, True, False),
]


def _many_groups(seed):
    groups = []
    for i, (b, t, h, kd, vd, chunk, offset, dtype, query, s0, deferred) in enumerate(MANY):
        q, k, v, g, beta, st = _inputs(b, t, h, kd, vd, dtype, seed + i, q=query, s0=s0)
        if deferred:
            qr = torch.randn(b, t, h, kd, generator=torch.Generator().manual_seed(seed + 50 + i)).to(dtype)
        else:
            qr = None
        leaves = [x.to(DEV).requires_grad_() if x is not None else None for x in (q, k, v, g, beta, st, qr)]
        groups.append((leaves, chunk, offset, deferred))
    return groups


def _many_loss(results, groups, seed):
    """A loss over every output, every chunk-start state (state injections) and
    every final state, with fixed random weights."""
    gen = torch.Generator().manual_seed(seed)
    loss = 0.
    for (leaves, _, _, deferred), res in zip(groups, results):
        if deferred:
            states, final, read = res
            out = read(leaves[6])
        else:
            out, states, final = res
        parts = [x for x in (out, states, final) if x is not None]
        for x in parts:
            wgt = torch.randn(x.shape, generator=gen).to(DEV)
            loss = loss + (x.float() * wgt).sum()
    return loss


def test_scan_many_matches_one_call_per_group():
    from gpa_amd.ops import gdn_scan_deferred, gdn_scan_hip, gdn_scan_many
    results = {}
    for packed in (True, False):
        groups = _many_groups(300)
        if packed:
            res = gdn_scan_many([dict(q=lv[0], k=lv[1], v=lv[2], g=lv[3], beta=lv[4], s0=lv[5], chunk=c, offset=o,
                                      deferred=d) for lv, c, o, d in groups])
        else:
            res = [gdn_scan_deferred(lv[1], lv[2], lv[3], lv[4], lv[5], chunk=c, offset=o) if d else
                   gdn_scan_hip(lv[0], lv[1], lv[2], lv[3], lv[4], lv[5], chunk=c, offset=o)
                   for lv, c, o, d in groups]
        loss = _many_loss(res, groups, 7)
        loss.backward()
        fwd = [x.detach() for r, (_, _, _, d) in zip(res, groups) for x in (r[:2] if d else r) if x is not None]
        grads = [x.grad for lv, _, _, _ in groups for x in lv if x is not None]
        results[packed] = (fwd, grads)
    (fa, ga), (fb, gb) = results[True], results[False]
    assert len(fa) == len(fb) and len(ga) == len(gb)
    for i, (a, b) in enumerate(zip(fa, fb)):
        assert _rel(a, b) < 1e-6, ("forward", i, _rel(a, b))
    for i, (a, b) in enumerate(zip(ga, gb)):
        assert a is not None and b is not None, ("grad", i)
        assert _rel(a, b) < 1e-5, ("grad", i, _rel(a, b))


def test_scan_many_refuses_too_many_groups():
    from gpa_amd.ops import gdn_scan_many
    q, k, v, g, beta, st = (x.to(DEV) if x is not None else None for x in _inputs(1, 8, 1, 16, 16, torch.bfloat16, 1))
    with pytest.raises(ValueError):
        gdn_scan_many([dict(q=q, k=k, v=v, g=g, beta=beta, s0=st, chunk=8)] * 13)
