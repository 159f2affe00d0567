"""Pin the counted-core oracle (oracle/paper.py) and the seeded construction of
`gpa_amd.paper_dense.PaperDenseGPA` to the reference.

Fixtures tests/golden/paper_*.npz and moment_*.npz were written by running the
reference on the CPU (tests/golden/make_paper_golden.py).  Besides them, the
oracle's recurrences are checked against closed forms that share no code with
them: the decayed sums written out over all earlier tokens.
"""
import pytest
import torch

from oracle import paper as op
from oracle import reference as oref
from tests.golden_cases import MomentCase, PaperCase, compare, compare_state, moment_names, paper_names

RTOL = {torch.float64: 1e-9, torch.float32: 2e-5, torch.bfloat16: 2e-2}


def _moment_run(case: MomentCase, x: dict):
    """The oracle on a moment fixture's inputs: (y, final, counts)."""
    axis = "value" if case.gate == "value" else "key"
    if case.gate == "none":
        y, final = oref.additive_scan(x["q"], x["k"], x["v"], x["s0"])
    else:
        y, final = op.moment_scan(x["q"], x["k"], x["v"], x["g"], x["s0"], axis=axis)
    counts = op.decayed_counts(x["p"], x["cg"], x["n0"])
    return y, final, counts


@pytest.mark.parametrize("name", moment_names())
def test_moment_oracle_matches_reference(name):
    case = MomentCase(name)
    rtol = RTOL[case.dtype]
    x = {n: t.requires_grad_() for n, t in case.inputs().items()}
    y, final, counts = _moment_run(case, x)
    errors = [compare(case, "out/y", y, rtol), compare(case, "out/final", final, rtol),
              compare(case, "out/counts", counts, rtol)]
    (y.float().square().mean() + final.float().square().mean() + counts.float().square().mean()).backward()
    g_rtol = rtol if case.dtype != torch.bfloat16 else 5e-2
    for n, t in x.items():
        assert case.has("grad/" + n) == (t.grad is not None), n
        if t.grad is not None:
            errors.append(compare(case, "grad/" + n, t.grad, g_rtol))
    assert not [e for e in errors if e], errors


def _closed_form(q, k, v, g, s0, axis):
    """y_t = sum_{s<=t} exp(G_t - G_s) o (k_s v_s^T), read with q_t, plus
    exp(G_t) o S_0, with G the inclusive cumulative log decay (elementwise on
    the decayed axis); no recurrence."""
    b, t, h, kd = q.shape
    vd = v.shape[-1]
    if g is None:
        lg = torch.zeros(b, t, h, 1, 1, dtype=q.dtype)
    elif g.ndim == 3:
        lg = g[..., None, None]
    elif axis == "value":
        lg = g[..., None, :]
    else:
        lg = g[..., :, None]
    G = lg.cumsum(1)  # [b,t,h,kd|1,vd|1]
    ys, finals = [], None
    for ti in range(t):
        s = (G[:, ti].exp() * s0).clone()
        for si in range(ti + 1):
            s = s + (G[:, ti] - G[:, si]).exp() * (k[:, si, :, :, None] * v[:, si, :, None, :])
        ys.append((q[:, ti, :, :, None] * s).sum(-2))
        finals = s
    return torch.stack(ys, 1), finals


@pytest.mark.parametrize("gate", ["none", "token", "key", "value"])
def test_moment_oracle_equals_closed_form(gate):
    g_ = torch.Generator().manual_seed(5)
    b, t, h, kd, vd = 2, 6, 3, 4, 5
    q, k = (torch.randn(b, t, h, kd, generator=g_, dtype=torch.float64) for _ in range(2))
    v = torch.randn(b, t, h, vd, generator=g_, dtype=torch.float64)
    s0 = torch.randn(b, h, kd, vd, generator=g_, dtype=torch.float64)
    shape = {"token": (b, t, h), "key": (b, t, h, kd), "value": (b, t, h, vd)}.get(gate)
    g = -torch.rand(*shape, generator=g_, dtype=torch.float64) if shape else None
    axis = "value" if gate == "value" else "key"
    y, final = op.moment_scan(q, k, v, g, s0, axis=axis)
    y2, final2 = _closed_form(q, k, v, g, s0, axis)
    torch.testing.assert_close(y, y2, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(final, final2, rtol=1e-12, atol=1e-12)
    if gate == "none":  # the DenseGPA oracle's additive scan is the same recurrence
        y3, f3 = oref.additive_scan(q, k, v, s0)
        torch.testing.assert_close(y3, y, rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(f3, final, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("vector", [False, True])
def test_decayed_counts_equal_the_cumulative_closed_form(vector):
    """n_t = exp(G_t) (n_0 + sum_{s<=t} p_s exp(-G_s)) (the reference's own two
    closed forms, paper_dense.py:50-58, evaluated independently here)."""
    g_ = torch.Generator().manual_seed(2)
    p = torch.rand(2, 7, 2, 3, generator=g_, dtype=torch.float64)
    n0 = torch.rand(2, 2, 3, generator=g_, dtype=torch.float64)
    g = -p * 2 if vector else -torch.rand(2, 7, 2, generator=g_, dtype=torch.float64) * .01
    G = g.cumsum(1) if vector else g.cumsum(1)[..., None]
    closed = G.exp() * (n0[:, None] + (p * (-G).exp()).cumsum(1))
    torch.testing.assert_close(op.decayed_counts(p, g, n0), closed, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("name", paper_names())
def test_paper_seeded_parameters_and_inputs_match_reference(name):
    case = PaperCase(name)
    model, q, k, v, ctrl = case.build()
    exact = 1e-12 if case.dtype == torch.float64 else 1e-6
    errors = [compare(case, "param/" + n, p, exact) for n, p in model.named_parameters()]
    stored = sorted(key[len("full/param/"):] if key.startswith("full/") else key[len("fp/param/"):]
                    for key in case.z if "/param/" in key)
    assert stored == sorted(n for n, _ in model.named_parameters())
    errors += [compare(case, "in/" + n, x, exact) for n, x in (("q", q), ("k", k), ("v", v), ("control", ctrl))
               if x is not None]
    assert not [e for e in errors if e], errors


@pytest.mark.parametrize("name", paper_names())
def test_paper_oracle_matches_reference(name):
    case = PaperCase(name)
    rtol = RTOL[case.dtype]
    model, q, k, v, ctrl = case.build()
    q, k, v = (x.requires_grad_() for x in (q, k, v))
    if ctrl is not None:
        ctrl.requires_grad_()
    out, state = op.forward(model, q, k, v, control_input=ctrl)
    errors = [compare(case, "out", out, rtol)] + compare_state(case, "state", state, rtol)
    out.float().square().mean().backward()
    g_rtol = rtol if case.dtype != torch.bfloat16 else 5e-2
    for n, p in model.named_parameters():
        assert case.has("grad/" + n) == (p.grad is not None), n
        if p.grad is not None:
            errors.append(compare(case, "grad/" + n, p.grad, g_rtol))
    for n, x in (("q", q), ("k", k), ("v", v), ("control", ctrl)):
        if x is not None:
            errors.append(compare(case, "grad/in_" + n, x.grad, g_rtol))
    if "partitions" in case.z:
        with torch.no_grad():
            running, parts = None, []
            for lo, hi in case.z["partitions"]:
                y, running = op.forward(model, q[:, lo:hi], k[:, lo:hi], v[:, lo:hi], running,
                                        control_input=ctrl[:, lo:hi] if ctrl is not None else None)
                parts.append(y)
            errors.append(compare(case, "partition_out", torch.cat(parts, 1), rtol))
            errors += compare_state(case, "partition_state", running, rtol)
    assert not [e for e in errors if e], errors


def test_paper_oracle_input_gradcheck():
    """The reference's gradcheck case (tests/test_paper_dense.py:43-48), on the oracle."""
    from gpa_amd.paper_dense import PaperConfig, PaperDenseGPA
    torch.manual_seed(4)
    model = PaperDenseGPA(PaperConfig(heads=1, key_dim=2, value_dim=2, slots=(2, 2), chunk_size=2)).double()
    xs = tuple(torch.randn(1, 2, 1, 2, dtype=torch.double, requires_grad=True) for _ in range(3))
    assert torch.autograd.gradcheck(lambda *x: op.forward(model, *x)[0], xs, atol=2e-4, rtol=2e-3)
