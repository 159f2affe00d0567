"""The gated moment-scan kernel and the counted dense core (`PaperDenseGPA`) on
the GPU, through the C ABI:

- `gpa_amd.moment.moment_scan` / `decayed_counts` against the reference's own
  numbers (tests/golden/moment_*.npz: outputs, final state and every input
  gradient; the float64 fixtures run in float32 here) and against the oracle's
  per-token recurrence for every shape class of the kernel, every decay form,
  long sequences, float32 (1e-4) and bfloat16 (2e-2);
- `PaperDenseGPA` against the oracle on the same parameters and inputs
  (output, carried state, every parameter and input gradient) for every read
  mode of the reference's tests, and against the reference's fixtures
  (tests/golden/paper_*.npz); cached-call partitions equal one call.
"""
import pytest
import torch

from gpa_amd import moment
from gpa_amd.paper_dense import PaperConfig, PaperDenseGPA
from gpa_amd.state import tensors
from oracle import paper as op
from oracle import reference as oref
from tests.golden_cases import MomentCase, PaperCase, compare, compare_state, moment_names, paper_names

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / max(b.norm().item(), 1e-30)).item()


@pytest.mark.parametrize("name", moment_names())
def test_moment_kernel_matches_reference_fixtures(name):
    case = MomentCase(name)
    dtype = torch.float32 if case.dtype == torch.float64 else case.dtype
    rtol = 2e-4 if dtype == torch.float32 else 2e-2
    print(f"moment fixture {name} as {dtype}", flush=True)
    x = {n: t.to(DEV).requires_grad_() for n, t in case.inputs(dtype, DEV).items()}
    axis = "value" if case.gate == "value" else "key"
    y, final = moment.moment_scan(x["q"], x["k"], x["v"], x.get("g"), x["s0"], axis=axis)
    counts = moment.decayed_counts(x["p"], x["cg"], x["n0"])
    errors = [compare(case, "out/y", y, rtol), compare(case, "out/final", final, rtol),
              compare(case, "out/counts", counts, rtol)]
    (y.float().square().mean() + final.float().square().mean() + counts.float().square().mean()).backward()
    g_rtol = rtol if dtype == torch.float32 else 5e-2
    for n, t in x.items():
        assert case.has("grad/" + n) == (t.grad is not None), n
        if t.grad is not None:
            errors.append(compare(case, "grad/" + n, t.grad, g_rtol))
    assert not [e for e in errors if e], errors


CASES = [  # (b, t, h, k, v, gate, s0)
    (2, 300, 2, 3, 5, "none", "full"), (1, 257, 3, 16, 64, "token", "broadcast"),
    (2, 200, 1, 32, 100, "key", "full"), (1, 130, 2, 48, 16, "value", None),
    (1, 1, 1, 64, 64, "key", "full"), (1, 333, 2, 128, 128, "value", "full"),
    (1, 129, 1, 100, 200, "token", "full"), (1, 96, 1, 256, 256, "key", "broadcast"),
    (1, 70, 2, 200, 33, "none", None),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("b,t,h,k,v,gate,s0", CASES)
def test_moment_kernel_forward_backward_against_oracle(b, t, h, k, v, gate, s0, dtype):
    print(f"moment b={b} t={t} h={h} k={k} v={v} gate={gate} s0={s0} {dtype}", flush=True)
    g_ = torch.Generator().manual_seed(b * 1000 + t + k)
    q = torch.randn(b, t, h, k, generator=g_).to(dtype)
    kk = torch.randn(b, t, h, k, generator=g_).to(dtype) / k ** .5
    vv = torch.randn(b, t, h, v, generator=g_).to(dtype)
    shape = {"token": (b, t, h), "key": (b, t, h, k), "value": (b, t, h, v)}.get(gate)
    g = -torch.rand(*shape, generator=g_) * .05 if shape else None
    init = {"full": torch.randn(b, h, k, v, generator=g_) * .3,
            "broadcast": (torch.randn(1, h, k, v, generator=g_) * .3).expand(b, h, k, v),
            None: torch.zeros(b, h, k, v)}[s0]
    wy = torch.randn(b, t, h, v, generator=g_)
    wf = torch.randn(b, h, k, v, generator=g_)
    axis = "value" if gate == "value" else "key"

    def run(fn, dev, init_):
        xs = [x.detach().to(dev).requires_grad_() for x in (q, kk, vv)]
        gg = g.detach().to(dev).requires_grad_() if g is not None else None
        s = init_.detach().to(dev).requires_grad_()
        y, final = fn(*xs, gg, s, axis=axis)
        ((y.float() * wy.to(dev)).sum() + (final.float() * wf.to(dev)).sum()).backward()
        return [y, final] + [x.grad for x in xs] + [gg.grad if gg is not None else None, s.grad]

    got = run(moment.moment_scan, DEV, init)
    want = run(op.moment_scan, "cpu", init.float())
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    for name, a, r in zip(("y", "final", "dq", "dk", "dv", "dg", "ds0"), got, want):
        if r is None:
            assert a is None, name
            continue
        assert torch.isfinite(a).all(), name
        assert _rel(a, r) < tol, (name, _rel(a, r))


def test_linear_scan_uses_the_kernel_and_matches_the_oracle():
    """positional moments (reference ops.py:88-118) through the kernel."""
    from gpa_amd.positional import linear_scan
    g_ = torch.Generator().manual_seed(9)
    q, k = (torch.randn(1, 150, 2, 32, generator=g_).bfloat16() for _ in range(2))
    v = torch.randn(1, 150, 2, 40, generator=g_).bfloat16()
    s0 = torch.randn(1, 2, 32, 40, generator=g_)
    y, final = linear_scan(q.to(DEV), k.to(DEV), v.to(DEV), s0.to(DEV))
    ry, rf = oref.additive_scan(q, k, v, s0)
    assert _rel(final, rf) < 1e-5 and _rel(y, ry) < 1e-2


def _paper_pair(case: PaperCase):
    """The fixture's model and inputs in float32 (or its bf16) on the GPU and,
    with the same parameters, on the CPU for the oracle."""
    model, q, k, v, ctrl = case.build()
    dtype = torch.float32 if case.dtype == torch.float64 else case.dtype
    model = model.float()
    gpu = PaperDenseGPA(model.config).to(DEV)
    gpu.load_state_dict(model.state_dict())
    xs = [x.to(dtype) if x is not None else None for x in (q, k, v, ctrl)]
    return model, gpu, xs, dtype


@pytest.mark.parametrize("name", paper_names())
def test_paper_module_matches_oracle_and_reference(name):
    case = PaperCase(name)
    print(f"paper case {name}", flush=True)
    cpu_model, model, xs, dtype = _paper_pair(case)
    xg = [x.to(DEV).requires_grad_() if x is not None else None for x in xs]
    xc = [x.clone().requires_grad_() if x is not None else None for x in xs]
    out, state = model(*xg[:3], control_input=xg[3])
    rout, rstate = op.forward(cpu_model, *xc[:3], control_input=xc[3])
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    errors = []
    if _rel(out, rout) > tol:
        errors.append(("out", _rel(out, rout)))
    for i, (a, r) in enumerate(zip(tensors(state), tensors(rstate))):
        if _rel(a, r) > tol:
            errors.append((f"state {i}", _rel(a, r)))
    out.float().square().mean().backward()
    rout.float().square().mean().backward()
    for (n, p), (_, rp) in zip(model.named_parameters(), cpu_model.named_parameters()):
        assert (p.grad is None) == (rp.grad is None), n
        if p.grad is not None and _rel(p.grad, rp.grad) > (tol if dtype == torch.float32 else 5e-2):
            errors.append((n, _rel(p.grad, rp.grad)))
    for n, a, r in zip(("q", "k", "v", "control"), xg, xc):
        if a is not None and _rel(a.grad, r.grad) > (tol if dtype == torch.float32 else 5e-2):
            errors.append(("in_" + n, _rel(a.grad, r.grad)))
    # and against the reference's own numbers (float32 and bf16 fixtures at their precision)
    if case.dtype != torch.float64:
        rtol = 2e-4 if dtype == torch.float32 else 2e-2
        fixture = [compare(case, "out", out, rtol)] + compare_state(case, "state", state, rtol)
        errors += [e for e in fixture if e]
    assert not errors, errors


def test_paper_partitions_equal_one_call_and_decode():
    torch.manual_seed(3)
    cfg = PaperConfig(heads=2, key_dim=32, value_dim=32, slots=(16, 16, 16), chunk_size=16,
                      dense_read="transport", slot_decay=True)
    model = PaperDenseGPA(cfg).to(DEV)
    q, k, v = (torch.randn(1, 61, 2, 32, device=DEV) for _ in range(3))
    with torch.no_grad():
        y, state = model(q, k, v)
        running, parts = None, []
        for lo, hi in ((0, 5), (5, 16), (16, 40), (40, 41), (41, 61)):
            yy, running = model(q[:, lo:hi], k[:, lo:hi], v[:, lo:hi], running)
            parts.append(yy)
    assert _rel(torch.cat(parts, 1), y) < 1e-5
    for a, r in zip(tensors(running), tensors(state)):
        assert _rel(a, r) < 1e-5
    assert running.position == 61 and running.chunk_offset == 61 % 16 and running.frozen is not None
