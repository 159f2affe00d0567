"""The reference-signature operators on the GPU vs the oracle (reference
src/gpa/ops.py:29-85, 140-163): gdn_scan, gdn_update, memory_read and
two_stage_gdn, in float32 (1e-4 relative) and bfloat16 (2e-2 relative)."""
import pytest
import torch

import oracle
from gpa_amd import TwoStageState, two_stage_gdn
from gpa_amd.ops import gdn_scan, gdn_update, memory_read
from tests.golden_cases import TwoStageCase, ops_names

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _scan_inputs(b, t, h, kd, vd, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, t, h, kd, generator=g).to(dtype)
    k = torch.randn(b, t, h, kd, generator=g).to(dtype)
    v = torch.randn(b, t, h, vd, generator=g).to(dtype)
    gate = -torch.rand(b, t, h, generator=g) * .3
    beta = torch.rand(b, t, h, generator=g)
    s0 = torch.randn(b, h, kd, vd, generator=g) * .2
    return q, k, v, gate, beta, s0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_gdn_scan_reference_signature(dtype):
    q, k, v, g, beta, s0 = _scan_inputs(2, 150, 3, 32, 24, dtype, 0)
    out, final = gdn_scan(*(x.to(DEV) for x in (q, k, v, g, beta, s0)))
    ref_out, ref_final = oracle.gdn_scan(q.double(), k.double(), v.double(), g.double(), beta.double(),
                                         s0.double())
    assert out.dtype == dtype and final.dtype == torch.float32
    assert _rel(out, ref_out) < TOL[dtype] and _rel(final, ref_final) < TOL[dtype]


def test_gdn_scan_empty_returns_initial_state():
    q, k, v, g, beta, s0 = _scan_inputs(1, 0, 2, 8, 4, torch.float32, 1)
    s0 = s0.to(DEV)
    out, final = gdn_scan(q.to(DEV), k.to(DEV), v.to(DEV), g.to(DEV), beta.to(DEV), s0)
    assert out.shape == (1, 0, 2, 4) and final is s0


def test_gdn_update_and_memory_read_match_one_step():
    q, k, v, g, beta, s0 = _scan_inputs(2, 1, 3, 16, 8, torch.float32, 2)
    s1 = gdn_update(s0.to(DEV), k[:, 0].to(DEV), v[:, 0].to(DEV), g[:, 0].to(DEV), beta[:, 0].to(DEV))
    ref = oracle.gdn_step(s0.double(), k[:, 0].double(), v[:, 0].double(), g[:, 0].double(), beta[:, 0].double())
    assert _rel(s1, ref) < 1e-5
    y = memory_read(q[:, 0].to(DEV), s1)
    assert _rel(y, oracle.gdn_read(q[:, 0].double(), ref)) < 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_two_stage_gdn_matches_oracle(dtype):
    b, t, h, dk, m, dv = 1, 70, 2, 16, 12, 10
    gen = torch.Generator().manual_seed(3)
    q = torch.randn(b, t, h, dk, generator=gen).to(dtype)
    k = torch.randn(b, t, h, dk, generator=gen).to(dtype)
    slots = torch.randn(b, t, h, m, generator=gen).to(dtype)
    v = torch.randn(b, t, h, dv, generator=gen).to(dtype)
    gates = [-torch.rand(b, t, h, generator=gen) * .2, torch.rand(b, t, h, generator=gen),
             -torch.rand(b, t, h, generator=gen) * .2, torch.rand(b, t, h, generator=gen)]
    inner = torch.randn(b, h, dk, m, generator=gen) * .1
    outer = torch.randn(b, h, m, dv, generator=gen) * .1
    rw = torch.randn(m, m, generator=gen) / m ** .5
    qw = torch.randn(m, dk, generator=gen) / dk ** .5
    out, st = two_stage_gdn(q.to(DEV), k.to(DEV), slots.to(DEV), v.to(DEV), *(x.to(DEV) for x in gates),
                            TwoStageState(inner.to(DEV), outer.to(DEV)), route_weight=rw.to(DEV),
                            query_weight=qw.to(DEV))
    ref_out, ref_a, ref_b = oracle.two_stage(q, k, slots, v, *gates, inner, outer, route_weight=rw,
                                             query_weight=qw)
    tol = TOL[dtype]
    assert _rel(out, ref_out) < tol and _rel(st.inner, ref_a) < tol and _rel(st.outer, ref_b) < tol


@pytest.mark.parametrize("name", ops_names("ops_two_stage"))
def test_two_stage_gdn_reproduces_reference_fixture(name):
    """HIP two_stage_gdn against the reference's own two_stage_gdn results
    (tests/golden/ops_two_stage_*.npz): output, both final states and the
    gradient of every input.  A float64 fixture runs in float32 at 1e-4."""
    case = TwoStageCase(name)
    dtype = torch.float32 if case.dtype == torch.float64 else case.dtype
    tol = TOL[dtype]
    x = {n: t.to(DEV).requires_grad_() for n, t in case.inputs(dtype).items()}
    out, st = two_stage_gdn(x["q"], x["k"], x["slots"], x["v"], x["gi"], x["bi"], x["go"], x["bo"],
                            TwoStageState(x["inner"], x["outer"]), route_weight=x.get("route_weight"),
                            query_weight=x.get("query_weight"))
    out.float().square().mean().backward()
    errors = {label: _rel(got, case.ref(label)) for label, got in (("out", out), ("inner", st.inner),
                                                                  ("outer", st.outer))}
    for n, t in x.items():
        errors["grad/" + n] = _rel(t.grad, case.ref("grad/" + n))
    print(name, "worst", max(errors.items(), key=lambda kv: kv[1]))
    bad = {k: e for k, e in errors.items() if e > tol}
    assert not bad, bad


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("n", [1, 2, 6, 8, 11])
def test_sum_many_matches_float32_sum(n, dtype):
    """gpa_sum_many (the packed backward's gradient sum of a shared input):
    float32 accumulation and one rounding, bit for bit against torch's float32
    sum rounded once; more than 8 sources in several passes."""
    from gpa_amd.ops import _sum_many
    g = torch.Generator().manual_seed(n)
    xs = [torch.randn(3, 40, 2, 16, generator=g).to(dtype).to("cuda") for _ in range(n)]
    got = _sum_many(xs)
    want = torch.stack([x.float() for x in xs]).sum(0)
    assert got.shape == want.shape and got.dtype == dtype
    err = (got.float() - want).abs()
    if dtype == torch.float32:
        assert (err <= 1e-6 * want.abs() + 1e-6).all()
    else:  # one rounding per pass (8 sources, then the partial sum and the rest): half an ulp each
        bound = 2 ** -8 * want.abs()
        if n > 8:
            bound = bound + 2 ** -8 * torch.stack([x.float() for x in xs[:8]]).sum(0).abs()
        assert (err <= bound + 1e-6).all()


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("levels,b,t,h,dv", [(4, 1, 70, 2, 24), (3, 2, 33, 16, 128), (1, 1, 5, 3, 8)])
def test_output_mix_train_matches_device_ops(levels, b, t, h, dv, dtype):
    """The trainable output mix (attention.py:340-341) against the same sum as
    device tensor operations: output bit for bit; the reads' gradients bit for
    bit (each one product rounded once), the weights' gradient to float32
    summation order."""
    from gpa_amd import glue
    g = torch.Generator().manual_seed(levels * 100 + t)
    reads = [torch.randn(b, t, h, dv, generator=g).to(dtype).cuda().requires_grad_() for _ in range(levels)]
    assert glue.output_mix_supported(reads)
    assert not glue.output_mix_supported([torch.zeros(b, t, h, 7, dtype=dtype, device="cuda")])
    logits = torch.randn(levels, h, generator=g).cuda().requires_grad_()
    dout = torch.randn(b, t, h, dv, generator=g).to(dtype).cuda()
    out = glue.output_mix_train(reads, logits.softmax(0))
    out.backward(dout)
    got = [out.detach()] + [r.grad.clone() for r in reads] + [logits.grad.clone()]
    for r in reads:
        r.grad = None
    logits.grad = None
    w = logits.softmax(0)
    ref = 0
    for j, r in enumerate(reads):
        ref = ref + w[j][..., None] * r
    ref = ref.to(dtype)
    ref.backward(dout)
    want = [ref.detach()] + [r.grad for r in reads] + [logits.grad]
    assert torch.equal(got[0], want[0])
    for a, r in zip(got[1:-1], want[1:-1]):
        assert torch.equal(a, r)
    assert torch.allclose(got[-1], want[-1], rtol=1e-5, atol=1e-6)  # one level: the softmax's gradient is 0


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("shape", [(2, 33, 3, 7), (1, 64, 16, 128), (1, 20, 2, 256), (3, 5, 1, 1000)])
def test_row_softmax_matches_device_ops(shape, dtype):
    """softmax(logits).to(dtype) of the local read distribution (attention.py:330)
    and its gradient against the same device ops: float32 to 1e-6 (the exp and
    the summation order), bf16 within one rounding."""
    from gpa_amd import glue
    g = torch.Generator().manual_seed(shape[-1])
    x = (torch.randn(*shape, generator=g) * 3).cuda().requires_grad_()
    dy = torch.randn(*shape, generator=g).to(dtype).cuda()
    y = glue.softmax_rows(x, dtype)
    y.backward(dy)
    gx = x.grad.clone()
    x.grad = None
    ref = x.softmax(-1).to(dtype)
    ref.backward(dy)
    assert y.dtype == dtype and y.shape == ref.shape
    if dtype == torch.float32:
        assert torch.allclose(y, ref, rtol=1e-6, atol=1e-7)
    else:
        assert ((y.float() - ref.float()).abs() <= 2 ** -8 * ref.float().abs() + 1e-7).all()
    assert ((gx - x.grad).norm() / x.grad.norm()).item() < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("decay_scale", [1.0, 0.01, 0.0])
def test_gate_act_train_matches_device_ops(dtype, decay_scale):
    """The gate nonlinearities with their gradient (attention.py:166-174)
    against the reference's device ops: decays -min(softplus(x), 10) * scale
    (inputs spanning the clamp and the softplus threshold), strengths
    beta_max sigmoid(x); gradients of the gate inputs and of the bias."""
    import torch.nn.functional as F
    from gpa_amd import glue
    g = torch.Generator().manual_seed(7)
    b, t, h = 2, 300, 5
    raw = (torch.randn(b, t, h, 4, generator=g) * 8).to(dtype).cuda().requires_grad_()
    bias = torch.randn(h, 4, generator=g).cuda().requires_grad_()
    ws = [torch.randn(b, t, h, generator=g).cuda() for _ in range(4)]
    outs = glue.gate_act_train(raw, bias, .9, decay_scale)
    sum((o * w).sum() for o, w in zip(outs, ws)).backward()
    got = [o.detach() for o in outs] + [raw.grad.clone(), bias.grad.clone()]
    raw.grad = bias.grad = None
    x = raw.float() + bias
    gi, bi, go, bo = x.unbind(-1)
    ref = (-F.softplus(gi).clamp(max=10.) * decay_scale, .9 * bi.sigmoid(),
           -F.softplus(go).clamp(max=10.) * decay_scale, .9 * bo.sigmoid())
    sum((o * w).sum() for o, w in zip(ref, ws)).backward()
    want = [o.detach() for o in ref] + [raw.grad, bias.grad]
    for i, (a, r) in enumerate(zip(got, want)):
        scale = r.abs().max().item()
        if i == 4 and dtype == torch.bfloat16:  # one rounding of the input gradient
            assert ((a.float() - r.float()).abs() <= 2 ** -8 * r.float().abs() + 1e-6 * max(scale, 1e-30)).all(), i
        else:
            assert (a.float() - r.float()).abs().max().item() <= 1e-5 * max(scale, 1e-30) + 1e-7, i
