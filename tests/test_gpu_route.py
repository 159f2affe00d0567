"""Route reader (gpa_route_forward / gpa_route_backward / gpa_route_weight_grads,
csrc/route_reader.hip) through the C ABI: the tiled bf16 path (row kernels
and 128-row MFMA products, taken when the widths are multiples of 64 and the
q, route and qo rows are uniformly strided) against the one-kernel path of the
same library on the same values (taken when q's rows are not uniformly
strided: a [B, T+1, H, Dk] buffer viewed as [B, T, H, Dk]).  Both round where
the reference's bf16 einsums round and contract in the same order, so every
output and saved row must agree bit for bit.  Calls with fewer than 1024 rows (one-token decode) keep the one-kernel
path.  The one-kernel path is itself
pinned to the oracle by the module tests (test_gpu_dense_gpa.py) and the
host-built kernel tests (test_route_emulated.py)."""
import pytest
import torch

from gpa_amd import _lib
from gpa_amd import route as rt

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


def _inputs(b, t, h, m, dk, n_in, seed):
    g = torch.Generator().manual_seed(seed)
    base = torch.randn(b, t, h, m, generator=g)
    q = torch.randn(b, t, h, dk, generator=g).to(BF)
    msgs = [torch.randn(b, t, h, m, generator=g).to(BF) for _ in range(n_in)]
    ew = torch.softmax(torch.randn(n_in, h, generator=g), 0) if n_in else torch.zeros(0, h)
    gain = torch.rand(h, generator=g) + .5
    mg = torch.rand(h, generator=g) + .5
    up = torch.randn(h, m, 2 * m, generator=g) / m ** .5
    down = torch.randn(h, 2 * m, m, generator=g) / (2 * m) ** .5
    rs = torch.eye(m).expand(h, m, m) + .05 * torch.randn(h, m, m, generator=g)
    qs = torch.randn(h, dk, m, generator=g) / dk ** .5
    return [x.to(DEV) for x in (base, q, ew, gain, mg, up, down, rs, qs)], [x.to(DEV) for x in msgs]


def _strided_copy(x):
    """The same values in a [B, T+1, ...] buffer, viewed as [B, T, ...]: the
    rows are then not uniformly strided when B > 1."""
    big = torch.zeros(x.shape[0], x.shape[1] + 1, *x.shape[2:], device=x.device, dtype=x.dtype)
    big[:, :x.shape[1]] = x
    return big[:, :x.shape[1]]


def _forward(args, msgs, q, query_scale=1 / 16):
    base, _, ew, gain, mg, up, down, rs, qs = args
    lib = _lib.load()
    b, t, h, _ = q.shape
    m = base.shape[-1]
    weights = {"up_t": rt._pack(up, BF, True), "down_t": rt._pack(down, BF, True),
               "rs_t": rt._pack(rs, BF, True), "qs_t": rt._pack(qs, BF, True)}
    qo = torch.empty(b, t, h, m, device=DEV, dtype=BF)
    route = torch.empty_like(qo)
    saved = tuple(torch.empty(h, b * t, w, device=DEV, dtype=BF) for w in (m, 2 * m, m))
    prob = rt._problem(base.contiguous(), q, ew.contiguous(), gain, mg, msgs, query_scale, weights,
                       (qo, route), saved)
    _lib.check(lib.gpa_route_forward(prob, _lib.stream_handle(q.device)), "gpa_route_forward")
    torch.cuda.synchronize()
    return {"qo": qo, "route": route, "r0": saved[0], "h1": saved[1], "hd": saved[2]}


# (rows b*t >= 1024 take the tiled path; none is a multiple of the 128-row tile)
SHAPES = [(2, 600, 3, 128, 128, 3), (2, 530, 2, 256, 128, 3), (2, 513, 2, 64, 64, 1), (2, 515, 1, 128, 64, 0)]


@pytest.mark.parametrize("b,t,h,m,dk,n_in", SHAPES)
def test_tiled_route_forward_matches_one_kernel_path(b, t, h, m, dk, n_in):
    args, msgs = _inputs(b, t, h, m, dk, n_in, seed=b * 100 + t + m)
    q = args[1]
    tiled = _forward(args, msgs, q)
    fused = _forward(args, msgs, _strided_copy(q))
    for name, x in tiled.items():
        y = fused[name]
        assert torch.equal(x, y), f"{name}: max |diff| {(x.float() - y.float()).abs().max().item()}"
    assert torch.isfinite(tiled["qo"].float()).all()


def _backward(args, msgs, q, fwd, dqo, droute, query_scale=1 / 16):
    base, _, ew, gain, mg, up, down, rs, qs = args
    lib = _lib.load()
    b, t, h, dk = q.shape
    m = base.shape[-1]
    rows = b * t
    weights = {"up": rt._pack(up, BF, False), "down": rt._pack(down, BF, False),
               "rs": rt._pack(rs, BF, False), "qs": rt._pack(qs, BF, False)}
    saved = (fwd["r0"], fwd["h1"], fwd["hd"])
    prob = rt._problem(base.contiguous(), q, ew.contiguous(), gain, mg, msgs, query_scale, weights,
                       (fwd["route"], fwd["route"]), saved)
    out = {"dbase": torch.empty(b, t, h, m, device=DEV), "dq": torch.empty(b, t, h, dk, device=DEV, dtype=BF),
           "dh1": torch.empty(h, rows, 2 * m, device=DEV, dtype=BF),
           "dhd": torch.empty(h, rows, m, device=DEV, dtype=BF),
           "dqs": torch.empty(h, rows, m, device=DEV, dtype=BF),
           "hg": torch.empty(h, rows, 2 * m, device=DEV, dtype=BF),
           "partials": torch.full(((rows + _lib.ROUTE_ROWS - 1) // _lib.ROUTE_ROWS, h, 2 + len(msgs)), float("nan"),
                                  device=DEV)}
    dmsgs = [torch.empty_like(x) for x in msgs]
    gr = _lib.RouteGrads()
    gr.dqo, gr.droute = _lib.operand(dqo), _lib.operand(droute)
    gr.dbase, gr.dq = _lib.operand(out["dbase"]), _lib.operand(out["dq"])
    for e, x in enumerate(dmsgs):
        gr.dmsg[e] = _lib.operand(x)
    gr.dh1, gr.dhd, gr.dqs = out["dh1"].data_ptr(), out["dhd"].data_ptr(), out["dqs"].data_ptr()
    gr.hg, gr.partials = out["hg"].data_ptr(), out["partials"].data_ptr()
    _lib.check(lib.gpa_route_backward(prob, gr, _lib.stream_handle(q.device)), "gpa_route_backward")
    torch.cuda.synchronize()
    for e, x in enumerate(dmsgs):
        out[f"dmsg{e}"] = x
    return out


@pytest.mark.parametrize("b,t,h,m,dk,n_in,with_droute", [s + (i % 2 == 0,) for i, s in enumerate(SHAPES)])
def test_tiled_route_backward_matches_one_kernel_path(b, t, h, m, dk, n_in, with_droute):
    """d base, d messages, d q, the saved gradient rows and every partial sum
    agree bit for bit, except d mlp_gain's partials (slot 0), which the tiled
    path sums over a block's rows in another order (relative 1e-5)."""
    args, msgs = _inputs(b, t, h, m, dk, n_in, seed=7 * b + t + m)
    q = args[1]
    fwd = _forward(args, msgs, q)
    g = torch.Generator().manual_seed(t)
    dqo = torch.randn(b, t, h, m, generator=g).to(BF).to(DEV)
    droute = torch.randn(b, t, h, m, generator=g).to(BF).to(DEV) if with_droute else None
    tiled = _backward(args, msgs, q, fwd, dqo, droute)
    fused = _backward(args, msgs, _strided_copy(q), fwd, dqo, droute)
    for name, x in tiled.items():
        y = fused[name]
        if name == "partials":
            assert torch.equal(x[..., 1:], y[..., 1:]), "partials of d gain / d w_e"
            assert torch.allclose(x[..., 0], y[..., 0], rtol=1e-5, atol=1e-6 * y[..., 0].abs().max().item())
            assert torch.isfinite(x).all()
        else:
            assert torch.equal(x, y), f"{name}: max |diff| {(x.float() - y.float()).abs().max().item()}"


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / max(b.norm().item(), 1e-30)).item()


def _product_ref(base, gexp, w, msgs, norms, counts):
    """The product relation read as the reference's tensor ops (attention.py:
    231-236), with the messages promoted from their dtype as there."""
    total = 0
    for e, (msg, n) in enumerate(zip(msgs, norms)):
        total = total + w[e][..., None] * msg * n[..., None]
    out = base + base.shape[-1] * gexp[..., None] * total
    if counts is not None:
        out = out - gexp[..., None] * counts.log1p()
    return out


@pytest.mark.parametrize("dtype", [torch.float32, BF], ids=["f32", "bf16"])
@pytest.mark.parametrize("b,t,h,m,n_in,marginal", [(2, 9, 3, 128, 3, True), (1, 130, 2, 256, 2, False),
                                                   (3, 5, 2, 12, 1, True), (64, 1, 16, 128, 3, True)])
def test_product_read_matches_reference_ops_with_gradients(b, t, h, m, n_in, marginal, dtype):
    """gpa_product_read_forward / _backward against the reference's tensor ops
    (float32 autograd on the CPU): output to 1e-6, and the gradients of the
    base, gain factor, edge weights, messages, norms and counts (1e-5 in
    float32; messages rounded to bfloat16 at 2e-2)."""
    g = torch.Generator().manual_seed(b * 31 + m + n_in)
    base = torch.randn(b, t, h, m, generator=g)
    gexp = torch.rand(h, generator=g) + .5
    w = torch.softmax(torch.randn(n_in, h, generator=g), 0)
    msgs = [torch.randn(b, t, h, m, generator=g).to(dtype) for _ in range(n_in)]
    norms = [torch.rand(b, t, h, generator=g) + .1 for _ in range(n_in)]
    counts = torch.rand(b, t, h, m, generator=g) * 9 if marginal else None
    dout = torch.randn(b, t, h, m, generator=g)
    ins = [base, gexp, w] + msgs + norms + ([counts] if marginal else [])
    ref_in = [x.clone().requires_grad_() for x in ins]
    hip_in = [x.to(DEV).requires_grad_() for x in ins]

    def split(xs):
        return xs[0], xs[1], xs[2], xs[3:3 + n_in], xs[3 + n_in:3 + 2 * n_in], (xs[-1] if marginal else None)

    ref = _product_ref(*split(ref_in))
    ref.backward(dout)
    got = rt.product_read(*split(hip_in))
    got.backward(dout.to(DEV))
    assert got.dtype == torch.float32 and got.shape == ref.shape
    assert _rel(got, ref) < 1e-6
    for i, (a, r) in enumerate(zip(hip_in, ref_in)):
        tol = 2e-2 if a.dtype == BF else 1e-5
        assert a.grad is not None and a.grad.dtype == r.grad.dtype, i
        assert _rel(a.grad, r.grad) < tol, (i, _rel(a.grad, r.grad))


LM_FLAGS = dict(rsa_update=True, balanced_bridge=True, paper_product_read=True, shared_query_center=True)


def _bridge_run(model, logits, incoming, q):
    """Routes, query outputs and every gradient of schedule._bridge under a
    seeded random loss."""
    from gpa_amd import schedule
    logits = [x.clone().requires_grad_() for x in logits]
    incoming = [[(e, m.clone().requires_grad_()) for e, m in group] for group in incoming]
    q = q.clone().requires_grad_()
    model.zero_grad(set_to_none=True)
    routes, queries = schedule._bridge(model, q, logits, incoming, [None] * len(logits))
    gen = torch.Generator(device=DEV).manual_seed(7)
    loss = sum((x.float() * torch.randn(x.shape, generator=gen, device=DEV)).sum() for x in routes + queries)
    loss.backward()
    grads = {f"logits{j}": x.grad for j, x in enumerate(logits)}
    grads.update({f"msg{e}": m.grad for group in incoming for e, m in group})
    grads["q"] = q.grad
    grads.update({n: p.grad for n, p in model.named_parameters() if p.grad is not None})
    return list(routes) + list(queries), grads


@pytest.mark.parametrize("t", [6, 1040], ids=["one_kernel", "tiled"])
@pytest.mark.parametrize("flags", [dict(rsa_update=True), dict(balanced_bridge=True), LM_FLAGS],
                         ids=["rsa", "balanced", "lm_flags"])
def test_route_flags_match_the_device_glue(flags, t, monkeypatch):
    """rsa_update's L1 rescale and balanced_bridge's unit mix inside the HIP
    route reader (attention.py:251-259), alone and with the LM flag set, at
    C3 widths in bf16, against the schedule's device glue (the reference's
    typed torch expressions) for the same read: every route and query output
    and the gradients of the logits, messages, q and every parameter
    (bridge_mix_raw included), relative L2 2e-2.  6 rows take the one-kernel
    reader, 1040 rows the tiled products with the flags' row kernels."""
    from gpa_amd import DenseGPA, GPAConfig, schedule
    torch.manual_seed(3)
    cfg = GPAConfig(heads=2, key_dim=128, value_dim=128, slots=(128, 128, 128, 256), chunk_size=64, **flags)
    model = DenseGPA(cfg).to(DEV)
    with torch.no_grad():
        for group in (model.route_weight, model.route_down):
            for w in group:
                w.add_(torch.randn_like(w) * .3)
        model.edge_logits.normal_(0, .7)
        model.relation_gain.normal_(0, .5)
        model.route_mlp_gain.normal_(.5, .2)
        if cfg.balanced_bridge:
            model.bridge_mix_raw.normal_(0, 1.)
        for w in model.query_weight:
            w.normal_(0, .05)
    g = torch.Generator(device=DEV).manual_seed(4)
    logits = [torch.randn(1, t, 2, m, generator=g, device=DEV) * 2 for m in cfg.slots]
    incoming = [[] for _ in cfg.slots]
    for e, (i, j) in enumerate(model.edges):
        incoming[j].append((e, torch.randn(1, t, 2, cfg.slots[j], generator=g, device=DEV).to(BF)))
    q = torch.randn(1, t, 2, 128, generator=g, device=DEV).to(BF)
    assert schedule.fused_route_supported(cfg, BF, 256)
    monkeypatch.setattr(schedule, "_FUSED_ROUTE", [False])
    ref_out, ref_grads = _bridge_run(model, logits, incoming, q)
    monkeypatch.setattr(schedule, "_FUSED_ROUTE", [True])
    out, grads = _bridge_run(model, logits, incoming, q)
    errors = {f"out{i}": _rel(a, b) for i, (a, b) in enumerate(zip(out, ref_out))}
    assert set(grads) == set(ref_grads)
    errors.update({"grad/" + n: _rel(grads[n], ref_grads[n]) for n in ref_grads})
    worst = max(errors.items(), key=lambda kv: kv[1])
    print(flags, t, "worst", worst)
    assert not {k: v for k, v in errors.items() if v > 2e-2}, errors
