"""The gated moment-scan kernel (gpa_amd/csrc/moment_scan.hip) built for the
host under AddressSanitizer (tests/host_emu/) and compared on the CPU with the
oracle's per-token recurrence (oracle/paper.py, reference
src/gpa/paper_dense.py:16-58 and src/gpa/ops.py:88-118):

- the forward for every shape class of the kernel (key widths 3 .. 256, value
  widths 1 .. 130, partial stages, one token), every decay form (none, per
  token, per key row, per value column), float32 and bfloat16, no initial
  state, a full one and a batch-broadcast one;
- the backward (three adjoint scans in one launch plus the decay gradient)
  against the oracle's autograd;
- the decayed counts (one key row).

Every access of the kernel is bounds-checked here before it runs on a GPU.
"""
import pytest
import torch

from gpa_amd import moment
from oracle import paper as op
from tests.host_emu import harness


@pytest.fixture
def host(host_runner, tmp_path, monkeypatch):
    lib = harness.HostLib(host_runner, str(tmp_path))
    harness.use_host(monkeypatch, lib)
    return lib


def _rel(a, b):
    a, b = a.detach().double(), b.detach().double()
    return ((a - b).norm() / max(b.norm().item(), 1e-30)).item()


def _inputs(seed, b, t, h, k, v, gate, dtype, s0):
    g_ = torch.Generator().manual_seed(seed)
    q = torch.randn(b, t, h, k, generator=g_).to(dtype)
    kk = torch.randn(b, t, h, k, generator=g_).to(dtype)
    vv = torch.randn(b, t, h, v, generator=g_).to(dtype)
    shape = {"token": (b, t, h), "key": (b, t, h, k), "value": (b, t, h, v)}.get(gate)
    g = -torch.rand(*shape, generator=g_) * .3 if shape else None
    init = {"full": torch.randn(b, h, k, v, generator=g_) * .3,
            "broadcast": (torch.randn(1, h, k, v, generator=g_) * .3).expand(b, h, k, v),
            None: torch.zeros(b, h, k, v)}[s0]
    return q, kk, vv, g, init


FWD = [  # (b, t, h, k, v, gate, s0)
    (2, 17, 1, 3, 5, "none", None), (1, 40, 2, 16, 64, "token", "full"), (2, 33, 1, 20, 1, "key", "broadcast"),
    (1, 1, 2, 32, 65, "value", "full"), (1, 40, 1, 33, 40, "key", "full"), (1, 16, 2, 64, 7, "value", None),
    (1, 20, 1, 100, 33, "token", "broadcast"), (1, 17, 1, 128, 32, "key", "full"),
    (1, 18, 1, 200, 17, "value", "full"), (1, 16, 1, 256, 16, "token", None), (1, 5, 1, 256, 130, "key", "full"),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("b,t,h,k,v,gate,s0", FWD)
def test_moment_forward_matches_oracle(host, b, t, h, k, v, gate, s0, dtype):
    q, kk, vv, g, init = _inputs(7, b, t, h, k, v, gate, dtype, s0)
    axis = "value" if gate == "value" else "key"
    y, final = moment.moment_scan(q, kk, vv, g, init, axis=axis)
    ry, rf = op.moment_scan(q, kk, vv, g, init.float(), axis=axis)
    assert y.dtype == dtype and final.dtype == torch.float32
    assert _rel(final, rf) < 1e-5
    assert _rel(y, ry) < (1e-5 if dtype == torch.float32 else 1e-2)


@pytest.mark.parametrize("b,t,h,k,v,gate,s0,dtype", [
    (1, 19, 2, 5, 3, "none", "full", torch.float32), (2, 17, 1, 20, 9, "token", "broadcast", torch.float32),
    (1, 33, 1, 40, 24, "key", "full", torch.float32), (1, 18, 2, 12, 70, "value", "full", torch.float32),
    (1, 17, 1, 130, 20, "key", "full", torch.float32), (1, 20, 1, 32, 16, "value", "full", torch.bfloat16),
    (1, 16, 1, 16, 32, "token", None, torch.bfloat16)])
def test_moment_backward_matches_oracle(host, b, t, h, k, v, gate, s0, dtype):
    q, kk, vv, g, init = _inputs(11, b, t, h, k, v, gate, dtype, s0)
    axis = "value" if gate == "value" else "key"
    g_ = torch.Generator().manual_seed(3)
    wy = torch.randn(b, t, h, v, generator=g_)
    wf = torch.randn(b, h, k, v, generator=g_)

    def run(fn, init_):
        xs = [x.detach().clone().requires_grad_() for x in (q, kk, vv)]
        gg = g.detach().clone().requires_grad_() if g is not None else None
        s = init_.detach().clone().requires_grad_()
        y, final = fn(*xs, gg, s, axis=axis)
        ((y.float() * wy).sum() + (final * wf).sum()).backward()
        return [x.grad for x in xs] + [gg.grad if gg is not None else None, s.grad]

    got = run(moment.moment_scan, init)
    want = run(op.moment_scan, init.float())
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    for name, a, r in zip(("dq", "dk", "dv", "dg", "ds0"), got, want):
        if r is None:
            assert a is None, name
            continue
        assert _rel(a, r) < tol, (name, _rel(a, r))


@pytest.mark.parametrize("vector", [False, True])
def test_decayed_counts_match_oracle(host, vector):
    g_ = torch.Generator().manual_seed(4)
    b, t, h, m = 2, 21, 2, 6
    p = torch.rand(b, t, h, m, generator=g_).bfloat16()
    g = -torch.rand(*((b, t, h, m) if vector else (b, t, h)), generator=g_) * .2
    n0 = torch.rand(b, h, m, generator=g_)
    got = moment.decayed_counts(p, g, n0)
    want = op.decayed_counts(p, g, n0)
    assert got.dtype == torch.float32
    assert _rel(got, want) < 1e-6
