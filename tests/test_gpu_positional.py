"""Positional moments on the GPU (gpa_amd/positional.py): the rotary
embedding and the additive moment scan against the oracle's restatements of
the reference (src/gpa/ops.py:88-137), including gradients, block-unaligned
lengths, [B,T] positions and an empty sequence."""
import pytest
import torch

import oracle.reference as ref
from gpa_amd.positional import additive_scan, linear_scan, rope

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / max(b.norm().item(), 1e-30)).item()


@pytest.mark.parametrize("shape,positions", [((2, 7, 3, 8), "range"), ((2, 5, 2, 16), "batch"),
                                             ((3, 4), "scalar")])
def test_rope_matches_reference(shape, positions):
    g = torch.Generator().manual_seed(1)
    x = torch.randn(*shape, generator=g)
    if positions == "range":
        pos = torch.arange(5, 5 + shape[1])
    elif positions == "batch":
        pos = torch.randint(0, 1000, shape[:2], generator=g)
    else:
        pos = torch.tensor(17)
    got = rope(x.to(DEV), pos.to(DEV))
    assert _rel(got, ref.rope(x, pos)) < 1e-5  # float32 sin/cos of angles up to 1000
    xb = x.bfloat16()
    assert got.dtype == torch.float32 and rope(xb.to(DEV), pos.to(DEV)).dtype == torch.bfloat16
    with pytest.raises(ValueError):
        rope(torch.randn(2, 3, 5, device=DEV), 1)


@pytest.mark.parametrize("b,t,h,k,v", [(2, 1, 2, 8, 5), (1, 63, 2, 16, 8), (2, 130, 3, 32, 48), (1, 256, 1, 128, 256)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_additive_scan_matches_reference_with_gradients(b, t, h, k, v, dtype):
    g = torch.Generator().manual_seed(b * 10 + t)
    q = torch.randn(b, t, h, k, generator=g).to(dtype)
    kk = (torch.randn(b, t, h, k, generator=g) * .3).to(dtype)
    vv = torch.randn(b, t, h, v, generator=g).to(dtype)
    s0 = torch.randn(b, h, k, v, generator=g) * .1
    xs = [x.to(DEV).requires_grad_() for x in (q, kk, vv, s0)]
    out, final = additive_scan(*xs)
    rs = [x.clone().double().requires_grad_() for x in (q, kk, vv, s0)]
    r_out, r_final = ref.additive_scan(*rs)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert out.dtype == dtype and out.shape == (b, t, h, v) and final.dtype == torch.float32
    assert _rel(out, r_out) < tol and _rel(final, r_final) < 1e-5
    wo = torch.randn(out.shape, generator=g)
    wf = torch.randn(final.shape, generator=g)
    ((out.float() * wo.to(DEV)).sum() + (final * wf.to(DEV)).sum()).backward()
    ((r_out * wo.double()).sum() + (r_final * wf.double()).sum()).backward()
    for x, r in zip(xs, rs):
        assert _rel(x.grad, r.grad) < (1e-5 if dtype == torch.float32 else 2e-2)


def test_linear_scan_signature_and_empty_sequence():
    q = torch.randn(2, 0, 3, 4, device=DEV)
    v = torch.randn(2, 0, 3, 5, device=DEV)
    s0 = torch.randn(2, 3, 4, 5, device=DEV)
    out, final = linear_scan(q, q, v, s0)
    assert out.shape == v.shape and final is s0
    with pytest.raises(ValueError):
        linear_scan(q, q[..., :3], v, s0)
    with pytest.raises(ValueError):
        linear_scan(torch.randn(1, 2, 1, 4, device=DEV), torch.randn(1, 2, 1, 4, device=DEV),
                    torch.randn(1, 2, 1, 5, device=DEV), torch.zeros(1, 1, 4, 5, device=DEV), backend="torch")
