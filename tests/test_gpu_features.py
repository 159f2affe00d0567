"""The quadratic Q/K feature map (gpa_amd/csrc/quad_features.hip, reference
src/gpa/features.py:17-25) on the GPU against the oracle's restatement on the
CPU: output and the gradients of x, both weight matrices and the gain, float32
(1e-5 forward, 1e-4 gradients) and bfloat16 (2e-2, 3e-2), for widths below, at
and above one 32-column block, partial row tiles, a zero row and C3's width
(128) at 2x1024 rows.  The module-level case (`features` in
tests/test_gpu_dense_gpa.py) runs the map inside DenseGPA against the oracle.
"""
import pytest
import torch

from gpa_amd.module import QuadraticFeatures
from oracle import reference as ref

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / max(b.norm().item(), 1e-30)).item()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("lead,heads,dim", [((37,), 2, 8), ((2, 16), 1, 32), ((65,), 3, 40), ((2, 1, 1024), 2, 128),
                                            ((33,), 1, 256), ((0,), 2, 16)])
def test_quad_features_match_oracle(lead, heads, dim, dtype):
    print(f"quad features lead={lead} heads={heads} dim={dim} {dtype}", flush=True)
    torch.manual_seed(dim + heads)
    fm = QuadraticFeatures(heads, dim)
    with torch.no_grad():
        fm.gain_raw.normal_(0, .5)
    gpu = QuadraticFeatures(heads, dim).cuda()
    gpu.load_state_dict(fm.state_dict())
    x = torch.randn(*lead, heads, dim).to(dtype)
    if x.numel():
        x.view(-1, heads, dim)[min(3, x.shape[0] - 1)] = 0
    w = torch.randn(*lead, heads, dim)

    def run(module, dev, fn):
        xx = x.to(dev).requires_grad_()
        y = fn(module, xx)
        (y.float() * w.to(dev)).sum().backward()
        return [y, xx.grad, module.left.grad, module.right.grad, module.gain_raw.grad]

    got = run(gpu, "cuda", lambda m, xx: m(xx))
    want = run(fm, "cpu", lambda m, xx: ref.quadratic_features(m, xx))
    assert got[0].shape == x.shape and got[0].dtype == dtype
    if not x.numel():
        return
    tol = (1e-5, 1e-4) if dtype == torch.float32 else (2e-2, 3e-2)
    for i, (name, a, r) in enumerate(zip(("out", "dx", "dleft", "dright", "dgain"), got, want)):
        assert torch.isfinite(a).all(), name
        assert _rel(a, r) < tol[min(i, 1)], (name, _rel(a, r))
