"""The quadratic feature-map kernels (gpa_amd/csrc/quad_features.hip) built for
the host under AddressSanitizer (tests/host_emu/) and compared on the CPU with
the oracle's restatement of the reference's map (oracle.reference
.quadratic_features, src/gpa/features.py:17-25): forward output and the
gradients of x and of every parameter, float32 (1e-5 / 1e-4) and bfloat16
(2e-2), for widths below, at and above one 32-column block (8, 32, 40, 128,
256), partial row tiles and a zero row.  Every access of the kernels is
bounds-checked here before they run on a GPU.
"""
import math

import pytest
import torch

from gpa_amd import features
from gpa_amd.module import QuadraticFeatures
from oracle import reference as ref
from tests.host_emu import harness


@pytest.fixture
def host(host_runner, tmp_path, monkeypatch):
    lib = harness.HostLib(host_runner, str(tmp_path))
    harness.use_host(monkeypatch, lib)
    return lib


def _rel(a, b):
    a, b = a.detach().double(), b.detach().double()
    return ((a - b).norm() / max(b.norm().item(), 1e-30)).item()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("rows,heads,dim", [(37, 2, 8), (32, 1, 32), (65, 2, 40), (40, 1, 128), (33, 1, 256)])
def test_quad_features_match_oracle(host, rows, heads, dim, dtype):
    torch.manual_seed(rows + dim)
    fm = QuadraticFeatures(heads, dim)
    with torch.no_grad():
        fm.gain_raw.normal_(0, .5)
    x = torch.randn(rows, heads, dim).to(dtype)
    x[3] = 0  # a zero row: both normalisations at their floors
    w = torch.randn(rows, heads, dim)

    def run(fn):
        xx = x.clone().requires_grad_()
        fm.zero_grad(set_to_none=True)
        y = fn(xx)
        (y.float() * w).sum().backward()
        return [y, xx.grad, fm.left.grad, fm.right.grad, fm.gain_raw.grad]

    def kernel(xx):
        gain = 2 * fm.gain_raw.sigmoid() * math.sqrt(dim)
        return features._QuadFeatures.apply(xx, fm.left, fm.right, gain)

    got = run(kernel)
    want = run(lambda xx: ref.quadratic_features(fm, xx))
    tol = (1e-5, 1e-4) if dtype == torch.float32 else (2e-2, 3e-2)
    for i, (name, a, r) in enumerate(zip(("out", "dx", "dleft", "dright", "dgain"), got, want)):
        assert _rel(a, r) < tol[min(i, 1)], (name, _rel(a, r))
