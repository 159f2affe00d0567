"""The allocation-free forward scan (gpa_gdn_scan_noalloc) against the
ordinary forward entry point (gpa_gdn_forward) on the same inputs.

Both run the same kernels; only where the intermediates live differs (the
library's static per-device scratch array instead of caller buffers), so the
outputs and final states must be identical, bit for bit.  Two calls in a row
share the scratch array; the second is smaller (fewer streams, tokens and
narrower widths, float32 instead of bf16), so stale contents of the first
call are present while it runs.  A problem larger than the array is rejected
with an error before any launch."""
import pytest
import torch

from gpa_amd import _lib
from gpa_amd.ops import gdn_scan_hip, gdn_scan_noalloc

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(b, t, h, kd, vd, dtype, seed, with_s0=True):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(b, t, h, kd, device=DEV, generator=g).to(dtype)
    k = torch.randn(b, t, h, kd, device=DEV, generator=g).to(dtype)
    v = torch.randn(b, t, h, vd, device=DEV, generator=g).to(dtype)
    gate = -torch.rand(b, t, h, device=DEV, generator=g) * .2
    beta = torch.rand(b, t, h, device=DEV, generator=g)
    s0 = torch.randn(b, h, kd, vd, device=DEV, generator=g) * .1 if with_s0 else None
    return q, k, v, gate, beta, s0


CALLS = [  # (B, T, H, K, V, dtype, chunk, offset, with query)
    (2, 300, 3, 128, 128, torch.bfloat16, 64, 0, True),
    (1, 70, 2, 64, 96, torch.float32, 32, 5, True),
    (1, 45, 2, 40, 24, torch.bfloat16, 16, 3, False),
]


def test_noalloc_matches_forward_on_consecutive_calls():
    with torch.no_grad():
        for i, (b, t, h, kd, vd, dtype, chunk, offset, with_q) in enumerate(CALLS):
            print("noalloc call", i, (b, t, h, kd, vd, dtype, chunk, offset, with_q), flush=True)
            q, k, v, gate, beta, s0 = _inputs(b, t, h, kd, vd, dtype, seed=10 + i)
            q = q if with_q else None
            out_ref, _, final_ref = gdn_scan_hip(q, k, v, gate, beta, s0, chunk=chunk, offset=offset)
            out, final = gdn_scan_noalloc(q, k, v, gate, beta, s0, chunk=chunk, offset=offset)
            torch.cuda.synchronize()
            assert torch.equal(final, final_ref), i
            if with_q:
                assert out.dtype == dtype and torch.equal(out, out_ref), i
            else:
                assert out is None


def test_noalloc_rejects_a_problem_above_its_scratch():
    q, k, v, gate, beta, s0 = _inputs(1, 64 * 200, 2, 128, 128, torch.bfloat16, seed=3, with_s0=False)
    with torch.no_grad(), pytest.raises(_lib.HipBackendError, match="scratch"):
        gdn_scan_noalloc(q, k, v, gate, beta, None, chunk=64)
