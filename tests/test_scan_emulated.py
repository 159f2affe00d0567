"""The chunked GDN scan's kernels (gdn_scan.hip and the prep, 256-key state,
out / dd0 and chunk-backward MFMA kernels) built for the host and run under
AddressSanitizer (tests/host_emu/), against the oracle's per-token
recurrence in float64 (reference ops.py:29-85), on the CPU.

The cases reach the float32 FMA path (state, out and dd0 kernels of
gdn_scan.hip, the chunk backward on fp32 MFMA, or the FMA chunk backward
when K is not a multiple of 4), the bfloat16 FMA path (K not a multiple of
16) and the bfloat16 MFMA path above 128 keys (gdn_state_fwd_mfma / gdn_state_bwd_mfma at 256 keys, with K
below and at the tile), with chunk offsets, ragged last chunks and tiny
shapes.  Every global access of those kernels is checked against the exact
extent of the buffer it addresses; the results are held to the GPU tests'
bar: relative L2 1e-4 in float32, 2e-2 in bfloat16.  The bfloat16 scans of
at most 128 keys take the strip state kernels, which the host build does not
emulate (their LDS loads are inline global_load_lds); the GPU tests cover
them.
"""
import pytest
import torch

from tests.host_emu import harness
from tests.test_gpu_gdn_scan import _inputs, _oracle_segments, _oracle_segments_autograd, _rel

CASES = [
    # (B, T, H, K, V, chunk, offset, dtype)
    (2, 9, 2, 4, 3, 4, 2, torch.float32),
    (2, 11, 1, 6, 5, 4, 1, torch.float32),  # K % 4 != 0: the FMA chunk backward at 64 keys
    (1, 40, 2, 40, 24, 16, 5, torch.bfloat16),  # K % 16 != 0: the bfloat16 FMA state path
    (1, 70, 2, 32, 48, 64, 17, torch.float32),
    (1, 40, 1, 256, 64, 16, 3, torch.float32),
    (1, 40, 1, 256, 64, 64, 3, torch.float32),
    (1, 40, 1, 128, 64, 16, 3, torch.float32),
    (1, 129, 1, 256, 96, 64, 1, torch.bfloat16),
    (1, 70, 1, 192, 128, 64, 5, torch.bfloat16),
]
IDS = [f"B{c[0]}T{c[1]}H{c[2]}K{c[3]}V{c[4]}C{c[5]}o{c[6]}{str(c[7])[6:]}" for c in CASES]


@pytest.fixture
def host(host_runner, monkeypatch, tmp_path):
    from gpa_amd import ops
    harness.use_host(monkeypatch, harness.HostLib(host_runner, str(tmp_path)))
    # host tensors belong to no stream: nothing to mark as in use
    monkeypatch.setattr(ops, "_in_use_here", lambda *tensors: None)


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_emulated_scan_forward_matches_recurrence(host, case):
    from gpa_amd.ops import gdn_scan_hip
    b, t, h, kd, vd, chunk, offset, dtype = case
    q, k, v, g, beta, s0 = _inputs(b, t, h, kd, vd, dtype, seed=11)
    out, states, final = gdn_scan_hip(q, k, v, g, beta, s0, chunk=chunk, offset=offset)
    ref_out, ref_states, ref_final = _oracle_segments(q, k, v, g, beta, s0, chunk, offset)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    errs = dict(out=_rel(out, ref_out), states=_rel(states, ref_states), final=_rel(final, ref_final))
    print(case, errs)
    assert all(e < tol for e in errs.values()), errs


@pytest.mark.parametrize("case", CASES, ids=IDS)
@pytest.mark.parametrize("with_q", [True, False], ids=["read", "noread"])
def test_emulated_scan_backward_matches_autograd_of_recurrence(host, case, with_q):
    """Gradients of a loss over the read, the chunk-start states (injected
    into the backward) and the final state.  The float32 cases above 128
    keys run the FMA chunk backward (gdn_chunk_bwd<float, 256>), whose dA
    product once read rows of an LDS matrix that other threads were already
    overwriting: a race the host build's independent threads expose."""
    from gpa_amd.ops import gdn_scan_hip
    b, t, h, kd, vd, chunk, offset, dtype = case
    q, k, v, g, beta, s0 = _inputs(b, t, h, kd, vd, dtype, seed=5, q=with_q)
    gen = torch.Generator().manual_seed(3)
    nch = (offset + t + chunk - 1) // chunk
    w_out = torch.randn(b, t, h, vd, generator=gen, dtype=torch.float64)
    w_states = torch.randn(b, h, nch, kd, vd, generator=gen, dtype=torch.float64) * .1
    w_final = torch.randn(b, h, kd, vd, generator=gen, dtype=torch.float64)

    def loss(out, states, final):
        total = (final.double() * w_final).sum() + (states.double() * w_states).sum()
        return total + (out.double() * w_out).sum() if out is not None else total

    leaves = [x.clone().requires_grad_() if x is not None else None for x in (q, k, v, g, beta, s0)]
    out, states, final = gdn_scan_hip(*leaves, chunk=chunk, offset=offset)
    loss(out if with_q else None, states, final).backward()
    refs = [x.detach().double().requires_grad_() if x is not None else None for x in (q, k, v, g, beta, s0)]
    ro, rs, rf = _oracle_segments_autograd(refs[:3], refs[3], refs[4], refs[5], chunk, offset)
    loss(ro if with_q else None, rs, rf).backward()
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    names = ["dq", "dk", "dv", "dg", "dbeta", "ds0"]
    errs = {n: _rel(a.grad, r.grad) for n, a, r in zip(names, leaves, refs) if a is not None}
    print(case, with_q, errs)
    assert all(e < tol for e in errs.values()), errs
