"""DenseGPA(backend="hip") on the GPU against the reference's own results.

Each fixture in tests/golden/ holds what the reference package computed on the
CPU for one seeded case (tests/golden/make_golden.py): outputs, every tensor of
the carried cache, the gradient of every parameter and input, cached-call
partitions and single-token continuations.  Here the same seeded model and
inputs run through the HIP backend and every entry is compared by relative L2
error: 1e-4 in float32, 2e-2 in bfloat16.  Entries stored as fingerprints (sum,
sum|x|, sum x^2 and 64 evenly spaced samples) are compared through sum|x|,
sum x^2 and the samples.  Gradients that vanish at initialisation are floored
at 1e-3 of the largest gradient norm of the case.  The HIP backend computes in
float32 or bfloat16, so a float64 fixture runs in float32 (the seeded float64
model and inputs rounded to float32) at the float32 bar, 1e-4.
"""
import math

import numpy as np
import pytest
import torch

from gpa_amd.state import tensors
from tests.golden_cases import Case, fingerprint, names

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}
CASES = names()


def _norm(case, name):
    if "full/" + name in case.z:
        return float(np.linalg.norm(case.z["full/" + name]))
    return math.sqrt(max(float(case.z["fp/" + name][2]), 0.))


def _rel(case, name, x, floor=0.):
    x = x.detach().double().cpu()
    if "full/" + name in case.z:
        ref = torch.from_numpy(case.z["full/" + name]).double()
        assert ref.shape == x.shape, (name, tuple(x.shape), tuple(ref.shape))
        return ((x - ref).norm() / max(ref.norm().item(), floor, 1e-30)).item()
    ref, got = case.z["fp/" + name], fingerprint(x)
    norm = math.sqrt(max(ref[2], 0.))
    # sample error scaled to the whole tensor, relative to its norm (or the floor)
    sample_err = np.linalg.norm(got[3:] - ref[3:]) * math.sqrt(max(x.numel(), 1) / (len(ref) - 3))
    rel_samples = sample_err / max(norm, floor, 1e-30)
    rel_abs = abs(got[1] - ref[1]) / max(abs(ref[1]), floor, 1e-30)
    rel_sq = abs(math.sqrt(max(got[2], 0.)) - norm) / max(norm, floor, 1e-30)
    return max(rel_samples, rel_abs, rel_sq)


@pytest.mark.parametrize("name", CASES)
def test_hip_backend_reproduces_reference_fixture(name):
    case = Case(name)
    dtype = torch.float32 if case.dtype == torch.float64 else case.dtype
    tol = TOL[dtype]
    model, q, k, v, ctrl = case.build()
    model = model.float().to(DEV)
    xs = [x.to(DEV, dtype).requires_grad_() for x in (q, k, v)]
    c = ctrl.to(DEV, torch.float32).requires_grad_() if ctrl is not None else None
    out, state = model(*xs, control_input=c)
    errors = {"out": _rel(case, "out", out)}
    meta = list(case.z["state/meta"])
    assert [state.position, state.chunk_size, state.chunk_offset, int(state.frozen is not None)] == meta
    for n, x in enumerate(tensors(state)):
        errors[f"state/{n:03d}"] = _rel(case, f"state/{n:03d}", x)
    out.float().square().mean().backward()
    grad_names = [n for n, p in model.named_parameters() if case.has("grad/" + n)]
    grad_names += ["in_" + n for n, x in zip("qkv", xs)] + (["in_control"] if c is not None else [])
    floor = 1e-3 * max(_norm(case, "grad/" + n) for n in grad_names)
    for n, p in model.named_parameters():
        if case.has("grad/" + n):
            assert p.grad is not None, n
            errors["grad/" + n] = _rel(case, "grad/" + n, p.grad, floor)
    for n, x in zip("qkv", xs):
        errors["grad/in_" + n] = _rel(case, "grad/in_" + n, x.grad, floor)
    if c is not None:
        errors["grad/in_control"] = _rel(case, "grad/in_control", c.grad, floor)
    with torch.no_grad():
        if "partitions" in case.z:
            running, parts = None, []
            for lo, hi in case.z["partitions"]:
                y, running = model(*(x[:, lo:hi] for x in xs), running,
                                   control_input=c[:, lo:hi] if c is not None else None)
                parts.append(y)
            errors["partition_out"] = _rel(case, "partition_out", torch.cat(parts, 1))
        if case.steps():
            dq, dk, dv = (x.to(DEV, dtype) for x in case.regen_decode_inputs())
            running, ys = state, []
            for t in range(case.steps()):
                y, running = model(dq[:, t:t + 1], dk[:, t:t + 1], dv[:, t:t + 1], running)
                ys.append(y)
            errors["decode/out"] = _rel(case, "decode/out", torch.cat(ys, 1))
            for n, x in enumerate(tensors(running)):
                errors[f"decode/state/{n:03d}"] = _rel(case, f"decode/state/{n:03d}", x)
    worst = max(errors.items(), key=lambda kv: kv[1])
    print(name, "worst", worst)
    bad = {k: e for k, e in errors.items() if e > tol}
    assert not bad, bad
