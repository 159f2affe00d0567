"""Pin the oracle (and the product's parameter initialisation) to the reference.

Every fixture in tests/golden/ was written by running the reference package on
the CPU (tests/golden/make_golden.py).  Here the same seeded construction must
give the same parameters and inputs, and the oracle must reproduce the
reference's outputs, carried state, gradients of every parameter and input,
cached-call partitions and single-token continuations.
"""
import pytest
import torch

import oracle
from tests.golden_cases import Case, TwoStageCase, compare, compare_state, grad_scale, names, ops_names

# Same arithmetic in a different association order: fp64 agrees to ~1e-12,
# fp32 to ~1e-6; bf16 activations agree except where an fp32 difference of
# one ulp flips a bf16 rounding.
RTOL = {torch.float64: 1e-9, torch.float32: 2e-5, torch.bfloat16: 2e-2}


@pytest.mark.parametrize("name", names())
def test_seeded_parameters_and_inputs_match_reference(name):
    case = Case(name)
    model, q, k, v, ctrl = case.build()
    exact = 1e-12 if case.dtype == torch.float64 else 1e-6
    errors = [compare(case, "param/" + n, p, exact) for n, p in model.named_parameters()]
    errors += [compare(case, "in/" + n, x, exact) for n, x in (("q", q), ("k", k), ("v", v), ("control", ctrl))
               if x is not None]
    assert not [e for e in errors if e], errors


@pytest.mark.parametrize("name", names())
def test_oracle_forward_state_and_gradients_match_reference(name):
    case = Case(name)
    rtol = RTOL[case.dtype]
    model, q, k, v, ctrl = case.build()
    q, k, v = (x.requires_grad_() for x in (q, k, v))
    if ctrl is not None:
        ctrl.requires_grad_()
    run = oracle.OracleRun(model, chunk_size=case.chunk_size)
    out, state = run(q, k, v, control_input=ctrl)
    errors = [compare(case, "out", out, rtol)] + compare_state(case, "state", state, rtol)
    out.float().square().mean().backward()
    # Gradients that vanish at initialisation (edge logits while every relation
    # memory is still zero) are pure roundoff: floor them at 1e-3*rtol of the
    # largest gradient of the case.
    g_rtol = rtol if case.dtype != torch.bfloat16 else 5e-2
    g_atol = 1e-3 * g_rtol * grad_scale(case)
    for n, p in model.named_parameters():
        if p.grad is not None:
            assert case.has("grad/" + n), n
            errors.append(compare(case, "grad/" + n, p.grad, g_rtol, g_atol))
        else:
            assert not case.has("grad/" + n), n
    for n, x in (("q", q), ("k", k), ("v", v), ("control", ctrl)):
        if x is not None:
            errors.append(compare(case, "grad/in_" + n, x.grad, g_rtol, g_atol))
    with torch.no_grad():
        if "partitions" in case.z:
            running, parts = None, []
            for lo, hi in case.z["partitions"]:
                y, running = run(q[:, lo:hi], k[:, lo:hi], v[:, lo:hi], running,
                                 control_input=ctrl[:, lo:hi] if ctrl is not None else None)
                parts.append(y)
            errors.append(compare(case, "partition_out", torch.cat(parts, 1), rtol))
        if case.steps():
            dq, dk, dv = case.regen_decode_inputs()
            running, ys = state, []
            for t in range(case.steps()):
                y, running = run(dq[:, t:t + 1], dk[:, t:t + 1], dv[:, t:t + 1], running)
                ys.append(y)
            errors.append(compare(case, "decode/out", torch.cat(ys, 1), rtol))
            errors += compare_state(case, "decode/state", running, rtol)
    errors = [e for e in errors if e]
    assert not errors, errors


@pytest.mark.parametrize("name", ops_names("ops_two_stage"))
def test_oracle_two_stage_matches_reference(name):
    """oracle.two_stage against the reference's two_stage_gdn on the same inputs:
    output, both final states and the gradient of every input."""
    case = TwoStageCase(name)
    rtol = RTOL[case.dtype]
    x = {n: t.requires_grad_() for n, t in case.inputs().items()}
    out, a, b = oracle.two_stage(x["q"], x["k"], x["slots"], x["v"], x["gi"], x["bi"], x["go"], x["bo"],
                                 x["inner"], x["outer"], route_weight=x.get("route_weight"),
                                 query_weight=x.get("query_weight"))
    out.float().square().mean().backward()
    errors = []
    for label, got in (("out", out), ("inner", a), ("outer", b)):
        rel = ((got.detach().double() - case.ref(label)).norm() / case.ref(label).norm()).item()
        if rel > rtol:
            errors.append(f"{label}: {rel:.3e}")
    g_rtol = rtol if case.dtype != torch.bfloat16 else 5e-2
    for n, t in x.items():
        ref = case.ref("grad/" + n)
        rel = ((t.grad.double() - ref).norm() / ref.norm()).item()
        if rel > g_rtol:
            errors.append(f"grad/{n}: {rel:.3e}")
    assert not errors, errors


def test_oracle_lm_matches_the_reference_lm():
    """oracle.lm.OracleLM (the all-GPA Qwen LM, src/gpa/hf_qwen.py) on the
    reference-written tiny checkpoint: training loss and every parameter
    gradient, full logits, a cached prefill with one-token and multi-token
    continuations (logits and every cache tensor), and the keep_rope variant,
    against the reference's numbers (float32)."""
    from gpa_amd.lm import GPALMForCausalLM
    from gpa_amd.state import tensors
    from oracle.lm import OracleLM
    from tests.lm_cases import CHECKPOINT, PIECES, LMCase
    case = LMCase()
    model = GPALMForCausalLM.from_pretrained(CHECKPOINT, attention_dtype=None)
    ids = case.ids
    run = OracleLM(model)
    loss, _, _ = run(ids, labels=ids)
    loss.backward()
    errors = [case.compare("train/loss", loss, 2e-5)]
    atol = 1e-3 * 2e-5 * case.grad_scale()
    got = [n for n, p in model.named_parameters() if p.grad is not None]
    assert got == case.grad_names
    errors += [case.compare("train/grad/" + n, p.grad, 2e-5, atol) for n, p in model.named_parameters()
               if p.grad is not None]
    with torch.no_grad():
        errors.append(case.compare("logits", run(ids)[1], 2e-5))
        cache = None
        for n, (lo, hi) in enumerate(PIECES):
            _, logits, cache = run(ids[:, lo:hi], cache=cache)
            errors.append(case.compare(f"cache/logits{n}", logits, 2e-5))
        assert cache["seen"] == int(case.z["full/cache/seen"])
        for i, (state, ptail, ctail) in enumerate(cache["layers"]):
            errors += [case.compare(f"cache/layer{i}/state{n:03d}", t, 2e-5) for n, t in enumerate(tensors(state))]
            errors += [case.compare(f"cache/layer{i}/ptail", ptail, 2e-5),
                       case.compare(f"cache/layer{i}/ctail", ctail, 2e-5)]
        rope_model = GPALMForCausalLM.from_pretrained(CHECKPOINT, attention_dtype=None, keep_rope=True)
        errors.append(case.compare("rope/logits", OracleLM(rope_model)(ids)[1], 2e-5))
    errors = [e for e in errors if e]
    assert not errors, errors
