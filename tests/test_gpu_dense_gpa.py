"""DenseGPA(backend="hip") on the GPU vs the oracle's reference forward on the CPU.

Same seeded parameters and inputs; compared: output, every tensor of the
carried cache, gradients of every parameter (prefixes and relation prefixes
included) and of q/k/v, cached-call partitions and single-token decode.
Tolerances (relative L2 per tensor): 1e-4 in float32, 2e-2 in bfloat16.
Gradients that vanish at initialisation (edge logits while relation memories
are zero) are compared against an absolute floor of 1e-3 * the largest
gradient norm instead, since their relative error is pure roundoff.

In bfloat16 some gradients are ill-conditioned in the reference algorithm
itself (at the config-5 flag set and a perturbed parameter point the
oracle's own bf16 gradient vector sits 14 % from its float32 one): there a
kernel whose roundings differ from the torch expressions' by an ulp here and
there cannot sit within 2e-2 of the oracle's bf16 numbers.  A bf16 gradient
that misses 2e-2 is then held to the float32 oracle by the oracle's own bf16
error, 1.25x + 1e-2, and so is the whole gradient vector.
"""
import copy

import pytest
import torch

import oracle
from gpa_amd import DenseGPA, GPAConfig
from gpa_amd.state import tensors

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}


def _rel(a, b, floor=0.):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / max(b.norm().item(), floor, 1e-30)).item()


# Scale of the seeded noise `perturb` adds to each parameter (by name prefix);
# parameters not listed move by 20 % of their mean magnitude.
PERTURB = {"relation_prefix": .1, "gate_weight": .3, "residual_raw": .8, "output_logits": .8,
           "edge_logits": .8, "bridge_mix_raw": .8, "inner_prefix": .05, "outer_prefix": .05}


def perturb(model, seed: int) -> None:
    """Move every parameter off its initial value with seeded N(0,1) noise:
    zero-initialised ones (relation prefixes, gate weights, residual steps,
    output and edge logits) get the absolute scales in PERTURB, the identity
    route weights get I + 0.2/sqrt(M) noise, the rest 20 % of their mean
    magnitude.  The gradients then leave the corner of parameter space that
    default initialisation sits in (constant gates, zero relation memories)."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            noise = torch.randn(p.shape, generator=g, dtype=torch.float64).to(p.dtype)
            key = name.split(".")[0]
            if key in PERTURB:
                scale = PERTURB[key]
            elif key == "route_weight":
                scale = .2 / p.shape[-1] ** .5
            else:
                scale = .2 * p.abs().mean().item()
            p.add_(noise * scale)


def _setup(cfg_kwargs, b, t, dtype, seed, normalize_k=False, gate_noise=0., control_dim=0, perturbed=False):
    torch.manual_seed(seed)
    model = DenseGPA(GPAConfig(**cfg_kwargs))
    if perturbed:
        perturb(model, seed + 100)
    if gate_noise:
        with torch.no_grad():
            for w in model.gate_weight:
                w.normal_(0, gate_noise)
    cfg = model.config
    q = torch.randn(b, t, cfg.heads, cfg.key_dim)
    k = torch.randn_like(q)
    v = torch.randn(b, t, cfg.heads, cfg.value_dim)
    if normalize_k:
        k = torch.nn.functional.normalize(k, dim=-1)
    ctrl = torch.randn(b, t, control_dim) if control_dim else None
    return model, q.to(dtype), k.to(dtype), v.to(dtype), ctrl


CONFIGS = {
    "tiny_unequal_c3": dict(cfg=dict(heads=2, key_dim=4, value_dim=3, slots=(3, 2, 4), chunk_size=3), b=2, t=9),
    "tiny_none_c4": dict(cfg=dict(heads=2, key_dim=4, value_dim=3, slots=(3, 2, 4), chunk_size=4,
                                  positional_mode="none"), b=2, t=11),
    "one_level": dict(cfg=dict(heads=2, key_dim=8, value_dim=5, slots=(6,), chunk_size=4), b=1, t=10),
    "lm_flags": dict(cfg=dict(heads=2, key_dim=8, value_dim=6, slots=(8, 8), chunk_size=4, control_dim=5,
                              rsa_update=True, paper_product_read=True, shared_query_center=True,
                              balanced_bridge=True, relation_marginal=True, read_scale=8., beta_init=.6,
                              decay_init=1e-4), b=1, t=10, gate_noise=.1, control_dim=5),
    "features": dict(cfg=dict(heads=2, key_dim=8, value_dim=6, slots=(5, 7, 5), chunk_size=3,
                              slot_feature="tanh", quadratic_features=True, learn_read_scale=True,
                              rsa_update=True), b=1, t=8),
    "softmax_slots": dict(cfg=dict(heads=1, key_dim=8, value_dim=8, slots=(8, 6), chunk_size=2,
                                   slot_feature="softmax"), b=2, t=5),
    "c2_dims": dict(cfg=dict(heads=4, key_dim=32, value_dim=48, slots=(64, 64, 64, 128), chunk_size=64),
                    b=1, t=130),
    "c2_dims_b8": dict(cfg=dict(heads=4, key_dim=32, value_dim=48, slots=(64, 64, 64, 128), chunk_size=64),
                       b=8, t=130),
    "c3_dims": dict(cfg=dict(heads=2, key_dim=128, value_dim=128, slots=(128, 128, 128, 256), chunk_size=64),
                    b=1, t=130, normalize_k=True),
    # positional moments (rotary query, additive moment state and its logit term)
    "moments": dict(cfg=dict(heads=2, key_dim=8, value_dim=6, slots=(5, 7, 5), chunk_size=4,
                             positional_mode="moments"), b=2, t=11),
    "moments_c3": dict(cfg=dict(heads=2, key_dim=128, value_dim=128, slots=(128, 128, 128, 256), chunk_size=64,
                                positional_mode="moments"), b=1, t=130, normalize_k=True),
    "tokenwise_moments": dict(cfg=dict(heads=2, key_dim=8, value_dim=6, slots=(5, 4), chunk_size=1,
                                       positional_mode="moments"), b=2, t=6),
    # the product relation read with and without the marginal term (HIP product_read + route reader)
    "product": dict(cfg=dict(heads=2, key_dim=8, value_dim=6, slots=(8, 8, 16), chunk_size=4,
                             paper_product_read=True), b=2, t=9),
    "product_marginal": dict(cfg=dict(heads=2, key_dim=8, value_dim=6, slots=(8, 16, 8), chunk_size=3,
                                      paper_product_read=True, relation_marginal=True, read_scale=8.), b=2, t=10),
    "product_marginal_c3": dict(cfg=dict(heads=2, key_dim=128, value_dim=128, slots=(128, 128, 128, 256),
                                         chunk_size=64, paper_product_read=True, relation_marginal=True),
                                b=1, t=130, normalize_k=True),
    "product_center": dict(cfg=dict(heads=2, key_dim=16, value_dim=8, slots=(16, 8, 8), chunk_size=4,
                                    paper_product_read=True, relation_marginal=True, shared_query_center=True,
                                    read_scale=8.), b=2, t=9),
    "tokenwise_product": dict(cfg=dict(heads=2, key_dim=8, value_dim=6, slots=(8, 8), chunk_size=1,
                                       paper_product_read=True, relation_marginal=True), b=2, t=5),
    # the tokenwise model (chunk_size 1)
    "tokenwise": dict(cfg=dict(heads=2, key_dim=16, value_dim=8, slots=(6, 4, 5), chunk_size=1), b=2, t=8),
    # config 1's widths (the reference's CPU case): every recurrence takes the one-token kernels in inference
    "tokenwise_c1": dict(cfg=dict(heads=4, key_dim=32, value_dim=48, slots=(64, 64, 64, 128), chunk_size=1),
                         b=2, t=6),
    "tokenwise_lm": dict(cfg=dict(heads=2, key_dim=8, value_dim=6, slots=(8, 8), chunk_size=1, control_dim=5,
                                  rsa_update=True, paper_product_read=True, shared_query_center=True,
                                  balanced_bridge=True, relation_marginal=True, read_scale=8., beta_init=.6,
                                  decay_init=1e-4), b=1, t=4, gate_noise=.1, control_dim=5),
    # the LM layer's flag set (reference hf_qwen.py:145-151: rsa_update, product read, shared query
    # centre, balanced bridge, read scale 8, beta .6, decay 1e-4, full hidden controls) at C3 widths
    "lm_c3": dict(cfg=dict(heads=2, key_dim=128, value_dim=128, slots=(128, 128, 128, 256), chunk_size=64,
                           control_dim=64, rsa_update=True, paper_product_read=True, shared_query_center=True,
                           balanced_bridge=True, read_scale=8., beta_init=.6, decay_init=1e-4),
                  b=1, t=130, gate_noise=.05, control_dim=64),
}


def _run_both(name, dtype, perturbed=False):
    spec = CONFIGS[name]
    model, q, k, v, ctrl = _setup(spec["cfg"], spec["b"], spec["t"], dtype, seed=5,
                                  normalize_k=spec.get("normalize_k", False),
                                  gate_noise=spec.get("gate_noise", 0.), control_dim=spec.get("control_dim", 0),
                                  perturbed=perturbed)
    if dtype == torch.bfloat16:  # for the float32 oracle on the same (bf16-valued) inputs, if needed
        _TRUTH[name] = (copy.deepcopy(model), q, k, v, ctrl)
    ref_model = copy.deepcopy(model)
    hip_model = model.to(DEV)
    xs = [x.to(DEV).requires_grad_() for x in (q, k, v)]
    c_hip = ctrl.to(DEV).requires_grad_() if ctrl is not None else None
    out, state = hip_model(*xs, control_input=c_hip)
    out.float().square().mean().backward()
    rs = [x.clone().requires_grad_() for x in (q, k, v)]
    c_ref = ctrl.clone().requires_grad_() if ctrl is not None else None
    ref_out, ref_state = oracle.OracleRun(ref_model)(*rs, control_input=c_ref)
    ref_out.float().square().mean().backward()
    return (hip_model, xs, c_hip, out, state), (ref_model, rs, c_ref, ref_out, ref_state)


_TRUTH = {}  # case -> (model, q, k, v, control) of the last bf16 run, before it ran


def _noise_aware(name, errors, tol, hm, xs, c_hip, rm, rs, c_ref):
    """bf16 gradients above `tol` against the oracle's bf16 ones, re-judged
    against the float32 oracle: each within 1.25x the oracle's own bf16 error
    + 1e-2, and the whole gradient vector too.  Returns the re-judged names."""
    m32, q, k, v, ctrl = _TRUTH.pop(name)
    if all(err <= tol for label, err in errors.items() if label.startswith("grad/")):
        return []
    xs32 = [x.float().requires_grad_() for x in (q, k, v)]
    c32 = ctrl.clone().requires_grad_() if ctrl is not None else None
    out32, _ = oracle.OracleRun(m32)(*xs32, control_input=c32)
    out32.float().square().mean().backward()
    params32 = {n: p.grad for n, p in m32.named_parameters() if p.grad is not None}
    xs32, c32 = [x.grad for x in xs32], c32.grad if c32 is not None else None
    ours = {n: p.grad for n, p in hm.named_parameters() if n in params32}
    theirs = {n: p.grad for n, p in rm.named_parameters() if n in params32}
    truth = dict(params32)
    for label, a, b, t in zip("qkv", xs, rs, xs32):
        ours["x/" + label], theirs["x/" + label], truth["x/" + label] = a.grad, b.grad, t
    if c32 is not None:
        ours["x/control"], theirs["x/control"], truth["x/control"] = c_hip.grad, c_ref.grad, c32
    names = list(truth)
    flat = lambda g: torch.cat([g[n].detach().double().cpu().reshape(-1) for n in names])  # noqa: E731
    ours_all, theirs_all = _rel(flat(ours), flat(truth)), _rel(flat(theirs), flat(truth))
    print(f"bf16 gradient vector vs the float32 oracle: ours {ours_all:.3e}, the oracle's bf16 {theirs_all:.3e}")
    assert ours_all <= 1.25 * theirs_all + 1e-2
    key = {("grad/" + n[2:] if n.startswith("x/") and n != "x/control" else
            "grad/control" if n == "x/control" else "grad/" + n): n for n in names}
    rejudged = []
    for label, err in list(errors.items()):
        if err <= tol or label not in key:
            continue
        n = key[label]
        e_ours, e_theirs = _rel(ours[n], truth[n]), _rel(theirs[n], truth[n])
        print(f"  {label}: {err:.2e} from the oracle's bf16; vs float32: ours {e_ours:.2e}, "
              f"the oracle's bf16 {e_theirs:.2e}")
        if e_ours <= 1.25 * e_theirs + 1e-2:
            errors[label] = 0.
            rejudged.append(label)
    return rejudged


def _compare(name, dtype, perturbed=False):
    """Relative errors of output, cache and every gradient; returns (errors,
    names of parameter gradients that passed only through the roundoff floor
    of 1e-3 * the largest parameter-gradient norm)."""
    tol = TOL[dtype]
    (hm, xs, c_hip, out, state), (rm, rs, c_ref, ref_out, ref_state) = _run_both(name, dtype, perturbed)
    errors = {"out": _rel(out, ref_out)}
    assert state.position == ref_state.position and state.chunk_offset == ref_state.chunk_offset
    assert (state.frozen is None) == (ref_state.frozen is None)
    for n, (a, b) in enumerate(zip(tensors(state), tensors(ref_state))):
        errors[f"state{n}"] = _rel(a, b)
    grads = {n: p.grad for n, p in rm.named_parameters() if p.grad is not None}
    top = max(g.norm().item() for g in grads.values())
    floored = []
    for (n, p) in hm.named_parameters():
        if n in grads:
            assert p.grad is not None, n
            errors["grad/" + n] = _rel(p.grad, grads[n], floor=1e-3 * top)
            if _rel(p.grad, grads[n]) > tol >= errors["grad/" + n]:
                floored.append(n)
    for label, a, b in zip("qkv", xs, rs):
        errors["grad/" + label] = _rel(a.grad, b.grad)
    if c_hip is not None:
        errors["grad/control"] = _rel(c_hip.grad, c_ref.grad)
    worst = max(errors.items(), key=lambda kv: kv[1])
    print(name, dtype, "perturbed" if perturbed else "init", "worst", worst, "out", errors["out"],
          "floored", floored or "none")
    if dtype == torch.bfloat16:
        rejudged = _noise_aware(name, errors, tol, hm, xs, c_hip, rm, rs, c_ref)
        print("held to the float32 oracle:", rejudged or "none")
    bad = {k: v for k, v in errors.items() if v > tol}
    assert not bad, bad
    return errors, floored


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("name", list(CONFIGS))
def test_dense_gpa_forward_backward_matches_oracle(name, dtype):
    if dtype == torch.bfloat16 and name not in ("c3_dims", "c2_dims", "c2_dims_b8", "tiny_unequal_c3", "lm_flags",
                                                "tokenwise", "moments_c3", "product_marginal_c3", "lm_c3"):
        pytest.skip("bf16 covered on the configuration-shaped cases")
    _compare(name, dtype)


PERTURBED = ["tiny_unequal_c3", "lm_flags", "tokenwise", "tokenwise_lm", "c2_dims", "c3_dims",
             "product_marginal_c3", "lm_c3", "moments", "features"]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("name", PERTURBED)
def test_dense_gpa_at_a_perturbed_parameter_point(name, dtype):
    """The module against the oracle away from default initialisation: every
    parameter carries seeded noise (`perturb`), so relation memories start
    non-zero, gates vary per token, residual steps, output and edge logits
    differ per level and head, and route weights are not the identity.  No
    gradient of a learnable initial state (inner, outer and relation
    prefixes) may pass through the roundoff floor."""
    if dtype == torch.bfloat16 and name not in ("c2_dims", "c3_dims", "lm_flags", "product_marginal_c3", "lm_c3"):
        pytest.skip("bf16 covered on the configuration-shaped cases")
    _, floored = _compare(name, dtype, perturbed=True)
    assert not [n for n in floored if "prefix" in n], floored


@pytest.mark.parametrize("name", ["tiny_unequal_c3", "tiny_none_c4", "lm_flags", "c2_dims", "c3_dims",
                                  "tokenwise", "tokenwise_c1", "moments", "tokenwise_moments", "product_marginal",
                                  "product_center"])
def test_cached_partitions_and_decode_match_oracle(name):
    """Cached calls cut at block-unaligned points, then three one-token decode
    calls (the T = 1 inference path: one-token scan steps, the one-token level
    kernel and the relation token steps, with the configuration's flags and
    control input), against the oracle's cached calls, in float32."""
    spec = CONFIGS[name]
    model, q, k, v, ctrl = _setup(spec["cfg"], spec["b"], spec["t"], torch.float32, seed=9,
                                  normalize_k=spec.get("normalize_k", False), gate_noise=spec.get("gate_noise", 0.),
                                  control_dim=spec.get("control_dim", 0))
    ref = oracle.OracleRun(copy.deepcopy(model))
    hip = model.to(DEV)
    t = spec["t"]
    cuts = [0, 2, 3, t // 2, t - 1, t]
    part = (lambda x, lo, hi: x[:, lo:hi]) if ctrl is not None else (lambda x, lo, hi: None)
    dev = (lambda x: x.to(DEV) if x is not None else None)
    with torch.no_grad():
        full, full_state = hip(q.to(DEV), k.to(DEV), v.to(DEV), control_input=dev(ctrl))
        state, parts = None, []
        for lo, hi in zip(cuts[:-1], cuts[1:]):
            y, state = hip(q[:, lo:hi].to(DEV), k[:, lo:hi].to(DEV), v[:, lo:hi].to(DEV), state,
                           control_input=dev(part(ctrl, lo, hi)))
            parts.append(y)
        ref_state, ref_parts = None, []
        for lo, hi in zip(cuts[:-1], cuts[1:]):
            y, ref_state = ref(q[:, lo:hi], k[:, lo:hi], v[:, lo:hi], ref_state, control_input=part(ctrl, lo, hi))
            ref_parts.append(y)
        hip_cat, ref_cat = torch.cat(parts, 1), torch.cat(ref_parts, 1)
        assert _rel(hip_cat, full) < 1e-5
        assert _rel(hip_cat, ref_cat) < 1e-4
        for a, b in zip(tensors(state), tensors(ref_state)):
            assert _rel(a, b) < 1e-4
        assert state.chunk_offset == ref_state.chunk_offset and state.position == ref_state.position
        # Single-token decode from the carried cache.
        g = torch.Generator().manual_seed(3)
        for _ in range(3):
            dq = torch.randn(q.shape[0], 1, *q.shape[2:], generator=g)
            dk = torch.nn.functional.normalize(torch.randn(dq.shape, generator=g), dim=-1)
            dv = torch.randn(v.shape[0], 1, *v.shape[2:], generator=g)
            dc = torch.randn(q.shape[0], 1, ctrl.shape[-1], generator=g) if ctrl is not None else None
            y, state = hip(dq.to(DEV), dk.to(DEV), dv.to(DEV), state, control_input=dev(dc))
            y_ref, ref_state = ref(dq, dk, dv, ref_state, control_input=dc)
            assert _rel(y, y_ref) < 1e-4
        for a, b in zip(tensors(state), tensors(ref_state)):
            assert _rel(a, b) < 1e-4


def test_empty_call_returns_same_state_and_state_is_query_independent():
    spec = CONFIGS["tiny_unequal_c3"]
    model, q, k, v, _ = _setup(spec["cfg"], spec["b"], spec["t"], torch.float32, seed=4)
    hip = model.to(DEV)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    with torch.no_grad():
        y1, s1 = hip(q, k, v)
        y2, s2 = hip(q * 3 + 1, k, v)
        z, same = hip(q[:, :0], k[:, :0], v[:, :0], s1)
    assert z.shape == (q.shape[0], 0, q.shape[2], v.shape[3]) and same is s1
    for a, b in zip(s1.levels, s2.levels):
        assert torch.equal(a.inner, b.inner) and torch.equal(a.outer, b.outer)
    assert not torch.allclose(y1, y2)


@pytest.mark.parametrize("name", ["c2_dims", "lm_flags", "c3_dims"])
def test_packed_scans_match_the_stream_schedule(name, monkeypatch):
    """The packed scan calls (a level's A/B pair and every edge in one library
    call, schedule._PACKED) against the same schedule with one call per scan
    group on side streams: output, every cache tensor and every gradient."""
    from gpa_amd import schedule
    spec = CONFIGS[name]
    dtype = torch.bfloat16 if name == "c3_dims" else torch.float32
    runs = {}
    for packed in (True, False):
        monkeypatch.setattr(schedule, "_PACKED", [packed])
        model, q, k, v, ctrl = _setup(spec["cfg"], spec["b"], spec["t"], dtype, seed=9,
                                      normalize_k=spec.get("normalize_k", False),
                                      gate_noise=spec.get("gate_noise", 0.), control_dim=spec.get("control_dim", 0))
        model = model.to(DEV)
        xs = [x.to(DEV).requires_grad_() for x in (q, k, v)]
        c = ctrl.to(DEV) if ctrl is not None else None
        out, state = model(*xs, control_input=c)
        out.float().square().mean().backward()
        runs[packed] = ([out] + list(tensors(state)), [p.grad for p in model.parameters()] + [x.grad for x in xs])
    tol = 1e-5 if dtype == torch.float32 else 5e-3
    for kind, a_list, b_list in (("forward", runs[True][0], runs[False][0]), ("grad", runs[True][1], runs[False][1])):
        for i, (a, b) in enumerate(zip(a_list, b_list)):
            if a is None or b is None:
                assert a is None and b is None, (kind, i)
                continue
            assert _rel(a, b) < tol, (kind, i, _rel(a, b))
