"""Fused single-token decode (`gpa_decode_step`) vs the level-major HIP
schedule and vs the oracle's reference forward.

A prefill leaves a cache part-way into a block; then tokens are decoded one by
one across at least one block boundary (where the residual snapshots refresh),
and every output and every tensor of the final cache is compared.  The decode
from an empty cache starts on broadcast prefixes (batch stride 0).
Tolerances (relative L2): 1e-4 in float32, 2e-2 in bfloat16; the two HIP paths
agree to 2e-5 in float32.
"""
import copy

import pytest
import torch

import oracle
from gpa_amd import DenseGPA, GPAConfig
from gpa_amd.decode import decode_supported
from gpa_amd.schedule import run_segment
from gpa_amd.state import tensors

pytestmark = [pytest.mark.gpu,
              pytest.mark.skip(reason="fused decode switched off: its first MI355X launch ended in a memory fault "
                                      "with no cause found yet; kernel logic is covered by test_decode_emulated.py")]
DEV = "cuda"
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}

CASES = {
    "tiny_unequal_c3": dict(cfg=dict(heads=2, key_dim=4, value_dim=3, slots=(3, 2, 4), chunk_size=3), b=2,
                            prefill=4, steps=5),
    "tiny_none_c4": dict(cfg=dict(heads=2, key_dim=4, value_dim=3, slots=(3, 2, 4), chunk_size=4,
                                  positional_mode="none"), b=3, prefill=0, steps=6),
    "one_level": dict(cfg=dict(heads=2, key_dim=8, value_dim=5, slots=(6,), chunk_size=4), b=1, prefill=2,
                      steps=4),
    "c2_dims": dict(cfg=dict(heads=4, key_dim=32, value_dim=48, slots=(64, 64, 64, 128), chunk_size=8), b=2,
                    prefill=13, steps=5),
    "c3_dims": dict(cfg=dict(heads=2, key_dim=128, value_dim=128, slots=(128, 128, 128, 256), chunk_size=4),
                    b=2, prefill=6, steps=4),
}


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / max(b.norm().item(), 1e-30)).item()


def _inputs(cfg, b, t, dtype, gen):
    q = torch.randn(b, t, cfg.heads, cfg.key_dim, generator=gen)
    k = torch.nn.functional.normalize(torch.randn(b, t, cfg.heads, cfg.key_dim, generator=gen), dim=-1)
    v = torch.randn(b, t, cfg.heads, cfg.value_dim, generator=gen)
    return q.to(dtype), k.to(dtype), v.to(dtype)


def _generic(model, q, k, v, state):
    pos = torch.arange(state.position, state.position + 1, device=q.device)
    out, new, _ = run_segment(model, q, k, v, state, pos, None)
    return out, new


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("name", list(CASES))
def test_fused_decode_matches_schedule_and_oracle(name, dtype):
    spec = CASES[name]
    torch.manual_seed(11)
    model = DenseGPA(GPAConfig(**spec["cfg"]))
    with torch.no_grad():
        for w in model.gate_weight:
            w.normal_(0, .1)
        for p in model.relation_prefix:
            p.normal_(0, .01)
        model.edge_logits.normal_(0, .5)
    ref = oracle.OracleRun(copy.deepcopy(model))
    hip = model.to(DEV)
    cfg = hip.config
    gen = torch.Generator().manual_seed(5)
    b, n0, steps = spec["b"], spec["prefill"], spec["steps"]
    q, k, v = _inputs(cfg, b, n0 + steps, dtype, gen)
    tol = TOL[dtype]
    with torch.no_grad():
        if n0:
            _, state = hip(q[:, :n0].to(DEV), k[:, :n0].to(DEV), v[:, :n0].to(DEV))
            _, ref_state = ref(q[:, :n0], k[:, :n0], v[:, :n0])
        else:
            state = hip.initial_state(b, device=DEV, dtype=dtype)
            ref_state = None
        plain = state
        for t in range(n0, n0 + steps):
            xs = [x[:, t:t + 1].to(DEV) for x in (q, k, v)]
            assert decode_supported(hip, *xs, state, None)
            y, state = hip(*xs, state)
            y_plain, plain = _generic(hip, *xs, plain)
            y_ref, ref_state = ref(q[:, t:t + 1], k[:, t:t + 1], v[:, t:t + 1], ref_state)
            assert y.dtype == dtype and y.shape == y_ref.shape
            assert _rel(y, y_plain) < (2e-5 if dtype == torch.float32 else tol), t
            assert _rel(y, y_ref) < tol, t
            assert state.chunk_offset == ref_state.chunk_offset and state.position == ref_state.position
            assert (state.frozen is None) == (ref_state.frozen is None)
        for n, (a, p, r) in enumerate(zip(tensors(state), tensors(plain), tensors(ref_state))):
            assert a.shape == r.shape, n
            assert _rel(a, p) < (2e-5 if dtype == torch.float32 else tol), n
            assert _rel(a, r) < tol, n


def test_decode_keeps_the_incoming_cache_and_falls_back_when_unsupported():
    spec = CASES["tiny_unequal_c3"]
    torch.manual_seed(2)
    hip = DenseGPA(GPAConfig(**spec["cfg"])).to(DEV)
    gen = torch.Generator().manual_seed(1)
    q, k, v = (x.to(DEV) for x in _inputs(hip.config, 2, 3, torch.float32, gen))
    with torch.no_grad():
        _, s0 = hip(q[:, :2], k[:, :2], v[:, :2])
        before = [t.clone() for t in tensors(s0)]
        y1, s1 = hip(q[:, 2:], k[:, 2:], v[:, 2:], s0)
        y2, _ = hip(q[:, 2:], k[:, 2:], v[:, 2:], s0)
    for a, b in zip(before, tensors(s0)):
        assert torch.equal(a, b)
    assert torch.equal(y1, y2)
    # A call that needs gradients takes the schedule, and agrees.
    xs = [x[:, 2:].clone().requires_grad_() for x in (q, k, v)]
    assert not decode_supported(hip, *xs, s0, None)
    y3, s3 = hip(*xs, s0)
    y3.square().sum().backward()
    assert _rel(y3, y1) < 2e-5
    for a, b in zip(tensors(s3), tensors(s1)):
        assert _rel(a, b) < 2e-5
    softmax = DenseGPA(GPAConfig(heads=1, key_dim=8, value_dim=8, slots=(8, 6), chunk_size=2,
                                 slot_feature="softmax")).to(DEV)
    x = torch.randn(1, 1, 1, 8, device=DEV)
    assert not decode_supported(softmax, x, x, x, softmax.initial_state(1, device=DEV), None)
