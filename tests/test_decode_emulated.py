"""The fused decode kernel (gpa_amd/csrc/gpa_decode.hip) built for the host and
compared with the oracle's reference forward, on the CPU.

The kernel source is compiled for the host with AddressSanitizer against the
HIP emulation in tests/host_emu/ (harness.py).  `decode.decode_step` builds its
`gpa_decode_problem` exactly as on the GPU; the call runs in a runner process
that gives every buffer the problem points into an allocation of its exact
size, so any out-of-bounds access aborts it.

Checked per decode step: the output and, at the end, every tensor of the cache,
against the oracle, from a prefill part-way into a block and across block
boundaries (residual snapshot refresh), and from an empty cache (broadcast
prefixes, batch stride 0).  Tolerances: 1e-5 relative in float32 and bfloat16
(both follow the reference's rounding points, so only fp32 summation order
differs).
"""
import copy

import pytest
import torch

import oracle
from gpa_amd import DenseGPA, GPAConfig
from gpa_amd import decode as dec
from gpa_amd.state import tensors
from tests.host_emu import harness

CASES = {
    "tiny_unequal_c3": dict(cfg=dict(heads=2, key_dim=4, value_dim=3, slots=(3, 2, 4), chunk_size=3), b=2,
                            prefill=4, steps=3),
    "tiny_none_c4": dict(cfg=dict(heads=1, key_dim=4, value_dim=3, slots=(3, 2, 4), chunk_size=4,
                                  positional_mode="none"), b=2, prefill=0, steps=5),
    "one_level": dict(cfg=dict(heads=2, key_dim=8, value_dim=5, slots=(6,), chunk_size=4), b=1, prefill=2,
                      steps=4),
    "c2_dims": dict(cfg=dict(heads=2, key_dim=32, value_dim=48, slots=(64, 64, 64, 128), chunk_size=8), b=1,
                    prefill=15, steps=2),
    "c3_dims": dict(cfg=dict(heads=1, key_dim=128, value_dim=128, slots=(128, 128, 128, 256), chunk_size=4),
                    b=1, prefill=3, steps=2),
}


@pytest.fixture
def runner(host_runner):
    return host_runner


def _rel(a, b):
    a, b = a.detach().double(), b.detach().double()
    return ((a - b).norm() / max(b.norm().item(), 1e-30)).item()


@pytest.mark.parametrize("name,dtype", [(n, torch.float32) for n in CASES]
                         + [(n, torch.bfloat16) for n in ("tiny_unequal_c3", "c3_dims")],
                         ids=[f"{n}-f32" for n in CASES] + ["tiny_unequal_c3-bf16", "c3_dims-bf16"])
def test_host_built_decode_kernel_matches_oracle(name, dtype, runner, tmp_path, monkeypatch):
    harness.use_host(monkeypatch, harness.HostLib(runner, str(tmp_path)))
    monkeypatch.setattr(dec, "FUSED_DECODE", True)
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
    cfg = model.config
    gen = torch.Generator().manual_seed(5)
    b, n0, steps = spec["b"], spec["prefill"], spec["steps"]
    q = torch.randn(b, n0 + steps, cfg.heads, cfg.key_dim, generator=gen)
    k = torch.nn.functional.normalize(torch.randn(q.shape, generator=gen), dim=-1)
    v = torch.randn(b, n0 + steps, cfg.heads, cfg.value_dim, generator=gen)
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    with torch.no_grad():
        if n0:
            _, ref_state = ref(q[:, :n0], k[:, :n0], v[:, :n0])
            state = copy.deepcopy(ref_state)
        else:
            ref_state, state = None, model.initial_state(b, dtype=dtype)
        for t in range(n0, n0 + steps):
            xs = [x[:, t:t + 1].contiguous() for x in (q, k, v)]
            assert dec.decode_supported(model, *xs, state, None)
            y, state = dec.decode_step(model, *xs, state)
            y_ref, ref_state = ref(*xs, ref_state)
            assert y.dtype == dtype
            assert _rel(y, y_ref) < 1e-5, t
            assert state.chunk_offset == ref_state.chunk_offset and state.position == ref_state.position
            assert (state.frozen is None) == (ref_state.frozen is None)
        for n, (a, r) in enumerate(zip(tensors(state), tensors(ref_state))):
            assert a.shape == r.shape, n
            assert _rel(a, r) < 1e-5, n
