"""Host-side behaviour of the gpa_amd module that needs no GPU: configuration
validation (reference attention.py:45-75 plus the HIP backend's own rules),
state_dict compatibility, cache topology checks and the no-fallback rule."""
from dataclasses import replace

import pytest
import torch

from gpa_amd import DenseGPA, GPAConfig, _lib


@pytest.mark.parametrize("bad", [
    dict(heads=0), dict(chunk_size=0), dict(backend="torch"), dict(backend="fla"), dict(slots=()),
    dict(slots=(4, 0)), dict(positional_mode="x"), dict(beta_init=.95), dict(relation_beta_init=1.),
    dict(decay_init=0.), dict(execution="fast"), dict(read_scale=0.), dict(relation_marginal=True),
    dict(slot_feature="relu"), dict(control_dim=-1), dict(positional_mode="moments", key_dim=5),
])
def test_config_rejects(bad):
    with pytest.raises(ValueError):
        GPAConfig(**bad)


def test_config_defaults_and_edges():
    cfg = GPAConfig()
    assert cfg.backend == "hip" and cfg.chunk_size == 1
    assert cfg.edges == tuple((i, j) for i in range(4) for j in range(4) if i != j)
    replace(cfg, execution="staged")  # accepted and ignored


def test_config_defaults_match_the_reference_field_by_field():
    """Every GPAConfig field, in declaration order, with the reference's
    default (src/gpa/attention.py:17-42, fixture written by
    tests/golden/make_config_defaults.py from that source); `backend` is the
    one deliberate difference ("hip" instead of "torch")."""
    import json
    import os
    from dataclasses import fields
    with open(os.path.join(os.path.dirname(__file__), "golden", "config_defaults.json")) as f:
        ref = json.load(f)["fields"]
    ours = [(fl.name, fl.default) for fl in fields(GPAConfig)]
    assert [n for n, _ in ours] == [n for n, _ in ref]
    for (name, mine), (_, theirs) in zip(ours, ref):
        if name == "backend":
            assert (mine, theirs) == ("hip", "torch")
        elif isinstance(mine, tuple):
            assert list(mine) == theirs, name
        else:
            assert mine == theirs and type(mine) is type(theirs), name


def test_parameter_derived_tensors_are_cached_only_inside_frozen():
    """params.derived recomputes on every call unless the caller opts in with
    params.frozen(store); inside, an entry is dropped when the parameter is
    replaced (p.data = ...), converted (.double()) or updated in place."""
    from gpa_amd import params
    p = torch.nn.Parameter(torch.ones(3))
    calls = []

    def fn():
        calls.append(1)
        return p.detach() * 2

    # outside frozen(): never cached, so in-place and .data updates are seen
    assert torch.equal(params.derived("k", (p,), fn), torch.full((3,), 2.))
    p.data.copy_(torch.full((3,), 5.))
    assert torch.equal(params.derived("k", (p,), fn), torch.full((3,), 10.))
    p.data = torch.full((3,), 7.)
    assert torch.equal(params.derived("k", (p,), fn), torch.full((3,), 14.))
    assert len(calls) == 3
    with params.frozen() as store:
        a = params.derived("k", (p,), fn)
        assert params.derived("k", (p,), fn) is a and len(calls) == 4 and len(store) == 1
        p.data = torch.full((3,), 1.)           # new storage
        assert torch.equal(params.derived("k", (p,), fn), torch.full((3,), 2.)) and len(calls) == 5
        with torch.no_grad():
            p.add_(1.)                           # version counter
        assert torch.equal(params.derived("k", (p,), fn), torch.full((3,), 4.)) and len(calls) == 6
        m = torch.nn.Linear(2, 2)
        m.weight.requires_grad_(False)
        w = params.derived("w", (m.weight,), lambda: m.weight * 1)
        m.double()                               # same Parameter object, new dtype
        assert params.derived("w", (m.weight,), lambda: m.weight * 1).dtype == torch.float64
        assert w.dtype == torch.float32
    # the store belongs to its scope: a new scope starts empty
    with params.frozen() as again:
        assert len(again) == 0
    prints = params.fingerprints([p])
    assert params.unchanged(prints)
    p.data = torch.zeros(3)
    assert not params.unchanged(prints)


def test_state_dict_round_trip_and_names():
    a = DenseGPA(GPAConfig(heads=2, key_dim=4, value_dim=3, slots=(3, 5), chunk_size=4, balanced_bridge=True,
                           learn_read_scale=True, quadratic_features=True))
    b = DenseGPA(a.config)
    b.load_state_dict(a.state_dict(), strict=True)
    # The reference's named_parameters() order (optimizer state is positional):
    # direct parameters first, then the per-level lists, then the feature map.
    names = [n for n, _ in a.named_parameters()]
    assert names == ['residual_raw', 'count_gain_raw', 'moment_gain', 'route_mlp_gain', 'output_logits',
                     'edge_logits', 'relation_gain', 'relation_decay_raw', 'relation_beta_raw', 'bridge_mix_raw',
                     'read_log_scale', 'center.0', 'center.1', 'inner_prefix.0', 'inner_prefix.1',
                     'outer_prefix.0', 'outer_prefix.1', 'route_weight.0', 'route_weight.1', 'query_weight.0',
                     'query_weight.1', 'route_up.0', 'route_up.1', 'route_down.0', 'route_down.1',
                     'gate_weight.0', 'gate_weight.1', 'gate_bias.0', 'gate_bias.1', 'relation_prefix.0',
                     'relation_prefix.1', 'feature_map.left', 'feature_map.right', 'feature_map.gain_raw']
    assert "_edge_source" not in a.state_dict()


def test_initial_state_layout():
    m = DenseGPA(GPAConfig(heads=2, key_dim=4, value_dim=3, slots=(3, 5), chunk_size=4))
    s = m.initial_state(3)
    assert s.levels[0].inner.shape == (3, 2, 4, 3) and s.levels[1].outer.shape == (3, 2, 5, 3)
    assert s.relations[0].memory.shape == (3, 2, 3, 5) and s.relations[1].memory.shape == (3, 2, 5, 3)
    assert s.numel() == 3 * 2 * (4 * 3 + 3 * 3 + 3 + 4 * 5 + 5 * 3 + 5 + 2 * 15)
    assert s.chunk_size == 4 and s.chunk_offset == 0 and s.frozen is None


def test_forward_validation_and_no_cpu_fallback():
    m = DenseGPA(GPAConfig(heads=2, key_dim=4, value_dim=3, slots=(3,), chunk_size=4))
    q = torch.randn(1, 5, 2, 4)
    v = torch.randn(1, 5, 2, 3)
    with pytest.raises(ValueError):
        m(q, q, torch.randn(1, 5, 2, 4))
    with pytest.raises(ValueError):
        m(q, q, v, position_ids=torch.arange(4))
    other = DenseGPA(GPAConfig(heads=2, key_dim=4, value_dim=3, slots=(3, 3), chunk_size=4)).initial_state(1)
    with pytest.raises(ValueError):
        m(q, q, v, other)
    with pytest.raises(_lib.HipBackendError):
        m(q, q, v)


def test_reference_signature_ops_validate_like_the_reference():
    from gpa_amd.ops import gdn_scan
    x = torch.zeros(1, 3, 2, 4)
    with pytest.raises(ValueError, match="q/k must share"):
        gdn_scan(x, torch.zeros(1, 3, 2, 5), x, torch.zeros(1, 3, 2), torch.zeros(1, 3, 2), None)
    with pytest.raises(ValueError, match="scalar per token"):
        gdn_scan(x, x, x, torch.zeros(1, 3, 2, 1), torch.zeros(1, 3, 2), None)
    s0 = torch.zeros(1, 2, 4, 4)
    out, final = gdn_scan(x[:, :0], x[:, :0], x[:, :0], torch.zeros(1, 0, 2), torch.zeros(1, 0, 2), s0)
    assert out.shape == (1, 0, 2, 4) and final is s0
    with pytest.raises(ValueError, match="unknown backend"):
        gdn_scan(x, x, x, torch.zeros(1, 3, 2), torch.zeros(1, 3, 2), s0, backend="torch")


def test_gradient_graph_refuses_captures_over_the_row_limit():
    """GradientGraph refuses steps of MAX_CAPTURE_ROWS rows (batch x tokens)
    or more before it touches the device: captures that large are switched
    off (the B=1, T=8192 training step's capture ended in a host segfault)."""
    from gpa_amd import GradientGraph
    from gpa_amd.graph import MAX_CAPTURE_ROWS
    model = DenseGPA(GPAConfig(heads=1, key_dim=8, value_dim=8, slots=(4, 4)))
    xs = [torch.zeros(2, MAX_CAPTURE_ROWS // 2, 1, 8) for _ in range(3)]
    with pytest.raises(NotImplementedError, match="switched off"):
        GradientGraph(model, xs, lambda *a: None)
