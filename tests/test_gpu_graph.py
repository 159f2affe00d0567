"""GradientGraph (reference src/gpa/training_graph.py:10-39) on the HIP backend:
a captured DenseGPA forward+backward replayed with fresh inputs reproduces an
eager run of an identical model, replay after replay, with eager work and
synchronisations in between (a graph node that only replays correctly once
would show up here)."""
import copy

import pytest
import torch

from gpa_amd import DenseGPA, GPAConfig, GradientGraph

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_captured_step_replays_match_eager(dtype):
    torch.manual_seed(0)
    cfg = GPAConfig(heads=2, key_dim=32, value_dim=48, slots=(64, 64, 64, 128), chunk_size=64)
    model = DenseGPA(cfg).to(DEV)
    eager = copy.deepcopy(model)
    shape_q, shape_v = (1, 130, 2, 32), (1, 130, 2, 48)

    def inputs(seed):
        g = torch.Generator().manual_seed(seed)
        return [torch.randn(shape_q, generator=g).to(DEV, dtype).requires_grad_(),
                torch.randn(shape_q, generator=g).to(DEV, dtype).requires_grad_(),
                torch.randn(shape_v, generator=g).to(DEV, dtype).requires_grad_()]

    def loss_fn(m):
        def f(q, k, v):
            out, _ = m(q, k, v)
            return out.float().square().mean(), out
        return f

    graph = GradientGraph(model, inputs(100), loss_fn(model), warmups=2)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    for seed in (1, 2, 3):
        xs = inputs(seed)
        loss, out = graph.replay(*xs)
        torch.cuda.synchronize()
        got_out, got_loss = out.clone(), loss.clone()
        got_grads = {n: p.grad.clone() for n, p in model.named_parameters() if p.grad is not None}
        got_in = [x.grad.clone() for x in graph.inputs]
        eager.zero_grad(set_to_none=True)
        ex = [x.detach().clone().requires_grad_() for x in xs]
        e_loss, e_out = loss_fn(eager)(*ex)
        e_loss.backward()
        torch.cuda.synchronize()
        assert _rel(got_out, e_out) < tol and _rel(got_loss, e_loss) < tol, seed
        top = max(p.grad.norm().item() for p in eager.parameters() if p.grad is not None)
        for n, p in eager.named_parameters():
            if p.grad is None:
                continue
            err = (got_grads[n] - p.grad).norm().item() / max(p.grad.norm().item(), 1e-3 * top)
            assert err < tol, (seed, n, err)
        for a, b in zip(got_in, ex):
            assert _rel(a, b.grad) < tol, seed


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_decode_graph_matches_eager_decode(dtype):
    """DecodeGraph: one graph per block position; three blocks of one-token
    steps (every graph replays three times, with the block-boundary state copy
    and eager checks in between) give the eager decode's outputs and cache."""
    from gpa_amd.graph import DecodeGraph
    from gpa_amd.state import tensors
    torch.manual_seed(3)
    cfg = GPAConfig(heads=2, key_dim=32, value_dim=48, slots=(64, 64, 64, 128), chunk_size=4)
    model = DenseGPA(cfg).to(DEV)
    b = 3
    g = torch.Generator(device=DEV).manual_seed(9)

    def token():
        q = torch.randn(b, 1, 2, 32, device=DEV, generator=g).to(dtype)
        k = torch.nn.functional.normalize(torch.randn(b, 1, 2, 32, device=DEV, generator=g), dim=-1).to(dtype)
        return q, k, torch.randn(b, 1, 2, 48, device=DEV, generator=g).to(dtype)

    toks = [token() for _ in range(12)]
    with torch.no_grad():
        state = model.initial_state(b, device=DEV, dtype=dtype)
        graphed = DecodeGraph(model, state, *toks[0])
        for i, x in enumerate(toks):
            y_graph = graphed.step(*x).clone()
            torch.cuda.synchronize()
            y_eager, state = model(*x, state)
            assert _rel(y_graph, y_eager) < 1e-6, i
            if (i + 1) % cfg.chunk_size == 0:
                got = graphed.state
                assert got.position == state.position == i + 1
                for a, r in zip(tensors(got), tensors(state)):
                    assert _rel(a, r) < 1e-6, i


def test_gradient_graph_replays_match_oracle():
    """Replays of a captured float32 forward+backward (C2 widths, two heads,
    two blocks and a partial one) against the oracle's forward and autograd on
    the CPU: output, loss, every parameter gradient and the input gradients,
    for two different inputs."""
    import oracle
    torch.manual_seed(1)
    cfg = GPAConfig(heads=2, key_dim=32, value_dim=48, slots=(64, 64, 64, 128), chunk_size=64)
    cpu_model = DenseGPA(cfg)
    model = copy.deepcopy(cpu_model).to(DEV)
    shape_q, shape_v = (2, 130, 2, 32), (2, 130, 2, 48)

    def inputs(seed):
        g = torch.Generator().manual_seed(seed)
        return [torch.randn(shape_q, generator=g), torch.randn(shape_q, generator=g),
                torch.randn(shape_v, generator=g)]

    def loss_fn(q, k, v):
        out, _ = model(q, k, v)
        return out.float().square().mean(), out

    graph = GradientGraph(model, [x.to(DEV).requires_grad_() for x in inputs(100)], loss_fn, warmups=2)
    for seed in (7, 8):
        xs = inputs(seed)
        loss, out = graph.replay(*(x.to(DEV) for x in xs))
        torch.cuda.synchronize()
        ref_model = copy.deepcopy(cpu_model)
        rs = [x.clone().requires_grad_() for x in xs]
        r_out, _ = oracle.OracleRun(ref_model)(*rs)
        r_loss = r_out.float().square().mean()
        r_loss.backward()
        assert _rel(out, r_out) < 1e-4 and _rel(loss, r_loss) < 1e-4, seed
        top = max(p.grad.norm().item() for p in ref_model.parameters() if p.grad is not None)
        for (n, p), (_, r) in zip(model.named_parameters(), ref_model.named_parameters()):
            if r.grad is None:
                continue
            err = (p.grad.cpu() - r.grad).norm().item() / max(r.grad.norm().item(), 1e-3 * top)
            assert err < 1e-4, (seed, n, err)
        for a, b in zip(graph.inputs, rs):
            assert _rel(a.grad, b.grad) < 1e-4, seed


def test_decode_graph_outputs_hold_until_their_position_replays():
    """The output of position o stays valid while the following positions of
    the block and the first positions of the next block replay (until o
    itself replays): kept without copies, it equals the eager decode's."""
    from gpa_amd.graph import DecodeGraph
    torch.manual_seed(4)
    cfg = GPAConfig(heads=2, key_dim=32, value_dim=48, slots=(64, 64, 64, 128), chunk_size=4)
    model = DenseGPA(cfg).to(DEV)
    b = 2
    g = torch.Generator(device=DEV).manual_seed(5)
    toks = [(torch.randn(b, 1, 2, 32, device=DEV, generator=g),
             torch.nn.functional.normalize(torch.randn(b, 1, 2, 32, device=DEV, generator=g), dim=-1),
             torch.randn(b, 1, 2, 48, device=DEV, generator=g)) for _ in range(6)]
    with torch.no_grad():
        state = model.initial_state(b, device=DEV, dtype=torch.float32)
        graphed = DecodeGraph(model, state, *toks[0])
        kept = [graphed.step(*x) for x in toks[:4]]        # one whole block, no clones
        later = [graphed.step(*x).clone() for x in toks[4:6]]  # positions 0 and 1 of the next block
        torch.cuda.synchronize()
        eager = []
        for x in toks:
            y, state = model(*x, state)
            eager.append(y)
    for o in (2, 3):  # not replayed since
        assert _rel(kept[o], eager[o]) < 1e-6, o
    for i, y in enumerate(later):
        assert _rel(y, eager[4 + i]) < 1e-6, i


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_decode_graph_matches_oracle_at_c3_widths(dtype):
    """The graphed decode the benchmark times, at config-3 widths (Dk = Dv =
    128, slots (128,128,128,256), chunk 64) with two heads and two sequences:
    a 64-token prefill, then 65 graphed one-token steps (a whole block and one
    step into the next), against the oracle's cached calls on the CPU: every
    step's output and the whole cache at the block boundary."""
    import oracle
    from gpa_amd.graph import DecodeGraph
    from gpa_amd.state import tensors
    torch.manual_seed(6)
    cfg = GPAConfig(heads=2, key_dim=128, value_dim=128, slots=(128, 128, 128, 256), chunk_size=64)
    cpu_model = DenseGPA(cfg)
    model = copy.deepcopy(cpu_model).to(DEV)
    ref = oracle.OracleRun(cpu_model)
    b, steps = 2, 65
    g = torch.Generator().manual_seed(7)

    def draw(t):
        q = torch.randn(b, t, 2, 128, generator=g)
        k = torch.nn.functional.normalize(torch.randn(b, t, 2, 128, generator=g), dim=-1)
        return q.to(dtype), k.to(dtype), torch.randn(b, t, 2, 128, generator=g).to(dtype)

    pre = draw(64)
    toks = [draw(1) for _ in range(steps)]
    tol = TOL_DEC[dtype]
    with torch.no_grad():
        _, state = model(*(x.to(DEV) for x in pre))
        _, r_state = ref(*pre)
        graphed = DecodeGraph(model, state, *(x.to(DEV) for x in toks[0]))
        for i, x in enumerate(toks):
            y = graphed.step(*(t.to(DEV) for t in x))
            y_ref, r_state = ref(*x, r_state)
            assert _rel(y, y_ref) < tol, (i, _rel(y, y_ref))
            if i == 63:
                got = graphed.state
                assert got.position == r_state.position == 128 and r_state.chunk_offset == 0
                for n, (a, r) in enumerate(zip(tensors(got), tensors(r_state))):
                    assert _rel(a, r) < tol, (n, _rel(a, r))


TOL_DEC = {torch.float32: 1e-4, torch.bfloat16: 2e-2}


@pytest.mark.parametrize("packed", [False, True], ids=["streams", "packed"])
def test_capture_keeps_the_schedule_on_the_capturing_stream(packed, monkeypatch):
    """Graphs are captured single-stream: while a GradientGraph or a
    DecodeGraph captures, the schedule runs its independent scans in order on
    the capturing stream and never takes its side streams (no cross-stream
    fork/join or allocator stream records inside a capture).  With one call
    per scan group the eager warm-up calls of the training step do take them;
    with packed scan calls (the default) no call takes a side stream."""
    from gpa_amd import schedule
    from gpa_amd.graph import DecodeGraph
    seen = []
    real = schedule._side_streams

    def spy(device):
        seen.append(torch.cuda.is_current_stream_capturing())
        return real(device)

    monkeypatch.setattr(schedule, "_side_streams", spy)
    monkeypatch.setattr(schedule, "_SERIAL", [False])
    monkeypatch.setattr(schedule, "_PACKED", [packed])
    torch.manual_seed(2)
    cfg = GPAConfig(heads=2, key_dim=32, value_dim=48, slots=(64, 64, 64, 128), chunk_size=4)
    model = DenseGPA(cfg).to(DEV)
    g = torch.Generator().manual_seed(3)
    xs = [torch.randn(2, 9, 2, d, generator=g).to(DEV).requires_grad_() for d in (32, 32, 48)]

    def loss_fn(q, k, v):
        out, _ = model(q, k, v)
        return out.float().square().mean(), out

    GradientGraph(model, xs, loss_fn, warmups=1)
    assert not any(seen), "side streams taken while capturing the training step"
    assert packed or seen, "the eager warm-up of the stream schedule took no side stream"
    eager_calls = len(seen)
    seen.clear()
    with torch.no_grad():
        tok = [x[:, :1].detach() for x in xs]
        DecodeGraph(model, model.initial_state(2, device=DEV, dtype=torch.float32), *tok, warmups=1)
    # (one-token decode packs its independent steps into single launches and
    # may take no side stream at all)
    assert not any(seen), "side streams taken while capturing a decode step"
    assert packed or eager_calls > 0


def test_gradient_graph_capture_accumulates_on_the_capturing_stream(monkeypatch):
    """The warm-up's autograd graph is released before the capture, so the
    captured backward creates its own gradient-accumulation nodes on the
    capturing stream.  A node reused from the warm-up keeps the warm-up
    stream, which would put the captured accumulation on a stream outside
    the capture; torch reports that reuse as a stream-mismatch warning.  (The
    warm-up runs on one stream here, so the capture is the only place such a
    mismatch can come from.)"""
    import warnings

    from gpa_amd import schedule
    monkeypatch.setattr(schedule, "_SERIAL", [True])
    torch.manual_seed(5)
    cfg = GPAConfig(heads=2, key_dim=32, value_dim=48, slots=(64, 64, 64, 128), chunk_size=4)
    model = DenseGPA(cfg).to(DEV)
    g = torch.Generator().manual_seed(6)
    xs = [torch.randn(1, 10, 2, d, generator=g).to(DEV).requires_grad_() for d in (32, 32, 48)]

    def loss_fn(q, k, v):
        out, _ = model(q, k, v)
        return out.float().square().mean(), out

    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter("always")
        graph = GradientGraph(model, xs, loss_fn, warmups=2)
        graph.replay(*xs)
        torch.cuda.synchronize()
    assert not [w for w in rec if "AccumulateGrad" in str(w.message)], [str(w.message)[:120] for w in rec]
