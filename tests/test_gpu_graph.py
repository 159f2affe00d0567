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
