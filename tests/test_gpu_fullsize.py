"""Size-independent properties of the HIP backend at the full benchmark sizes.

The oracle cannot run these sizes in seconds, so they are checked through
properties the model guarantees at any size:
  * config 3 (B=1, T=8192, H=16, Dk=Dv=128, slots (128,128,128,256), chunk 64,
    bf16, K L2-normalised): forward+backward gives finite outputs and finite
    gradients of every parameter and input; a call split into cached calls
    (at 4096, block-aligned, and at 4100, inside a block) gives the output and
    cache of the whole call; the level memories do not depend on Q
    (attention.py:309-329 never reads it, reference tests/test_gpa.py:107-115);
  * config 4 (the same layer, batch 64, a 2048-token prefill, then one-token
    steps): the prefill split at 1024 equals the whole prefill, and the graphed
    decode equals eager decode for a block's first steps;
  * config 2 (B=8, T=1024, H=4, Dk=32, Dv=48, slots (64,64,64,128), chunk 64,
    fp32): the same finiteness, partition and Q-independence properties.
The kernels at these shapes are compared with the oracle at reduced head
counts and lengths elsewhere (test_gpu_dense_gpa.py, test_gpu_graph.py)."""
import pytest
import torch

from gpa_amd import DenseGPA, GPAConfig
from gpa_amd.state import tensors

pytestmark = pytest.mark.gpu
DEV = "cuda"
C3 = dict(heads=16, key_dim=128, value_dim=128, slots=(128, 128, 128, 256), chunk_size=64)


def _rel(a, b):
    a, b = a.detach().double(), b.detach().double()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _inputs(b, t, seed, dtype=torch.bfloat16):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(b, t, 16, 128, device=DEV, generator=g)
    k = torch.nn.functional.normalize(torch.randn(b, t, 16, 128, device=DEV, generator=g), dim=-1)
    v = torch.randn(b, t, 16, 128, device=DEV, generator=g)
    return q.to(dtype), k.to(dtype), v.to(dtype)


@pytest.fixture(scope="module")
def c3_model():
    torch.manual_seed(0)
    return DenseGPA(GPAConfig(**C3)).to(DEV)


def test_c3_forward_backward_is_finite(c3_model):
    print("C3 full size: B=1 T=8192 H=16 bf16 forward+backward", flush=True)
    c3_model.zero_grad(set_to_none=True)
    xs = [x.requires_grad_() for x in _inputs(1, 8192, 1)]
    out, state = c3_model(*xs)
    loss = out.float().square().mean()
    loss.backward()
    torch.cuda.synchronize()
    assert out.shape == (1, 8192, 16, 128) and out.dtype == torch.bfloat16
    assert torch.isfinite(out).all() and torch.isfinite(loss)
    assert all(torch.isfinite(t).all() for t in tensors(state))
    for n, p in c3_model.named_parameters():
        if n == "moment_gain":  # read only by positional_mode="moments" (attention.py:202-203)
            assert p.grad is None
            continue
        assert p.grad is not None and torch.isfinite(p.grad).all(), n
    for x in xs:
        assert torch.isfinite(x.grad).all() and x.grad.abs().sum() > 0
    c3_model.zero_grad(set_to_none=True)


@pytest.mark.parametrize("cut", [4096, 4100])
def test_c3_cached_calls_equal_the_whole_call(c3_model, cut):
    print("C3 full size: partition at", cut, flush=True)
    q, k, v = _inputs(1, 8192, 2)
    with torch.no_grad():
        whole, s_whole = c3_model(q, k, v)
        y1, s1 = c3_model(q[:, :cut], k[:, :cut], v[:, :cut])
        y2, s2 = c3_model(q[:, cut:], k[:, cut:], v[:, cut:], s1)
    assert s2.position == 8192 and s2.chunk_offset == s_whole.chunk_offset == 0
    assert _rel(torch.cat((y1, y2), 1), whole) < 1e-2
    for a, b in zip(tensors(s2), tensors(s_whole)):
        assert _rel(a, b) < 1e-3


def test_c3_level_memories_do_not_depend_on_q(c3_model):
    print("C3 full size: Q-independence of the level memories", flush=True)
    q, k, v = _inputs(1, 8192, 3)
    with torch.no_grad():
        y1, s1 = c3_model(q, k, v)
        y2, s2 = c3_model((q.float() * -2 + .5).to(q.dtype), k, v)
    for a, b in zip(s1.levels, s2.levels):
        assert torch.equal(a.inner, b.inner) and torch.equal(a.outer, b.outer) and torch.equal(a.count, b.count)
    assert not torch.equal(y1, y2)


def test_c4_prefill_partition_and_graphed_decode(c3_model):
    print("C4 full size: B=64 prefill 2048 (split at 1024) then graphed decode", flush=True)
    from gpa_amd.graph import DecodeGraph
    q, k, v = _inputs(64, 2048, 4)
    with torch.no_grad():
        _, s_whole = c3_model(q, k, v)
        _, s1 = c3_model(q[:, :1024], k[:, :1024], v[:, :1024])
        _, s2 = c3_model(q[:, 1024:], k[:, 1024:], v[:, 1024:], s1)
        del s1
        for a, b in zip(tensors(s2), tensors(s_whole)):
            assert _rel(a, b) < 1e-3
        del s2
        toks = [_inputs(64, 1, 10 + i) for i in range(4)]
        graphed = DecodeGraph(c3_model, s_whole, *toks[0])
        state = s_whole
        for i, x in enumerate(toks):
            y_graph = graphed.step(*x)
            y_eager, state = c3_model(*x, state)
            assert torch.isfinite(y_eager).all()
            assert _rel(y_graph, y_eager) < 1e-6, i


C2 = dict(heads=4, key_dim=32, value_dim=48, slots=(64, 64, 64, 128), chunk_size=64)


def _c2_inputs(seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(8, 1024, 4, 32, device=DEV, generator=g)
    k = torch.randn(8, 1024, 4, 32, device=DEV, generator=g)
    v = torch.randn(8, 1024, 4, 48, device=DEV, generator=g)
    return q, k, v


def test_c2_full_size_properties():
    """Config 2 at its full size (B=8, T=1024, H=4, Dk=32, Dv=48, slots
    (64,64,64,128), chunk 64, fp32): forward+backward is finite with a
    gradient for every parameter; the call split into cached calls at 512
    (block-aligned) and 515 (inside a block) gives the whole call's output and
    cache; the level memories do not depend on Q."""
    print("C2 full size: B=8 T=1024 H=4 fp32 forward+backward", flush=True)
    torch.manual_seed(0)
    model = DenseGPA(GPAConfig(**C2)).to(DEV)
    xs = [x.requires_grad_() for x in _c2_inputs(5)]
    out, state = model(*xs)
    loss = out.square().mean()
    loss.backward()
    assert out.shape == (8, 1024, 4, 48) and out.dtype == torch.float32
    assert torch.isfinite(out).all() and torch.isfinite(loss)
    assert all(torch.isfinite(t).all() for t in tensors(state))
    for n, p in model.named_parameters():
        if n == "moment_gain":
            continue
        assert p.grad is not None and torch.isfinite(p.grad).all(), n
    for x in xs:
        assert torch.isfinite(x.grad).all() and x.grad.abs().sum() > 0
    q, k, v = (x.detach() for x in xs)
    with torch.no_grad():
        whole, s_whole = model(q, k, v)
        assert _rel(whole, out) < 1e-6
        for cut in (512, 515):
            print("C2 full size: partition at", cut, flush=True)
            y1, s1 = model(q[:, :cut], k[:, :cut], v[:, :cut])
            y2, s2 = model(q[:, cut:], k[:, cut:], v[:, cut:], s1)
            assert s2.position == 1024 and s2.chunk_offset == 0
            assert _rel(torch.cat((y1, y2), 1), whole) < 1e-5
            for a, b in zip(tensors(s2), tensors(s_whole)):
                assert _rel(a, b) < 1e-5
        y3, s3 = model(q * -2 + .5, k, v)
    for a, b in zip(s_whole.levels, s3.levels):
        assert torch.equal(a.inner, b.inner) and torch.equal(a.outer, b.outer) and torch.equal(a.count, b.count)
    assert not torch.equal(y3, whole)
