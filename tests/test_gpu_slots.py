"""Fused slot products and gate inputs (gpa_amd/slots.py, csrc/slot_gates.hip)
against the oracle's restatement of the reference's bf16 einsums on the CPU
(`OracleRun.slot`, attention.py:176-177, and `OracleRun.gate_inputs`, :162-165):
slot, raw and the gradients of key, center and gate_weight, at the bf16 bar 2e-2.
Also the row tails (T not a multiple of 64), several heads and batches, and
the widest shapes (Dk = M = 256)."""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _reference(key, center, gate_w):
    """The oracle's slot product and gate input of one level with these weights."""
    from types import SimpleNamespace

    import oracle
    from gpa_amd import GPAConfig
    h, m, d = center.shape
    cfg = GPAConfig(heads=h, key_dim=d, value_dim=8, slots=(m,), chunk_size=64)
    run = oracle.OracleRun(SimpleNamespace(config=cfg, center=[center], gate_weight=[gate_w]))
    return run.slot(key, 0), run.gate_inputs(key, 0, None)


@pytest.mark.parametrize("b,t,h,d,m", [(1, 130, 2, 128, 128), (2, 64, 3, 64, 96), (1, 200, 1, 256, 256),
                                       (3, 5, 2, 32, 32), (64, 1, 16, 128, 256), (1, 2048, 16, 128, 128)])
def test_slot_gates_match_typed_einsums(b, t, h, d, m):
    from gpa_amd.slots import slot_gates
    g = torch.Generator().manual_seed(b * 1000 + t + d)
    key = torch.nn.functional.normalize(torch.randn(b, t, h, d, generator=g), dim=-1).to(torch.bfloat16)
    key[0, 0, 0] = 0  # a zero row: the clamped-norm branch of unit()
    center = torch.randn(h, m, d, generator=g) / d ** .5
    gate_w = torch.randn(h, d, 4, generator=g) * .3
    ws = torch.randn(b, t, h, m, generator=g)
    wr = torch.randn(b, t, h, 4, generator=g)

    def run(fn, dev):
        xs = [x.to(dev).requires_grad_() for x in (key, center, gate_w)]
        slot, raw = fn(*xs)
        loss = (slot.float() * ws.to(dev)).sum() + (raw.float() * wr.to(dev)).sum()
        loss.backward()
        return [slot, raw] + [x.grad for x in xs]

    got = run(slot_gates, DEV)
    ref = run(_reference, "cpu")
    names = ["slot", "raw", "dkey", "dcenter", "dgate_w"]
    for n, a, r in zip(names, got, ref):
        assert a.shape == r.shape and a.dtype == r.dtype, n
        assert torch.isfinite(a).all(), n
        err = _rel(a, r)
        assert err < 2e-2, (n, err)


def test_slot_gates_repeated_calls_clear_their_sums():
    """dgate_w and dcenter are sums the library clears itself: two backward
    passes give the same gradients."""
    from gpa_amd.slots import slot_gates
    g = torch.Generator().manual_seed(7)
    key = torch.randn(1, 96, 2, 64, generator=g).to(torch.bfloat16).to(DEV)
    center = (torch.randn(2, 64, 64, generator=g) / 8).to(DEV)
    gate_w = torch.randn(2, 64, 4, generator=g).to(DEV)
    grads = []
    for _ in range(2):
        xs = [x.clone().requires_grad_() for x in (key, center, gate_w)]
        slot, raw = slot_gates(*xs)
        (slot.float().square().sum() + raw.float().sum()).backward()
        grads.append([x.grad.clone() for x in xs])
    for a, b in zip(*grads):
        assert torch.equal(a, b)
