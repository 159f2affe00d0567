"""Fused slot counts and base logits (gpa_amd/counts.py, csrc/count_logits.hip)
against the reference's torch expression (attention.py:196-204 with the
counts of :318-319) on the GPU: logits, final counts and the gradients of raw,
write, count0, gain and scale; float32 at 1e-5, bfloat16 at 2e-2 (the
gradients of raw and write are rounded to bf16 in both)."""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _torch_ref(raw, write, count0, gain, scale):
    counts = count0[:, None] + write.float().cumsum(1)
    logits = scale[:, None] * raw.float() + gain[:, None] * counts.log1p()
    return logits, counts[:, -1]


@pytest.mark.parametrize("b,t,h,m", [(1, 130, 2, 128), (2, 64, 3, 48), (1, 200, 1, 256), (3, 5, 2, 7)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("with_final", [True, False], ids=["dfinal", "nodfinal"])
def test_count_logits_matches_torch(b, t, h, m, dtype, with_final):
    from gpa_amd.counts import count_logits
    g = torch.Generator().manual_seed(b * 100 + t)
    raw = torch.randn(b, t, h, m, generator=g).to(dtype)
    write = torch.rand(b, t, h, m, generator=g).softmax(-1).to(dtype)
    count0 = torch.rand(b, h, m, generator=g) * 5
    gain = torch.rand(h, generator=g) + .1
    scale = torch.rand(h, generator=g) + .5
    wl = torch.randn(b, t, h, m, generator=g)
    wf = torch.randn(b, h, m, generator=g)

    def run(fn, dev):
        xs = [x.to(dev).requires_grad_() for x in (raw, write, count0, gain, scale)]
        logits, final = fn(*xs)
        loss = (logits * wl.to(dev)).sum()
        if with_final:
            loss = loss + (final * wf.to(dev)).sum()
        loss.backward()
        return logits, final, [x.grad for x in xs]

    lg, fc, grads = run(count_logits, DEV)
    lr, fr, refs = run(_torch_ref, "cpu")
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert _rel(lg, lr) < 1e-5 and _rel(fc, fr) < 1e-5
    errs = {n: _rel(a, r) for n, a, r in zip(("raw", "write", "count0", "gain", "scale"), grads, refs)}
    print(b, t, h, m, dtype, errs)
    assert all(e < tol for e in errs.values()), errs
