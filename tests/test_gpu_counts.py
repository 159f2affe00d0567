"""Fused slot counts and base logits (gpa_amd/counts.py, csrc/count_logits.hip)
against the oracle's restatement on the CPU (`OracleRun.counts`,
attention.py:316, and `OracleRun.base_logits` with a learned read scale,
:196-204): logits, final counts and the gradients of raw, write, count0 and of
the raw count gain and log read scale; float32 at 1e-5, bfloat16 at 2e-2 (the
gradients of raw and write are rounded to bf16 in both)."""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _oracle(raw, write, count0, gain_raw, log_scale):
    """The oracle's counts and base logits of one level (learned read scale)."""
    from types import SimpleNamespace

    import oracle
    from gpa_amd import GPAConfig
    h, m = count0.shape[1:]
    cfg = GPAConfig(heads=h, key_dim=8, value_dim=8, slots=(m,), chunk_size=64, learn_read_scale=True)
    run = oracle.OracleRun(SimpleNamespace(config=cfg, count_gain_raw=[gain_raw], read_log_scale=[log_scale]))
    counts = run.counts(count0, write)
    return run.base_logits(raw, counts, None, 0), counts[:, -1]


def _hip(raw, write, count0, gain_raw, log_scale):
    from gpa_amd.counts import count_logits
    return count_logits(raw, write, count0, torch.nn.functional.softplus(gain_raw), log_scale.exp())


@pytest.mark.parametrize("b,t,h,m", [(1, 130, 2, 128), (2, 64, 3, 48), (1, 200, 1, 256), (3, 5, 2, 7)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("with_final", [True, False], ids=["dfinal", "nodfinal"])
def test_count_logits_matches_oracle(b, t, h, m, dtype, with_final):
    g = torch.Generator().manual_seed(b * 100 + t)
    raw = torch.randn(b, t, h, m, generator=g).to(dtype)
    write = torch.rand(b, t, h, m, generator=g).softmax(-1).to(dtype)
    count0 = torch.rand(b, h, m, generator=g) * 5
    gain = torch.rand(h, generator=g) - .5        # raw count gain (softplus inside)
    scale = torch.rand(h, generator=g) - .5       # log read scale, inside its clamp [log .25, log 64]
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

    lg, fc, grads = run(_hip, DEV)
    lr, fr, refs = run(_oracle, "cpu")
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert _rel(lg, lr) < 1e-5 and _rel(fc, fr) < 1e-5
    errs = {n: _rel(a, r) for n, a, r in zip(("raw", "write", "count0", "gain", "scale"), grads, refs)}
    print(b, t, h, m, dtype, errs)
    assert all(e < tol for e in errs.values()), errs
