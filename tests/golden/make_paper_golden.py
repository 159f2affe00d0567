"""Write golden vectors of the reference's counted dense core and its moment
recurrences (src/gpa/paper_dense.py, src/gpa/ops.py:88-118).

Run in the build container only (the reference is not present elsewhere):

    python tests/golden/make_paper_golden.py

It imports the reference `gpa` package from /root/reference/src, runs the
cases below on the CPU with ``backend="torch"`` and stores inputs, outputs,
carried state and gradients under tests/golden/paper_*.npz and
tests/golden/moment_*.npz, in the storage format of make_golden.py (small
tensors whole, large ones as fingerprints).  Nothing from the reference other
than these numbers is written.
"""
from __future__ import annotations

import json
import os
import sys
from dataclasses import asdict

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
from make_golden import REFERENCE, put, put_state  # noqa: E402


def run_paper(name, cfg_kwargs, *, seed, batch, length, dtype, control_dim=0, partitions=None, perturb=0.0):
    from gpa.paper_dense import PaperConfig, PaperDenseGPA
    torch.manual_seed(seed)
    cfg = PaperConfig(**cfg_kwargs)
    model = PaperDenseGPA(cfg)
    if dtype == torch.float64:
        model = model.double()
    if perturb:  # move the zero-initialised parameters off their initial values
        g = torch.Generator().manual_seed(seed + 100)
        with torch.no_grad():
            for pname in ("control_weight", "mlp_down", "relation_prefix", "residual_raw", "level_logits"):
                p = getattr(model, pname)
                p.add_(torch.randn(p.shape, generator=g, dtype=p.dtype) * perturb)
    h, dk, dv = cfg.heads, cfg.key_dim, cfg.value_dim
    gen = torch.float64 if dtype == torch.float64 else torch.float32
    q = torch.randn(batch, length, h, dk, dtype=gen)
    k = torch.randn_like(q)
    v = torch.randn(batch, length, h, dv, dtype=gen)
    ctrl = torch.randn(batch, length, control_dim, dtype=gen) if control_dim else None
    q, k, v = (x.to(dtype).requires_grad_() for x in (q, k, v))
    if ctrl is not None:
        ctrl = ctrl.to(dtype).requires_grad_()
    store: dict = {"config": np.array(json.dumps({a: b for a, b in asdict(cfg).items() if a != "backend"})),
                   "meta": np.array([seed, batch, length, control_dim]),
                   "dtype": np.array(str(dtype).replace("torch.", "")),
                   "perturb": np.array(perturb)}
    for pname, p in model.named_parameters():
        put(store, "param/" + pname, p)
    for label, x in (("q", q), ("k", k), ("v", v), ("control", ctrl)):
        put(store, "in/" + label, x)
    out, state = model(q, k, v, control_input=ctrl)
    put(store, "out", out)
    put_state(store, "state", state)
    out.float().square().mean().backward()
    for pname, p in model.named_parameters():
        if p.grad is not None:
            put(store, "grad/" + pname, p.grad)
    for label, x in (("q", q), ("k", k), ("v", v), ("control", ctrl)):
        if x is not None:
            put(store, "grad/in_" + label, x.grad)
    if partitions:
        with torch.no_grad():
            running, parts = None, []
            for lo, hi in partitions:
                y, running = model(q[:, lo:hi], k[:, lo:hi], v[:, lo:hi], running,
                                   control_input=ctrl[:, lo:hi] if ctrl is not None else None)
                parts.append(y)
            put(store, "partition_out", torch.cat(parts, 1))
            put_state(store, "partition_state", running)
            store["partitions"] = np.array(partitions)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **store)
    print(name, "arrays:", len(store), flush=True)


def run_moment(name, *, seed, batch, length, heads, kdim, vdim, gate, dtype):
    """moment_scan (gate "token", "key", "value") or linear_scan (gate "none") and
    decayed_counts on seeded inputs: outputs, final state and every input gradient
    of y.square().mean() + final.square().mean()."""
    from gpa.ops import linear_scan
    from gpa.paper_dense import decayed_counts, moment_scan
    g = torch.Generator().manual_seed(seed)
    work = torch.float64 if dtype == torch.float64 else torch.float32
    b, t, h = batch, length, heads
    x = {"q": torch.randn(b, t, h, kdim, generator=g, dtype=torch.float64),
         "k": torch.randn(b, t, h, kdim, generator=g, dtype=torch.float64),
         "v": torch.randn(b, t, h, vdim, generator=g, dtype=torch.float64),
         "s0": torch.randn(b, h, kdim, vdim, generator=g, dtype=torch.float64) * .1}
    shape = {"token": (b, t, h), "key": (b, t, h, kdim), "value": (b, t, h, vdim)}.get(gate)
    if shape:
        x["g"] = -torch.rand(*shape, generator=g, dtype=torch.float64) * .3
    x["p"] = torch.rand(b, t, h, vdim, generator=g, dtype=torch.float64)
    x["n0"] = torch.rand(b, h, vdim, generator=g, dtype=torch.float64)
    x["cg"] = -torch.rand(*(shape if gate == "value" else (b, t, h)), generator=g, dtype=torch.float64) * .3
    act = ("q", "k", "v", "p")
    x = {n: t_.to(dtype if n in act else work).requires_grad_() for n, t_ in x.items()}
    if gate == "none":
        y, final = linear_scan(x["q"], x["k"], x["v"], x["s0"])
    else:
        y, final = moment_scan(x["q"], x["k"], x["v"], x["g"], x["s0"], "torch",
                               axis="value" if gate == "value" else "key")
    counts = decayed_counts(x["p"], x["cg"], x["n0"])
    loss = y.float().square().mean() + final.float().square().mean() + counts.float().square().mean()
    loss.backward()
    store = {"meta": np.array(json.dumps(dict(seed=seed, batch=b, length=t, heads=h, kdim=kdim, vdim=vdim,
                                                gate=gate, dtype=str(dtype).replace("torch.", ""))))}
    for n, t_ in x.items():
        put(store, "in/" + n, t_)
        if t_.grad is not None:
            put(store, "grad/" + n, t_.grad)
    put(store, "out/y", y)
    put(store, "out/final", final)
    put(store, "out/counts", counts)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **store)
    print(name, "arrays:", len(store), flush=True)


PAPER = {
    # The reference test's shapes (tests/test_paper_dense.py:23-28), one per read mode.
    "paper_local_fp64": dict(cfg_kwargs=dict(heads=2, key_dim=4, value_dim=3, slots=(3, 3, 3), chunk_size=3),
                             seed=3, batch=2, length=7, dtype=torch.float64, partitions=[(0, 2), (2, 7)]),
    "paper_transport_fp64": dict(cfg_kwargs=dict(heads=2, key_dim=4, value_dim=3, slots=(3, 3, 3), chunk_size=3,
                                                 dense_read="transport"),
                                 seed=3, batch=2, length=7, dtype=torch.float64, partitions=[(0, 4), (4, 7)]),
    "paper_slot_fp64": dict(cfg_kwargs=dict(heads=2, key_dim=4, value_dim=3, slots=(3, 3, 3), chunk_size=3,
                                            dense_read="transport", slot_decay=True),
                            seed=3, batch=2, length=7, dtype=torch.float64, perturb=.1),
    "paper_strong_fp64": dict(cfg_kwargs=dict(heads=2, key_dim=4, value_dim=3, slots=(3, 3, 3), chunk_size=3,
                                              dense_read="transport", slot_decay=True, strong_relations=True),
                              seed=3, batch=2, length=7, dtype=torch.float64, perturb=.1),
    "paper_control_fp64": dict(cfg_kwargs=dict(heads=2, key_dim=4, value_dim=3, slots=(4, 4), chunk_size=4,
                                               control_dim=5, normalize_features=False, use_relations=False),
                               seed=5, batch=1, length=9, dtype=torch.float64, control_dim=5, perturb=.1),
    # Default widths, two full blocks of 64 and a partial one, fp32.
    "paper_default_fp32": dict(cfg_kwargs=dict(heads=2, key_dim=32, value_dim=32, slots=(16, 16, 16, 16),
                                               chunk_size=64),
                               seed=6, batch=1, length=130, dtype=torch.float32, perturb=.05,
                               partitions=[(0, 70), (70, 130)]),
    # The reference's FLA parity shape (tests/test_paper_dense.py:53-56) in bf16, with slot decay.
    "paper_slot_bf16": dict(cfg_kwargs=dict(heads=2, key_dim=32, value_dim=32, slots=(16, 16), chunk_size=64,
                                            slot_decay=True),
                            seed=7, batch=1, length=128, dtype=torch.bfloat16),
}

MOMENT = {
    "moment_none_fp64": dict(seed=21, batch=2, length=9, heads=2, kdim=5, vdim=3, gate="none", dtype=torch.float64),
    "moment_token_fp64": dict(seed=22, batch=2, length=9, heads=2, kdim=5, vdim=3, gate="token",
                              dtype=torch.float64),
    "moment_key_fp64": dict(seed=23, batch=2, length=9, heads=2, kdim=5, vdim=3, gate="key", dtype=torch.float64),
    "moment_value_fp64": dict(seed=24, batch=2, length=9, heads=2, kdim=5, vdim=3, gate="value",
                              dtype=torch.float64),
    "moment_key_fp32": dict(seed=25, batch=1, length=70, heads=2, kdim=32, vdim=16, gate="key", dtype=torch.float32),
    "moment_value_bf16": dict(seed=26, batch=1, length=70, heads=2, kdim=32, vdim=16, gate="value",
                              dtype=torch.bfloat16),
}


def main():
    sys.path.insert(0, REFERENCE)
    torch.set_num_threads(4)
    for name, kw in MOMENT.items():
        run_moment(name, **kw)
    for name, kw in PAPER.items():
        run_paper(name, **kw)


if __name__ == "__main__":
    main()
