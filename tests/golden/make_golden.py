"""Write golden vectors for the oracle from the reference package.

Run in the build container only (the reference is not present elsewhere):

    python tests/golden/make_golden.py

It imports the reference `gpa` package from /root/reference/src, runs the
cases below on the CPU with ``backend="torch"`` and stores inputs, outputs,
carried state and gradients under tests/golden/*.npz.  Small tensors are stored
whole; large ones as a fingerprint (sum, sum|x|, sum x^2 and 64 strided
samples, see `fingerprint`).  Nothing from the reference other than these
numbers is written.
"""
from __future__ import annotations

import json
import os
import sys
from dataclasses import asdict

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REFERENCE = "/root/reference/src"
FULL_LIMIT = 2_048  # larger tensors are fingerprinted ...
WHOLE = ("out", "partition_out", "decode/out", "grad/in_")  # ... except these
SAMPLES = 64


def fingerprint(x: torch.Tensor) -> np.ndarray:
    """[sum, sum|x|, sum x^2, x.flat[idx] for 64 evenly spaced idx]."""
    flat = x.detach().double().reshape(-1)
    idx = torch.linspace(0, max(flat.numel() - 1, 0), SAMPLES).round().long()
    head = torch.stack((flat.sum(), flat.abs().sum(), flat.square().sum()))
    return torch.cat((head, flat[idx] if flat.numel() else torch.zeros(SAMPLES, dtype=torch.double))).numpy()


def put(store: dict, name: str, x: torch.Tensor | None):
    if x is None:
        return
    x = x.detach()
    if x.numel() <= FULL_LIMIT or name.startswith(WHOLE):
        store["full/" + name] = x.float().numpy() if x.dtype == torch.bfloat16 else x.numpy()
    else:
        store["fp/" + name] = fingerprint(x)


def put_state(store: dict, prefix: str, state):
    from gpa.state import tensors  # reference package
    for n, x in enumerate(tensors(state)):
        put(store, f"{prefix}/{n:03d}", x)
    store[f"{prefix}/meta"] = np.array([state.position, state.chunk_size, state.chunk_offset,
                                        0 if state.frozen is None else 1])


def run_case(name, cfg_kwargs, *, seed, batch, length, dtype, normalize_k=False, control_dim=0,
             gate_noise=0.0, partitions=None, decode_steps=0, grads=True):
    from gpa import DenseGPA, GPAConfig
    torch.manual_seed(seed)
    cfg = GPAConfig(**cfg_kwargs)
    model = DenseGPA(cfg)
    if dtype == torch.float64:
        model = model.double()
    if gate_noise:
        with torch.no_grad():
            for w in model.gate_weight:
                w.normal_(0, gate_noise)
    h, dk, dv = cfg.heads, cfg.key_dim, cfg.value_dim
    gen_dtype = torch.float64 if dtype == torch.float64 else torch.float32
    q = torch.randn(batch, length, h, dk, dtype=gen_dtype)
    k = torch.randn_like(q)
    v = torch.randn(batch, length, h, dv, dtype=gen_dtype)
    if normalize_k:
        k = torch.nn.functional.normalize(k, dim=-1)
    ctrl = torch.randn(batch, length, control_dim, dtype=gen_dtype) if control_dim else None
    q, k, v = (x.to(dtype).requires_grad_(grads) for x in (q, k, v))
    if ctrl is not None:
        ctrl = ctrl.to(dtype if dtype != torch.bfloat16 else torch.float32).requires_grad_(grads)
    store: dict = {"config": np.array(json.dumps({k2: v2 for k2, v2 in asdict(cfg).items()
                                                  if k2 not in ("backend", "execution")})),
                   "meta": np.array([seed, batch, length, int(normalize_k), control_dim]),
                   "dtype": np.array(str(dtype).replace("torch.", "")),
                   "gate_noise": np.array(gate_noise)}
    for pname, p in model.named_parameters():
        put(store, "param/" + pname, p)
    put(store, "in/q", q)
    put(store, "in/k", k)
    put(store, "in/v", v)
    put(store, "in/control", ctrl)
    out, state = model(q, k, v, control_input=ctrl)
    put(store, "out", out)
    put_state(store, "state", state)
    if grads:
        out.float().square().mean().backward()
        for pname, p in model.named_parameters():
            if p.grad is not None:
                put(store, "grad/" + pname, p.grad)
        for label, x in (("q", q), ("k", k), ("v", v), ("control", ctrl)):
            if x is not None:
                put(store, "grad/in_" + label, x.grad)
    with torch.no_grad():
        if partitions:
            running, parts = None, []
            for lo, hi in partitions:
                y, running = model(q[:, lo:hi], k[:, lo:hi], v[:, lo:hi], running,
                                   control_input=ctrl[:, lo:hi] if ctrl is not None else None)
                parts.append(y)
            put(store, "partition_out", torch.cat(parts, 1))
            store["partitions"] = np.array(partitions)
        if decode_steps:
            torch.manual_seed(seed + 1)
            dq = torch.randn(batch, decode_steps, h, dk, dtype=gen_dtype)
            dkk = torch.randn_like(dq)
            dvv = torch.randn(batch, decode_steps, h, dv, dtype=gen_dtype)
            if normalize_k:
                dkk = torch.nn.functional.normalize(dkk, dim=-1)
            dq, dkk, dvv = (x.to(dtype) for x in (dq, dkk, dvv))
            put(store, "decode/q", dq)
            put(store, "decode/k", dkk)
            put(store, "decode/v", dvv)
            running, ys = state, []
            for t in range(decode_steps):
                y, running = model(dq[:, t:t + 1], dkk[:, t:t + 1], dvv[:, t:t + 1], running)
                ys.append(y)
            put(store, "decode/out", torch.cat(ys, 1))
            put_state(store, "decode/state", running)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **store)
    print(name, "arrays:", len(store), flush=True)


CASES = {
    # The reference's own CPU case: tokenwise recurrent model, fp32.
    "c1_token_fp32": dict(cfg_kwargs=dict(heads=4, key_dim=32, value_dim=48, slots=(64, 64, 64, 128),
                                          positional_mode="gated", chunk_size=1),
                          seed=0, batch=2, length=16, dtype=torch.float32, decode_steps=1),
    # Block-lagged chunk model, tiny dims, three positional modes, cached partitions.
    "chunk_gated_fp64": dict(cfg_kwargs=dict(heads=2, key_dim=4, value_dim=3, slots=(3, 2, 4), chunk_size=3),
                             seed=11, batch=2, length=9, dtype=torch.float64,
                             partitions=[(0, 2), (2, 3), (3, 7), (7, 9)], decode_steps=2),
    "chunk_none_fp64": dict(cfg_kwargs=dict(heads=2, key_dim=4, value_dim=3, slots=(3, 2, 4), chunk_size=4,
                                            positional_mode="none"),
                            seed=12, batch=2, length=9, dtype=torch.float64, partitions=[(0, 5), (5, 9)]),
    "chunk_moments_fp64": dict(cfg_kwargs=dict(heads=2, key_dim=4, value_dim=3, slots=(3, 2, 4), chunk_size=4,
                                               positional_mode="moments"),
                               seed=13, batch=2, length=9, dtype=torch.float64, partitions=[(0, 6), (6, 9)]),
    # The flags an all-GPA LM layer enables, with full hidden controls.
    "chunk_lmflags_fp64": dict(cfg_kwargs=dict(heads=2, key_dim=4, value_dim=3, slots=(4, 4), chunk_size=4,
                                               control_dim=5, rsa_update=True, paper_product_read=True,
                                               shared_query_center=True, balanced_bridge=True,
                                               relation_marginal=True, read_scale=8., beta_init=.6,
                                               decay_init=1e-4),
                               seed=14, batch=1, length=10, dtype=torch.float64, control_dim=5,
                               gate_noise=.1, partitions=[(0, 3), (3, 10)]),
    "chunk_features_fp64": dict(cfg_kwargs=dict(heads=2, key_dim=4, value_dim=3, slots=(3, 5, 3), chunk_size=3,
                                                slot_feature="tanh", quadratic_features=True,
                                                learn_read_scale=True, rsa_update=True),
                                seed=15, batch=1, length=8, dtype=torch.float64),
    "chunk_softmaxslot_fp64": dict(cfg_kwargs=dict(heads=1, key_dim=4, value_dim=4, slots=(4, 3), chunk_size=2,
                                                   slot_feature="softmax"),
                                   seed=16, batch=2, length=5, dtype=torch.float64),
    # Config-2 dimensions, two full blocks plus a partial one.
    "c2_dims_fp64": dict(cfg_kwargs=dict(heads=4, key_dim=32, value_dim=48, slots=(64, 64, 64, 128),
                                         chunk_size=64),
                         seed=2, batch=1, length=130, dtype=torch.float64, partitions=[(0, 70), (70, 130)]),
    # Config-3 dimensions at two heads, fp32 and bf16, with a 3-token decode.
    "c3_dims_fp32": dict(cfg_kwargs=dict(heads=2, key_dim=128, value_dim=128, slots=(128, 128, 128, 256),
                                         chunk_size=64),
                         seed=3, batch=1, length=130, dtype=torch.float32, normalize_k=True, decode_steps=3),
    "c3_dims_bf16": dict(cfg_kwargs=dict(heads=2, key_dim=128, value_dim=128, slots=(128, 128, 128, 256),
                                         chunk_size=64),
                         seed=4, batch=1, length=70, dtype=torch.bfloat16, normalize_k=True),
}


def run_two_stage(name, *, seed, batch, length, heads, key_dim, slots, value_dim, dtype, weights=True):
    """The reference's two_stage_gdn (ops.py:146-163) on seeded inputs: output,
    both final states and the gradient of every input of out.square().mean()."""
    from gpa import TwoStageState, two_stage_gdn
    g = torch.Generator().manual_seed(seed)
    b, t, h, dk, m, dv = batch, length, heads, key_dim, slots, value_dim
    raw = {"q": torch.randn(b, t, h, dk, generator=g, dtype=torch.float64),
           "k": torch.randn(b, t, h, dk, generator=g, dtype=torch.float64),
           "slots": torch.randn(b, t, h, m, generator=g, dtype=torch.float64),
           "v": torch.randn(b, t, h, dv, generator=g, dtype=torch.float64),
           "gi": -torch.rand(b, t, h, generator=g, dtype=torch.float64) * .3,
           "bi": torch.rand(b, t, h, generator=g, dtype=torch.float64),
           "go": -torch.rand(b, t, h, generator=g, dtype=torch.float64) * .3,
           "bo": torch.rand(b, t, h, generator=g, dtype=torch.float64),
           "inner": torch.randn(b, h, dk, m, generator=g, dtype=torch.float64) * .1,
           "outer": torch.randn(b, h, m, dv, generator=g, dtype=torch.float64) * .1}
    if weights:
        raw["route_weight"] = torch.randn(m, m, generator=g, dtype=torch.float64) / m ** .5
        raw["query_weight"] = torch.randn(m, dk, generator=g, dtype=torch.float64) / dk ** .5
    act = ("q", "k", "slots", "v")
    work = torch.float64 if dtype == torch.float64 else torch.float32
    x = {n: t_.to(dtype if n in act else work).requires_grad_() for n, t_ in raw.items()}
    state = TwoStageState(x["inner"], x["outer"])
    out, new = two_stage_gdn(x["q"], x["k"], x["slots"], x["v"], x["gi"], x["bi"], x["go"], x["bo"], state,
                             route_weight=x.get("route_weight"), query_weight=x.get("query_weight"))
    out.float().square().mean().backward()
    store = {"dtype": np.array(str(dtype).replace("torch.", ""))}
    for n, t_ in x.items():
        store["in/" + n] = t_.detach().float().numpy() if t_.dtype == torch.bfloat16 else t_.detach().numpy()
        store["grad/" + n] = (t_.grad.float() if t_.grad.dtype == torch.bfloat16 else t_.grad).numpy()
    store["out"] = out.detach().float().numpy() if out.dtype == torch.bfloat16 else out.detach().numpy()
    store["inner"] = new.inner.detach().numpy()
    store["outer"] = new.outer.detach().numpy()
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **store)
    print(name, "arrays:", len(store), flush=True)


# Operator-level fixtures (names start with "ops_"; not DenseGPA cases).
OPS_CASES = {
    "ops_two_stage_fp64": dict(seed=21, batch=2, length=37, heads=2, key_dim=8, slots=6, value_dim=5,
                               dtype=torch.float64),
    "ops_two_stage_fp32": dict(seed=22, batch=1, length=70, heads=2, key_dim=16, slots=12, value_dim=10,
                               dtype=torch.float32),
    "ops_two_stage_plain_fp32": dict(seed=23, batch=2, length=20, heads=3, key_dim=8, slots=5, value_dim=7,
                                     dtype=torch.float32, weights=False),
    "ops_two_stage_bf16": dict(seed=24, batch=1, length=70, heads=2, key_dim=16, slots=12, value_dim=10,
                               dtype=torch.bfloat16),
}


def main(names):
    if not os.path.isdir(REFERENCE):
        raise SystemExit("reference package not found; golden vectors are written in the build container")
    sys.path.insert(0, REFERENCE)
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    for name in names or [*CASES, *OPS_CASES]:
        if name in OPS_CASES:
            run_two_stage(name, **OPS_CASES[name])
        else:
            run_case(name, **CASES[name])


if __name__ == "__main__":
    main(sys.argv[1:])
