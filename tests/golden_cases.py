"""Loading and comparing the golden fixtures in tests/golden/*.npz.

A fixture holds the reference's inputs, outputs, carried state and gradients
for one seeded case (written by tests/golden/make_golden.py).  Tensors are
stored whole ("full/<name>") or as a fingerprint ("fp/<name>": sum, sum|x|,
sum x^2 and 64 evenly spaced samples of the flattened tensor).
"""
from __future__ import annotations

import json
import os

import numpy as np
import torch

from gpa_amd import DenseGPA, GPAConfig
from gpa_amd.state import tensors

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SAMPLES = 64
DTYPES = {"float32": torch.float32, "float64": torch.float64, "bfloat16": torch.bfloat16}


def names():
    """The DenseGPA fixtures (operator fixtures start with "ops_" or "moment_", LM
    fixtures with "lm_", counted-core fixtures with "paper_")."""
    return sorted(f[:-4] for f in os.listdir(GOLDEN)
                  if f.endswith(".npz") and not f.startswith(("ops_", "lm_", "paper_", "moment_")))


def ops_names(prefix: str):
    """The operator fixtures whose names start with `prefix` (e.g. "ops_two_stage")."""
    return sorted(f[:-4] for f in os.listdir(GOLDEN) if f.endswith(".npz") and f.startswith(prefix))


class TwoStageCase:
    """A two_stage_gdn fixture (reference src/gpa/ops.py:146-163): inputs, output,
    final states and the input gradients of out.square().mean()."""

    ACT = ("q", "k", "slots", "v")
    ORDER = ("q", "k", "slots", "v", "gi", "bi", "go", "bo", "inner", "outer", "route_weight", "query_weight")

    def __init__(self, name: str):
        self.name = name
        with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
            self.z = {k: z[k] for k in z.files}
        self.dtype = DTYPES[str(self.z["dtype"])]

    def inputs(self, dtype=None):
        """Input tensors by name, activations in `dtype` (default: the fixture's),
        the rest in its work type (float64 for a float64 case, else float32)."""
        dtype = dtype or self.dtype
        work = torch.float64 if dtype == torch.float64 else torch.float32
        return {n: torch.from_numpy(self.z["in/" + n]).to(dtype if n in self.ACT else work)
                for n in self.ORDER if "in/" + n in self.z}

    def ref(self, name: str) -> torch.Tensor:
        return torch.from_numpy(self.z[name]).double()


class Case:
    def __init__(self, name: str):
        self.name = name
        with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
            self.z = {k: z[k] for k in z.files}
        self.cfg = json.loads(str(self.z["config"]))
        self.cfg["slots"] = tuple(self.cfg["slots"])
        self.seed, self.batch, self.length, self.normalize_k, self.control_dim = (
            int(x) for x in self.z["meta"])
        self.dtype = DTYPES[str(self.z["dtype"])]
        self.gate_noise = float(self.z["gate_noise"])
        self.chunk_size = self.cfg["chunk_size"]

    def has(self, name: str) -> bool:
        return ("full/" + name) in self.z or ("fp/" + name) in self.z

    def build(self):
        """Seeded model and inputs, drawn in the fixture script's RNG order."""
        cfg = dict(self.cfg)
        torch.manual_seed(self.seed)
        model = DenseGPA(GPAConfig(**cfg))
        if self.dtype == torch.float64:
            model = model.double()
        if self.gate_noise:
            with torch.no_grad():
                for w in model.gate_weight:
                    w.normal_(0, self.gate_noise)
        gen = torch.float64 if self.dtype == torch.float64 else torch.float32
        h, dk, dv = cfg["heads"], cfg["key_dim"], cfg["value_dim"]
        q = torch.randn(self.batch, self.length, h, dk, dtype=gen)
        k = torch.randn_like(q)
        v = torch.randn(self.batch, self.length, h, dv, dtype=gen)
        if self.normalize_k:
            k = torch.nn.functional.normalize(k, dim=-1)
        ctrl = torch.randn(self.batch, self.length, self.control_dim, dtype=gen) if self.control_dim else None
        q, k, v = (x.to(self.dtype) for x in (q, k, v))
        if ctrl is not None and self.dtype == torch.bfloat16:
            ctrl = ctrl.float()
        return model, q, k, v, ctrl

    def decode_inputs(self):
        return tuple(torch.from_numpy(self.z["full/decode/" + n]).to(self.dtype) if ("full/decode/" + n) in self.z
                     else None for n in ("q", "k", "v"))

    def regen_decode_inputs(self):
        torch.manual_seed(self.seed + 1)
        gen = torch.float64 if self.dtype == torch.float64 else torch.float32
        steps = self.steps()
        h, dk, dv = self.cfg["heads"], self.cfg["key_dim"], self.cfg["value_dim"]
        dq = torch.randn(self.batch, steps, h, dk, dtype=gen)
        dk_ = torch.randn_like(dq)
        dv_ = torch.randn(self.batch, steps, h, dv, dtype=gen)
        if self.normalize_k:
            dk_ = torch.nn.functional.normalize(dk_, dim=-1)
        return tuple(x.to(self.dtype) for x in (dq, dk_, dv_))

    def steps(self) -> int:
        return int(self.z["full/decode/out"].shape[1]) if "full/decode/out" in self.z else 0


def fingerprint(x: torch.Tensor) -> np.ndarray:
    flat = x.detach().double().reshape(-1)
    idx = torch.linspace(0, max(flat.numel() - 1, 0), SAMPLES).round().long()
    head = torch.stack((flat.sum(), flat.abs().sum(), flat.square().sum()))
    return torch.cat((head, flat[idx])).numpy()


def grad_scale(case: Case) -> float:
    """Largest |gradient| stored for the case (whole tensors and fingerprint samples)."""
    top = 0.
    for key, val in case.z.items():
        if key.startswith("full/grad/"):
            top = max(top, float(np.abs(val).max()) if val.size else 0.)
        elif key.startswith("fp/grad/"):
            top = max(top, float(np.abs(val[3:]).max()))
    return top


def compare(case: Case, name: str, x: torch.Tensor, rtol: float, atol: float = 0.) -> str | None:
    """None if `x` matches the fixture entry, else a message.

    Whole tensors: elementwise |d| <= atol + rtol*(|ref| + 0.1*max|ref|), and a
    relative L2 error <= 10*rtol unless the tensor is itself at the `atol`
    (roundoff) level.  Fingerprints: the sum within atol*n + rtol*sum|x|,
    sum|x| and sum x^2 relatively, and the samples elementwise as above.
    """
    x = x.detach().double().cpu()
    if "full/" + name in case.z:
        ref = torch.from_numpy(case.z["full/" + name]).double()
        if ref.shape != x.shape:
            return f"{name}: shape {tuple(x.shape)} != {tuple(ref.shape)}"
        if not ref.numel():
            return None
        scale = ref.abs().max().item()
        rel = ((x - ref).norm() / ref.norm().clamp_min(1e-300)).item()
        worst = ((x - ref).abs() - atol - rtol * (ref.abs() + .1 * scale)).max().item()
        tiny = ref.norm().item() <= 100 * atol * ref.numel() ** .5
        if (rel > 10 * rtol and not tiny) or worst > 0:
            return f"{name}: rel L2 {rel:.3e}, worst excess {worst:.3e} (rtol {rtol}, atol {atol:.1e})"
        return None
    ref = case.z["fp/" + name]
    got = fingerprint(x)
    n = x.numel()
    bad = []
    if abs(got[0] - ref[0]) > atol * n + rtol * max(abs(ref[1]), 1e-300):
        bad.append(f"sum {got[0]:.6e} vs {ref[0]:.6e}")
    for i, label, floor in ((1, "abs-sum", atol * n), (2, "sq-sum", 2 * atol * abs(ref[1]) + atol * atol * n)):
        if abs(got[i] - ref[i]) > floor + rtol * abs(ref[i]):
            bad.append(f"{label} {got[i]:.6e} vs {ref[i]:.6e}")
    err = np.abs(got[3:] - ref[3:]) - atol - rtol * (np.abs(ref[3:]) + .1 * np.abs(ref[3:]).max())
    if (err > 0).any():
        bad.append(f"samples worst excess {err.max():.3e}")
    return f"{name}: " + "; ".join(bad) if bad else None


def compare_state(case: Case, prefix: str, state, rtol: float) -> list[str]:
    errors = []
    meta = case.z[prefix + "/meta"]
    got_meta = [state.position, state.chunk_size, state.chunk_offset, 0 if state.frozen is None else 1]
    if list(meta) != got_meta:
        errors.append(f"{prefix} meta {got_meta} != {list(meta)}")
    for n, x in enumerate(tensors(state)):
        key = f"{prefix}/{n:03d}"
        if not case.has(key):
            errors.append(f"{key}: not in fixture")
            continue
        msg = compare(case, key, x, rtol)
        if msg:
            errors.append(msg)
    return errors


class MomentCase:
    """A moment-scan fixture (reference paper_dense.py:16-58, ops.py:88-118):
    inputs, y, final state and counts, and the input gradients of
    y.square().mean() + final.square().mean() + counts.square().mean()."""

    ACT = ("q", "k", "v", "p")

    def __init__(self, name: str):
        self.name = name
        with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
            self.z = {k: z[k] for k in z.files}
        self.meta = json.loads(str(self.z["meta"]))
        self.dtype = DTYPES[self.meta["dtype"]]
        self.gate = self.meta["gate"]

    def has(self, name: str) -> bool:
        return ("full/" + name) in self.z or ("fp/" + name) in self.z

    def inputs(self, dtype=None, device=None):
        """The seeded inputs in the fixture script's draw order, activations in
        `dtype` (default: the fixture's), the rest in its work type."""
        dtype = dtype or self.dtype
        work = torch.float64 if dtype == torch.float64 else torch.float32
        m = self.meta
        g = torch.Generator().manual_seed(m["seed"])
        b, t, h, kd, vd = m["batch"], m["length"], m["heads"], m["kdim"], m["vdim"]
        f64 = dict(generator=g, dtype=torch.float64)
        x = {"q": torch.randn(b, t, h, kd, **f64), "k": torch.randn(b, t, h, kd, **f64),
             "v": torch.randn(b, t, h, vd, **f64), "s0": torch.randn(b, h, kd, vd, **f64) * .1}
        shape = {"token": (b, t, h), "key": (b, t, h, kd), "value": (b, t, h, vd)}.get(self.gate)
        if shape:
            x["g"] = -torch.rand(*shape, **f64) * .3
        x["p"] = torch.rand(b, t, h, vd, **f64)
        x["n0"] = torch.rand(b, h, vd, **f64)
        x["cg"] = -torch.rand(*(shape if self.gate == "value" else (b, t, h)), **f64) * .3
        return {n: v.to(device=device, dtype=dtype if n in self.ACT else work) for n, v in x.items()}


class PaperCase:
    """A counted-core fixture (reference paper_dense.py:87-278), seeded like
    tests/golden/make_paper_golden.py."""

    def __init__(self, name: str):
        self.name = name
        with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
            self.z = {k: z[k] for k in z.files}
        self.cfg = json.loads(str(self.z["config"]))
        self.cfg["slots"] = tuple(self.cfg["slots"])
        if self.cfg.get("decay_tiers") is not None:
            self.cfg["decay_tiers"] = tuple(self.cfg["decay_tiers"])
        self.seed, self.batch, self.length, self.control_dim = (int(x) for x in self.z["meta"])
        self.dtype = DTYPES[str(self.z["dtype"])]
        self.perturb = float(self.z["perturb"])

    def has(self, name: str) -> bool:
        return ("full/" + name) in self.z or ("fp/" + name) in self.z

    def build(self):
        from gpa_amd.paper_dense import PaperConfig, PaperDenseGPA
        torch.manual_seed(self.seed)
        model = PaperDenseGPA(PaperConfig(**self.cfg))
        if self.dtype == torch.float64:
            model = model.double()
        if self.perturb:
            g = torch.Generator().manual_seed(self.seed + 100)
            with torch.no_grad():
                for pname in ("control_weight", "mlp_down", "relation_prefix", "residual_raw", "level_logits"):
                    p = getattr(model, pname)
                    p.add_(torch.randn(p.shape, generator=g, dtype=p.dtype) * self.perturb)
        gen = torch.float64 if self.dtype == torch.float64 else torch.float32
        h, dk, dv = self.cfg["heads"], self.cfg["key_dim"], self.cfg["value_dim"]
        q = torch.randn(self.batch, self.length, h, dk, dtype=gen)
        k = torch.randn_like(q)
        v = torch.randn(self.batch, self.length, h, dv, dtype=gen)
        ctrl = torch.randn(self.batch, self.length, self.control_dim, dtype=gen) if self.control_dim else None
        q, k, v = (x.to(self.dtype) for x in (q, k, v))
        if ctrl is not None:
            ctrl = ctrl.to(self.dtype)
        return model, q, k, v, ctrl


def paper_names():
    return sorted(f[:-4] for f in os.listdir(GOLDEN) if f.endswith(".npz") and f.startswith("paper_"))


def moment_names():
    return sorted(f[:-4] for f in os.listdir(GOLDEN) if f.endswith(".npz") and f.startswith("moment_"))
