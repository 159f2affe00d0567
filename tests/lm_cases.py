"""The LM-shell fixtures written by tests/golden/make_lm_golden.py.

tests/golden/lm_tiny/ is a reference-written checkpoint (config.json +
model.safetensors) of a tiny all-GPA Qwen3 LM; tests/golden/lm_tiny_fp32.npz
holds the reference's numbers for it.  Entries named in FINGERPRINTED are
fingerprints (sum, sum|x|, sum x^2, 64 samples); the rest are whole arrays.
`LMCase` exposes them through the keys `golden_cases.compare` reads.
"""
from __future__ import annotations

import json
import os

import numpy as np
import torch

from tests.golden_cases import GOLDEN, compare

CHECKPOINT = os.path.join(GOLDEN, "lm_tiny")
FINGERPRINTED = ("train/grad/", "cache/layer")
PIECES = [(0, 6), (6, 7), (7, 8), (8, 9), (9, 13)]  # the cached calls of cache/logits{n}


class LMCase:
    def __init__(self):
        with np.load(os.path.join(GOLDEN, "lm_tiny_fp32.npz"), allow_pickle=False) as z:
            raw = {k: z[k] for k in z.files}
        self.z = {}
        for k, v in raw.items():
            fp = k.startswith(FINGERPRINTED) and not k.endswith(("ptail", "ctail"))
            self.z[("fp/" if fp else "full/") + k] = v
        self.ids = torch.from_numpy(raw["ids"]).long()
        self.grad_names = json.loads(str(raw["train/names"]))

    def compare(self, name: str, x: torch.Tensor, rtol: float, atol: float = 0.) -> str | None:
        return compare(self, name, x, rtol, atol)

    def grad_scale(self) -> float:
        return max(float(np.abs(v[3:]).max()) for k, v in self.z.items() if k.startswith("fp/train/grad/"))


def perturb(model, seed: int) -> None:
    """Seeded noise on every parameter of an LM (the scheme the fixture
    script applies): absolute scales for the zero- or identity-initialised
    ones, 20 % of the mean magnitude for the rest."""
    absolute = {"relation_prefix": .1, "gate_weight": .05, "residual_raw": .8, "output_logits": .8,
                "edge_logits": .8, "bridge_mix_raw": .8, "query_weight": .05, "projected_conv": .2,
                "control_conv": .1}
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            noise = torch.randn(p.shape, generator=g, dtype=torch.float64).float()
            parts = name.split(".")
            key = next((k for k in absolute if k in parts), None)
            if key is not None:
                scale = absolute[key]
            elif "route_weight" in parts:
                scale = .2 / p.shape[-1] ** .5
            else:
                scale = .2 * p.abs().mean().item()
            p.add_(noise.to(p.device) * scale)
