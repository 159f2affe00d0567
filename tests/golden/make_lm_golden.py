"""Write golden vectors for the LM shell from the reference's GPAQwenForCausalLM.

Run in the build container only (the reference and transformers' Qwen3 are
needed; nothing is downloaded):

    python tests/golden/make_lm_golden.py

A tiny Qwen3-architecture all-GPA LM (2 layers, hidden 64, 4 query / 2 KV
heads of width 16, slots (16,16,16,32), chunk 4, vocab 96) is built by the
reference (src/gpa/hf_qwen.py, backend="torch" on the CPU, float32), every
parameter is moved off its initial value with seeded noise, and the
checkpoint is written as tests/golden/lm_tiny/{config.json, model.safetensors}
(the reference config's to_dict() and its state_dict; the reference's own
save_pretrained is not used because it would copy its source file next to the
weights).  tests/golden/lm_tiny_fp32.npz holds the inputs and:
  * train/*: the chunked-CE loss (labels = inputs) in training mode and the
    fingerprint of every parameter gradient;
  * logits: the full logits of the same tokens;
  * cache/*: a 6-token prefill, three one-token calls and a 4-token call
    through GPAQwenCache (logits of each), then every tensor of the cache;
  * rope/logits: the same tokens with keep_rope=True.
Nothing from the reference other than these numbers is written.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REFERENCE = "/root/reference/src"
SAMPLES = 64
BASE = dict(model_type="qwen3", vocab_size=96, hidden_size=64, intermediate_size=96, num_hidden_layers=2,
            num_attention_heads=4, num_key_value_heads=2, head_dim=16, max_position_embeddings=256)
GPA = dict(slots=(16, 16, 16, 32), chunk_size=4, backend="torch", execution="reference")


def fingerprint(x: torch.Tensor) -> np.ndarray:
    """[sum, sum|x|, sum x^2, x.flat[idx] for 64 evenly spaced idx]."""
    flat = x.detach().double().reshape(-1)
    idx = torch.linspace(0, max(flat.numel() - 1, 0), SAMPLES).round().long()
    head = torch.stack((flat.sum(), flat.abs().sum(), flat.square().sum()))
    return torch.cat((head, flat[idx])).numpy()


def perturb(model, seed: int) -> None:
    """Seeded noise on every parameter: absolute scales for the zero or
    identity initialised ones, 20 % of the mean magnitude for the rest."""
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
            p.add_(noise * scale)


def main() -> None:
    sys.path.insert(0, REFERENCE)
    from safetensors.torch import save_file

    from gpa.hf_qwen import GPAQwenConfig, GPAQwenForCausalLM
    torch.manual_seed(0)
    cfg = GPAQwenConfig(base_config=dict(BASE), gpa=dict(GPA), loss_chunk_size=5)
    model = GPAQwenForCausalLM(cfg)
    perturb(model, 1234)
    out_dir = os.path.join(HERE, "lm_tiny")
    os.makedirs(out_dir, exist_ok=True)
    with open(os.path.join(out_dir, "config.json"), "w") as f:
        json.dump(model.config.to_dict(), f, indent=1)
    save_file({k: v.detach().contiguous() for k, v in model.state_dict().items()},
              os.path.join(out_dir, "model.safetensors"), metadata={"format": "pt"})

    g = torch.Generator().manual_seed(7)
    ids = torch.randint(0, BASE["vocab_size"], (2, 13), generator=g)
    store = {"ids": ids.numpy()}
    model.train()
    out = model(ids, labels=ids, use_cache=False)
    out.loss.backward()
    store["train/loss"] = out.loss.detach().numpy()
    names = []
    for name, p in model.named_parameters():
        if p.grad is not None:
            store["train/grad/" + name] = fingerprint(p.grad)
            names.append(name)
    store["train/names"] = np.array(json.dumps(names))
    model.eval()
    with torch.no_grad():
        store["logits"] = model(ids, use_cache=False).logits.numpy()
        cache = None
        pieces = [(0, 6), (6, 7), (7, 8), (8, 9), (9, 13)]
        for n, (lo, hi) in enumerate(pieces):
            res = model(ids[:, lo:hi], past_key_values=cache, use_cache=True)
            cache = res.past_key_values
            store[f"cache/logits{n}"] = res.logits.numpy()
        store["cache/seen"] = np.array(cache.seen_tokens)
        from gpa.state import tensors
        for i, mem in enumerate(cache.layers):
            for n, t in enumerate(tensors(mem.state)):
                store[f"cache/layer{i}/state{n:03d}"] = fingerprint(t)
            store[f"cache/layer{i}/ptail"] = mem.projected_tail.numpy()
            store[f"cache/layer{i}/ctail"] = mem.control_tail.numpy()
        rope_cfg = GPAQwenConfig(base_config=dict(BASE), gpa=dict(GPA), loss_chunk_size=5, keep_rope=True)
        rope_model = GPAQwenForCausalLM(rope_cfg)
        rope_model.load_state_dict(model.state_dict(), strict=True)
        rope_model.eval()
        store["rope/logits"] = rope_model(ids, use_cache=False).logits.numpy()
    np.savez_compressed(os.path.join(HERE, "lm_tiny_fp32.npz"), **store)
    print("wrote", out_dir, "and lm_tiny_fp32.npz:", len(store), "arrays")


if __name__ == "__main__":
    main()
