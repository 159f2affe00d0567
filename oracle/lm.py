"""CPU restatement of the reference's all-GPA Qwen LM (src/gpa/hf_qwen.py).

TEST INFRASTRUCTURE ONLY, like the rest of `oracle`: imported by tests/ and
never by the `gpa_amd` product.

`OracleLM(lm)` reads the weights of any module with the reference's parameter
names (`gpa_amd.lm.GPALMForCausalLM` on the CPU is one) and runs the
reference's forward with plain tensor ops, every GPA core through the DenseGPA
oracle (`oracle.reference.OracleRun`).  Autograd reaches the module's
parameters, so gradients compare too.  Pinned by the reference-written
fixtures of tests/golden/make_lm_golden.py (tests/test_oracle_golden.py).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor

from .reference import OracleRun


def rms_norm(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    """Qwen RMSNorm: statistics in float32, the normalised value rounded to
    x's dtype, then times the weight (transformers Qwen3RMSNorm, used by
    hf_qwen.py:137-138, :195-197, :216)."""
    h = x.float()
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    return weight * h.to(x.dtype)


def causal_conv(x: Tensor, weight: Tensor, tail: Tensor | None):
    """hf_qwen.py:118-124: depthwise causal convolution with a carried tail."""
    width = weight.shape[-1] - 1
    prefix = x.new_zeros(x.shape[0], x.shape[-1], width) if tail is None else tail.to(x.dtype)
    joined = torch.cat((prefix, x.transpose(1, 2)), -1)
    out = F.conv1d(joined, weight.to(x.dtype), groups=x.shape[-1]).transpose(1, 2)
    return out, joined[:, :, -width:] if width else joined[:, :, :0]


def rotate_half(x: Tensor) -> Tensor:
    """hf_qwen.py:127-129."""
    a, b = x.chunk(2, -1)
    return torch.cat((-b, a), -1)


def rotary(head_dim: int, theta: float, positions: Tensor, dtype) -> tuple[Tensor, Tensor]:
    """The Qwen rotary embedding (cos, sin) at positions [B,T]: inverse
    frequencies theta^(-2i/d), the angle table repeated over both halves."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    emb = torch.cat([positions.float()[..., None] * inv] * 2, -1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


class OracleLM:
    def __init__(self, lm, attention_dtype: torch.dtype | None = None):
        self.lm = lm
        self.cfg = lm.config
        self.attention_dtype = attention_dtype
        self.cores = [OracleRun(layer.self_attn.gpa) for layer in lm.model.layers]

    def attention(self, i: int, hidden: Tensor, rope, memory):
        """GPAQwenAttention.forward (hf_qwen.py:161-190); memory = (state,
        projected_tail, control_tail) or None."""
        att = self.lm.model.layers[i].self_attn
        cfg = self.cfg
        b, t, _ = hidden.shape
        h, kv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim

        def linear(mod, x):
            return F.linear(x, mod.weight, mod.bias)

        projected = torch.cat((linear(att.q_proj, hidden), linear(att.k_proj, hidden), linear(att.v_proj, hidden)),
                              -1)
        projected, ptail = causal_conv(projected, att.projected_conv, None if memory is None else memory[1])
        control, ctail = causal_conv(hidden, att.control_conv, None if memory is None else memory[2])
        q, k, v = projected.split((h * d, kv * d, kv * d), -1)
        q, k, v = q.reshape(b, t, h, d), k.reshape(b, t, kv, d), v.reshape(b, t, kv, d)
        if cfg.model_type == "qwen3":
            q = rms_norm(q, att.q_norm.weight, cfg.rms_norm_eps)
            k = rms_norm(k, att.k_norm.weight, cfg.rms_norm_eps)
        if rope is not None:
            cos, sin = (x[:, :, None].to(q.dtype) for x in rope)
            q = q * cos + rotate_half(q) * sin
            k = k * cos + rotate_half(k) * sin
        k, v = (x.repeat_interleave(h // kv, dim=2) for x in (k, v))
        if self.attention_dtype is not None:
            q, k, v = (x.to(self.attention_dtype) for x in (q, k, v))
        out, state = self.cores[i](q, k, v, None if memory is None else memory[0], control_input=F.silu(control))
        out = linear(att.o_proj, out.reshape(b, t, -1).to(hidden.dtype))
        return out, (state, ptail, ctail)

    def __call__(self, ids: Tensor, labels: Tensor | None = None, cache: dict | None = None):
        """(loss, logits, cache) of GPAQwenForCausalLM.forward (hf_qwen.py:
        348-407); cache = {"layers": [...], "seen": n} or None for a fresh
        stream.  The loss is the chunked mean cross entropy of :388-400."""
        cfg, lm = self.cfg, self.lm
        hidden = F.embedding(ids, lm.model.embed_tokens.weight)
        b, t, _ = hidden.shape
        seen = 0 if cache is None else cache["seen"]
        rope = None
        if cfg.keep_rope:
            pos = torch.arange(seen, seen + t)[None].expand(b, -1)
            rope = rotary(cfg.head_dim, cfg.rope_theta, pos, hidden.dtype)
        new_layers = []
        for i, layer in enumerate(lm.model.layers):
            x = rms_norm(hidden, layer.input_layernorm.weight, cfg.rms_norm_eps)
            branch, memory = self.attention(i, x, rope, None if cache is None else cache["layers"][i])
            new_layers.append(memory)
            hidden = hidden + branch
            x = rms_norm(hidden, layer.post_attention_layernorm.weight, cfg.rms_norm_eps)
            mlp = layer.mlp
            hidden = hidden + F.linear(F.silu(F.linear(x, mlp.gate_proj.weight)) * F.linear(x, mlp.up_proj.weight),
                                       mlp.down_proj.weight)
        hidden = rms_norm(hidden, lm.model.norm.weight, cfg.rms_norm_eps)
        head = lm.lm_head.weight
        loss = logits = None
        if labels is not None:
            count = (labels[:, 1:] != -100).sum().clamp_min(1)
            loss = hidden.sum() * 0.
            for start in range(0, t - 1, cfg.loss_chunk_size):
                stop = min(t - 1, start + cfg.loss_chunk_size)
                x, y = hidden[:, start:stop], labels[:, start + 1:stop + 1]
                value = F.cross_entropy(F.linear(x, head).float().reshape(-1, cfg.vocab_size), y.reshape(-1),
                                        reduction="sum", ignore_index=-100)
                loss = loss + value / count
        else:
            logits = F.linear(hidden, head)
        return loss, logits, {"layers": new_layers, "seen": seen + t}
