"""A Qwen2/Qwen3-architecture causal LM whose attention layers are DenseGPA cores on the HIP backend.

The reference's consumer of the attention core is its Hugging Face wrapper
`GPAQwenForCausalLM` (src/gpa/hf_qwen.py:20-407).  This module rebuilds that
model in plain PyTorch around `gpa_amd.DenseGPA`, keeping what a user of the
reference relies on:

* the same module tree and parameter names, so checkpoints load strictly both
  ways (``model.layers.N.self_attn.gpa.center.0``, ``...self_attn.projected_conv``,
  ``...mlp.gate_proj.weight``, ``lm_head.weight`` ...);
* the same attention block (hf_qwen.py:132-190): q/k/v projections, a causal
  depthwise short convolution over the projected channels and another over
  the hidden state (the GPA gate control), both carrying their tails across
  cached calls; q/k RMSNorm; grouped K/V heads repeated to the query heads;
  the GPA defaults of hf_qwen.py:145-151 (rsa_update, product read, shared
  query centre, balanced bridge, read scale 8, beta .6, decay 1e-4, chunk 64,
  control_dim = hidden); newly added query weights start at zero;
* the recurrent cache (`GPALMCache`, hf_qwen.py:92-115): no growing K/V, only
  the convolution tails and every layer's GPA state, with reorder / repeat /
  detach;
* per-layer activation checkpointing for training (hf_qwen.py:376-383) and
  the chunked cross entropy (hf_qwen.py:388-400);
* the checkpoint format: ``config.json`` in the reference config's layout and
  ``model.safetensors`` (hf_qwen.py:249-289), see `save_pretrained` /
  `from_pretrained`.

The GPA core runs with its own precision policy: q, k and v are handed over in
`attention_dtype` (bfloat16 by default, as the reference hands its GPU core
bfloat16, hf_qwen.py:184-186) and the core runs outside autocast, so its
rounding points are the core's own whatever the caller's autocast state.
Everything else is ordinary PyTorch (GEMMs on hipBLASLt).
"""
from __future__ import annotations

import json
import os
from dataclasses import asdict, dataclass, field, fields, is_dataclass

import torch
import torch.nn.functional as F
from torch import Tensor, nn
from torch.utils.checkpoint import checkpoint as _checkpoint

from .config import GPAConfig
from .module import DenseGPA

# GPA options an LM layer takes unless `gpa` overrides them (hf_qwen.py:145-151).
LAYER_DEFAULTS = dict(chunk_size=64, rsa_update=True, paper_product_read=True, shared_query_center=True,
                      balanced_bridge=True, beta_init=.6, decay_init=.0001, read_scale=8.)

# Native-architecture defaults of the two supported families (the Hugging Face
# Qwen3Config / Qwen2Config defaults), used for fields a base config omits.
_NATIVE_DEFAULTS = {
    "qwen3": dict(vocab_size=151936, hidden_size=4096, intermediate_size=22016, num_hidden_layers=32,
                  num_attention_heads=32, num_key_value_heads=32, head_dim=128, rms_norm_eps=1e-6,
                  rope_theta=10000., tie_word_embeddings=False, initializer_range=.02, attention_bias=False,
                  max_position_embeddings=32768),
    "qwen2": dict(vocab_size=151936, hidden_size=4096, intermediate_size=22016, num_hidden_layers=32,
                  num_attention_heads=32, num_key_value_heads=32, head_dim=None, rms_norm_eps=1e-6,
                  rope_theta=10000., tie_word_embeddings=False, initializer_range=.02, attention_bias=True,
                  max_position_embeddings=32768),
}


@dataclass
class GPALMConfig:
    """Architecture of the LM (defaults: Qwen3-0.6B) plus the GPA-wrapper
    fields of the reference's GPAQwenConfig (hf_qwen.py:20-46)."""
    model_type: str = "qwen3"
    vocab_size: int = 151936
    hidden_size: int = 1024
    intermediate_size: int = 3072
    num_hidden_layers: int = 28
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    head_dim: int = 128
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1000000.
    tie_word_embeddings: bool = True
    initializer_range: float = .02
    attention_bias: bool = False
    max_position_embeddings: int = 40960
    convolution: int = 4
    loss_chunk_size: int = 512
    keep_rope: bool = False
    gpa: dict = field(default_factory=dict)
    gpa_last_slots: tuple | None = None
    attention_dtype: str | None = "bfloat16"

    def __post_init__(self):
        if self.model_type not in _NATIVE_DEFAULTS:
            raise ValueError("Only native Qwen2/Qwen2.5 and Qwen3 causal LMs are supported")
        if self.convolution < 1 or self.loss_chunk_size < 1:
            raise ValueError("convolution and loss_chunk_size must be positive")
        if self.num_attention_heads % self.num_key_value_heads:
            raise ValueError("Query heads must be divisible by KV heads")
        if self.attention_dtype not in (None, "bfloat16", "float32"):
            raise ValueError("attention_dtype must be None, 'bfloat16' or 'float32'")
        self.gpa = dict(self.gpa)
        if self.gpa_last_slots is not None:
            self.gpa_last_slots = tuple(self.gpa_last_slots)

    @property
    def qk_norm(self) -> bool:
        """Qwen3 normalises q and k per head; Qwen2 does not (hf_qwen.py:137-138)."""
        return self.model_type == "qwen3"

    def layer_gpa(self, index: int) -> GPAConfig:
        """The GPAConfig of layer `index` (hf_qwen.py:140-155, :205-212)."""
        options = dict(self.gpa)
        options.setdefault("slots", (self.head_dim, self.head_dim))
        if index == self.num_hidden_layers - 1 and self.gpa_last_slots is not None:
            options["slots"] = self.gpa_last_slots
        options["slots"] = tuple(options["slots"])
        inherited = dict(heads=self.num_attention_heads, key_dim=self.head_dim, value_dim=self.head_dim,
                         control_dim=self.hidden_size)
        for key, value in inherited.items():
            if options.setdefault(key, value) != value:
                raise ValueError(f"{key} must match the inherited native Qwen projections")
        for key, value in LAYER_DEFAULTS.items():
            options.setdefault(key, value)
        # this package is the HIP backend; the reference's backend/execution
        # choices (fla, staged) name its own schedules
        options["backend"] = "hip"
        return GPAConfig(**options)

    # ------------------------------------------------------------ reference layout
    def to_reference_dict(self) -> dict:
        """config.json in the layout of the reference's GPAQwenConfig.to_dict()."""
        base = {"model_type": self.model_type, "vocab_size": self.vocab_size, "hidden_size": self.hidden_size,
                "intermediate_size": self.intermediate_size, "num_hidden_layers": self.num_hidden_layers,
                "num_attention_heads": self.num_attention_heads, "num_key_value_heads": self.num_key_value_heads,
                "head_dim": self.head_dim, "rms_norm_eps": self.rms_norm_eps, "rope_theta": self.rope_theta,
                "tie_word_embeddings": self.tie_word_embeddings, "initializer_range": self.initializer_range,
                "attention_bias": self.attention_bias, "max_position_embeddings": self.max_position_embeddings}
        gpa = asdict(self.layer_gpa(0))
        gpa["slots"] = list(gpa["slots"])
        gpa.update(backend="hip")
        out = {k: base[k] for k in ("vocab_size", "hidden_size", "num_hidden_layers", "num_attention_heads",
                                     "num_key_value_heads", "max_position_embeddings", "initializer_range",
                                     "tie_word_embeddings")}
        out.update(model_type="gpa_qwen", base_config=base, gpa=gpa,
                   gpa_last_slots=list(self.gpa_last_slots) if self.gpa_last_slots is not None else None,
                   lora={"rank": 0, "alpha": 64., "dropout": 0.}, keep_rope=self.keep_rope,
                   convolution=self.convolution, loss_chunk_size=self.loss_chunk_size,
                   attention_dtype=self.attention_dtype)
        return out

    @classmethod
    def from_reference_dict(cls, d: dict) -> "GPALMConfig":
        """Read a reference GPAQwenConfig dict (its config.json): the native
        fields from `base_config`, filled with the family's defaults
        (hf_qwen.py:24-33), and the wrapper fields."""
        if d.get("model_type") not in ("gpa_qwen", None):
            raise ValueError("expected a gpa_qwen config")
        base = dict(d.get("base_config") or {"model_type": "qwen3"})
        kind = base.pop("model_type", None)
        if kind not in _NATIVE_DEFAULTS:
            raise ValueError("Only native Qwen2/Qwen2.5 and Qwen3 causal LMs are supported")
        native = dict(_NATIVE_DEFAULTS[kind])
        native.update({k: v for k, v in base.items() if k in native})
        for k in ("vocab_size", "hidden_size", "num_hidden_layers", "num_attention_heads", "num_key_value_heads",
                  "tie_word_embeddings", "initializer_range", "max_position_embeddings"):
            if d.get(k) is not None:
                native[k] = d[k]
        if native["head_dim"] is None:
            native["head_dim"] = native["hidden_size"] // native["num_attention_heads"]
        if int((d.get("lora") or {}).get("rank", 0)):
            raise ValueError("LoRA adapters are not supported: merge them into the base weights first")
        gpa = dict(d.get("gpa") or {})
        gpa.pop("backend", None)
        gpa.pop("execution", None)
        return cls(model_type=kind, **native, convolution=int(d.get("convolution", 4)),
                   loss_chunk_size=int(d.get("loss_chunk_size", 512)), keep_rope=bool(d.get("keep_rope", False)),
                   gpa=gpa, gpa_last_slots=d.get("gpa_last_slots"),
                   attention_dtype=d.get("attention_dtype", "bfloat16"))


class RMSNorm(nn.Module):
    """weight * x / sqrt(mean(x^2) + eps), statistics in float32, the
    normalised value rounded back to x's dtype before the weight (the Qwen
    RMSNorm)."""

    def __init__(self, dim: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.variance_epsilon = eps

    def forward(self, x: Tensor) -> Tensor:
        dtype = x.dtype
        h = x.float()
        h = h * torch.rsqrt(h.square().mean(-1, keepdim=True) + self.variance_epsilon)
        return self.weight * h.to(dtype)


def causal_conv(x: Tensor, weight: Tensor, tail: Tensor | None) -> tuple[Tensor, Tensor]:
    """Depthwise causal convolution of x [B,T,C] with weight [C,1,W], the last
    W-1 inputs of the previous call prepended (zeros when `tail` is None).
    Returns (out [B,T,C], the new tail [B,C,W-1]) (hf_qwen.py:118-124)."""
    width = weight.shape[-1] - 1
    prefix = x.new_zeros(x.shape[0], x.shape[-1], width) if tail is None else tail.to(x.dtype)
    joined = torch.cat((prefix, x.transpose(1, 2)), -1)
    if x.shape[1] == 1:
        # one token (decode): the window's dot product per channel, accumulated
        # in float32 like the convolution, without a convolution library call
        out = (joined.float() * weight[:, 0].float()).sum(-1, keepdim=True).to(x.dtype).transpose(1, 2)
    else:
        out = F.conv1d(joined, weight.to(x.dtype), groups=x.shape[-1]).transpose(1, 2)
    return out, (joined[:, :, -width:] if width else joined[:, :, :0])


def _rotate_half(x: Tensor) -> Tensor:
    a, b = x.chunk(2, -1)
    return torch.cat((-b, a), -1)


def rotary(config: GPALMConfig, positions: Tensor, dtype: torch.dtype) -> tuple[Tensor, Tensor]:
    """(cos, sin) [B,T,head_dim] of the Qwen rotary embedding at `positions` [B,T]."""
    d = config.head_dim
    inv = 1.0 / (config.rope_theta ** (torch.arange(0, d, 2, device=positions.device, dtype=torch.float32) / d))
    freqs = positions.float()[..., None] * inv
    emb = torch.cat((freqs, freqs), -1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


@dataclass(frozen=True)
class AttentionMemory:
    """One layer's cache entry: the GPA state and both convolution tails (hf_qwen.py:84-88)."""
    state: object
    projected_tail: Tensor
    control_tail: Tensor


def _map_tensors(value, fn):
    if isinstance(value, Tensor):
        return fn(value)
    if isinstance(value, tuple):
        return tuple(_map_tensors(v, fn) for v in value)
    if is_dataclass(value):
        return type(value)(**{f.name: _map_tensors(getattr(value, f.name), fn) for f in fields(value)})
    return value


class GPALMCache:
    """No growing K/V tensors: the short-convolution tails and every layer's
    A/B/R states (hf_qwen.py:92-115)."""

    def __init__(self, layers: int):
        self.layers = [None] * layers
        self.seen_tokens = 0

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.seen_tokens

    def reorder_cache(self, beam_idx: Tensor) -> None:
        self.layers = [_map_tensors(s, lambda x: x.index_select(0, beam_idx.to(x.device))) for s in self.layers]

    def batch_repeat_interleave(self, repeats: int) -> None:
        self.layers = [_map_tensors(s, lambda x: x.repeat_interleave(repeats, dim=0)) for s in self.layers]

    def detach(self) -> "GPALMCache":
        result = GPALMCache(len(self.layers))
        result.seen_tokens = self.seen_tokens
        result.layers = [_map_tensors(s, lambda x: x.detach()) for s in self.layers]
        return result


class GPALMAttention(nn.Module):
    """The attention block of one layer (hf_qwen.py:132-190)."""

    def __init__(self, config: GPALMConfig, index: int):
        super().__init__()
        h, kv, d, hid = config.num_attention_heads, config.num_key_value_heads, config.head_dim, config.hidden_size
        bias = config.attention_bias
        self.q_proj = nn.Linear(hid, h * d, bias=bias)
        self.k_proj = nn.Linear(hid, kv * d, bias=bias)
        self.v_proj = nn.Linear(hid, kv * d, bias=bias)
        self.o_proj = nn.Linear(h * d, hid, bias=False if config.model_type == "qwen2" else bias)
        if config.qk_norm:
            self.q_norm = RMSNorm(d, config.rms_norm_eps)
            self.k_norm = RMSNorm(d, config.rms_norm_eps)
        else:
            self.q_norm = self.k_norm = nn.Identity()
        self.heads, self.kv_heads, self.head_dim = h, kv, d
        self.attention_dtype = getattr(torch, config.attention_dtype) if config.attention_dtype else None
        self.gpa = DenseGPA(config.layer_gpa(index))
        with torch.no_grad():  # aligned direct query: these start at zero (hf_qwen.py:157-159)
            for q in self.gpa.query_weight:
                q.zero_()
        channels = (h + 2 * kv) * d
        self.projected_conv = nn.Parameter(torch.zeros(channels, 1, config.convolution))
        self.control_conv = nn.Parameter(torch.full((hid, 1, config.convolution), 1 / config.convolution))
        with torch.no_grad():
            self.projected_conv[:, :, -1] = 1.

    def forward(self, hidden: Tensor, rotary_emb=None, memory: AttentionMemory | None = None):
        b, t, _ = hidden.shape
        sizes = (self.q_proj.out_features, self.k_proj.out_features, self.v_proj.out_features)
        projected = torch.cat((self.q_proj(hidden), self.k_proj(hidden), self.v_proj(hidden)), -1)
        projected, ptail = causal_conv(projected, self.projected_conv, None if memory is None else memory.projected_tail)
        control, ctail = causal_conv(hidden, self.control_conv, None if memory is None else memory.control_tail)
        q, k, v = projected.split(sizes, -1)
        q = self.q_norm(q.reshape(b, t, self.heads, self.head_dim))
        k = self.k_norm(k.reshape(b, t, self.kv_heads, self.head_dim))
        v = v.reshape(b, t, self.kv_heads, self.head_dim)
        if rotary_emb is not None:
            cos, sin = (x[:, :, None].to(q.dtype) for x in rotary_emb)
            q = q * cos + _rotate_half(q) * sin
            k = k * cos + _rotate_half(k) * sin
        # each K/V head serves `groups` consecutive query heads (repeat_interleave
        # on the head axis, written as an expand so that no size is read back)
        groups = self.heads // self.kv_heads
        k, v = (x.unsqueeze(3).expand(b, t, self.kv_heads, groups, self.head_dim).reshape(b, t, self.heads,
                                                                                          self.head_dim)
                for x in (k, v))
        if self.attention_dtype is not None:
            q, k, v = (x.to(self.attention_dtype) for x in (q, k, v))
        control = F.silu(control)
        with torch.autocast(device_type=q.device.type, enabled=False):
            output, state = self.gpa(q, k, v, None if memory is None else memory.state, control_input=control)
        output = self.o_proj(output.reshape(b, t, -1).to(hidden.dtype))
        return output, AttentionMemory(state, ptail, ctail)


class GPALMMLP(nn.Module):
    """down(silu(gate(x)) * up(x)) (the Qwen SwiGLU MLP)."""

    def __init__(self, config: GPALMConfig):
        super().__init__()
        self.gate_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=False)
        self.up_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=False)
        self.down_proj = nn.Linear(config.intermediate_size, config.hidden_size, bias=False)

    def forward(self, x: Tensor) -> Tensor:
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class GPALMDecoderLayer(nn.Module):
    """Pre-norm residual layer (hf_qwen.py:193-203)."""

    def __init__(self, config: GPALMConfig, index: int):
        super().__init__()
        self.input_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.self_attn = GPALMAttention(config, index)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.mlp = GPALMMLP(config)

    def forward(self, hidden: Tensor, rotary_emb=None, memory=None):
        branch, memory = self.self_attn(self.input_layernorm(hidden), rotary_emb, memory)
        hidden = hidden + branch
        return hidden + self.mlp(self.post_attention_layernorm(hidden)), memory


class GPALMDecoder(nn.Module):
    def __init__(self, config: GPALMConfig):
        super().__init__()
        # registration order = the reference's parameter order (positional optimizer state)
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)
        self.norm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.layers = nn.ModuleList(GPALMDecoderLayer(config, i) for i in range(config.num_hidden_layers))


@dataclass
class LMOutput:
    loss: Tensor | None
    logits: Tensor | None
    past_key_values: GPALMCache | None


class GPALMForCausalLM(nn.Module):
    """Causal LM: embeddings, `num_hidden_layers` GPA decoder layers, final
    RMSNorm and LM head (tied to the embeddings when tie_word_embeddings).
    `forward` follows GPAQwenForCausalLM.forward (hf_qwen.py:348-407)."""

    def __init__(self, config: GPALMConfig):
        super().__init__()
        self.config = config
        self.model = GPALMDecoder(config)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        self._init_native(config)
        if config.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight
        self.gradient_checkpointing = False

    def _init_native(self, config: GPALMConfig) -> None:
        """Random init of the native (Qwen) weights: N(0, initializer_range)
        for projections and embeddings, zero biases; norms start at one."""
        std = config.initializer_range
        with torch.no_grad():
            for name, module in self.named_modules():
                if ".gpa" in name or name.endswith("gpa"):
                    continue
                if isinstance(module, (nn.Linear, nn.Embedding)):
                    module.weight.normal_(0., std)
                    if getattr(module, "bias", None) is not None:
                        module.bias.zero_()

    # --------------------------------------------------------------- training
    def gradient_checkpointing_enable(self, gradient_checkpointing_kwargs=None) -> None:
        opts = dict(gradient_checkpointing_kwargs or {"use_reentrant": False})
        if opts.get("use_reentrant", False):
            raise ValueError("Use non-reentrant checkpointing for GPA")
        self.gradient_checkpointing = True

    def gradient_checkpointing_disable(self) -> None:
        self.gradient_checkpointing = False

    def rebuild_runtime_buffers(self) -> None:
        """Restore the deterministic non-persistent buffers (the edge index
        tables of every GPA core) after a meta-device materialisation
        (hf_qwen.py:275-289); learned tensors are left alone."""
        for layer in self.model.layers:
            core = layer.self_attn.gpa
            device = core.center[0].device
            core._edge_source = torch.tensor([i for i, _ in core.edges], dtype=torch.long, device=device)
            core._edge_target = torch.tensor([j for _, j in core.edges], dtype=torch.long, device=device)

    # ---------------------------------------------------------------- forward
    def forward(self, input_ids: Tensor | None = None, *, labels: Tensor | None = None,
                past_key_values: GPALMCache | None = None, use_cache: bool | None = None,
                position_ids: Tensor | None = None, inputs_embeds: Tensor | None = None,
                attention_mask: Tensor | None = None, logits_to_keep: int = 0) -> LMOutput:
        if (input_ids is None) == (inputs_embeds is None):
            raise ValueError("Supply exactly one of input_ids or inputs_embeds")
        hidden = self.model.embed_tokens(input_ids) if inputs_embeds is None else inputs_embeds
        b, t, _ = hidden.shape
        if t < 1:
            raise ValueError("Empty token input")
        if attention_mask is not None:
            if attention_mask.ndim != 2 or attention_mask.shape[0] != b or attention_mask.shape[1] < t:
                raise ValueError("Expected a 2D all-valid attention_mask")
            if not bool((attention_mask == 1).all()):
                raise ValueError("Padding/packed-document masks are unsupported: use unpadded equal-length streams")
        if past_key_values is not None and not isinstance(past_key_values, GPALMCache):
            raise TypeError("GPA requires GPALMCache, not a Transformer KV cache")
        use_cache = True if use_cache is None else use_cache
        checkpointed = self.training and self.gradient_checkpointing
        if checkpointed:
            if past_key_values is not None:
                raise ValueError("Checkpointed training requires a fresh stream")
            use_cache = False
        cache = past_key_values
        if use_cache and cache is None:
            cache = GPALMCache(len(self.model.layers))
        seen = 0 if cache is None else cache.seen_tokens
        rotary_emb = None
        if self.config.keep_rope:
            if position_ids is None:
                position_ids = torch.arange(seen, seen + t, device=hidden.device)[None].expand(b, -1)
            rotary_emb = rotary(self.config, position_ids, hidden.dtype)
        for i, layer in enumerate(self.model.layers):
            old = None if cache is None else cache.layers[i]
            if checkpointed:
                def run(x, layer=layer):
                    return layer(x, rotary_emb, None)[0]
                hidden = _checkpoint(run, hidden, use_reentrant=False)
            else:
                hidden, memory = layer(hidden, rotary_emb, old)
                if use_cache:
                    cache.layers[i] = memory
        hidden = self.model.norm(hidden)
        if use_cache:
            cache.seen_tokens += t
        loss = logits = None
        if labels is not None:
            loss = self.chunked_loss(hidden, labels)
        else:
            keep = logits_to_keep
            logits = self.lm_head(hidden[:, -keep:] if keep > 0 else hidden)
        return LMOutput(loss, logits, cache if use_cache else None)

    def chunked_loss(self, hidden: Tensor, labels: Tensor) -> Tensor:
        """Mean next-token cross entropy over `loss_chunk_size`-token pieces,
        each piece's logits recomputed in the backward when training
        (hf_qwen.py:388-400)."""
        b, t = hidden.shape[:2]
        if labels.shape != (b, t):
            raise ValueError("labels must match this input block")
        count = (labels[:, 1:] != -100).sum().clamp_min(1)
        loss = hidden.sum() * 0.
        vocab = self.config.vocab_size

        def ce(x, y):
            return F.cross_entropy(self.lm_head(x).float().reshape(-1, vocab), y.reshape(-1), reduction="sum",
                                   ignore_index=-100)

        for start in range(0, t - 1, self.config.loss_chunk_size):
            stop = min(t - 1, start + self.config.loss_chunk_size)
            x, y = hidden[:, start:stop], labels[:, start + 1:stop + 1]
            value = _checkpoint(ce, x, y, use_reentrant=False) if self.training else ce(x, y)
            loss = loss + value / count
        return loss

    @torch.no_grad()
    def generate_greedy(self, input_ids: Tensor, max_new_tokens: int, cache: GPALMCache | None = None,
                        prefill_chunk: int | None = None) -> tuple[Tensor, GPALMCache]:
        """Greedy decoding: the prompt through the cache (in `prefill_chunk`-token
        calls, or one call), then one token per call.  Returns (new tokens
        [B,max_new_tokens], cache); the last new token is returned but not
        fed, so the cache has seen the prompt and all new tokens but the last."""
        cache = GPALMCache(len(self.model.layers)) if cache is None else cache
        step = prefill_chunk or input_ids.shape[1]
        logits = None
        for start in range(0, input_ids.shape[1], step):
            logits = self(input_ids[:, start:start + step], past_key_values=cache, logits_to_keep=1).logits
        tokens = []
        for i in range(max_new_tokens):
            nxt = logits[:, -1].argmax(-1, keepdim=True)
            tokens.append(nxt)
            if i + 1 < max_new_tokens:
                logits = self(nxt, past_key_values=cache, logits_to_keep=1).logits
        return torch.cat(tokens, 1), cache

    # ------------------------------------------------------------ checkpoints
    def save_pretrained(self, path: str) -> None:
        """config.json (reference GPAQwenConfig layout) and model.safetensors
        (parameters by name; the LM head is omitted when tied, as the
        reference's tied checkpoints omit it)."""
        from safetensors.torch import save_file
        os.makedirs(path, exist_ok=True)
        with open(os.path.join(path, "config.json"), "w") as f:
            json.dump(self.config.to_reference_dict(), f, indent=1)
        state = {k: v.detach().contiguous().cpu() for k, v in self.state_dict().items()}
        if self.config.tie_word_embeddings:
            state.pop("lm_head.weight", None)
        save_file(state, os.path.join(path, "model.safetensors"), metadata={"format": "pt"})

    @classmethod
    def from_pretrained(cls, path: str, **overrides) -> "GPALMForCausalLM":
        """Build from a checkpoint directory (ours or the reference's:
        config.json + model.safetensors) with float32 master weights, loading
        every tensor strictly (hf_qwen.py:257-273)."""
        from safetensors.torch import load_file
        with open(os.path.join(path, "config.json")) as f:
            config = GPALMConfig.from_reference_dict(json.load(f))
        for k, v in overrides.items():
            setattr(config, k, v)
        config.__post_init__()
        model = cls(config)
        state = load_file(os.path.join(path, "model.safetensors"))
        if config.tie_word_embeddings:
            state.pop("lm_head.weight", None)
            state["lm_head.weight"] = state["model.embed_tokens.weight"]
        model.load_state_dict({k: v.float() for k, v in state.items()}, strict=True)
        model.rebuild_runtime_buffers()
        return model


class LMDecodeGraph:
    """Greedy one-token decode of the LM on HIP graphs (inference, no autograd).

    A one-token call depends on its position in the GPA block (which
    snapshots it reads), so there is one graph per position: `chunk_size`
    graphs captured in replay order into one memory pool.  Each runs the
    whole LM for one token of every stream (embedding; every layer's
    projections, short convolutions, GPA core and MLP; final norm; LM head),
    stores the logits in its own buffer and writes the greedy choice into the
    static token buffer that the next replay reads.  A decode loop is then one
    replay per token with nothing read back.

    The cache must start at a block boundary of every layer.  Its tensors are
    copied into static buffers that the first graph reads; after the last
    position of a block the new cache is copied back into them.  Parameters
    must not change while the graphs are in use (their derived tensors are
    computed once, `params.frozen`); `step` raises if one has.  `autocast` is
    the dtype the graphs run the native layers under (None: none).  The
    decode depends on positions only through the block offset, so keep_rope
    and positional moments are refused.
    """

    def __init__(self, lm: GPALMForCausalLM, cache: GPALMCache, token: Tensor,
                 autocast: torch.dtype | None = torch.bfloat16, warmups: int = 2):
        from . import params
        from .state import _apply
        cores = [layer.self_attn.gpa.config for layer in lm.model.layers]
        self.chunk = cores[0].chunk_size
        if lm.config.keep_rope or any(c.positional_mode == "moments" for c in cores):
            raise ValueError("LMDecodeGraph: rotary positions depend on the absolute position; decode eagerly")
        if any(c.chunk_size != self.chunk for c in cores) or any(
                m is None or m.state.chunk_offset != 0 for m in cache.layers):
            raise ValueError("LMDecodeGraph: every layer's cache must start at a block boundary of one chunk size")
        if token.shape != (token.shape[0], 1):
            raise ValueError("LMDecodeGraph: one token per stream, [B, 1]")
        self.lm, self.autocast = lm, autocast
        self.seen = cache.seen_tokens
        self.offset = 0
        self.ids = token.detach().clone()
        clone = lambda t: t.detach().clone(memory_format=torch.contiguous_format)  # noqa: E731
        self.start = [AttentionMemory(_apply(m.state, clone), clone(m.projected_tail), clone(m.control_tail))
                      for m in cache.layers]
        self._params = params.fingerprints(list(lm.parameters()))
        self._derived = params.Store()
        current = torch.cuda.current_stream()
        side = torch.cuda.Stream()
        side.wait_stream(current)
        with torch.cuda.stream(side), self._context(), params.frozen(self._derived):
            layers = self.start
            for _ in range(warmups):
                c = GPALMCache(len(layers))
                c.layers = list(layers)
                lm(self.ids.clone(), past_key_values=c, logits_to_keep=1)
                layers = c.layers
            del layers, c
        current.wait_stream(side)
        self.pool = torch.cuda.graph_pool_handle()
        self.graphs = []
        self.logits = [torch.empty(token.shape[0], lm.config.vocab_size, device=token.device)
                       for _ in range(self.chunk)]
        layers = self.start
        with self._context(), params.frozen(self._derived):
            for o in range(self.chunk):
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, pool=self.pool):
                    c = GPALMCache(len(layers))
                    c.layers = list(layers)
                    logits = lm(self.ids, past_key_values=c, logits_to_keep=1).logits[:, -1]
                    self.logits[o].copy_(logits)
                    self.ids.copy_(logits.argmax(-1, keepdim=True))
                    del logits
                layers = c.layers
                self.graphs.append(graph)
        self.last = layers
        from .state import tensors
        for a, b in zip(self.start, self.last):
            if b.state.chunk_offset != 0 or [t.shape for t in tensors(a.state)] != [t.shape for t in tensors(b.state)]:
                raise RuntimeError("LMDecodeGraph: the cache after a block does not match the cache it started from")

    def _context(self):
        import contextlib
        stack = contextlib.ExitStack()
        stack.enter_context(torch.no_grad())
        if self.autocast is not None:
            stack.enter_context(torch.autocast("cuda", dtype=self.autocast, cache_enabled=False))
        return stack

    def step(self) -> Tensor:
        """Feed the current token of every stream; returns the static [B, 1]
        buffer, which now holds the greedy next token (and `logits[o]` its
        logits)."""
        from . import params
        if not params.unchanged(self._params):
            raise RuntimeError("LMDecodeGraph: a parameter changed after capture; build a new graph")
        o = self.offset
        self.graphs[o].replay()
        self.offset = (o + 1) % self.chunk
        self.seen += 1
        if self.offset == 0:
            from .state import tensors
            with torch.no_grad():
                for a, b in zip(self.start, self.last):
                    for dst, src in zip(tensors(a.state), tensors(b.state)):
                        dst.copy_(src)
                    a.projected_tail.copy_(b.projected_tail)
                    a.control_tail.copy_(b.control_tail)
        return self.ids

    def generate(self, steps: int) -> Tensor:
        """`steps` greedy tokens [B, steps]: the current token of the static
        buffer first, then one replay per further token (the last one is
        returned, not fed)."""
        out = torch.empty(self.ids.shape[0], steps, dtype=self.ids.dtype, device=self.ids.device)
        for i in range(steps):
            out[:, i:i + 1].copy_(self.ids)
            if i + 1 < steps:
                self.step()
        return out

    @property
    def cache(self) -> GPALMCache:
        """The cache at a block boundary (its tensors are the static buffers: clone to keep them)."""
        if self.offset != 0:
            raise RuntimeError("LMDecodeGraph.cache is available at block boundaries")
        c = GPALMCache(len(self.start))
        c.layers = list(self.start)
        c.seen_tokens = self.seen
        return c


__all__ = ["GPALMConfig", "GPALMForCausalLM", "GPALMCache", "AttentionMemory", "RMSNorm", "causal_conv",
           "LAYER_DEFAULTS", "LMOutput", "LMDecodeGraph"]
