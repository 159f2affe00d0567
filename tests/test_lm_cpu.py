"""Host-side behaviour of the LM shell (gpa_amd.lm) that needs no GPU: the
checkpoint format against a reference-written checkpoint, our own save/load
round trip, tied embeddings, the config contract and the cache operations."""
import json
import os

import pytest
import torch
from safetensors.torch import load_file

from gpa_amd import _lib
from gpa_amd.lm import AttentionMemory, GPALMCache, GPALMConfig, GPALMForCausalLM
from tests.lm_cases import CHECKPOINT

TINY = dict(vocab_size=96, hidden_size=64, intermediate_size=96, num_hidden_layers=2, num_attention_heads=4,
            num_key_value_heads=2, head_dim=16, gpa=dict(slots=(16, 16, 16, 32), chunk_size=4))


def test_reference_checkpoint_loads_strictly():
    """The reference-written checkpoint (config.json + model.safetensors of
    GPAQwenForCausalLM) loads with every tensor, by name, in the reference's
    order, and the GPA layers take the reference wrapper's defaults
    (hf_qwen.py:145-151) plus the checkpoint's overrides."""
    model = GPALMForCausalLM.from_pretrained(CHECKPOINT)
    ref = load_file(os.path.join(CHECKPOINT, "model.safetensors"))
    ours = model.state_dict()
    assert list(ours) == [k for k in ours if k in ref] and set(ours) == set(ref)
    for k, v in ref.items():
        assert torch.equal(ours[k], v), k
    cfg = model.model.layers[0].self_attn.gpa.config
    assert (cfg.rsa_update, cfg.paper_product_read, cfg.shared_query_center, cfg.balanced_bridge) == (True,) * 4
    assert (cfg.read_scale, cfg.beta_init, cfg.decay_init, cfg.chunk_size) == (8., .6, 1e-4, 4)
    assert cfg.control_dim == 64 and cfg.slots == (16, 16, 16, 32) and cfg.backend == "hip"
    assert model.config.loss_chunk_size == 5 and not model.config.tie_word_embeddings


def test_save_and_load_round_trip(tmp_path):
    model = GPALMForCausalLM.from_pretrained(CHECKPOINT)
    model.save_pretrained(str(tmp_path))
    with open(tmp_path / "config.json") as f:
        saved = json.load(f)
    with open(os.path.join(CHECKPOINT, "config.json")) as f:
        ref = json.load(f)
    # the reference config's layout: every key it writes that describes the model
    for key in ("model_type", "base_config", "gpa", "gpa_last_slots", "lora", "keep_rope", "convolution",
                "loss_chunk_size", "vocab_size", "hidden_size", "num_hidden_layers", "num_attention_heads",
                "num_key_value_heads", "tie_word_embeddings"):
        assert key in saved and key in ref, key
    assert {k: v for k, v in saved["gpa"].items() if k != "backend"} == \
        {k: v for k, v in ref["gpa"].items() if k not in ("backend", "execution")} | {"execution": "reference"}
    again = GPALMForCausalLM.from_pretrained(str(tmp_path))
    a, b = model.state_dict(), again.state_dict()
    assert list(a) == list(b) and all(torch.equal(a[k], b[k]) for k in a)


def test_tied_embeddings_are_saved_once_and_retied(tmp_path):
    torch.manual_seed(0)
    model = GPALMForCausalLM(GPALMConfig(**TINY, tie_word_embeddings=True))
    assert model.lm_head.weight is model.model.embed_tokens.weight
    model.save_pretrained(str(tmp_path))
    assert "lm_head.weight" not in load_file(str(tmp_path / "model.safetensors"))
    again = GPALMForCausalLM.from_pretrained(str(tmp_path))
    assert again.lm_head.weight is again.model.embed_tokens.weight
    assert torch.equal(again.lm_head.weight, model.lm_head.weight)


def test_layer_defaults_and_config_contract():
    cfg = GPALMConfig(**TINY, gpa_last_slots=(8, 8))
    first, last = cfg.layer_gpa(0), cfg.layer_gpa(1)
    assert first.slots == (16, 16, 16, 32) and last.slots == (8, 8)
    assert first.heads == 4 and first.key_dim == first.value_dim == 16 and first.control_dim == 64
    default = GPALMConfig()
    assert default.layer_gpa(0).slots == (128, 128)  # the reference's (head_dim, head_dim) default
    with pytest.raises(ValueError, match="inherited"):
        GPALMConfig(**{**TINY, "gpa": dict(heads=3)}).layer_gpa(0)
    with pytest.raises(ValueError):
        GPALMConfig(model_type="llama")
    with pytest.raises(ValueError):
        GPALMConfig(num_attention_heads=6, num_key_value_heads=4)
    with pytest.raises(ValueError):
        GPALMConfig(convolution=0)
    with pytest.raises(ValueError, match="LoRA"):
        GPALMConfig.from_reference_dict({"model_type": "gpa_qwen", "base_config": {"model_type": "qwen3"},
                                         "lora": {"rank": 4}})
    qwen2 = GPALMConfig.from_reference_dict({"model_type": "gpa_qwen", "base_config": {
        "model_type": "qwen2", "hidden_size": 64, "num_attention_heads": 4, "num_key_value_heads": 2,
        "num_hidden_layers": 1, "vocab_size": 32, "intermediate_size": 96}})
    assert qwen2.head_dim == 16 and qwen2.attention_bias and not qwen2.qk_norm
    m = GPALMForCausalLM(qwen2)
    assert m.model.layers[0].self_attn.q_proj.bias is not None and m.model.layers[0].self_attn.o_proj.bias is None


def test_new_query_weights_start_at_zero_and_conv_is_identity():
    torch.manual_seed(0)
    m = GPALMForCausalLM(GPALMConfig(**TINY))
    att = m.model.layers[0].self_attn
    assert all(not q.any() for q in att.gpa.query_weight)
    assert torch.equal(att.projected_conv[:, 0, -1], torch.ones(att.projected_conv.shape[0]))
    assert not att.projected_conv[:, :, :-1].any()
    assert torch.allclose(att.control_conv, torch.full_like(att.control_conv, .25))


def test_forward_input_checks_and_no_cpu_fallback():
    torch.manual_seed(0)
    m = GPALMForCausalLM(GPALMConfig(**TINY))
    ids = torch.zeros(1, 3, dtype=torch.long)
    with pytest.raises(ValueError, match="exactly one"):
        m()
    with pytest.raises(ValueError, match="Empty"):
        m(ids[:, :0])
    with pytest.raises(ValueError, match="mask"):
        m(ids, attention_mask=torch.tensor([[1, 0, 1]]))
    with pytest.raises(TypeError):
        m(ids, past_key_values=[])
    m.train()
    m.gradient_checkpointing_enable()
    with pytest.raises(ValueError, match="fresh stream"):
        m(ids, past_key_values=GPALMCache(2))
    with pytest.raises(ValueError, match="non-reentrant"):
        m.gradient_checkpointing_enable({"use_reentrant": True})
    m.eval()
    with pytest.raises(_lib.HipBackendError):
        m(ids)


def test_cache_reorder_repeat_detach():
    state = torch.arange(6.).reshape(3, 2).requires_grad_()
    cache = GPALMCache(1)
    cache.seen_tokens = 5
    cache.layers[0] = AttentionMemory(state * 1, torch.arange(3.)[:, None], torch.arange(3.)[:, None] * 2)
    cache.reorder_cache(torch.tensor([2, 0]))
    assert torch.equal(cache.layers[0].projected_tail[:, 0], torch.tensor([2., 0.]))
    cache.batch_repeat_interleave(2)
    assert cache.layers[0].control_tail[:, 0].tolist() == [4., 4., 0., 0.]
    d = cache.detach()
    assert d.seen_tokens == 5 and not d.layers[0].state.requires_grad and cache.layers[0].state.requires_grad
