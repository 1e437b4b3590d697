"""Tiny random Qwen2 / Qwen3 models (no weights needed), like the reference's fixture
(tests/tiny_models.py:12-45), with head_dim 64 so the MFMA attention tiles apply."""

from __future__ import annotations

import torch

DIMS = dict(vocab_size=128, hidden_size=256, intermediate_size=256, num_attention_heads=4,
            num_key_value_heads=2, head_dim=64, max_position_embeddings=1024,
            tie_word_embeddings=False)


def _finish(model, seed: int):
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        model.lm_head.weight.copy_(torch.randn(model.lm_head.weight.shape, generator=g))
    model.eval()
    model.requires_grad_(False)
    return model


def tiny_qwen3(num_layers: int = 2, seed: int = 0):
    from transformers import Qwen3Config, Qwen3ForCausalLM
    torch.manual_seed(seed)
    model = Qwen3ForCausalLM(Qwen3Config(num_hidden_layers=num_layers, **DIMS))
    g = torch.Generator().manual_seed(seed + 2)
    with torch.no_grad():
        for layer in model.model.layers:
            for norm in (layer.self_attn.q_norm, layer.self_attn.k_norm):
                norm.weight.copy_(1.0 + 0.3 * torch.randn(norm.weight.shape, generator=g))
    return _finish(model, seed)


def tiny_qwen2(num_layers: int = 2, seed: int = 0):
    from transformers import Qwen2Config, Qwen2ForCausalLM
    torch.manual_seed(seed)
    return _finish(Qwen2ForCausalLM(Qwen2Config(num_hidden_layers=num_layers, **DIMS)), seed)
