"""Seeded toy causal LMs of the two families the model runner serves (Qwen2: biased QKV,
no q/k norm; Qwen3: q/k RMSNorm), built from a config alone -- no checkpoint exists on
the test machines.

Every parameter is drawn from one seeded generator in name order, so a model is a pure
function of (family, layers, seed) whatever torch's global RNG state is:
  * matrices (embeddings, projections, lm_head): N(0, 1/fan_in), which keeps hidden states
    and logits O(1) through the layers;
  * RMSNorm gains (input/post-attention/final norms and Qwen3's q/k norms): U[0.75, 1.25],
    so a kernel that skips a norm or applies the wrong head's weight is visible;
  * biases (Qwen2's QKV): N(0, 0.05^2).
Head geometry: 4 query heads over 2 KV heads (G = 2) of head_dim 64, so the attention
paths under test run their MFMA tiles.
"""

from __future__ import annotations

import math

import torch

GEOMETRY = dict(vocab_size=128, hidden_size=256, intermediate_size=256,
                num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                max_position_embeddings=1024, tie_word_embeddings=False)


def _draw(model: torch.nn.Module, seed: int) -> torch.nn.Module:
    gen = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in sorted(model.named_parameters()):
            if name.endswith("norm.weight"):
                p.copy_(0.75 + 0.5 * torch.rand(p.shape, generator=gen))
            elif p.dim() == 2:
                p.copy_(torch.randn(p.shape, generator=gen) / math.sqrt(p.shape[1]))
            else:
                p.copy_(0.05 * torch.randn(p.shape, generator=gen))
    return model.eval().requires_grad_(False)


def toy_lm(family: str, num_layers: int = 2, seed: int = 0) -> torch.nn.Module:
    """A random `family` ("qwen2" | "qwen3") causal LM with `num_layers` layers."""
    import transformers
    kinds = {"qwen2": ("Qwen2Config", "Qwen2ForCausalLM"),
             "qwen3": ("Qwen3Config", "Qwen3ForCausalLM")}
    if family not in kinds:
        raise ValueError(f"unknown family {family!r}; expected one of {sorted(kinds)}")
    cfg_cls, lm_cls = (getattr(transformers, n) for n in kinds[family])
    return _draw(lm_cls(cfg_cls(num_hidden_layers=num_layers, **GEOMETRY)), seed)
