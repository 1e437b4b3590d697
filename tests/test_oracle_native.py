"""Pins the oracle's restatement of the reference native forward (CPU only).

A fresh prefill through oracle.ref_torch.native_forward must reproduce the HF model's own
forward (the reference's bar: tests/test_qwen3.py:54-89, tiny Qwen3 vs HF at 1e-4), and a
chunked prefill must equal one prefill (tests/test_prefill_attention.py:72-82).
"""

import pytest
import torch

from oracle import ref_torch
from tests.toy_lm import toy_lm


def _pool(model, nb=16, bs=16):
    cfg = model.config
    shape = (cfg.num_hidden_layers, nb * bs, cfg.num_key_value_heads, cfg.head_dim)
    return torch.zeros(shape), torch.zeros(shape)


@pytest.mark.parametrize("family", ["qwen3", "qwen2"])
def test_native_forward_matches_hf(family):
    model = toy_lm(family)
    ids = torch.randint(0, 128, (37,), generator=torch.Generator().manual_seed(3))
    key, value = _pool(model)
    blocks = [5, 9, 2]
    slots = ref_torch.context_slots(blocks, 37, 16)
    h = ref_torch.native_forward(model, ids, torch.arange(37), slots, [(blocks, 37, 37)],
                                 key, value, 16)
    ours = model.lm_head(h)
    with torch.inference_mode():
        theirs = model(ids[None]).logits[0]
    torch.testing.assert_close(ours, theirs, atol=1e-4, rtol=1e-4)


def test_native_forward_chunked_equals_whole():
    model = toy_lm("qwen3")
    ids = torch.randint(0, 128, (40,), generator=torch.Generator().manual_seed(1))
    blocks = [3, 7, 1]
    key, value = _pool(model)
    whole = ref_torch.native_forward(model, ids, torch.arange(40),
                                     ref_torch.context_slots(blocks, 40, 16),
                                     [(blocks, 40, 40)], key, value, 16)
    key, value = _pool(model)
    s = ref_torch.context_slots(blocks, 40, 16)
    first = ref_torch.native_forward(model, ids[:17], torch.arange(17), s[:17],
                                     [(blocks, 17, 17)], key, value, 16)
    rest = ref_torch.native_forward(model, ids[17:], torch.arange(17, 40), s[17:],
                                    [(blocks, 23, 40)], key, value, 16)
    torch.testing.assert_close(torch.cat([first, rest]), whole, atol=1e-4, rtol=1e-4)
