"""ModelRunner's host side on the CPU: the attn_backend string switch and fuse=True's
in-place fusion (reference dispec/engine/model_runner.py:48-52, :93-118).  Building a
runner touches no GPU; running one does (tests/test_gpu_model_runner.py)."""

import pytest
import torch

from tests.toy_lm import toy_lm


def test_backend_switch():
    from dispec_amd.engine.model_runner import ModelRunner
    assert ModelRunner(toy_lm("qwen3")).attn_backend == "hip"
    assert ModelRunner(toy_lm("qwen3"), attn_backend="native").attn_backend == "native"
    with pytest.raises(ValueError, match="use attn_backend='hip'"):
        ModelRunner(toy_lm("qwen3"), attn_backend="triton")
    with pytest.raises(ValueError, match="not one of"):
        ModelRunner(toy_lm("qwen3"), attn_backend="flash")


@pytest.mark.parametrize("family", ["qwen2", "qwen3"])
def test_fuse_concatenates_in_place(family):
    from dispec_amd.engine.model_runner import ModelRunner
    model = toy_lm(family)
    layer = model.model.layers[1]
    q, k, v = (getattr(layer.self_attn, n).weight.clone() for n in ("q_proj", "k_proj", "v_proj"))
    gate, up = layer.mlp.gate_proj.weight.clone(), layer.mlp.up_proj.weight.clone()
    bias = layer.self_attn.q_proj.bias
    runner = ModelRunner(model, fuse=True)
    assert runner.fused
    f = runner._fused[1]
    assert torch.equal(f.qkv_weight, torch.cat([q, k, v]))
    assert torch.equal(f.gate_up_weight, torch.cat([gate, up]))
    assert (f.qkv_bias is None) == (bias is None)
    assert isinstance(layer.self_attn.q_proj, torch.nn.Identity)
    assert isinstance(layer.mlp.up_proj, torch.nn.Identity)
    with pytest.raises(ValueError, match="already fused"):
        ModelRunner(model, fuse=True)


def test_fused_projection_views_match_separate_projections():
    """_project_qkv and _mlp with fuse=True give the same q/k/v heads and MLP output as
    the separate modules (CPU float32, so any mismatch is a layout error, not rounding)."""
    from dispec_amd.engine.model_runner import ModelRunner
    plain_model, fused_model = toy_lm("qwen2"), toy_lm("qwen2")
    plain, fused = ModelRunner(plain_model), ModelRunner(fused_model, fuse=True)
    x = torch.randn(5, plain_model.config.hidden_size, generator=torch.Generator().manual_seed(3))
    for i in range(2):
        a = plain._project_qkv(plain.layers[i].self_attn, x, i)
        b = fused._project_qkv(fused.layers[i].self_attn, x, i)
        for ta, tb in zip(a, b):
            assert ta.shape == tb.shape
            torch.testing.assert_close(ta, tb, rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(plain._mlp(plain.layers[i], x, i),
                                   fused._mlp(fused.layers[i], x, i), rtol=1e-5, atol=1e-5)
    h = torch.randn(3, plain_model.config.hidden_size)
    torch.testing.assert_close(plain.logits(h, torch.tensor([2, 0])), plain.lm_head(h)[[2, 0]])


def test_graph_decoder_needs_the_hip_backend():
    """A HIP graph replays device-side batch metadata; the native backend reads the host
    sequence list every step, so the graph decoder refuses it up front."""
    from types import SimpleNamespace

    from dispec_amd.engine.hip_graph import HipGraphDecoder
    from dispec_amd.engine.model_runner import ModelRunner
    runner = ModelRunner(toy_lm("qwen3"), attn_backend="native")
    fake_cache = SimpleNamespace(key=torch.zeros(1))
    with pytest.raises(ValueError, match="attn_backend='hip'"):
        HipGraphDecoder(runner, fake_cache)
