"""Map files, validation and host-side behaviour of dispec_amd.kv.transfer (CPU only).

Restates the reference's CPU tests of the file format and validation
(tests/test_kv_transfer.py:79-87, :138-182) against dispec_amd's loader.  Loading with
device="cpu" runs only host code; applying a map needs the GPU and must say so.
"""

import json
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch

from dispec_amd.kv.transfer import CrossModelKVMap

H, D = 2, 4
KV_DIM = H * D


def _config(n_layers, vocab=100, heads=H, head_dim=D, name="org/model"):
    return SimpleNamespace(num_hidden_layers=n_layers, num_key_value_heads=heads,
                           head_dim=head_dim, hidden_size=16, num_attention_heads=4,
                           vocab_size=vocab, _name_or_path=name)


def _write_maps(path: Path, n_src, n_tgt, k=2, seed=0, source="org/src", target="org/tgt"):
    """A map directory in kvxfer's save_maps format (tests/test_kv_transfer.py:49-62)."""
    g = torch.Generator().manual_seed(seed)
    for kind in ("keys", "values"):
        state = {}
        for t in range(n_tgt):
            layers = sorted(torch.randperm(n_src, generator=g)[:k].tolist())
            state[t] = {"weight": torch.randn(k * KV_DIM, KV_DIM, generator=g),
                        "bias": torch.randn(KV_DIM, generator=g), "source_layers": layers,
                        "target_layer": t, "r2": 0.5, "rank": None, "factors": None}
        torch.save(state, path / f"ridge__{kind}.pt")
    (path / "maps.json").write_text(json.dumps(
        {"source": source, "target": target, "variants": ["ridge"]}))
    return path


def _load(path, n_src, n_tgt, **kw):
    return CrossModelKVMap.load(path, _config(n_src, name="org/src"),
                                _config(n_tgt, name="org/tgt"), device="cpu", **kw)


def test_load_reads_kvxfer_map_format(tmp_path):
    _write_maps(tmp_path, n_src=3, n_tgt=4)
    kv_map = _load(tmp_path, 3, 4)
    saved = torch.load(tmp_path / "ridge__keys.pt", weights_only=True)
    assert len(kv_map.keys) == len(kv_map.values) == 4
    assert kv_map.dtype == torch.bfloat16
    for t, m in enumerate(kv_map.keys):
        assert m.source_layers == tuple(saved[t]["source_layers"])
        torch.testing.assert_close(m.weight, saved[t]["weight"].to(torch.bfloat16))


def test_residual_loads_from_kvxfer_format(tmp_path):
    _write_maps(tmp_path, n_src=3, n_tgt=2)
    hidden, design = 5, 2 * KV_DIM
    sd = lambda: {f"{i}.{name}": torch.randn(shape)  # noqa: E731
                  for i in range(2) for name, shape in
                  (("down.weight", (hidden, design)), ("down.bias", (hidden,)),
                   ("up.weight", (KV_DIM, hidden)))}
    res = tmp_path / "residual"
    res.mkdir()
    state = {"key_residual": sd(), "value_residual": sd(), "hidden": hidden, "design_dim": design}
    torch.save(state, res / "residual.pt")
    kv_map = _load(tmp_path, 3, 2, residual_dir=res)
    assert kv_map.has_residual
    torch.testing.assert_close(kv_map.values[1].residual[2],
                               state["value_residual"]["1.up.weight"].to(torch.bfloat16))


def test_missing_manifest_and_variant(tmp_path):
    with pytest.raises(FileNotFoundError, match="maps.json"):
        _load(tmp_path, 3, 2)
    _write_maps(tmp_path, 3, 2)
    with pytest.raises(ValueError, match="variant 'lasso'"):
        _load(tmp_path, 3, 2, variant="lasso")


def test_rejects_models_without_a_shared_tokenizer(tmp_path):
    _write_maps(tmp_path, 3, 2)
    with pytest.raises(ValueError, match="tokenizer"):
        CrossModelKVMap.load(tmp_path, _config(3), _config(2, vocab=101), device="cpu")


def test_rejects_mismatched_kv_geometry(tmp_path):
    _write_maps(tmp_path, 3, 2)
    with pytest.raises(ValueError, match="head_dim"):
        CrossModelKVMap.load(tmp_path, _config(3, head_dim=8), _config(2), device="cpu")
    with pytest.raises(ValueError, match="num_key_value_heads"):
        CrossModelKVMap.load(tmp_path, _config(3, heads=4), _config(2), device="cpu")


def test_rejects_maps_that_do_not_fit_the_models(tmp_path):
    _write_maps(tmp_path, n_src=3, n_tgt=2)
    with pytest.raises(ValueError, match="2 layer maps for a 3-layer target"):
        CrossModelKVMap.load(tmp_path, _config(3), _config(3), device="cpu")
    with pytest.raises(ValueError, match="source has 1"):
        CrossModelKVMap.load(tmp_path, _config(1), _config(2), device="cpu")


def test_warns_when_maps_were_fitted_for_other_models(tmp_path):
    _write_maps(tmp_path, 3, 2, source="org/other")
    with pytest.warns(UserWarning, match="fitted with source"):
        CrossModelKVMap.load(tmp_path, _config(3, name="org/src"), _config(2, name="org/tgt"),
                             device="cpu")


def test_map_needs_the_gpu(tmp_path):
    _write_maps(tmp_path, 3, 2)
    kv_map = _load(tmp_path, 3, 2)
    k = torch.zeros(3, 5, H, D)
    rope = (torch.ones(5, D), torch.zeros(5, D))
    with pytest.raises(RuntimeError, match="GPU only"):
        kv_map.map(k, k, rope, rope)
