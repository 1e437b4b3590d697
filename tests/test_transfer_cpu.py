"""Host side of dispec_amd.kv.transfer on the CPU: kvxfer's map-file format, validation and
the GPU-only guard of the apply path.

The format (maps.json + {variant}__{keys|values}.pt + residual/residual.pt) and the error
texts are what the reference's loader reads and raises (dispec/kv/transfer.py:144-230);
the reference's own CPU tests of them are tests/test_kv_transfer.py:79-87, :138-182.
Loading with device="cpu" runs only host code; applying a map needs the GPU.
"""

import json
from types import SimpleNamespace

import pytest
import torch

from dispec_amd.kv.transfer import CrossModelKVMap

HEADS, HEAD_DIM = 2, 4
KV = HEADS * HEAD_DIM


def model_config(layers, *, name, vocab=64, heads=HEADS, head_dim=HEAD_DIM):
    return SimpleNamespace(num_hidden_layers=layers, num_key_value_heads=heads,
                           head_dim=head_dim, hidden_size=32, num_attention_heads=8,
                           vocab_size=vocab, _name_or_path=name)


class MapFiles:
    """Writes a map directory the way kvxfer's save_maps lays it out.

    Layer t of either kind reads source layers `sources(t)`; layers listed in `factored`
    are stored as low-rank (left, right) factors instead of a dense weight.  Every tensor
    is filled with distinct values so a mix-up between layers or kinds is visible.
    """

    def __init__(self, root, n_src, n_tgt, *, fan_in=2, factored=(), rank=3,
                 fitted=("team/src-model", "team/tgt-model"), variants=("ridge",)):
        self.root, self.n_src, self.n_tgt = root, n_src, n_tgt
        self.fan_in, self.factored, self.rank = fan_in, set(factored), rank
        self.fitted, self.variants = fitted, variants
        self.saved = {}

    def sources(self, t):
        return [(t + j) % self.n_src for j in range(self.fan_in)]

    def _tensor(self, *shape, tag):
        n = 1
        for d in shape:
            n *= d
        return (torch.arange(n, dtype=torch.float32).reshape(shape) / 64 + tag)

    def write(self, variant="ridge", weight_rows=None, bias_len=KV):
        for kid, kind in enumerate(("keys", "values")):
            entries = {}
            for t in range(self.n_tgt):
                rows = weight_rows or self.fan_in * KV
                tag = 10 * kid + t
                e = {"source_layers": self.sources(t), "target_layer": t,
                     "bias": self._tensor(bias_len, tag=-tag), "r2": 0.9}
                if t in self.factored:
                    e["weight"], e["rank"] = None, self.rank
                    e["factors"] = (self._tensor(rows, self.rank, tag=tag),
                                    self._tensor(self.rank, KV, tag=tag + 0.5))
                else:
                    e["weight"], e["rank"], e["factors"] = self._tensor(rows, KV, tag=tag), None, None
                entries[t] = e
            torch.save(entries, self.root / f"{variant}__{kind}.pt")
            self.saved[kind] = entries
        self.root.joinpath("maps.json").write_text(json.dumps(
            {"source": self.fitted[0], "target": self.fitted[1],
             "variants": list(self.variants)}))
        return self

    def write_residual(self, hidden=5, design=None):
        design = design or self.fan_in * KV
        out = self.root / "residual"
        out.mkdir(exist_ok=True)
        state = {"hidden": hidden, "design_dim": design}
        for kid, key in enumerate(("key_residual", "value_residual")):
            state[key] = {}
            for t in range(self.n_tgt):
                tag = 100 + 10 * kid + t
                state[key][f"{t}.down.weight"] = self._tensor(hidden, design, tag=tag)
                state[key][f"{t}.down.bias"] = self._tensor(hidden, tag=-tag)
                state[key][f"{t}.up.weight"] = self._tensor(KV, hidden, tag=tag + 0.25)
        torch.save(state, out / "residual.pt")
        self.residual = state
        return out

    def load(self, src=None, tgt=None, **kw):
        src = src or model_config(self.n_src, name="team/src-model")
        tgt = tgt or model_config(self.n_tgt, name="team/tgt-model")
        return CrossModelKVMap.load(self.root, src, tgt, device="cpu", **kw)


def bf16(t):
    return t.to(torch.bfloat16)


def test_every_layer_of_both_kinds_loads_as_written(tmp_path):
    files = MapFiles(tmp_path, n_src=5, n_tgt=4, factored=(1, 3)).write()
    kv_map = files.load()
    assert kv_map.dtype == torch.bfloat16 and not kv_map.has_residual
    for kind, loaded in (("keys", kv_map.keys), ("values", kv_map.values)):
        assert len(loaded) == 4
        for t, m in enumerate(loaded):
            want = files.saved[kind][t]
            assert m.source_layers == tuple(files.sources(t))
            assert torch.equal(m.bias, bf16(want["bias"]))
            if t in files.factored:
                assert m.weight is None
                assert all(torch.equal(a, bf16(b)) for a, b in zip(m.factors, want["factors"]))
            else:
                assert m.factors is None and torch.equal(m.weight, bf16(want["weight"]))


def test_load_honours_dtype(tmp_path):
    kv_map = MapFiles(tmp_path, 3, 2).write().load(dtype=torch.float32)
    assert kv_map.dtype == torch.float32
    assert all(m.weight.dtype == torch.float32 for m in kv_map.keys + kv_map.values)


def test_residual_attaches_to_the_right_layer_and_kind(tmp_path):
    files = MapFiles(tmp_path, n_src=3, n_tgt=3).write()
    kv_map = files.load(residual_dir=files.write_residual())
    assert kv_map.has_residual
    for kind, key in (("keys", "key_residual"), ("values", "value_residual")):
        for t, m in enumerate(getattr(kv_map, kind)):
            sd = files.residual[key]
            for got, part in zip(m.residual, ("down.weight", "down.bias", "up.weight")):
                assert torch.equal(got, bf16(sd[f"{t}.{part}"]))


@pytest.mark.parametrize("case", ["no manifest", "unknown variant"])
def test_missing_files_are_named(tmp_path, case):
    if case == "no manifest":
        with pytest.raises(FileNotFoundError, match="no maps.json in"):
            MapFiles(tmp_path, 3, 2).load()
    else:
        MapFiles(tmp_path, 3, 2, variants=("ridge", "lowrank")).write()
        with pytest.raises(ValueError, match=r"variant 'pca' not in \['ridge', 'lowrank'\]"):
            MapFiles(tmp_path, 3, 2).load(variant="pca")


GEOMETRY_CASES = {
    "vocab": (dict(vocab=65), {}, "vocab_size differs .* do not share a tokenizer"),
    "head_dim": ({}, dict(head_dim=8), "head_dim differs .*cannot map onto a target head"),
    "kv_heads": (dict(heads=4), {}, "num_key_value_heads differs"),
}


@pytest.mark.parametrize("case", sorted(GEOMETRY_CASES))
def test_models_that_cannot_exchange_kv_are_rejected(tmp_path, case):
    src_kw, tgt_kw, msg = GEOMETRY_CASES[case]
    files = MapFiles(tmp_path, 3, 2).write()
    with pytest.raises(ValueError, match="cannot transfer KV: " + msg):
        files.load(src=model_config(3, name="a/s", **src_kw),
                   tgt=model_config(2, name="a/t", **tgt_kw))


def test_maps_that_do_not_fit_the_models_are_rejected(tmp_path):
    files = MapFiles(tmp_path, n_src=4, n_tgt=2, fan_in=2).write()
    with pytest.raises(ValueError, match="keys: 2 layer maps for a 5-layer target"):
        files.load(tgt=model_config(5, name="team/tgt-model"))
    # target layer 1 reads source layers 1 and 2; a 2-layer source lacks layer 2
    with pytest.raises(ValueError, match=r"target layer 1 reads source layers \[2\], "
                                         "but the source has 2"):
        files.load(src=model_config(2, name="team/src-model"))
    files.write(weight_rows=3 * KV)
    with pytest.raises(ValueError, match=r"keys map for target layer 0 has shape \(24, 8\), "
                                         r"expected \(16, 8\)"):
        files.load()
    files.write(bias_len=KV + 1)
    with pytest.raises(ValueError, match="has shape"):
        files.load()
    files.write()
    with pytest.raises(ValueError, match="residual for target layer 0 does not match a "
                                         "16->8 map"):
        files.load(residual_dir=files.write_residual(design=3 * KV))


@pytest.mark.parametrize("side", ["source", "target"])
def test_maps_fitted_for_other_checkpoints_warn(tmp_path, side):
    fitted = {"source": ("team/other", "team/tgt-model"),
              "target": ("team/src-model", "team/other")}[side]
    files = MapFiles(tmp_path, 3, 2, fitted=fitted).write()
    with pytest.warns(UserWarning, match=f"maps were fitted with {side} 'team/other'"):
        files.load()


def test_same_checkpoint_under_another_directory_does_not_warn(tmp_path, recwarn):
    MapFiles(tmp_path, 3, 2, fitted=("hub/src-model", "/data/ckpt/tgt-model/")).write()
    MapFiles(tmp_path, 3, 2).load()
    assert not [w for w in recwarn if "fitted with" in str(w.message)]


def test_applying_a_map_requires_the_gpu(tmp_path):
    kv_map = MapFiles(tmp_path, 3, 2).write().load()
    k = torch.zeros(3, 5, HEADS, HEAD_DIM)
    rope = (torch.ones(5, HEAD_DIM), torch.zeros(5, HEAD_DIM))
    with pytest.raises(RuntimeError, match="GPU only"):
        kv_map.map(k, k, rope, rope)
