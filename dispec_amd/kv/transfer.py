"""Cross-model KV transfer on the GPU: map one model's KV cache into another's layout.

Drop-in for the reference module (dispec/kv/transfer.py): the same map file format
(kvxfer's `maps.json` + `{variant}__{keys|values}.pt`, optional `residual/residual.pt`,
:187-230), the same validation and messages (:144-183), the same apply semantics -- strip
RoPE from the source keys in fp32, concatenate the selected source layers into one design
row per token ordered layer -> head -> dim, y = x @ W + b (or (x @ L) @ R + b) plus an
optional up(gelu(down(x))) residual, re-apply RoPE in fp32 (:15-25, :243-283).

Every step runs on the HIP kernels of libdispec_hip.so:
  strip_rope / apply_rope   -> dsp_kv_rope (fp32 math, one launch for all layers)
  LayerMap.apply            -> dsp_kv_map_gemm (MFMA; the design row is read in place
                               from the source buffer, never concatenated in memory)
and the bf16 result is rounded at the same points the reference's bf16 torch ops round
(x @ W, then + b; F.linear's bias fused; gelu; the residual add).

Maps live on the GPU in bf16 (the reference's default map dtype, :189); weights are kept
transposed once at load so both GEMM operands are read along K.
"""

from __future__ import annotations

import ctypes
import json
import warnings
from dataclasses import dataclass, field
from pathlib import Path

import torch

from dispec_amd import _lib
from dispec_amd.kv.paged_cache import check_prefix_coverage

KINDS = ("keys", "values")


def head_dim_of(config) -> int:
    return getattr(config, "head_dim", None) or config.hidden_size // config.num_attention_heads


# -- RoPE in and out of content space --------------------------------------------------
def rope_tables(rotary_emb, positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(cos, sin), (T, head_dim) float32, from a model's own rotary module (:50-58)."""
    probe = torch.zeros(1, 1, dtype=torch.float32, device=positions.device)
    cos, sin = rotary_emb(probe, positions[None, :])
    return cos[0].float().contiguous(), sin[0].float().contiguous()


def _rope(keys: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, direction: int,
          out_dtype: torch.dtype = torch.float32, out: torch.Tensor | None = None) -> torch.Tensor:
    _lib.require_gpu(keys, cos, sin)
    if keys.dim() != 4:
        raise ValueError(f"keys must be (L, T, H, D), got {tuple(keys.shape)}")
    L, T, H, D = keys.shape
    if tuple(cos.shape) != (T, D) or tuple(sin.shape) != (T, D):
        raise ValueError(f"rope tables {tuple(cos.shape)}/{tuple(sin.shape)} do not match "
                         f"{T} positions of head_dim {D}")
    if keys.dtype not in (torch.bfloat16, torch.float32):
        keys = keys.float()
    if keys.stride(3) != 1 or keys.stride(2) != D or keys.stride(1) != H * D:
        keys = keys.contiguous()
    cos = cos.float().contiguous()
    sin = sin.float().contiguous()
    if out is None:
        out = torch.empty((L, T, H, D), dtype=out_dtype, device=keys.device)
    _lib.check(_lib.lib().dsp_kv_rope(
        keys.data_ptr(), keys.stride(0), out.data_ptr(), out.stride(0), L, T, H, D,
        cos.data_ptr(), sin.data_ptr(), direction, _lib.dtype_code(keys.dtype),
        _lib.dtype_code(out.dtype), _lib.stream_of(keys)), "dsp_kv_rope")
    return out


def strip_rope(keys: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotated keys (L, T, H, D) -> content-space keys, float32 (:66-73)."""
    return _rope(keys, cos, sin, -1)


def apply_rope(keys: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Content-space keys (L, T, H, D) -> rotated keys, float32 (:76-80)."""
    return _rope(keys, cos, sin, +1)


# -- the GEMM --------------------------------------------------------------------------------
def _gemm(a: torch.Tensor, seg_offsets: list[int], seg_len: int, lda: int, M: int,
          bt: torch.Tensor, out: torch.Tensor, bias: torch.Tensor | None = None,
          bias_mode: int = 0, act: int = 0, accumulate: bool = False, batch: int = 1,
          a_batch_stride: int = 0, c_batch_stride: int = 0) -> torch.Tensor:
    """out[z, M, N] = epilogue(A_z . bt^T) for z < batch; A_z's column k is
    a[z*a_batch_stride + seg_offsets[k // seg_len] + m*lda + k % seg_len]; bt is (N, K) with
    K contiguous; out's rows are out.stride(-2) apart, problems c_batch_stride apart."""
    N, K = bt.shape
    if bt.stride(1) != 1:
        raise ValueError("Bt must be K-contiguous")
    if out.stride(-1) != 1 or tuple(out.shape[-2:]) != (M, N):
        raise ValueError(f"out must be row-major (..., {M}, {N})")
    offs = (ctypes.c_int64 * len(seg_offsets))(*seg_offsets)
    _lib.check(_lib.lib().dsp_kv_map_gemm(
        a.data_ptr(), offs, len(seg_offsets), seg_len, lda, bt.data_ptr(), bt.stride(0),
        out.data_ptr(), out.stride(-2), M, N, K, batch, a_batch_stride, c_batch_stride,
        _lib.ptr(bias), bias_mode, act, int(accumulate), _lib.DSP_BF16, _lib.stream_of(out)),
        "dsp_kv_map_gemm")
    return out


# -- the map ------------------------------------------------------------------------------
@dataclass
class LayerMap:
    """The affine map producing one target layer's keys or values (:84-123).

    source_layers: source layers concatenated into the design, in order.
    bias: (kv_dim,).  weight: (k * kv_dim, kv_dim), row-vector convention (x @ weight),
    or None when stored as low-rank factors (left, right) with x @ left @ right.
    residual: (down.weight, down.bias, up.weight) of up(gelu(down(x))), or None.
    """

    source_layers: tuple[int, ...]
    bias: torch.Tensor
    weight: torch.Tensor | None = None
    factors: tuple[torch.Tensor, torch.Tensor] | None = None
    residual: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = field(default=None)

    def __post_init__(self):
        self._kernel_ready = False

    def to(self, device, dtype) -> "LayerMap":
        move = lambda t: t.to(device=device, dtype=dtype)  # noqa: E731
        self.bias = move(self.bias)
        if self.weight is not None:
            self.weight = move(self.weight)
        if self.factors is not None:
            self.factors = tuple(move(t) for t in self.factors)
        if self.residual is not None:
            self.residual = tuple(move(t) for t in self.residual)
        self._kernel_ready = False
        return self

    def _prepare(self) -> None:
        """Kernel-side copies: every matrix as (N, K) with K contiguous, bf16, on the GPU."""
        if self._kernel_ready:
            return
        if self.bias.dtype != torch.bfloat16 or not self.bias.is_cuda:
            raise ValueError("the HIP map runs bf16 maps on the GPU: call .to('cuda', "
                             "torch.bfloat16) first")
        self._b = self.bias.contiguous()
        if self.factors is not None:
            self._lt = self.factors[0].t().contiguous()        # (r, K)
            self._rt = self.factors[1].t().contiguous()        # (N, r)
        else:
            self._wt = self.weight.t().contiguous()            # (N, K)
        if self.residual is not None:
            down_w, down_b, up_w = self.residual
            self._down = (down_w.contiguous(), down_b.contiguous())   # (hidden, K)
            self._up = up_w.contiguous()                              # (N, hidden)
        self._kernel_ready = True

    def apply_into(self, a: torch.Tensor, seg_offsets: list[int], seg_len: int, lda: int,
                   rows: int, out: torch.Tensor, use_residual: bool = True, batch: int = 1,
                   a_batch_stride: int = 0, c_batch_stride: int = 0) -> torch.Tensor:
        """out (rows, N) = x @ W + b (+ residual) with x's design rows read in place; with
        batch > 1, `batch` problems a_batch_stride / c_batch_stride elements apart."""
        self._prepare()
        bs = dict(batch=batch, a_batch_stride=a_batch_stride, c_batch_stride=c_batch_stride)
        if self.factors is not None:
            r = self._lt.shape[0]
            tmp = torch.empty((batch, rows, r), dtype=torch.bfloat16, device=out.device)
            _gemm(a, seg_offsets, seg_len, lda, rows, self._lt, tmp, batch=batch,
                  a_batch_stride=a_batch_stride, c_batch_stride=rows * r)
            _gemm(tmp, [0], r, r, rows, self._rt, out, self._b, bias_mode=1, batch=batch,
                  a_batch_stride=rows * r, c_batch_stride=c_batch_stride)
        else:
            _gemm(a, seg_offsets, seg_len, lda, rows, self._wt, out, self._b, bias_mode=1, **bs)
        if use_residual and self.residual is not None:
            down_w, down_b = self._down
            hid = down_w.shape[0]
            hidden = torch.empty((batch, rows, hid), dtype=torch.bfloat16, device=out.device)
            _gemm(a, seg_offsets, seg_len, lda, rows, down_w, hidden, down_b, bias_mode=2, act=1,
                  batch=batch, a_batch_stride=a_batch_stride, c_batch_stride=rows * hid)
            _gemm(hidden, [0], hid, hid, rows, self._up, out, accumulate=True, batch=batch,
                  a_batch_stride=rows * hid, c_batch_stride=c_batch_stride)
        return out

    def apply_to_pool(self, a: torch.Tensor, seg_offsets: list[int], seg_len: int, lda: int,
                      rows: int, pool_layer: torch.Tensor, block_table: torch.Tensor,
                      block_size: int, rope: tuple[torch.Tensor, torch.Tensor] | None = None,
                      batch: int = 1, a_batch_stride: int = 0,
                      err: torch.Tensor | None = None) -> bool:
        """apply_into, then (keys) RoPE with the target tables, then the scatter of each
        problem's rows into its blocks of one pool layer -- one GEMM launch writing straight
        into the pool (dsp_kv_map_gemm_to_pool).  Returns False, having done nothing, when
        this map or shape has no fused form (residual maps; shapes the large-tile GEMM does
        not take): the caller then runs apply_into + RoPE + scatter.  A row whose block id
        lies outside the pool is skipped and counted in `err` (at least once per row: once
        per 128-column tile of the row)."""
        self._prepare()
        if self.residual is not None:
            return False
        N = self._b.shape[0]
        H, D = pool_layer.shape[-2], pool_layer.shape[-1]
        if H * D != N or pool_layer.stride(-1) != 1 or pool_layer.stride(-2) != D:
            return False
        if self.factors is not None:
            r = self._lt.shape[0]
            if r % 64:
                # the fused launch steps K (= the rank here) 64 at a time: decide before the
                # first GEMM runs, or the caller's fallback would run it a second time
                return False
            tmp = torch.empty((batch, rows, r), dtype=torch.bfloat16, device=a.device)
            _gemm(a, seg_offsets, seg_len, lda, rows, self._lt, tmp, batch=batch,
                  a_batch_stride=a_batch_stride, c_batch_stride=rows * r)
            a, seg_offsets, seg_len, lda, a_batch_stride, bt = tmp, [0], r, r, rows * r, self._rt
        else:
            bt = self._wt
        cos, sin = (None, None) if rope is None else (rope[0].float().contiguous(),
                                                      rope[1].float().contiguous())
        if cos is not None and tuple(cos.shape) != (rows, D):
            raise ValueError(f"rope tables {tuple(cos.shape)} do not match {rows} rows of "
                             f"head_dim {D}")
        offs = (ctypes.c_int64 * len(seg_offsets))(*seg_offsets)
        st = _lib.lib().dsp_kv_map_gemm_to_pool(
            a.data_ptr(), offs, len(seg_offsets), seg_len, lda, bt.data_ptr(), bt.stride(0),
            pool_layer.data_ptr(), pool_layer.stride(0), pool_layer.shape[0],
            block_table.data_ptr(), block_table.stride(0), block_size, rows, N, bt.shape[1],
            batch, a_batch_stride, self._b.data_ptr(), _lib.ptr(cos), _lib.ptr(sin), D,
            _lib.DSP_BF16, _lib.ptr(err), _lib.stream_of(pool_layer))
        if st == _lib.DSP_EUNSUPPORTED:
            return False
        _lib.check(st, "dsp_kv_map_gemm_to_pool")
        return True

    def apply(self, x: torch.Tensor, use_residual: bool = True) -> torch.Tensor:
        """y = x @ W + b (+ up(gelu(down(x)))) for x (T, K) bf16 on the GPU (:104-112)."""
        _lib.require_gpu(x)
        x = x.to(torch.bfloat16).contiguous()
        T, K = x.shape
        out = torch.empty((T, self.bias.shape[0]), dtype=torch.bfloat16, device=x.device)
        return self.apply_into(x, [0], K, K, T, out, use_residual)


# -- map files and their validation ------------------------------------------------------
# The on-disk format is kvxfer's (reference loader: dispec/kv/transfer.py:187-230):
#   maps_dir/maps.json                  {"variants": [...], "source": name, "target": name, ...}
#   maps_dir/{variant}__{keys|values}.pt  list over target layers of
#                                       {"source_layers", "bias", "weight" | "factors"}
#   residual_dir/residual.pt            {"key_residual"|"value_residual":
#                                        {"{layer}.down.weight", "{layer}.down.bias",
#                                         "{layer}.up.weight"}}
# The error and warning texts are the reference's (:151-183, :197-200): callers and tests
# match on them.
_RESIDUAL_KEYS = {"keys": "key_residual", "values": "value_residual"}
_GEOMETRY = (  # (config attribute, how to read it, why a mismatch is fatal)
    ("num_key_value_heads", lambda c: c.num_key_value_heads,
     "a source head cannot map onto a target head"),
    ("head_dim", head_dim_of, "a source head cannot map onto a target head"),
    ("vocab_size", lambda c: c.vocab_size, "the models do not share a tokenizer"),
)


def _model_name(path: str) -> str:
    return path.rstrip("/").rpartition("/")[2]


def _layer_map_from_state(entry: dict) -> LayerMap:
    factors = entry.get("factors")
    return LayerMap(source_layers=tuple(map(int, entry["source_layers"])), bias=entry["bias"],
                    weight=entry.get("weight"),
                    factors=None if factors is None else tuple(factors))


def _read_stack(path: Path) -> list[LayerMap]:
    """One kind's per-target-layer maps: entries 0..n-1 of a safe-loaded dict (or list)."""
    state = torch.load(path, map_location="cpu", weights_only=True)
    return [_layer_map_from_state(state[i]) for i in range(len(state))]


def _stack_problems(kind: str, maps: list[LayerMap], n_src: int, n_tgt: int, kv_dim: int):
    """Yield the message of every way `maps` cannot produce an n_tgt-layer target."""
    if len(maps) != n_tgt:
        yield f"{kind}: {len(maps)} layer maps for a {n_tgt}-layer target"
        return
    for layer, m in enumerate(maps):
        outside = [i for i in m.source_layers if i < 0 or i >= n_src]
        if outside:
            yield (f"{kind} map for target layer {layer} reads source layers {outside}, "
                   f"but the source has {n_src}")
            continue
        rows = kv_dim * len(m.source_layers)
        if m.weight is not None:
            got = tuple(m.weight.shape)
        else:
            got = (m.factors[0].shape[0], m.factors[1].shape[1])
        if got != (rows, kv_dim) or tuple(m.bias.shape) != (kv_dim,):
            yield (f"{kind} map for target layer {layer} has shape {got}, "
                   f"expected {(rows, kv_dim)}")
        elif m.residual is not None and (m.residual[0].shape[1] != rows
                                         or m.residual[2].shape[0] != kv_dim):
            yield (f"{kind} residual for target layer {layer} does not match a "
                   f"{rows}->{kv_dim} map")


def _scatter_one_plane(cache, layer_pool: torch.Tensor, table: torch.Tensor, cu: torch.Tensor,
                       T: int, rows: torch.Tensor) -> None:
    """Scatter (T, H, D) rows into one layer of one pool plane (K or V) with the import
    kernel (dsp_kv_scatter over one layer; both of its planes name this one, so the rows
    are written twice -- the path of maps without a fused form only)."""
    _lib.check(_lib.lib().dsp_kv_scatter(
        layer_pool.data_ptr(), layer_pool.data_ptr(), 1, cache.layer_bytes, cache.num_blocks,
        cache.row_bytes, cache.block_size, table.data_ptr(), table.stride(0), cu.data_ptr(), 1,
        T, rows.data_ptr(), rows.data_ptr(), cache._err.data_ptr(), _lib.stream_of(rows)),
        "dsp_kv_scatter")


class CrossModelKVMap:
    """Maps a source model's contiguous KV (L, T, H, D) into a target model's (:126-283)."""

    def __init__(self, keys: list[LayerMap], values: list[LayerMap], source_config,
                 target_config, metadata: dict | None = None):
        for attr, read, why in _GEOMETRY:
            a, b = read(source_config), read(target_config)
            if a != b:
                raise ValueError(f"cannot transfer KV: {attr} differs ({a} vs {b}); {why}")
        self.keys, self.values = keys, values
        self.metadata = dict(metadata or {})
        self.num_kv_heads = target_config.num_key_value_heads
        self.head_dim = head_dim_of(target_config)
        kv_dim = self.num_kv_heads * self.head_dim
        for kind, maps in zip(KINDS, (keys, values)):
            problem = next(_stack_problems(kind, maps, source_config.num_hidden_layers,
                                           target_config.num_hidden_layers, kv_dim), None)
            if problem is not None:
                raise ValueError(problem)
        self.dtype = keys[0].bias.dtype if keys else torch.float32
        self._warn_if_other_models(source_config, target_config)

    def _warn_if_other_models(self, source_config, target_config) -> None:
        """Warn when the configs name other checkpoints than the maps were fitted on."""
        for side, cfg in (("source", source_config), ("target", target_config)):
            fitted = self.metadata.get(side) or ""
            loaded = (getattr(cfg, "_name_or_path", "") or getattr(cfg, "name_or_path", "")
                      or "")
            if fitted and loaded and _model_name(fitted) != _model_name(loaded):
                warnings.warn(f"maps were fitted with {side} {fitted!r} but {loaded!r} is "
                              "loaded; geometry matches, quality is not guaranteed",
                              stacklevel=4)

    @classmethod
    def load(cls, maps_dir, source_config, target_config, residual_dir=None,
             variant: str = "ridge", device="cuda",
             dtype: torch.dtype = torch.bfloat16) -> "CrossModelKVMap":
        """Read kvxfer's map files (and an optional trained residual) onto the GPU."""
        root = Path(maps_dir)
        try:
            manifest = json.loads((root / "maps.json").read_text())
        except FileNotFoundError:
            raise FileNotFoundError(f"no maps.json in {root}") from None
        offered = manifest.get("variants", [])
        if variant not in offered:
            raise ValueError(f"variant {variant!r} not in {manifest.get('variants')}")
        stacks = {kind: _read_stack(root / f"{variant}__{kind}.pt") for kind in KINDS}
        if residual_dir is not None:
            trained = torch.load(Path(residual_dir) / "residual.pt", map_location="cpu",
                                 weights_only=True)
            for kind, maps in stacks.items():
                sd = trained[_RESIDUAL_KEYS[kind]]
                for i, m in enumerate(maps):
                    m.residual = tuple(sd[f"{i}.{part}"] for part in
                                       ("down.weight", "down.bias", "up.weight"))
        return cls(stacks["keys"], stacks["values"], source_config, target_config,
                   manifest).to(device, dtype)

    def to(self, device, dtype: torch.dtype) -> "CrossModelKVMap":
        """Move every layer map to `device` / `dtype` (done once, at load)."""
        for m in self.keys + self.values:
            m.to(device, dtype)
        self.dtype = dtype
        return self

    @property
    def has_residual(self) -> bool:
        """Whether trained residual maps are attached (decided by the first key map)."""
        return bool(self.keys) and self.keys[0].residual is not None

    def _apply(self, source: torch.Tensor, maps: list[LayerMap], use_residual: bool,
               rope: tuple[torch.Tensor, torch.Tensor] | None = None,
               out: torch.Tensor | None = None) -> torch.Tensor:
        """Target layers (L_tgt, T, H, D) from contiguous source layers (L_src, T, H, D)."""
        L_src, T, H, D = source.shape
        kv = H * D
        if out is None:
            out = torch.empty((len(maps), T, H, D), dtype=torch.bfloat16, device=source.device)
        for layer, m in enumerate(maps):
            m.apply_into(source, [s * T * kv for s in m.source_layers], kv, kv, T,
                         out[layer].view(T, kv), use_residual)
        if rope is not None:
            _rope(out, rope[0], rope[1], +1, out=out)
        return out

    @torch.inference_mode()
    def map_into(self, k: torch.Tensor, v: torch.Tensor,
                 source_rope: tuple[torch.Tensor, torch.Tensor],
                 target_rope: tuple[torch.Tensor, torch.Tensor], cache, block_ids: list[int],
                 use_residual: bool = True, prompt_len: int | None = None) -> None:
        """map() followed by cache.import_contiguous(block_ids, keys, values), with each
        target layer's GEMM writing its rows (keys re-rotated) straight into the cache's
        blocks: no (L_tgt, T, H, D) intermediate.  Layers whose map has no fused form (a
        trained residual) take map's path for that layer and are then scattered.

        With `prompt_len`, this is an admission (the target request's prompt has
        prompt_len tokens): the T mapped tokens must cover at least one and fewer than
        all of them, checked before any launch with the reference scheduler's message
        (dispec/sched/scheduler.py:110-112)."""
        L_src, T, H, D = k.shape
        if prompt_len is not None:
            check_prefix_coverage(T, prompt_len)
        _lib.require_gpu(k, v)
        if self.dtype != torch.bfloat16:
            raise ValueError("the HIP map runs bf16 maps (load with dtype=torch.bfloat16)")
        if len(self.keys) != cache.num_layers or (cache.num_kv_heads, cache.head_dim) != (H, D):
            raise ValueError(f"a {len(self.keys)}-layer map of {H}x{D} heads cannot fill a "
                             f"{cache.num_layers}-layer cache of {cache.num_kv_heads}x"
                             f"{cache.head_dim}")
        if cache.dtype != torch.bfloat16:
            raise ValueError("map_into fills bf16 caches")
        cache._check_blocks(block_ids, T)
        table = cache.block_table([block_ids])
        kv = H * D
        content = _rope(k, *source_rope, direction=-1, out_dtype=torch.bfloat16)
        vals = v.to(torch.bfloat16).contiguous()
        tcos, tsin = target_rope[0].float().contiguous(), target_rope[1].float().contiguous()
        cu = torch.tensor([0, T], dtype=torch.long).to(k.device)
        for layer in range(cache.num_layers):
            jobs = ((self.keys[layer], content, cache.key, (tcos, tsin)),
                    (self.values[layer], vals, cache.value, None))
            for m, src, pool, rope in jobs:
                offs = [s * T * kv for s in m.source_layers]
                if (not use_residual or m.residual is None) and m.apply_to_pool(
                        src, offs, kv, kv, T, pool[layer], table, cache.block_size, rope,
                        err=cache._err):
                    continue
                # no fused form: the map's own output, rotated, then this layer's scatter
                out = torch.empty((T, H, D), dtype=torch.bfloat16, device=k.device)
                m.apply_into(src, offs, kv, kv, T, out.view(T, kv), use_residual)
                if rope is not None:
                    _rope(out[None], tcos, tsin, +1, out=out[None])
                _scatter_one_plane(cache, pool[layer], table, cu, T, out)
        cache._after()

    @torch.inference_mode()
    def map(self, k: torch.Tensor, v: torch.Tensor,
            source_rope: tuple[torch.Tensor, torch.Tensor],
            target_rope: tuple[torch.Tensor, torch.Tensor],
            use_residual: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
        """Map contiguous source KV (L_src, T, H, D) to target KV (L_tgt, T, H, D).

        Keys are RoPE-stripped with the source tables (fp32, stored bf16), mapped, and
        re-rotated with the target tables; values are mapped only.  Returned in the
        input dtypes.
        """
        _lib.require_gpu(k, v)
        if self.dtype != torch.bfloat16:
            raise ValueError("the HIP map runs bf16 maps (load with dtype=torch.bfloat16)")
        content = _rope(k, *source_rope, direction=-1, out_dtype=torch.bfloat16)
        keys = self._apply(content, self.keys, use_residual, rope=target_rope)
        del content
        values = self._apply(v.to(torch.bfloat16).contiguous(), self.values, use_residual)
        return keys.to(k.dtype), values.to(v.dtype)
