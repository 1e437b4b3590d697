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

    def apply(self, x: torch.Tensor, use_residual: bool = True) -> torch.Tensor:
        """y = x @ W + b (+ up(gelu(down(x)))) for x (T, K) bf16 on the GPU (:104-112)."""
        _lib.require_gpu(x)
        x = x.to(torch.bfloat16).contiguous()
        T, K = x.shape
        out = torch.empty((T, self.bias.shape[0]), dtype=torch.bfloat16, device=x.device)
        return self.apply_into(x, [0], K, K, T, out, use_residual)


class CrossModelKVMap:
    """Maps a source model's contiguous KV (L, T, H, D) into a target model's (:126-283)."""

    def __init__(self, keys: list[LayerMap], values: list[LayerMap], source_config,
                 target_config, metadata: dict | None = None):
        self.keys = keys
        self.values = values
        self.metadata = metadata or {}
        self.num_kv_heads = target_config.num_key_value_heads
        self.head_dim = head_dim_of(target_config)
        self.dtype = keys[0].bias.dtype if keys else torch.float32
        self._check(source_config, target_config)

    def _check(self, source_config, target_config) -> None:
        src, tgt = source_config, target_config
        for attr, a, b in (
            ("num_key_value_heads", src.num_key_value_heads, tgt.num_key_value_heads),
            ("head_dim", head_dim_of(src), head_dim_of(tgt)),
            ("vocab_size", src.vocab_size, tgt.vocab_size),
        ):
            if a != b:
                reason = ("the models do not share a tokenizer" if attr == "vocab_size"
                          else "a source head cannot map onto a target head")
                raise ValueError(f"cannot transfer KV: {attr} differs ({a} vs {b}); {reason}")
        n_src, n_tgt = src.num_hidden_layers, tgt.num_hidden_layers
        kv_dim = self.num_kv_heads * self.head_dim
        for kind, maps in (("keys", self.keys), ("values", self.values)):
            if len(maps) != n_tgt:
                raise ValueError(f"{kind}: {len(maps)} layer maps for a {n_tgt}-layer target")
            for layer, m in enumerate(maps):
                bad = [s for s in m.source_layers if not 0 <= s < n_src]
                if bad:
                    raise ValueError(f"{kind} map for target layer {layer} reads source "
                                     f"layers {bad}, but the source has {n_src}")
                design = len(m.source_layers) * kv_dim
                shape = (m.weight.shape if m.weight is not None
                         else (m.factors[0].shape[0], m.factors[1].shape[1]))
                if tuple(shape) != (design, kv_dim) or tuple(m.bias.shape) != (kv_dim,):
                    raise ValueError(f"{kind} map for target layer {layer} has shape "
                                     f"{tuple(shape)}, expected {(design, kv_dim)}")
                if m.residual is not None:
                    down_w, _, up_w = m.residual
                    if down_w.shape[1] != design or up_w.shape[0] != kv_dim:
                        raise ValueError(f"{kind} residual for target layer {layer} does "
                                         f"not match a {design}->{kv_dim} map")
        for side, config in (("source", src), ("target", tgt)):
            recorded = self.metadata.get(side)
            loaded = getattr(config, "_name_or_path", "") or getattr(config, "name_or_path", "")
            if recorded and loaded and (recorded.rstrip("/").split("/")[-1]
                                        != loaded.rstrip("/").split("/")[-1]):
                warnings.warn(f"maps were fitted with {side} {recorded!r} but {loaded!r} is "
                              "loaded; geometry matches, quality is not guaranteed", stacklevel=3)

    @classmethod
    def load(cls, maps_dir, source_config, target_config, residual_dir=None,
             variant: str = "ridge", device="cuda",
             dtype: torch.dtype = torch.bfloat16) -> "CrossModelKVMap":
        """Read kvxfer's map files (and an optional trained residual) onto the GPU."""
        maps_dir = Path(maps_dir)
        manifest = maps_dir / "maps.json"
        if not manifest.exists():
            raise FileNotFoundError(f"no maps.json in {maps_dir}")
        metadata = json.loads(manifest.read_text())
        if variant not in metadata.get("variants", []):
            raise ValueError(f"variant {variant!r} not in {metadata.get('variants')}")
        per_kind = {}
        for kind in KINDS:
            state = torch.load(maps_dir / f"{variant}__{kind}.pt", map_location="cpu",
                               weights_only=True)
            layers = []
            for layer in range(len(state)):
                s = state[layer]
                factors = s.get("factors")
                layers.append(LayerMap(
                    source_layers=tuple(int(i) for i in s["source_layers"]), bias=s["bias"],
                    weight=s.get("weight"),
                    factors=tuple(factors) if factors is not None else None))
            per_kind[kind] = layers
        if residual_dir is not None:
            res = torch.load(Path(residual_dir) / "residual.pt", map_location="cpu",
                             weights_only=True)
            for kind, key in (("keys", "key_residual"), ("values", "value_residual")):
                sd = res[key]
                for layer, m in enumerate(per_kind[kind]):
                    m.residual = (sd[f"{layer}.down.weight"], sd[f"{layer}.down.bias"],
                                  sd[f"{layer}.up.weight"])
        kv_map = cls(per_kind["keys"], per_kind["values"], source_config, target_config,
                     metadata)
        return kv_map.to(device, dtype)

    def to(self, device, dtype: torch.dtype) -> "CrossModelKVMap":
        for m in (*self.keys, *self.values):
            m.to(device, dtype)
        self.dtype = dtype
        return self

    @property
    def has_residual(self) -> bool:
        return self.keys[0].residual is not None

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
