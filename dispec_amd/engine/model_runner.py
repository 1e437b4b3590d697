"""Qwen2/Qwen3 forward over the paged cache with attention on the HIP kernels.

Drop-in for the reference ModelRunner (dispec/engine/model_runner.py:26-231) with a new
backend string, attn_backend="hip".  The model math around attention -- embeddings,
RMSNorms, q/k/v/o projections (optionally fused, :93-118), SwiGLU MLP, lm_head -- is
the HF modules, unchanged.  What the backend replaces is the KV path inside `_attention`
(:127-185) and the per-forward batch build in `forward` (:189-212):

  * q_norm / k_norm, RoPE on q and k,  -> dsp_qk_norm_rope_append (one launch; the torch
    cache.write (:142-148)               ops' rounding points)
  * all-decode batch (every q_len 1)  -> dsp_paged_decode, split-K over a device block
                                        table built once per forward (one H2D copy, no
                                        per-token slot table and no per-sequence loop)
  * anything else (fresh or chunked   -> dsp_paged_mq_attention, one launch for the whole
    prefill, speculative verify,        ragged batch with the bottom-right causal mask
    mixed decode + prefill)             (the reference loops over sequences with SDPA);
                                        when the sequences' tables start with the same
                                        blocks (copy-on-write forks of one prompt,
                                        prefix-cache hits) the shared-prefix variant
                                        attends those blocks once for the whole batch

attn_backend is a string switch as in the reference (:48-52): "hip" (the default here)
runs the kernels above; "native" keeps the reference's torch attention -- per sequence, the
context gathered from the pool (by the slot-gather kernel) and torch's SDPA with the
bottom-right causal mask and grouped heads (:160-185) -- on the same projections, prologue
and cache, as the baseline a deployment can switch back to.  "triton" names the
reference's Triton decode kernel, which this package does not carry: it is refused with a
message pointing at "hip", its replacement.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from dispec_amd import _lib
from dispec_amd.engine.hip_attn import (decode_workspace, mq_workspace,
                                       paged_decode_attention_blocks, paged_mq_attention)
from dispec_amd.engine.hip_prologue import qk_norm_rope_append
from dispec_amd.kv.paged_cache import PagedKVCache


@dataclass
class SeqMeta:
    """One sequence's slice of a flat batch (model_runner.py:26-32)."""

    block_ids: list[int]
    q_len: int      # new (query) tokens this step
    ctx_len: int    # context length including the new tokens


@dataclass
class _Batch:
    """Per-forward device metadata shared by every layer."""

    block_table: torch.Tensor
    ctx_lens: torch.Tensor
    cu_q: torch.Tensor
    max_q_len: int
    max_ctx: int
    decode: bool
    workspace: torch.Tensor | None = None
    shared_prefix: int = 0   # leading context tokens all sequences share (0: none used)
    balanced: bool = False   # short query blocks on the balanced split-K kernel
    seqs: tuple = ()         # the host SeqMeta list (attn_backend="native" walks it)


_BACKENDS = ("hip", "native")


def _compute_dtype(model) -> torch.dtype:
    """The model's arithmetic type: its first floating-point parameter's (quantised models
    keep integer-packed weights beside float scales)."""
    for p in model.parameters():
        if p.is_floating_point():
            return p.dtype
    return torch.float16


@dataclass(frozen=True)
class _FusedLayer:
    """One layer's projections concatenated for one GEMM each (fuse=True)."""

    qkv_weight: torch.Tensor              # rows: q heads, then k heads, then v heads
    qkv_bias: torch.Tensor | None
    gate_up_weight: torch.Tensor          # rows: gate, then up


class ModelRunner:
    def __init__(self, model, attn_backend: str = "hip", fuse: bool = False):
        if attn_backend not in _BACKENDS:
            hint = (" (the Triton decode kernel is replaced by this package's HIP kernels: "
                    "use attn_backend='hip')" if attn_backend == "triton" else "")
            raise ValueError(f"attn_backend {attn_backend!r} is not one of {_BACKENDS}{hint}")
        self.model, self.attn_backend = model, attn_backend
        self.cfg = cfg = model.config
        self.dtype = _compute_dtype(model)
        self.device = next(model.parameters()).device
        backbone = model.model
        self.embed = backbone.embed_tokens
        self.layers = backbone.layers
        self.norm = backbone.norm
        self.rotary_emb = backbone.rotary_emb    # the model's own cos/sin tables
        self.lm_head = model.lm_head
        self.num_heads = cfg.num_attention_heads
        self.num_kv_heads = cfg.num_key_value_heads
        self.head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // self.num_heads
        self.kv_groups = self.num_heads // self.num_kv_heads
        self.scale = 1.0 / self.head_dim ** 0.5
        if "sliding_attention" in (getattr(cfg, "layer_types", None) or ()):
            raise ValueError(f"{type(model).__name__} uses sliding-window attention layers, which "
                             "the paged attention path does not implement")
        first = self.layers[0].self_attn
        self.qk_norm = all(hasattr(first, n) for n in ("q_norm", "k_norm"))   # Qwen3
        # the MFMA attention kernels (and with them the balanced verify split and the shared
        # prefix) serve bf16 / fp16; fp32 models attend through the generic kernel
        self._tuned_attention = self.dtype in (torch.bfloat16, torch.float16)
        self._rope_dummy = torch.zeros(1, 1, device=self.device, dtype=self.dtype)
        self._fused: list[_FusedLayer] = self._fuse_projections() if fuse else []
        self.fused = bool(self._fused)
        # shared-prefix attention: used when at least this many sequences share at least
        # this many leading tokens (fewer gain nothing over per-sequence attention)
        self.shared_prefix_min_seqs = 4
        self.shared_prefix_min_tokens = 512
        # balanced split for verify batches whose keys per resident workgroup fall below
        # this fraction of the fixed split's partition (see _prefer_balanced)
        self.balanced_key_fraction = 0.6
        self._cus = (torch.cuda.get_device_properties(self.device).multi_processor_count
                     if self.device.type == "cuda" else 256)

    def _fuse_projections(self) -> list[_FusedLayer]:
        """fuse=True (model_runner.py:93-118): per layer, q/k/v become one GEMM and gate/up
        another; the separate projection modules are replaced by nn.Identity, so the model
        is changed in place and serves one fused runner.  Quantised projections (not float
        nn.Linear) are left as they are: returns [] and the runner stays unfused."""
        probe = self.layers[0].self_attn.q_proj
        if isinstance(probe, nn.Identity):
            raise ValueError("model already fused by another ModelRunner; fuse=True mutates "
                             "the model in place -- use one fused runner per model instance")
        if not isinstance(probe, nn.Linear) or not probe.weight.is_floating_point():
            return []
        fused = []
        for layer in self.layers:
            attn, mlp = layer.self_attn, layer.mlp
            projs = (attn.q_proj, attn.k_proj, attn.v_proj)
            biases = [p.bias for p in projs]
            fused.append(_FusedLayer(
                qkv_weight=torch.cat([p.weight for p in projs]),
                qkv_bias=None if biases[0] is None else torch.cat(biases),
                gate_up_weight=torch.cat([mlp.gate_proj.weight, mlp.up_proj.weight])))
            for name in ("q_proj", "k_proj", "v_proj"):
                setattr(attn, name, nn.Identity())
            for name in ("gate_proj", "up_proj"):
                setattr(mlp, name, nn.Identity())
        return fused

    def rope(self, positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        cos, sin = self.rotary_emb(self._rope_dummy, positions[None, :])
        return cos[0].to(self.dtype), sin[0].to(self.dtype)

    # -- batch metadata ---------------------------------------------------------------
    def _batch(self, seq_meta: list[SeqMeta], cache: PagedKVCache) -> _Batch:
        B = len(seq_meta)
        width = max(max((len(m.block_ids) for m in seq_meta), default=1), 1)
        host = torch.zeros((2 * B + 1 + B * width,), dtype=torch.int32)
        cu = 0
        for i, m in enumerate(seq_meta):
            if m.ctx_len > len(m.block_ids) * cache.block_size:
                raise ValueError(f"sequence {i}: ctx_len {m.ctx_len} exceeds its "
                                 f"{len(m.block_ids)} blocks")
            host[i] = m.ctx_len
            host[B + 1 + i] = cu = cu + m.q_len
            if m.block_ids:
                host[2 * B + 1 + i * width: 2 * B + 1 + i * width + len(m.block_ids)] = \
                    torch.tensor(m.block_ids, dtype=torch.int32)
        dev = host.to(cache.key.device)                 # one H2D copy for all metadata
        decode = all(m.q_len == 1 for m in seq_meta)
        shared = self._shared_prefix(seq_meta, host[2 * B + 1:].view(B, width),
                                     cache.block_size)
        max_q_len = max(m.q_len for m in seq_meta)
        max_ctx = width * cache.block_size
        balanced = (not decode and not shared and
                    self._prefer_balanced(seq_meta, max_q_len, max_ctx, cache.block_size))
        return _Batch(block_table=dev[2 * B + 1:].view(B, width), ctx_lens=dev[:B],
                      cu_q=dev[B:2 * B + 1], max_q_len=max_q_len, max_ctx=max_ctx,
                      decode=decode, shared_prefix=shared, balanced=balanced,
                      seqs=tuple(seq_meta))

    def _prefer_balanced(self, seq_meta: list[SeqMeta], max_q_len: int, max_ctx: int,
                         bs: int) -> bool:
        """Whether a batch of short query blocks (verify) runs on the balanced split-K
        kernel rather than fixed key partitions.  Fixed partitions are sized from max_ctx
        for every sequence; when the batch's keys per resident 16-row workgroup (three per
        CU) fall below `balanced_key_fraction` of that partition, the longest sequence's
        partitions run as a tail on a mostly idle GPU, and the balanced split, which gives
        every wave the same share of the keys, wins (one 32k context among 15 of 512, Qwen3
        heads, 5 queries: 44 against 93 us; similar lengths: fixed partitions 0-5 %
        faster)."""
        B = len(seq_meta)
        if (max_q_len * self.kv_groups > 16 or B > 512 or bs < 16 or not self._tuned_attention
                or self.head_dim not in (32, 64, 128)):
            return False
        P = _lib.lib().dsp_paged_mq_partition_tokens(B, self.num_heads, self.num_kv_heads,
                                                     self.head_dim, max_q_len, max_ctx)
        keys = sum(m.ctx_len for m in seq_meta) * self.num_kv_heads
        return keys < self.balanced_key_fraction * P * 3 * self._cus

    def _shared_prefix(self, seq_meta: list[SeqMeta], table: torch.Tensor, bs: int) -> int:
        """Leading context tokens whose blocks every sequence's table shares and every query
        sees, rounded down to a multiple of 128 -- or 0 when the batch is too small, the
        prefix too short, or the shape one the shared-prefix kernels do not serve."""
        B = len(seq_meta)
        if (B < self.shared_prefix_min_seqs or B > 1024 or bs < 16 or not self._tuned_attention
                or self.head_dim not in (64, 128)):
            return 0
        limit = min(m.ctx_len - m.q_len for m in seq_meta) // bs   # full blocks all queries see
        if limit * bs < self.shared_prefix_min_tokens:
            return 0
        same = (table[:, :limit] == table[0, :limit]).all(0)
        n = limit if bool(same.all()) else int(torch.argmin(same.to(torch.int8)))
        tokens = n * bs // 128 * 128
        return tokens if tokens >= self.shared_prefix_min_tokens else 0

    # -- attention for one layer --------------------------------------------------------
    def _project_qkv(self, attn, x: torch.Tensor, layer_idx: int):
        """q (T, Hq, D), k and v (T, KVH, D) of one layer; with fuse=True, views of one
        GEMM's output (heads laid out q, then k, then v, each row-strided)."""
        heads = (self.num_heads, self.num_kv_heads, self.num_kv_heads)
        if self._fused:
            f = self._fused[layer_idx]
            qkv = F.linear(x, f.qkv_weight, f.qkv_bias).unflatten(-1, (-1, self.head_dim))
            return qkv.split(heads, dim=1)
        projs = (attn.q_proj, attn.k_proj, attn.v_proj)
        return tuple(p(x).unflatten(-1, (n, self.head_dim)) for p, n in zip(projs, heads))

    def _attention(self, layer, x, cos, sin, write_slots, cache, layer_idx, batch: _Batch):
        attn = layer.self_attn
        q, k, v = self._project_qkv(attn, x, layer_idx)
        # q_norm / k_norm (Qwen3), RoPE on q and k, and cache.write(k, v): one launch
        q = qk_norm_rope_append(q, k, v, cos, sin, write_slots, cache, layer_idx,
                                attn.q_norm if self.qk_norm else None,
                                attn.k_norm if self.qk_norm else None)
        if self.attn_backend == "native":
            o = self._torch_attention(q, cache, layer_idx, batch.seqs)
        elif batch.decode and not batch.shared_prefix:
            o = paged_decode_attention_blocks(
                q, cache.key[layer_idx], cache.value[layer_idx], batch.block_table,
                batch.ctx_lens, self.kv_groups, block_size=cache.block_size, scale=self.scale,
                max_ctx=batch.max_ctx, workspace=batch.workspace)
        else:
            o = paged_mq_attention(
                q, cache.key[layer_idx], cache.value[layer_idx], batch.block_table, batch.cu_q,
                batch.ctx_lens, self.kv_groups, block_size=cache.block_size, scale=self.scale,
                max_q_len=batch.max_q_len, max_ctx=batch.max_ctx, workspace=batch.workspace,
                shared_prefix_tokens=batch.shared_prefix, balanced=batch.balanced)
        return attn.o_proj(o.flatten(1))

    def _torch_attention(self, q: torch.Tensor, cache: PagedKVCache, layer_idx: int,
                         seqs) -> torch.Tensor:
        """attn_backend="native": the reference's per-sequence attention
        (model_runner.py:160-185) -- the sequence's context rows gathered from the pool
        (the prologue has already appended this step's k and v, so a fresh prefill reads
        back exactly the rows it projected), then torch SDPA with the bottom-right causal
        mask and grouped KV heads.  SDPA runs in float32: torch's bf16 batched matmul on
        the transposed key operand SDPA forms is avoided on this platform; the output is
        rounded to the model dtype."""
        from torch.nn.attention.bias import causal_lower_right
        out = torch.empty_like(q)
        end = 0
        for m in seqs:
            start, end = end, end + m.q_len
            keys, vals = cache.gather(layer_idx, cache.context_slots(m.block_ids, m.ctx_len))
            as_bhd = lambda t: t.float().transpose(0, 1).unsqueeze(0)  # noqa: E731
            o = F.scaled_dot_product_attention(
                as_bhd(q[start:end]), as_bhd(keys), as_bhd(vals),
                attn_mask=causal_lower_right(m.q_len, m.ctx_len), scale=self.scale,
                enable_gqa=True)
            out[start:end] = o[0].transpose(0, 1)
        return out

    @torch.inference_mode()
    def forward(self, token_ids: torch.Tensor, positions: torch.Tensor,
                write_slots: torch.Tensor, seq_meta: list[SeqMeta],
                cache: PagedKVCache) -> torch.Tensor:
        """Normalized hidden states (T, hidden); `logits()` projects them."""
        return self.run_batch(token_ids, positions, write_slots, self._batch(seq_meta, cache),
                              cache)

    def run_batch(self, token_ids: torch.Tensor, positions: torch.Tensor,
                  write_slots: torch.Tensor, batch: _Batch, cache: PagedKVCache) -> torch.Tensor:
        """The layer loop of `forward` over batch metadata already on the device.

        No host sync and, for a batch that brings its own workspace, no allocation outside
        torch's allocator: this is the body a HIP graph captures.  Decode batches whose
        sequences share leading blocks (copy-on-write forks) take the shared-prefix
        multi-query kernel, which reads those blocks once for the batch."""
        cos, sin = self.rope(positions)
        x = self.embed(token_ids)
        if batch.workspace is None and self.attn_backend == "hip":
            B = batch.ctx_lens.shape[0]
            if batch.decode and not batch.shared_prefix:
                batch.workspace = decode_workspace(B, self.num_heads, self.num_kv_heads,
                                                   self.head_dim, batch.max_ctx,
                                                   cache.key.device)
            else:
                batch.workspace = mq_workspace(B, self.num_heads, self.num_kv_heads,
                                               self.head_dim, batch.max_q_len, batch.max_ctx,
                                               cache.key.device, batch.shared_prefix,
                                               batch.balanced)
        for i, layer in enumerate(self.layers):
            h = layer.input_layernorm(x)
            x = x + self._attention(layer, h, cos, sin, write_slots, cache, i, batch)
            h = layer.post_attention_layernorm(x)
            x = x + self._mlp(layer, h, i)
        return self.norm(x)

    def _mlp(self, layer, h, i):
        mlp = layer.mlp
        if not self._fused:
            return mlp(h)
        gate_up = F.linear(h, self._fused[i].gate_up_weight).unflatten(-1, (2, -1))
        return mlp.down_proj(mlp.act_fn(gate_up[..., 0, :]) * gate_up[..., 1, :])

    def logits(self, hidden: torch.Tensor, indices: torch.Tensor | None = None) -> torch.Tensor:
        """lm_head over the hidden states (of the rows `indices` selects, when given)."""
        return self.lm_head(hidden if indices is None else hidden[indices])
