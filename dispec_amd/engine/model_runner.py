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

Only "hip" is accepted: the reference's "native"/"triton" backends are torch/Triton
code paths this package does not carry.
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


class ModelRunner:
    def __init__(self, model, attn_backend: str = "hip", fuse: bool = False):
        if attn_backend != "hip":
            raise ValueError(f"attn_backend {attn_backend!r}: dispec_amd runs attention on its "
                             "HIP kernels only (attn_backend='hip')")
        self.model = model
        self.attn_backend = attn_backend
        cfg = model.config
        self.cfg = cfg
        self.device = next(model.parameters()).device
        self.dtype = next((p.dtype for p in model.parameters() if p.is_floating_point()),
                          torch.float16)
        core = model.model
        self.embed, self.layers, self.norm = core.embed_tokens, core.layers, core.norm
        self.lm_head = model.lm_head
        self.num_heads = cfg.num_attention_heads
        self.num_kv_heads = cfg.num_key_value_heads
        self.head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        self.kv_groups = self.num_heads // self.num_kv_heads
        self.scale = self.head_dim ** -0.5
        # the MFMA attention kernels (and with them the balanced verify split and the shared
        # prefix) serve bf16 / fp16; fp32 models attend through the generic kernel
        self._tuned_attention = self.dtype in (torch.bfloat16, torch.float16)
        attn0 = self.layers[0].self_attn
        self.qk_norm = hasattr(attn0, "q_norm") and hasattr(attn0, "k_norm")
        if "sliding_attention" in (getattr(cfg, "layer_types", None) or []):
            raise ValueError(f"{type(model).__name__} uses sliding-window attention layers, which "
                             "the paged attention path does not implement")
        self.rotary_emb = core.rotary_emb
        self._rope_dummy = torch.zeros(1, 1, device=self.device, dtype=self.dtype)
        self.fused = self._build_fused() if fuse else False
        # shared-prefix attention: used when at least this many sequences share at least
        # this many leading tokens (fewer gain nothing over per-sequence attention)
        self.shared_prefix_min_seqs = 4
        self.shared_prefix_min_tokens = 512
        # balanced split for verify batches whose keys per resident workgroup fall below
        # this fraction of the fixed split's partition (see _prefer_balanced)
        self.balanced_key_fraction = 0.6
        self._cus = (torch.cuda.get_device_properties(self.device).multi_processor_count
                     if self.device.type == "cuda" else 256)

    def _build_fused(self) -> bool:
        """One GEMM for q/k/v and one for gate/up per layer (model_runner.py:93-118)."""
        a0 = self.layers[0].self_attn
        if isinstance(a0.q_proj, nn.Identity):
            raise ValueError("model already fused by another ModelRunner; fuse=True mutates "
                             "the model in place -- use one fused runner per model instance")
        if not (isinstance(a0.q_proj, nn.Linear) and a0.q_proj.weight.is_floating_point()):
            return False
        self._qkv_w, self._qkv_b, self._gate_up_w = [], [], []
        for layer in self.layers:
            a, m = layer.self_attn, layer.mlp
            self._qkv_w.append(torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight], 0))
            self._qkv_b.append(torch.cat([a.q_proj.bias, a.k_proj.bias, a.v_proj.bias], 0)
                               if a.q_proj.bias is not None else None)
            self._gate_up_w.append(torch.cat([m.gate_proj.weight, m.up_proj.weight], 0))
            a.q_proj = a.k_proj = a.v_proj = nn.Identity()
            m.gate_proj = m.up_proj = nn.Identity()
        self._qsz = self.num_heads * self.head_dim
        self._kvsz = self.num_kv_heads * self.head_dim
        return True

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
                      decode=decode, shared_prefix=shared, balanced=balanced)

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
    def _attention(self, layer, x, cos, sin, write_slots, cache, layer_idx, batch: _Batch):
        attn = layer.self_attn
        T = x.shape[0]
        if self.fused:
            qkv = F.linear(x, self._qkv_w[layer_idx], self._qkv_b[layer_idx])
            q, k, v = qkv.split([self._qsz, self._kvsz, self._kvsz], dim=-1)
            q = q.view(T, self.num_heads, self.head_dim)
            k = k.view(T, self.num_kv_heads, self.head_dim)
            v = v.view(T, self.num_kv_heads, self.head_dim)
        else:
            q = attn.q_proj(x).view(T, self.num_heads, self.head_dim)
            k = attn.k_proj(x).view(T, self.num_kv_heads, self.head_dim)
            v = attn.v_proj(x).view(T, self.num_kv_heads, self.head_dim)
        # q_norm / k_norm (Qwen3), RoPE on q and k, and cache.write(k, v): one launch
        q = qk_norm_rope_append(q, k, v, cos, sin, write_slots, cache, layer_idx,
                                attn.q_norm if self.qk_norm else None,
                                attn.k_norm if self.qk_norm else None)
        if batch.decode and not batch.shared_prefix:
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
        return attn.o_proj(o.reshape(T, self.num_heads * self.head_dim))

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
        if batch.workspace is None:
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
        if not self.fused:
            return layer.mlp(h)
        gate, up = F.linear(h, self._gate_up_w[i]).chunk(2, dim=-1)
        return layer.mlp.down_proj(layer.mlp.act_fn(gate) * up)

    def logits(self, hidden: torch.Tensor, indices: torch.Tensor | None = None) -> torch.Tensor:
        if indices is not None:
            hidden = hidden[indices]
        return self.lm_head(hidden)
