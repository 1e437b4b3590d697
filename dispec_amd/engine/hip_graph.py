"""HIP-graph capture of the batched decode step.

Drop-in for the reference's CudaGraphDecoder (dispec/engine/cuda_graph.py:39-117): the
same constructor (runner, cache, buckets), `capture()`, `can_handle(ctx_len)` and the
batch-1 `decode(token, position, write_slot, ctx_slots)` returning (1, vocab) logits.
What changes is the body that is captured and the batch it covers:

  * The captured body is `ModelRunner.run_batch`, the eager forward itself: K/V append
    through dsp_kv_append and split-K paged decode through dsp_paged_decode over a device
    block table.  The reference captures a second copy of the forward whose attention is
    gather + repeat_interleave + SDPA over a masked window (cuda_graph.py:48-79), so its
    graph does work proportional to the bucket; here the kernels read ctx_lens from
    device memory and skip partitions past each sequence's end, so a replay costs what
    the real context costs.
  * Any batch size, not only 1: `decode_batch(token_ids, positions, write_slots,
    seq_meta)` has ModelRunner.forward's signature for an all-decode batch.  One graph is
    captured per (batch size, context bucket), on first use or by `capture()`.
  * All per-step metadata (tokens, positions, write slots, context lengths and the block
    table) is packed into one pinned host buffer and sent with ONE host-to-device copy
    into the graph's static buffers, then the graph is replayed on the same stream.  The
    reference fills five static tensors with separate copies (cuda_graph.py:108-115).
  * Capture is safe while the cache holds live data: the warm-up passes run with every
    write slot set to -1 and every context length 0, so they neither write nor read the
    pool (the reference warms up by writing slot 0, cuda_graph.py:93-94).  The append
    kernel counts the -1 slots as skipped rows; the cache's error counter is restored
    afterwards.

Buckets are context lengths; a bucket of C tokens gives the graph a block table of
ceil(C / block_size) columns and sizes the split-K grid for C.  Contexts past the largest
bucket are not handled (`can_handle` is False): the caller runs the eager ModelRunner.
Logits returned by a replay live in the graph's output buffer and stay valid until the
next replay of the same (batch size, bucket) graph.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from dispec_amd.engine.model_runner import ModelRunner, SeqMeta, _Batch
from dispec_amd.engine.hip_attn import decode_workspace
from dispec_amd.kv.paged_cache import PagedKVCache

DEFAULT_BUCKETS = (256, 512, 1024, 2048)
_WARMUP = 2


@dataclass
class _Graph:
    """Static buffers and the captured graph of one (batch size, bucket)."""

    batch: int
    width: int               # block-table columns
    host: torch.Tensor       # pinned int32 staging: [tok i64 | pos i64 | slot i64 | ctx | cu_q | table]
    dev: torch.Tensor        # device copy of `host`; the graph reads only this
    tok: torch.Tensor
    pos: torch.Tensor
    wslot: torch.Tensor
    meta: _Batch
    copied: torch.cuda.Event  # recorded after the last host->device copy of `host`
    graph: torch.cuda.CUDAGraph | None = None
    out: torch.Tensor | None = None


def _layout(B: int, W: int) -> tuple[int, int, int]:
    """int32 offsets in the staging buffer: ctx_lens, cu_q, table; and the total length."""
    ctx = 6 * B                   # three int64 vectors of B first (8-byte aligned)
    cu = ctx + B
    table = cu + B + 1
    return ctx, table, table + B * W


class HipGraphDecoder:
    def __init__(self, runner: ModelRunner, cache: PagedKVCache,
                 buckets: tuple[int, ...] = DEFAULT_BUCKETS):
        if not buckets or min(buckets) <= 0:
            raise ValueError(f"buckets must be positive context lengths, got {buckets}")
        if runner.attn_backend != "hip":
            # the native backend walks the host-side sequence list every step: a replay
            # would attend with the lengths of the step that was captured
            raise ValueError(f"HipGraphDecoder captures attn_backend='hip' (device-side batch "
                             f"metadata); this runner uses {runner.attn_backend!r}")
        if cache.key.device.type != "cuda":
            raise RuntimeError("HipGraphDecoder needs the cache on a GPU")
        self.r = runner
        self.cache = cache
        self.buckets = sorted(set(int(b) for b in buckets))
        self.max_ctx = self.buckets[-1]
        self._g: dict[tuple[int, int], _Graph] = {}

    # -- capture ------------------------------------------------------------------------
    def _bucket(self, ctx_len: int) -> int:
        for b in self.buckets:
            if b >= ctx_len:
                return b
        raise ValueError(f"context length {ctx_len} exceeds the largest bucket "
                         f"{self.max_ctx}; run the eager ModelRunner for it")

    def _new(self, B: int, bucket: int) -> _Graph:
        bs = self.cache.block_size
        W = -(-bucket // bs)
        dev_ = self.cache.key.device
        ctx_off, tab_off, n = _layout(B, W)
        host = torch.zeros(n, dtype=torch.int32, pin_memory=True)
        host[ctx_off + B: tab_off] = torch.arange(B + 1, dtype=torch.int32)   # cu_q: one row each
        dev = torch.zeros(n, dtype=torch.int32, device=dev_)
        i64 = dev[:6 * B].view(torch.int64)
        meta = _Batch(block_table=dev[tab_off:].view(B, W), ctx_lens=dev[ctx_off:ctx_off + B],
                      cu_q=dev[ctx_off + B:tab_off], max_q_len=1, max_ctx=W * bs, decode=True,
                      workspace=decode_workspace(B, self.r.num_heads, self.r.num_kv_heads,
                                                 self.r.head_dim, W * bs, dev_))
        return _Graph(B, W, host, dev, i64[:B], i64[B:2 * B], i64[2 * B:], meta,
                      torch.cuda.Event())

    def _body(self, g: _Graph) -> torch.Tensor:
        hidden = self.r.run_batch(g.tok, g.pos, g.wslot, g.meta, self.cache)
        return self.r.lm_head(hidden)

    @torch.inference_mode()
    def _capture_one(self, B: int, bucket: int) -> _Graph:
        g = self._new(B, bucket)
        # Warm-up passes that touch no cache data: slot -1 is skipped by the append kernel
        # (and counted), context length 0 makes attention read nothing.
        g.host[:6 * B].view(torch.int64)[2 * B:] = -1
        g.dev.copy_(g.host)
        err = self.cache._err.clone()
        for _ in range(_WARMUP):
            self._body(g)
        torch.cuda.synchronize()
        self.cache._err.copy_(err)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = self._body(g)
        torch.cuda.synchronize()
        g.graph, g.out = graph, out
        self._g[(B, bucket)] = g
        return g

    def capture(self, batch_sizes: tuple[int, ...] = (1,)) -> None:
        """Capture one graph per (batch size, bucket).  Live cache data is left intact."""
        for B in batch_sizes:
            for bucket in self.buckets:
                if (B, bucket) not in self._g:
                    self._capture_one(B, bucket)

    def can_handle(self, ctx_len: int) -> bool:
        return ctx_len <= self.max_ctx

    # -- replay -------------------------------------------------------------------------
    @staticmethod
    def _put(host_view: torch.Tensor, vals, name: str, B: int):
        """Stage a host value list / tensor, or return a device tensor to copy after."""
        if isinstance(vals, torch.Tensor) and vals.device.type != "cpu":
            if vals.numel() != B:
                raise ValueError(f"{name} has {vals.numel()} entries for a batch of {B}")
            return vals
        t = torch.as_tensor(vals, dtype=torch.int64).reshape(-1)
        if t.numel() != B:
            raise ValueError(f"{name} has {t.numel()} entries for a batch of {B}")
        host_view.copy_(t)
        return None

    @torch.inference_mode()
    def decode_batch(self, token_ids, positions, write_slots,
                     seq_meta: list[SeqMeta]) -> torch.Tensor:
        """Logits (B, vocab) of one decode step: each sequence appends one token.

        token_ids, positions, write_slots: B ints each, as lists, host tensors or device
        tensors (a device tensor, e.g. the previous step's argmax, is copied on the
        stream and never read by the host).  seq_meta: ModelRunner's per-sequence
        metadata with q_len 1; ctx_len counts the new token."""
        bs = self.cache.block_size
        for i, m in enumerate(seq_meta):
            if m.q_len != 1:
                raise ValueError(f"sequence {i}: q_len {m.q_len}; the graph runs decode only")
            if not 1 <= m.ctx_len <= len(m.block_ids) * bs:
                raise ValueError(f"sequence {i}: ctx_len {m.ctx_len} needs 1..{len(m.block_ids)} "
                                 f"blocks of {bs} tokens")
        return self._step(token_ids, positions, write_slots, [m.ctx_len for m in seq_meta],
                          [m.block_ids for m in seq_meta])

    @torch.inference_mode()
    def decode(self, token: int, position: int, write_slot: int,
               ctx_slots: torch.Tensor) -> torch.Tensor:
        """Batch-1 step with the reference's signature (cuda_graph.py:102-117).

        ctx_slots: the (ctx_len,) flat slots of the context, new token included, as
        `PagedKVCache.context_slots` returns them (slot = block * block_size + offset,
        so the block ids are slots[::block_size] // block_size).  A device tensor is
        turned into block ids on the stream, without a host sync."""
        n = int(ctx_slots.numel())
        if n < 1:
            raise ValueError("ctx_slots is empty: the context includes the new token")
        blocks = ctx_slots.reshape(-1)[::self.cache.block_size] // self.cache.block_size
        if blocks.device.type == "cpu":
            return self._step([token], [position], [write_slot], [n], [blocks.tolist()])
        return self._step([token], [position], [write_slot], [n], [None], dev_row0=blocks)

    def _step(self, token_ids, positions, write_slots, ctx_lens: list[int],
              tables: list, dev_row0: torch.Tensor | None = None) -> torch.Tensor:
        B = len(ctx_lens)
        if B == 0:
            raise ValueError("empty batch")
        bs = self.cache.block_size
        bucket = self._bucket(max(ctx_lens))
        g = self._g.get((B, bucket)) or self._capture_one(B, bucket)
        g.copied.synchronize()                  # the previous step's copy has left `host`
        ctx_off, tab_off, _ = _layout(B, g.width)
        h64 = g.host[:6 * B].view(torch.int64)
        late = [(dv, self._put(h64[k * B:(k + 1) * B], vals, name, B))
                for k, (dv, vals, name) in enumerate(((g.tok, token_ids, "token_ids"),
                                                      (g.pos, positions, "positions"),
                                                      (g.wslot, write_slots, "write_slots")))]
        g.host[ctx_off:ctx_off + B] = torch.tensor(ctx_lens, dtype=torch.int32)
        table = g.host[tab_off:].view(B, g.width)
        for i, ids in enumerate(tables):
            if ids is not None:
                nb = -(-ctx_lens[i] // bs)
                table[i, :nb] = torch.tensor(ids[:nb], dtype=torch.int32)
        g.dev.copy_(g.host, non_blocking=True)  # one H2D copy of all metadata
        g.copied.record()
        for dv, src in late:
            if src is not None:
                dv.copy_(src.reshape(-1))
        if dev_row0 is not None:
            g.meta.block_table[0, :dev_row0.numel()].copy_(dev_row0)
        g.graph.replay()
        return g.out
