"""Paged KV pool in HBM, read and written by the HIP kernels of libdispec_hip.so.

Drop-in for the reference `PagedKVCache` (dispec/kv/paged_cache.py:20-96): the same
constructor, the same per-cache layout -- K and V are separate tensors of shape
[num_layers, num_blocks * block_size, num_kv_heads, head_dim] (:39-41) -- and the same
slot definition, slot = block_id * block_size + offset (:6-7).  `cache.key[layer]` is
still the tensor an attention kernel reads, so code that indexes the pool directly keeps
working.  What changes is who moves the bytes:

  write              -> dsp_kv_append        (one launch for K and V; :61-68 used two
                                              index_copy_ launches)
  gather             -> dsp_kv_gather_slots  (:70-72)
  export_contiguous  -> dsp_kv_gather        (block-table gather over all layers, :87-90)
  import_contiguous  -> dsp_kv_scatter_ordered (:92-96)
  copy_blocks        -> dsp_kv_copy_blocks   (new: the data move behind copy-on-write
                                              fork and prefix-cache spill)

Kernels never read or write out of the pool: an out-of-range slot or block id is
skipped and counted in a device counter; `check_errors()` (or DISPEC_HIP_CHECK=1, which
checks after every call) raises IndexError for it, like index_copy_ does on the CPU.
"""

from __future__ import annotations

import os

import torch

from dispec_amd import _lib
from dispec_amd.kv.block_manager import BlockManager

_CHECK_EVERY_CALL = os.environ.get("DISPEC_HIP_CHECK", "0") not in ("", "0")


def check_prefix_kv(cache, prefix_kv, prompt_len: int) -> None:
    """Validate transferred KV before a request is admitted with it.

    The admission check of the reference scheduler (dispec/sched/scheduler.py:103-112):
    `prefix_kv` = (k, v), each (num_layers, T, num_kv_heads, head_dim) of `cache`'s
    layout, must cover at least one and fewer than all of the prompt's tokens -- the
    last prompt token is forwarded by the target itself to produce the first output
    token's logits.  Only the geometry attributes of `cache` are read, so the check runs
    on the host before anything reaches the GPU.  The messages are the reference's:
    callers and tests match on them.
    """
    k, v = prefix_kv
    covered = k.shape[1] if k.dim() > 1 else -1
    layout = (cache.num_layers, covered, cache.num_kv_heads, cache.head_dim)
    if tuple(k.shape) != layout or tuple(v.shape) != layout:
        raise ValueError(f"prefix_kv shapes {tuple(k.shape)}/{tuple(v.shape)} do not "
                         f"match this model's cache layout {layout}")
    check_prefix_coverage(covered, prompt_len)


def check_prefix_coverage(covered: int, prompt_len: int) -> None:
    """The coverage half of `check_prefix_kv`: 0 < covered < prompt_len."""
    if not 0 < covered < prompt_len:
        raise ValueError(f"prefix_kv covers {covered} tokens of a {prompt_len}-token "
                         "prompt; it must cover at least one and fewer than all of them")


class PagedKVCache:
    def __init__(self, num_layers: int, num_blocks: int, block_size: int, num_kv_heads: int,
                 head_dim: int, dtype: torch.dtype = torch.bfloat16, device: str = "cuda"):
        self.num_layers = num_layers
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = device
        shape = (num_layers, num_blocks * block_size, num_kv_heads, head_dim)
        self.key = torch.zeros(shape, dtype=dtype, device=device)
        self.value = torch.zeros(shape, dtype=dtype, device=device)
        _lib.require_gpu(self.key)
        self.manager = BlockManager(num_blocks, block_size)
        self._err = torch.zeros(1, dtype=torch.int32, device=self.key.device)

    @classmethod
    def for_model(cls, config, num_blocks: int, block_size: int, dtype,
                  device="cuda") -> "PagedKVCache":
        head_dim = getattr(config, "head_dim", None) or (
            config.hidden_size // config.num_attention_heads)
        return cls(num_layers=config.num_hidden_layers, num_blocks=num_blocks,
                   block_size=block_size, num_kv_heads=config.num_key_value_heads,
                   head_dim=head_dim, dtype=dtype, device=device)

    # -- geometry -------------------------------------------------------------------
    def memory_bytes(self) -> int:
        return self.key.numel() * self.key.element_size() * 2

    @property
    def num_slots(self) -> int:
        return self.num_blocks * self.block_size

    @property
    def row_bytes(self) -> int:
        """Bytes of one slot of one layer (all KV heads)."""
        return self.num_kv_heads * self.head_dim * self.key.element_size()

    @property
    def block_bytes(self) -> int:
        return self.block_size * self.row_bytes

    @property
    def layer_bytes(self) -> int:
        return self.num_slots * self.row_bytes

    def _stream(self) -> int:
        return _lib.stream_of(self.key)

    def _layer_ptrs(self, layer_idx: int) -> tuple[int, int]:
        """Device addresses of layer `layer_idx` of the K and V pools: what
        key[layer_idx].data_ptr() gives, without building the two views per call."""
        if not -self.num_layers <= layer_idx < self.num_layers:
            raise IndexError(f"layer {layer_idx} is out of range for {self.num_layers} layers")
        off = (layer_idx % self.num_layers) * self.layer_bytes
        return self.key.data_ptr() + off, self.value.data_ptr() + off

    # -- error reporting -----------------------------------------------------------
    def check_errors(self) -> None:
        """Raise IndexError if any kernel met an out-of-range slot or block id."""
        n = int(self._err.item())
        if n:
            self._err.zero_()
            raise IndexError(f"{n} out-of-range slot/block ids were skipped by the KV kernels "
                             f"(pool has {self.num_blocks} blocks of {self.block_size})")

    def _after(self) -> None:
        if _CHECK_EVERY_CALL:
            self.check_errors()

    def _rows(self, x: torch.Tensor, name: str, n: int) -> torch.Tensor:
        """Validate a (n, KVH, D) tensor whose token rows are each contiguous."""
        if tuple(x.shape) != (n, self.num_kv_heads, self.head_dim):
            raise ValueError(f"{name} has shape {tuple(x.shape)}, expected "
                             f"{(n, self.num_kv_heads, self.head_dim)}")
        if x.dtype != self.dtype:
            raise RuntimeError(f"{name} dtype {x.dtype} does not match the cache dtype {self.dtype}")
        if x.device != self.key.device:
            raise RuntimeError(f"{name} is on {x.device}, the cache on {self.key.device}")
        if n > 1 and not (x.stride(2) == 1 and x.stride(1) == self.head_dim):
            x = x.contiguous()
        elif n <= 1 and not x.is_contiguous():
            x = x.contiguous()
        return x

    @staticmethod
    def _as_slots(slots: torch.Tensor, device) -> torch.Tensor:
        if slots.dtype != torch.long or slots.device != device or not slots.is_contiguous():
            slots = slots.to(device=device, dtype=torch.long).contiguous()
        return slots

    # -- per-step IO ------------------------------------------------------------------
    def write(self, layer_idx: int, slots: torch.Tensor, k: torch.Tensor,
              v: torch.Tensor) -> None:
        """Append token rows: key[layer][slots] = k, value[layer][slots] = v.

        slots: (T,) long flat slot ids (unique); k, v: (T, num_kv_heads, head_dim).
        """
        n = slots.numel()
        k, v = self._rows(k, "k", n), self._rows(v, "v", n)
        if k.stride(0) != v.stride(0):
            k, v = k.contiguous(), v.contiguous()
        slots = self._as_slots(slots.reshape(-1), self.key.device)
        kp, vp = self._layer_ptrs(layer_idx)
        rb = self.row_bytes
        _lib.check(_lib.calls().dsp_kv_append(
            kp, vp, self.num_slots, rb, k.data_ptr(), v.data_ptr(),
            k.stride(0) * k.element_size(), slots.data_ptr(), n, rb, self._err.data_ptr(),
            self._stream()), "dsp_kv_append")
        self._after()

    def gather(self, layer_idx: int, slots: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """(k, v) rows of the given flat slots, each (len(slots), KVH, D)."""
        slots = self._as_slots(slots.reshape(-1), self.key.device)
        n = slots.numel()
        k = torch.empty((n, self.num_kv_heads, self.head_dim), dtype=self.dtype,
                        device=self.key.device)
        v = torch.empty_like(k)
        _lib.check(_lib.lib().dsp_kv_gather_slots(
            self.key[layer_idx].data_ptr(), self.value[layer_idx].data_ptr(), self.num_slots,
            self.row_bytes, slots.data_ptr(), n, self.row_bytes, k.data_ptr(), v.data_ptr(),
            self.row_bytes, self._err.data_ptr(), self._stream()), "dsp_kv_gather_slots")
        self._after()
        return k, v

    # -- slot helpers (host index math, same as paged_cache.py:75-84) -------------------
    def slots_for_positions(self, block_ids: list[int], positions: torch.Tensor) -> torch.Tensor:
        bt = torch.tensor(block_ids, device=positions.device, dtype=torch.long)
        return bt[positions // self.block_size] * self.block_size + positions % self.block_size

    def context_slots(self, block_ids: list[int], num_tokens: int) -> torch.Tensor:
        pos = torch.arange(num_tokens, device=self.key.device)
        return self.slots_for_positions(block_ids, pos)

    def block_table(self, tables: list[list[int]], width: int | None = None) -> torch.Tensor:
        """Device int32 [len(tables), width] block table, padded with zeros."""
        width = max([len(t) for t in tables] + [1]) if width is None else width
        host = torch.zeros((len(tables), width), dtype=torch.int32)
        for i, ids in enumerate(tables):
            if len(ids) > width:
                raise ValueError(f"sequence {i} has {len(ids)} blocks, table width {width}")
            if ids:
                host[i, :len(ids)] = torch.tensor(ids, dtype=torch.int32)
        return host.to(self.key.device, non_blocking=False)

    # -- whole-sequence export / import (P/D disaggregation, escalation) ------------------
    def _check_blocks(self, block_ids: list[int], num_tokens: int) -> None:
        need = -(-num_tokens // self.block_size)
        if len(block_ids) < need:
            raise IndexError(f"{num_tokens} tokens need {need} blocks, table has {len(block_ids)}")
        bad = [b for b in block_ids[:need] if not 0 <= b < self.num_blocks]
        if bad:
            raise IndexError(f"block ids {bad} outside a pool of {self.num_blocks} blocks")

    def export_batch(self, seqs: list[tuple[list[int], int]]) -> tuple[torch.Tensor, torch.Tensor, list[int]]:
        """Gather several sequences in one launch.

        seqs: (block_ids, seq_len) per sequence.  Returns flat K and V buffers and the
        token offsets; sequence b is buffer[L*cu[b] : L*cu[b+1]] viewed as (L, T_b, H, D).
        """
        for ids, n in seqs:
            self._check_blocks(ids, n)
        cu = [0]
        for _, n in seqs:
            cu.append(cu[-1] + n)
        rows = self.num_layers * cu[-1]
        kbuf = torch.empty((rows, self.num_kv_heads, self.head_dim), dtype=self.dtype,
                           device=self.key.device)
        vbuf = torch.empty_like(kbuf)
        if cu[-1]:
            table = self.block_table([ids for ids, _ in seqs])
            cu_t = torch.tensor(cu, dtype=torch.long).to(self.key.device)
            _lib.check(_lib.lib().dsp_kv_gather(
                self.key.data_ptr(), self.value.data_ptr(), self.num_layers, self.layer_bytes,
                self.num_blocks, self.row_bytes, self.block_size, table.data_ptr(),
                table.stride(0), cu_t.data_ptr(), len(seqs), max(n for _, n in seqs),
                kbuf.data_ptr(), vbuf.data_ptr(), self._err.data_ptr(), self._stream()),
                "dsp_kv_gather")
            self._after()
        return kbuf, vbuf, cu

    def export_contiguous(self, block_ids: list[int], seq_len: int) -> tuple[torch.Tensor, torch.Tensor]:
        """A sequence's first seq_len tokens as contiguous (num_layers, seq_len, H, D)."""
        kbuf, vbuf, _ = self.export_batch([(block_ids, seq_len)])
        shape = (self.num_layers, seq_len, self.num_kv_heads, self.head_dim)
        return kbuf.view(shape), vbuf.view(shape)

    def import_batch(self, tables: list[list[int]], k: torch.Tensor, v: torch.Tensor,
                     cu: list[int]) -> None:
        """Scatter flat buffers laid out as export_batch's into the given block tables."""
        for ids, a, b in zip(tables, cu[:-1], cu[1:]):
            self._check_blocks(ids, b - a)
        if not cu[-1]:
            return
        k, v = k.contiguous(), v.contiguous()
        table = self.block_table(tables)
        cu_t = torch.tensor(cu, dtype=torch.long).to(self.key.device)
        self._scatter(table, cu_t, max(b - a for a, b in zip(cu[:-1], cu[1:])), k, v)
        self._after()

    def _scatter(self, table: torch.Tensor, cu_t: torch.Tensor, max_seqlen: int,
                 k: torch.Tensor, v: torch.Tensor) -> None:
        """dsp_kv_scatter_ordered: the copies in destination-block order when the tables
        name at least half the pool's blocks (the library decides), with a block-owner
        workspace from torch's stream-ordered allocator."""
        owner = torch.empty(self.num_blocks, dtype=torch.int32, device=self.key.device)
        _lib.check(_lib.lib().dsp_kv_scatter_ordered(
            self.key.data_ptr(), self.value.data_ptr(), self.num_layers, self.layer_bytes,
            self.num_blocks, self.row_bytes, self.block_size, table.data_ptr(), table.stride(0),
            cu_t.data_ptr(), table.shape[0], int(max_seqlen), k.data_ptr(), v.data_ptr(),
            owner.data_ptr(), self._err.data_ptr(), self._stream()), "dsp_kv_scatter_ordered")

    def import_contiguous(self, block_ids: list[int], k: torch.Tensor, v: torch.Tensor) -> None:
        """Scatter contiguous (num_layers, T, H, D) K/V into the sequence's blocks."""
        shape = (self.num_layers, k.shape[1], self.num_kv_heads, self.head_dim)
        if tuple(k.shape) != shape or tuple(v.shape) != shape:
            raise ValueError(f"import shapes {tuple(k.shape)}/{tuple(v.shape)} do not match the "
                             f"cache layout {shape}")
        k = k.to(device=self.key.device, dtype=self.dtype)
        v = v.to(device=self.key.device, dtype=self.dtype)
        self.import_batch([block_ids], k, v, [0, k.shape[1]])

    def check_prefix_kv(self, prefix_kv, prompt_len: int) -> None:
        """Raise ValueError unless prefix_kv fits this cache and covers 0 < T < prompt_len
        of the prompt (dispec/sched/scheduler.py:103-112)."""
        check_prefix_kv(self, prefix_kv, prompt_len)

    def admit_prefix(self, block_ids: list[int], prefix_kv, prompt_len: int) -> int:
        """Admit a request with transferred KV: check it, scatter it into the request's
        blocks and return the number of prompt tokens it covers -- the tokens the block
        table now holds and the position prefill resumes from (scheduler.py:96-97,
        :165-170)."""
        self.check_prefix_kv(prefix_kv, prompt_len)
        self.import_contiguous(block_ids, *prefix_kv)
        return prefix_kv[0].shape[1]

    # -- device-table forms (no host round trip; what graph-captured callers use) ---------
    def gather_into(self, block_table: torch.Tensor, cu_seqlens: torch.Tensor, max_seqlen: int,
                    k_buf: torch.Tensor, v_buf: torch.Tensor) -> None:
        """export_batch with the int32 block table and int64 token offsets already on the
        GPU; k_buf/v_buf hold num_layers * cu_seqlens[-1] contiguous rows."""
        _lib.check(_lib.lib().dsp_kv_gather(
            self.key.data_ptr(), self.value.data_ptr(), self.num_layers, self.layer_bytes,
            self.num_blocks, self.row_bytes, self.block_size, block_table.data_ptr(),
            block_table.stride(0), cu_seqlens.data_ptr(), block_table.shape[0], int(max_seqlen),
            k_buf.data_ptr(), v_buf.data_ptr(), self._err.data_ptr(), self._stream()),
            "dsp_kv_gather")

    def scatter_from(self, block_table: torch.Tensor, cu_seqlens: torch.Tensor, max_seqlen: int,
                     k_buf: torch.Tensor, v_buf: torch.Tensor) -> None:
        """import_batch with device-side tables (the inverse of gather_into)."""
        self._scatter(block_table, cu_seqlens, max_seqlen, k_buf, v_buf)

    def copy_blocks_device(self, src: "PagedKVCache", src_ids: torch.Tensor,
                           dst_ids: torch.Tensor) -> None:
        """Block copy src -> self with int32 id arrays already on the GPU."""
        _lib.check(_lib.lib().dsp_kv_copy_blocks(
            src.key.data_ptr(), src.value.data_ptr(), src.layer_bytes, src.num_blocks,
            self.key.data_ptr(), self.value.data_ptr(), self.layer_bytes, self.num_blocks,
            self.num_layers, self.block_bytes, src_ids.data_ptr(), dst_ids.data_ptr(),
            src_ids.numel(), self._err.data_ptr(), self._stream()), "dsp_kv_copy_blocks")

    def copy_block_fanout_device(self, src: "PagedKVCache", src_block: int,
                                 dst_ids: torch.Tensor) -> None:
        """Block src_block of src copied into every block of dst_ids (int32, on the GPU)."""
        _lib.check(_lib.lib().dsp_kv_copy_block_fanout(
            src.key.data_ptr(), src.value.data_ptr(), src.layer_bytes, src.num_blocks,
            self.key.data_ptr(), self.value.data_ptr(), self.layer_bytes, self.num_blocks,
            self.num_layers, self.block_bytes, int(src_block), dst_ids.data_ptr(),
            dst_ids.numel(), self._err.data_ptr(), self._stream()), "dsp_kv_copy_block_fanout")

    # -- block copies (copy-on-write, prefix-cache spill) ----------------------------------
    def copy_blocks_from(self, src: "PagedKVCache", src_ids: list[int], dst_ids: list[int]) -> None:
        """dst[l, block d] = src[l, block s] for every layer, K and V."""
        if len(src_ids) != len(dst_ids):
            raise ValueError("src_ids and dst_ids differ in length")
        if (src.num_layers, src.block_bytes) != (self.num_layers, self.block_bytes):
            raise ValueError("block copy between pools of different geometry")
        if not src_ids:
            return
        if src is self and set(src_ids) & set(dst_ids):
            raise ValueError("a block is both copied from and written in one copy_blocks call")
        if len(src_ids) > 1 and len(set(src_ids)) == 1 and 0 <= src_ids[0] < src.num_blocks:
            # one block forked into many (copy-on-write children of one prompt): read it
            # once per group of copies
            dst = torch.tensor(list(dst_ids), dtype=torch.int32).to(self.key.device)
            self.copy_block_fanout_device(src, src_ids[0], dst)
            self._after()
            return
        ids = torch.tensor([list(src_ids), list(dst_ids)], dtype=torch.int32).to(self.key.device)
        _lib.check(_lib.lib().dsp_kv_copy_blocks(
            src.key.data_ptr(), src.value.data_ptr(), src.layer_bytes, src.num_blocks,
            self.key.data_ptr(), self.value.data_ptr(), self.layer_bytes, self.num_blocks,
            self.num_layers, self.block_bytes, ids[0].data_ptr(), ids[1].data_ptr(), len(src_ids),
            self._err.data_ptr(), self._stream()), "dsp_kv_copy_blocks")
        self._after()

    def copy_blocks(self, pairs: list[tuple[int, int]]) -> None:
        """In-pool block copies, e.g. the pairs BlockManager.cow_fork returns."""
        self.copy_blocks_from(self, [s for s, _ in pairs], [d for _, d in pairs])

    # -- copy-on-write helpers ---------------------------------------------------------
    def cow_fork(self, parent_id: int, child_id: int):
        """BlockManager.cow_fork plus the copy of the parent's partial block."""
        table, pairs = self.manager.cow_fork(parent_id, child_id)
        self.copy_blocks(pairs)
        return table

    def append_token(self, seq_id: int) -> tuple[int, int]:
        """Reserve the next token's slot, un-sharing a shared last block first."""
        self.copy_blocks(self.manager.ensure_writable(seq_id))
        return self.manager.append_token(seq_id)
