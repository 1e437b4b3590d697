"""Paged attention on the HIP kernels of libdispec_hip.so.

`batched_paged_decode_attention` and `paged_decode_attention` keep the signatures and
semantics of the reference's Triton wrappers (dispec/engine/triton_attn.py:98-139): the
same argument meaning, the per-token int32 slot table, `scale = scale or D ** -0.5`, and
an output allocated like `torch.empty_like(q)`.  They call `dsp_paged_decode`, a
GQA-packed split-K kernel with a log-sum-exp combine, instead of one Triton program per
(sequence, query head).  Like the Triton kernel they take any power-of-two head_dim from 8
to 256 and fp32 caches as well as bf16 / fp16: shapes outside the tuned kernels (fp32, head
dims 8 and 256, more than 8 query heads per KV head) run on a generic wave-per-row kernel.

`paged_decode_attention_blocks` is the block-table form (the table is
[B, max_blocks] int32 instead of [B, max_ctx] slots), the one `ModelRunner` uses.
"""

from __future__ import annotations

import functools

import torch

from dispec_amd import _lib

_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


@functools.lru_cache(maxsize=256)
def _decode_ws_bytes(B, Hq, KVH, D, max_ctx, P) -> int:
    return _lib.lib().dsp_paged_decode_workspace_bytes(B, Hq, KVH, D, max_ctx, P)


@functools.lru_cache(maxsize=256)
def _mq_ws_bytes(B, Hq, KVH, D, max_q_len, max_ctx, P) -> int:
    return _lib.lib().dsp_paged_mq_workspace_bytes(B, Hq, KVH, D, max_q_len, max_ctx, P)


# Split-K workspaces of calls that bring none, one per (device, stream): kernels on one
# stream run in order, so consecutive calls can share it; it grows to the largest need.
# Under graph capture a call allocates its own (from the graph's pool), so that no captured
# graph keeps the address of a cached workspace that a later, larger call replaces.
_WS: dict = {}


def _workspace(need: int, device, stream: int) -> torch.Tensor:
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(need // 4 + 1, dtype=torch.float32, device=device)
    key = (device, stream)
    ws = _WS.get(key)
    if ws is None or ws.numel() * 4 < need:
        ws = torch.empty(need // 4 + 1, dtype=torch.float32, device=device)
        _WS[key] = ws
    return ws


def _i32(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.int32 and t.is_contiguous() else t.to(torch.int32).contiguous()


def _decode(q, k_cache, v_cache, ctx_lens, kv_groups, scale, *, slot_table=None,
            block_table=None, block_size=16, max_ctx=None, partition_tokens=0, out=None,
            workspace=None, err=None):
    _lib.require_gpu(q, k_cache, v_cache, ctx_lens)
    if q.dim() != 3 or k_cache.dim() != 3 or v_cache.shape != k_cache.shape:
        raise ValueError(f"expected q (B, Hq, D) and caches (S, KVH, D); got {tuple(q.shape)}, "
                         f"{tuple(k_cache.shape)}, {tuple(v_cache.shape)}")
    B, Hq, D = q.shape
    S, KVH, Dk = k_cache.shape
    if Dk != D or Hq != KVH * kv_groups:
        raise ValueError(f"q has {Hq} heads of {D}, cache {KVH} heads of {Dk}, kv_groups {kv_groups}")
    if q.dtype not in _DTYPES or k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
        raise ValueError(f"q/k/v dtypes {q.dtype}/{k_cache.dtype}/{v_cache.dtype}: "
                         "the HIP decode kernels take bf16, fp16 or fp32, all the same")
    if k_cache.stride() != v_cache.stride() or k_cache.stride(2) != 1:
        raise ValueError("k_cache and v_cache need the same strides with head_dim contiguous")
    scale = scale or D ** -0.5
    if q.stride(2) != 1:
        q = q.contiguous()
    ctx_lens = _i32(ctx_lens)
    table = _i32(slot_table if slot_table is not None else block_table)
    if max_ctx is None:
        max_ctx = table.shape[1] if slot_table is not None else table.shape[1] * block_size
    out = torch.empty_like(q) if out is None else out
    if out.shape != q.shape or out.dtype != q.dtype or out.stride(2) != 1:
        raise ValueError("out must have q's shape and dtype with head_dim contiguous")
    L = _lib.calls()
    P = int(partition_tokens)  # 0: the library's automatic split
    stream = _lib.stream_of(q)
    need = _decode_ws_bytes(B, Hq, KVH, D, int(max_ctx), P)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = _workspace(need, q.device, stream)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    by_block = slot_table is None
    _lib.check(L.dsp_paged_decode(
        q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(), S,
        k_cache.stride(0), k_cache.stride(1),
        table.data_ptr() if by_block else None, table.stride(0) if by_block else 0,
        block_size, None if by_block else table.data_ptr(),
        0 if by_block else table.stride(0), ctx_lens.data_ptr(), B, Hq, KVH, D,
        float(scale), int(max_ctx), int(P), _lib.ptr(workspace), ws_bytes, out.data_ptr(),
        out.stride(0), out.stride(1), _lib.dtype_code(q.dtype), _lib.ptr(err), stream),
        "dsp_paged_decode")
    return out


def batched_paged_decode_attention(q, k_cache, v_cache, slot_table, ctx_lens, kv_groups,
                                   scale=None):
    """Paged attention for a batch of single-token queries, one launch (plus combine).

    q:          (B, num_heads, head_dim)
    k_cache:    (num_slots, num_kv_heads, head_dim), v_cache the same
    slot_table: (B, max_ctx) int32 slot of each context position (padding ignored)
    ctx_lens:   (B,) int32 context length of each sequence
    returns:    (B, num_heads, head_dim) in q's dtype
    """
    return _decode(q, k_cache, v_cache, ctx_lens, kv_groups, scale, slot_table=slot_table)


def paged_decode_attention(q, k_cache, v_cache, slots, kv_groups, scale=None):
    """Paged attention for one query token over `slots` (ctx,) of the cache.

    q: (num_heads, head_dim); returns (num_heads, head_dim).
    """
    ctx = slots.shape[0]
    table = slots.to(torch.int32).reshape(1, ctx)
    ctx_lens = torch.full((1,), ctx, dtype=torch.int32, device=q.device)
    return _decode(q.unsqueeze(0), k_cache, v_cache, ctx_lens, kv_groups, scale,
                   slot_table=table)[0]


def paged_decode_attention_blocks(q, k_cache, v_cache, block_table, ctx_lens, kv_groups,
                                  block_size=16, scale=None, max_ctx=None, partition_tokens=0,
                                  out=None, workspace=None, err=None):
    """Decode attention addressed by a block table.

    block_table: (B, max_blocks) int32 physical block ids; token j of sequence b lives
    in slot block_table[b, j // block_size] * block_size + j % block_size.
    max_ctx: upper bound of ctx_lens (defaults to max_blocks * block_size); it sizes the
    split-K grid, so a tight bound saves empty workgroups.
    err: optional int32 device counter, incremented for a context length outside
    [0, max_ctx] (clamped) and for block ids whose slots lie outside the cache (skipped).
    """
    return _decode(q, k_cache, v_cache, ctx_lens, kv_groups, scale, block_table=block_table,
                   block_size=block_size, max_ctx=max_ctx, partition_tokens=partition_tokens,
                   out=out, workspace=workspace, err=err)


def decode_workspace(batch, num_heads, num_kv_heads, head_dim, max_ctx, device):
    """A float32 split-K workspace big enough for every decode launch of this shape (the
    automatic split), or None when the launch needs none.  One buffer serves all layers of
    a forward: the launches run in stream order."""
    L = _lib.calls()
    need = L.dsp_paged_decode_workspace_bytes(batch, num_heads, num_kv_heads, head_dim,
                                              max_ctx, 0)
    return torch.empty(need // 4 + 1, dtype=torch.float32, device=device) if need else None


def mq_workspace(batch, num_heads, num_kv_heads, head_dim, max_q_len, max_ctx, device,
                 shared_prefix_tokens=0, balanced=False):
    """A float32 split-K workspace for every `paged_mq_attention` launch of this shape with
    the automatic partition (or the balanced split), or None when it needs none.  One
    buffer serves all layers of a forward: the launches run in stream order."""
    L = _lib.calls()
    if shared_prefix_tokens:
        P = L.dsp_paged_mq_shared_prefix_partition_tokens(
            batch, num_heads, num_kv_heads, head_dim, max_q_len, max_ctx, shared_prefix_tokens)
    else:
        P = _lib.DSP_SPLIT_BALANCED if balanced else 0
    need = L.dsp_paged_mq_workspace_bytes(batch, num_heads, num_kv_heads, head_dim, max_q_len,
                                          max_ctx, P)
    return torch.empty(need // 4 + 1, dtype=torch.float32, device=device) if need else None


def paged_mq_attention(q, k_cache, v_cache, block_table, cu_q, ctx_lens, kv_groups,
                       block_size=16, scale=None, max_q_len=None, max_ctx=None, out=None,
                       err=None, partition_tokens=0, workspace=None, shared_prefix_tokens=0,
                       balanced=False):
    """Multi-query paged attention: speculative verify, chunked and fresh prefill.

    Per sequence b, rows q[cu_q[b]:cu_q[b+1]] are the last q_len_b tokens of a ctx_b-token
    context already in the cache, attended with the bottom-right causal mask and GQA
    (the native path of the reference runner, model_runner.py:160-185).

    q:           (sum q_len, num_heads, head_dim), packed by sequence
    block_table: (B, max_blocks) int32
    cu_q:        (B+1,) int32 query offsets;  ctx_lens: (B,) int32 context lengths
    max_q_len, max_ctx: host-side bounds (computed from cu_q / the table if omitted,
                 which costs a device->host copy)
    partition_tokens: split-K key partition (0: chosen from the shape); workspace: an
                 optional preallocated fp32 buffer for the partial results
    balanced:    short query blocks (max_q_len * kv_groups <= 16) on the balanced split-K
                 kernel instead of key partitions: every wave takes an equal share of the
                 keys, which pays when one context is much longer than the others
                 (DSP_SPLIT_BALANCED)
    shared_prefix_tokens: > 0 when the first that many context tokens of every sequence
                 are the same physical blocks (copy-on-write forks, prefix-cache hits) and
                 every query sees them all: they are attended once for the whole batch
                 (a multiple of 128, < max_ctx; dsp_paged_mq_attention_shared_prefix)
    returns:     (sum q_len, num_heads, head_dim) in q's dtype
    """
    _lib.require_gpu(q, k_cache, v_cache, block_table, cu_q, ctx_lens)
    if q.dim() != 3 or k_cache.dim() != 3 or v_cache.shape != k_cache.shape:
        raise ValueError(f"expected q (T, Hq, D) and caches (S, KVH, D); got {tuple(q.shape)}, "
                         f"{tuple(k_cache.shape)}")
    T, Hq, D = q.shape
    S, KVH, Dk = k_cache.shape
    if Dk != D or Hq != KVH * kv_groups:
        raise ValueError(f"q has {Hq} heads of {D}, cache {KVH} heads of {Dk}, kv_groups {kv_groups}")
    if q.dtype not in _DTYPES or k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
        raise ValueError(f"q/k/v dtypes {q.dtype}/{k_cache.dtype}/{v_cache.dtype}: "
                         "the HIP kernels take bf16, fp16 or fp32, all the same")
    if k_cache.stride() != v_cache.stride() or k_cache.stride(2) != 1:
        raise ValueError("k_cache and v_cache need the same strides with head_dim contiguous")
    scale = scale or D ** -0.5
    if q.stride(2) != 1:
        q = q.contiguous()
    cu_q = _i32(cu_q)
    ctx_lens = _i32(ctx_lens)
    block_table = _i32(block_table)
    B = ctx_lens.numel()
    if cu_q.numel() != B + 1:
        raise ValueError(f"cu_q has {cu_q.numel()} entries for {B} sequences")
    if max_q_len is None:
        max_q_len = int((cu_q[1:] - cu_q[:-1]).max().item()) if B else 0
    if max_ctx is None:
        max_ctx = block_table.shape[1] * block_size
    out = torch.empty_like(q) if out is None else out
    if out.shape != q.shape or out.dtype != q.dtype or out.stride(2) != 1:
        raise ValueError("out must have q's shape and dtype with head_dim contiguous")
    L = _lib.calls()
    sp = int(shared_prefix_tokens)
    if balanced and (sp or partition_tokens):
        raise ValueError("balanced excludes shared_prefix_tokens and partition_tokens")
    if sp:
        P = partition_tokens or L.dsp_paged_mq_shared_prefix_partition_tokens(
            B, Hq, KVH, D, int(max_q_len), int(max_ctx), sp)
    elif balanced:
        P = _lib.DSP_SPLIT_BALANCED
    else:
        P = int(partition_tokens)   # 0: the library picks the partition
    stream = _lib.stream_of(q)
    need = _mq_ws_bytes(B, Hq, KVH, D, int(max_q_len), int(max_ctx), P)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = _workspace(need, q.device, stream)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    head = (q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(), S,
            k_cache.stride(0), k_cache.stride(1), block_table.data_ptr(), block_table.stride(0),
            block_size, cu_q.data_ptr(), ctx_lens.data_ptr(), B, Hq, KVH, D, float(scale),
            int(max_q_len), int(max_ctx))
    tail = (_lib.ptr(workspace), ws_bytes, out.data_ptr(), out.stride(0), out.stride(1),
            _lib.dtype_code(q.dtype), _lib.ptr(err), stream)
    if sp:
        _lib.check(L.dsp_paged_mq_attention_shared_prefix(*head, sp, int(P), *tail),
                   "dsp_paged_mq_attention_shared_prefix")
    else:
        _lib.check(L.dsp_paged_mq_attention(*head, int(P), *tail), "dsp_paged_mq_attention")
    return out
