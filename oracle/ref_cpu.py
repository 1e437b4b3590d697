"""CPU oracle of DiSpec's KV-cache data path (numpy).  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import this
module, and only as the checker -- never as the thing measured or shipped.  The product
path (dispec_amd) has no CPU code path and never imports it.

Each function restates one step of the reference algorithm and cites the reference
file:line it follows.  bf16 data is carried as uint16 bit patterns (numpy has no bf16);
`bf16_to_f32` widens exactly and `f32_to_bf16` rounds to nearest even, as torch does.

How each function is pinned (tests/test_oracle*.py; tests/test_oracle_mutants.py runs
edited copies of this module's source -- wrong KV head, dropped scale, swapped operand,
wrong softmax axis, short causal mask, wrong block index, reversed append or copy, wrong
RoPE frequency or sign, wrong feature order, dropped bias, GELU or norm weight, k
normalised with q's weight, a bf16 map rounding or RoPE step missed -- through the same
kinds of checks and requires each to fail one):
  slot math ............ known answers of tests/test_block_manager.py:8-27 and a
                         brute-force walk of the block table
  append/gather/export/
  import/copy_blocks ... torch index_copy_ / advanced indexing / index_put (library
                         routines) on the same bytes, round-trip and untouched-row
                         invariants, hand-built known answers
  decode_attention ..... torch SDPA with enable_gqa (library routine), closed forms
                         (equal keys -> mean of V; one dominant key -> that V; ctx=1)
  mq_attention ......... causal_lower_right == right-aligned bool mask (reference
                         tests/test_prefill_attention.py:58-69), q_len=1 == decode,
                         q_len=ctx == ordinary causal attention (torch SDPA is_causal)
  rope ................. textbook inverse-frequency formula checked against the
                         Qwen3 rotary module of transformers; strip(apply(x)) == x
  qk_norm_rope_append .. transformers' Qwen3RMSNorm module, the runner's rotate-half
                         RoPE and index_copy_ run as torch bf16 ops on the CPU (library
                         routines); closed forms (unit weight + zero angle = normalise only)
  layer_map / map ...... known-answer feature order (tests/test_kv_transfer.py:89-100),
                         factored == dense (:103-109), residual formula (:112-126),
                         identity map reproduces its input (:234-252)
"""

from __future__ import annotations

import numpy as np

# --------------------------------------------------------------------- bf16 bit helpers


def bf16_to_f32(u: np.ndarray) -> np.ndarray:
    """Exact widening of bf16 bit patterns (uint16) to float32."""
    return (np.asarray(u, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 to bf16 bit patterns, nearest-even; NaN stays NaN."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 value, returned as float32."""
    return bf16_to_f32(f32_to_bf16(x))


# --------------------------------------------------------------------------- slot math


def slots_for_positions(block_ids, positions, block_size: int) -> np.ndarray:
    """slot = block_ids[p // bs] * bs + p % bs  (paged_cache.py:75-79, block_manager.py:29-31)."""
    bt = np.asarray(block_ids, dtype=np.int64)
    p = np.asarray(positions, dtype=np.int64)
    return bt[p // block_size] * block_size + p % block_size


def context_slots(block_ids, num_tokens: int, block_size: int) -> np.ndarray:
    """Slots of the first num_tokens tokens (paged_cache.py:81-84)."""
    return slots_for_positions(block_ids, np.arange(num_tokens), block_size)


# ------------------------------------------------------------------ byte moves (J1/J2/J5)


def append(pool_layer: np.ndarray, slots, rows: np.ndarray) -> None:
    """pool_layer.index_copy_(0, slots, rows) in place (paged_cache.py:67-68)."""
    slots = np.asarray(slots, dtype=np.int64)
    if slots.size and (slots.min() < 0 or slots.max() >= pool_layer.shape[0]):
        raise IndexError("slot out of range")
    pool_layer[slots] = rows


def gather(pool_layer: np.ndarray, slots) -> np.ndarray:
    """pool_layer[slots] (paged_cache.py:70-72)."""
    return pool_layer[np.asarray(slots, dtype=np.int64)].copy()


def export_contiguous(pool: np.ndarray, block_ids, seq_len: int, block_size: int) -> np.ndarray:
    """pool[:, context_slots(block_ids, seq_len)] as a contiguous copy (paged_cache.py:87-90)."""
    return np.ascontiguousarray(pool[:, context_slots(block_ids, seq_len, block_size)])


def import_contiguous(pool: np.ndarray, block_ids, x: np.ndarray, block_size: int) -> None:
    """pool[:, context_slots(block_ids, T)] = x in place (paged_cache.py:92-96)."""
    pool[:, context_slots(block_ids, x.shape[1], block_size)] = x


def copy_blocks(src_pool: np.ndarray, dst_pool: np.ndarray, pairs, block_size: int) -> None:
    """For every layer: dst[l, d*bs:(d+1)*bs] = src[l, s*bs:(s+1)*bs].

    The reference's fork/evict move no data (block_manager.py:119-126,
    prefix_cache.py:64-70); this is the copy its refcount-shared blocks stand for.
    """
    for s, d in pairs:
        dst_pool[:, d * block_size:(d + 1) * block_size] = \
            src_pool[:, s * block_size:(s + 1) * block_size]


# ----------------------------------------------------------------------- attention (J3/J4)


def decode_attention(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, slot_table,
                     ctx_lens, kv_groups: int, scale: float | None = None) -> np.ndarray:
    """Decode attention in float64, the gather + repeat_kv + softmax form.

    Follows dispec/engine/cuda_graph.py:72-76 and the reference test's brute force
    (tests/test_triton_attn.py:55-59): for sequence b, K = k_cache[slots_b] with KV head
    h // G serving query head h (triton_attn.py:70), o = softmax(scale q.K^T) V.
    q (B, Hq, D) float; caches (S, KVH, D) float; returns float64 (B, Hq, D).
    ctx_len 0 gives zeros (the kernels' documented convention).
    """
    q = np.asarray(q, dtype=np.float64)
    B, Hq, D = q.shape
    scale = scale or D ** -0.5
    out = np.zeros((B, Hq, D))
    for b in range(B):
        n = int(ctx_lens[b])
        if n == 0:
            continue
        slots = np.asarray(slot_table[b][:n], dtype=np.int64)
        k = np.repeat(np.asarray(k_cache[slots], dtype=np.float64), kv_groups, axis=1)  # (n,Hq,D)
        v = np.repeat(np.asarray(v_cache[slots], dtype=np.float64), kv_groups, axis=1)
        # per head: s = q . K^T, o = softmax(s) . V (batched matmuls over the heads)
        s = np.matmul(k.transpose(1, 0, 2), q[b][:, :, None])[:, :, 0] * scale  # (Hq, n)
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=1, keepdims=True)
        out[b] = np.matmul(p[:, None, :], v.transpose(1, 0, 2))[:, 0, :]
    return out


def causal_lower_right_mask(q_len: int, ctx_len: int) -> np.ndarray:
    """Query i sees keys j <= ctx_len - q_len + i (torch causal_lower_right;
    reference tests/test_prefill_attention.py:62-63)."""
    past = ctx_len - q_len
    return np.arange(ctx_len)[None, :] <= np.arange(q_len)[:, None] + past


def mq_attention(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, slot_lists,
                 q_lens, kv_groups: int, scale: float | None = None) -> np.ndarray:
    """Multi-query paged attention in float64 (model_runner.py:160-185).

    q: (sum(q_lens), Hq, D) packed by sequence; slot_lists[b] are the ctx_b context
    slots of sequence b whose last q_lens[b] tokens are its queries.  Each sequence is
    SDPA(q, K, V, causal_lower_right(q_len, ctx), enable_gqa=True).
    """
    q = np.asarray(q, dtype=np.float64)
    T, Hq, D = q.shape
    scale = scale or D ** -0.5
    out = np.zeros((T, Hq, D))
    off = 0
    for slots, ql in zip(slot_lists, q_lens):
        slots = np.asarray(slots, dtype=np.int64)
        n = slots.size
        k = np.repeat(np.asarray(k_cache[slots], dtype=np.float64), kv_groups, axis=1)
        v = np.repeat(np.asarray(v_cache[slots], dtype=np.float64), kv_groups, axis=1)
        # per head: s = Q . K^T (Hq, q_len, n), masked, softmax, o = P . V
        s = np.matmul(q[off:off + ql].transpose(1, 0, 2), k.transpose(1, 2, 0)) * scale
        s = np.where(causal_lower_right_mask(ql, n)[None], s, -np.inf)
        s -= s.max(axis=2, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=2, keepdims=True)
        out[off:off + ql] = np.matmul(p, v.transpose(1, 0, 2)).transpose(1, 0, 2)
        off += ql
    return out


# ------------------------------------------------- attention prologue (model_runner.py)


def rms_norm_bf16(x_bits: np.ndarray, w_bits: np.ndarray, eps: float) -> np.ndarray:
    """Qwen3RMSNorm on bf16 rows (transformers' modeling_qwen3, as q_norm / k_norm at
    model_runner.py:142-144): var = mean(x^2) in fp32, bf16(x * rsqrt(var + eps)), times the
    bf16 weight rounded to bf16.  Returns bf16-representable float32."""
    x = bf16_to_f32(x_bits)
    var = np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32)
    inv = (np.float32(1.0) / np.sqrt(var + np.float32(eps))).astype(np.float32)
    return round_bf16(bf16_to_f32(w_bits) * round_bf16((x * inv).astype(np.float32)))


def rope_bf16(x: np.ndarray, cos_bits: np.ndarray, sin_bits: np.ndarray) -> np.ndarray:
    """The runner's _apply_rope on bf16 tensors (model_runner.py:49-50, 145-146):
    x * cos + rotate_half(x) * sin with cos/sin (T, D) broadcast over heads, each product
    and the sum rounded to bf16.  x: (T, H, D) bf16-representable float32."""
    c, s = bf16_to_f32(cos_bits)[:, None, :], bf16_to_f32(sin_bits)[:, None, :]
    return round_bf16(round_bf16(x * c) + round_bf16(_rotate_half(x) * s))


def qk_norm_rope_append(q_bits, k_bits, v_bits, qw_bits, kw_bits, eps, cos_bits, sin_bits,
                        slots, k_pool_bits, v_pool_bits) -> np.ndarray:
    """ModelRunner._attention between projections and attention (model_runner.py:142-148):
    optional q_norm / k_norm (weights None: none), RoPE on q and k, cache.write(k, v).
    Writes the pools in place (bf16 bits) and returns the rotated q as bf16 bits."""
    q, k = bf16_to_f32(q_bits), bf16_to_f32(k_bits)
    if qw_bits is not None:
        q, k = rms_norm_bf16(q_bits, qw_bits, eps), rms_norm_bf16(k_bits, kw_bits, eps)
    q, k = rope_bf16(q, cos_bits, sin_bits), rope_bf16(k, cos_bits, sin_bits)
    append(k_pool_bits, slots, f32_to_bf16(k))
    append(v_pool_bits, slots, np.asarray(v_bits, dtype=np.uint16))
    return f32_to_bf16(q)


# ------------------------------------------------------------------ RoPE (transfer.py)


def rope_tables(positions, head_dim: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """(cos, sin), (T, head_dim) float32, for default (unscaled) rotary embedding.

    inv_freq_i = theta^(-2i/D), angle = p * inv_freq, halves duplicated -- what the
    model's rotary module returns for rope_type "default" (transfer.py:50-58 reads it).
    """
    inv = 1.0 / (theta ** (np.arange(0, head_dim, 2, dtype=np.int64).astype(np.float32) / head_dim))
    ang = np.asarray(positions, dtype=np.float32)[:, None] * inv[None, :].astype(np.float32)
    emb = np.concatenate([ang, ang], axis=-1)
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


def _rotate_half(x: np.ndarray) -> np.ndarray:
    h = x.shape[-1] // 2
    return np.concatenate([-x[..., h:], x[..., :h]], axis=-1)


def strip_rope(keys: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """(L, T, H, D) rotated keys -> content keys, float32: x cos - rot(x) sin (transfer.py:66-73)."""
    x = np.asarray(keys, dtype=np.float32)
    c, s = cos[None, :, None, :], sin[None, :, None, :]
    return (x * c - _rotate_half(x) * s).astype(np.float32)


def apply_rope(keys: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """(L, T, H, D) content keys -> rotated, float32: x cos + rot(x) sin (transfer.py:76-80)."""
    x = np.asarray(keys, dtype=np.float32)
    c, s = cos[None, :, None, :], sin[None, :, None, :]
    return (x * c + _rotate_half(x) * s).astype(np.float32)


# -------------------------------------------------------------- cross-model map (J5b)


def _gelu(x):
    from math import erf, sqrt
    return 0.5 * x * (1.0 + np.vectorize(erf)(x / sqrt(2.0)))


def layer_map_apply(x: np.ndarray, weight=None, bias=None, factors=None, residual=None,
                    use_residual: bool = True) -> np.ndarray:
    """y = x @ W + b, or (x @ L) @ R + b, plus up(gelu(down(x))) (transfer.py:104-112).

    float64 throughout (the exact value the bf16 kernels round).
    """
    x = np.asarray(x, dtype=np.float64)
    if factors is not None:
        y = (x @ np.asarray(factors[0], np.float64)) @ np.asarray(factors[1], np.float64)
    else:
        y = x @ np.asarray(weight, np.float64)
    y = y + np.asarray(bias, np.float64)
    if use_residual and residual is not None:
        down_w, down_b, up_w = (np.asarray(t, np.float64) for t in residual)
        y = y + _gelu(x @ down_w.T + down_b) @ up_w.T
    return y


def design_rows(source: np.ndarray, source_layers) -> np.ndarray:
    """(T, k*H*D) rows: source[list(layers)].permute(1,0,2,3).reshape(T,-1) (transfer.py:249)."""
    sel = np.asarray(source)[list(source_layers)]          # (k, T, H, D)
    return np.ascontiguousarray(sel.transpose(1, 0, 2, 3)).reshape(sel.shape[1], -1)


def cross_model_map_bf16(k_bits: np.ndarray, v_bits: np.ndarray, key_maps, value_maps,
                         source_rope, target_rope) -> tuple[np.ndarray, np.ndarray]:
    """CrossModelKVMap.map with a bf16 map, rounding where the reference rounds.

    transfer.py:257-283 with self.dtype = bf16: keys are RoPE-stripped in fp32 and stored
    as bf16 (:277-279); each target layer's design row is multiplied by W (bf16 GEMM:
    fp32 accumulate, bf16 result), the bias is added in bf16 (:108), RoPE re-applied in
    fp32 and stored as bf16 (:251-253).  Values skip RoPE (:282).
    maps: list of dicts {source_layers, weight (K, N) float, bias (N,) float} whose
    weight/bias are already bf16-representable.  Inputs/outputs are bf16 bit patterns
    (L, T, H, D).  The GEMM is evaluated in float64 before its bf16 rounding.
    """
    L, T, H, D = k_bits.shape
    content = f32_to_bf16(strip_rope(bf16_to_f32(k_bits), *source_rope))
    vals = np.asarray(v_bits, dtype=np.uint16)

    def run(src_bits, maps, rope):
        src = bf16_to_f32(src_bits)
        out = np.empty((len(maps), T, H, D), dtype=np.uint16)
        for t, m in enumerate(maps):
            x = design_rows(src, m["source_layers"]).astype(np.float64)
            y = round_bf16((x @ np.asarray(m["weight"], np.float64)).astype(np.float32))
            y = round_bf16(y + np.asarray(m["bias"], np.float32))
            y = y.reshape(1, T, H, D)
            if rope is not None:
                y = apply_rope(y, *rope)
            out[t] = f32_to_bf16(y[0])
        return out

    return run(content, key_maps, target_rope), run(vals, value_maps, None)
