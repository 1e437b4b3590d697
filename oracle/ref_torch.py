"""The reference's own torch path for the KV data path, restated on the CPU.

TEST INFRASTRUCTURE ONLY: used by tests/ to pin the numpy oracle against the torch
library routines the reference calls, and by bench.py's CPU-baseline leg, which times
this path on the host cores ("the reference CPU torch path").  Nothing in dispec_amd
imports it.

Every function is the torch op sequence of the cited reference lines, on CPU tensors.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch.nn.attention.bias import causal_lower_right


def context_slots(block_ids, num_tokens: int, block_size: int) -> torch.Tensor:
    """paged_cache.py:75-84."""
    bt = torch.tensor(block_ids, dtype=torch.long)
    pos = torch.arange(num_tokens)
    return bt[pos // block_size] * block_size + pos % block_size


def append(key_layer: torch.Tensor, value_layer: torch.Tensor, slots, k, v) -> None:
    """PagedKVCache.write: two index_copy_ calls (paged_cache.py:67-68)."""
    key_layer.index_copy_(0, slots, k)
    value_layer.index_copy_(0, slots, v)


def gather(key_layer, value_layer, slots):
    """PagedKVCache.gather (paged_cache.py:70-72)."""
    return key_layer[slots], value_layer[slots]


def export_contiguous(key, value, block_ids, seq_len: int, block_size: int):
    """paged_cache.py:87-90."""
    slots = context_slots(block_ids, seq_len, block_size)
    return key[:, slots].contiguous(), value[:, slots].contiguous()


def import_contiguous(key, value, block_ids, k, v, block_size: int) -> None:
    """paged_cache.py:92-96."""
    slots = context_slots(block_ids, k.shape[1], block_size)
    key[:, slots] = k.to(key.dtype)
    value[:, slots] = v.to(value.dtype)


def copy_blocks(key, value, pairs, block_size: int) -> None:
    """pool[:, dst] = pool[:, src] for each block pair (the copy fork/evict imply)."""
    for s, d in pairs:
        key[:, d * block_size:(d + 1) * block_size] = key[:, s * block_size:(s + 1) * block_size]
        value[:, d * block_size:(d + 1) * block_size] = value[:, s * block_size:(s + 1) * block_size]


def decode_repeat_kv_sdpa(q, k_cache, v_cache, slot_lists, kv_groups: int, scale=None):
    """Decode as the graph decoder does it: gather + repeat_interleave + SDPA
    (cuda_graph.py:72-76), one sequence at a time.  q (B, Hq, D) -> (B, Hq, D)."""
    out = torch.empty_like(q)
    for b, slots in enumerate(slot_lists):
        ki = k_cache[slots].repeat_interleave(kv_groups, dim=1)
        vi = v_cache[slots].repeat_interleave(kv_groups, dim=1)
        oh = F.scaled_dot_product_attention(q[b][:, None], ki.transpose(0, 1), vi.transpose(0, 1),
                                            scale=scale)
        out[b] = oh[:, 0]
    return out


def native_attention(q, k_cache, v_cache, slot_lists, q_lens, scale=None):
    """ModelRunner._attention's native branch (model_runner.py:160-185): per sequence,
    gather then SDPA with causal_lower_right(q_len, ctx) and enable_gqa.
    q (sum q_lens, Hq, D) packed by sequence."""
    out = torch.empty_like(q)
    off = 0
    for slots, ql in zip(slot_lists, q_lens):
        ki, vi = k_cache[slots], v_cache[slots]
        oh = F.scaled_dot_product_attention(
            q[off:off + ql].transpose(0, 1)[None], ki.transpose(0, 1)[None],
            vi.transpose(0, 1)[None], attn_mask=causal_lower_right(ql, len(slots)),
            enable_gqa=True, scale=scale)
        out[off:off + ql] = oh[0].transpose(0, 1)
        off += ql
    return out


def layer_map(x, weight, bias):
    """LayerMap.apply, dense form (transfer.py:108): x @ W + b in the map dtype."""
    return x @ weight + bias


def _rotate_half(x):
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat((-x2, x1), dim=-1)


def _apply_rope(x, cos, sin):
    return x * cos.unsqueeze(1) + _rotate_half(x) * sin.unsqueeze(1)


@torch.inference_mode()
def native_forward(model, token_ids, positions, write_slots, seq_meta, key, value,
                   block_size: int):
    """ModelRunner.forward with attn_backend="native" (model_runner.py:127-220), on the
    CPU: per layer, project, q/k-norm (Qwen3), RoPE, index_copy_ the new K/V into the
    pool (`key`/`value`: [L, S, KVH, D]), then per sequence SDPA with
    causal_lower_right over the gathered context.  seq_meta: (block_ids, q_len, ctx_len)
    tuples.  Returns the normalized hidden states (T, hidden)."""
    cfg = model.config
    core = model.model
    H, KVH = cfg.num_attention_heads, cfg.num_key_value_heads
    D = getattr(cfg, "head_dim", None) or cfg.hidden_size // H
    dtype = next(p.dtype for p in model.parameters() if p.is_floating_point())
    cos, sin = core.rotary_emb(torch.zeros(1, 1, dtype=dtype), positions[None, :])
    cos, sin = cos[0].to(dtype), sin[0].to(dtype)
    x = core.embed_tokens(token_ids)
    T = x.shape[0]
    for li, layer in enumerate(core.layers):
        attn = layer.self_attn
        h = layer.input_layernorm(x)
        q = attn.q_proj(h).view(T, H, D)
        k = attn.k_proj(h).view(T, KVH, D)
        v = attn.v_proj(h).view(T, KVH, D)
        if hasattr(attn, "q_norm"):
            q, k = attn.q_norm(q), attn.k_norm(k)
        q, k = _apply_rope(q, cos, sin), _apply_rope(k, cos, sin)
        append(key[li], value[li], write_slots, k, v)
        slot_lists = [context_slots(ids, ctx, block_size) for ids, _, ctx in seq_meta]
        o = native_attention(q, key[li], value[li], slot_lists, [ql for _, ql, _ in seq_meta])
        x = x + attn.o_proj(o.reshape(T, H * D))
        x = x + layer.mlp(layer.post_attention_layernorm(x))
    return core.norm(x)


# --------------------------------------------- TCP transport (dispec/transport/tcp.py)


def tcp_send_pickle(sock, tokens, k, v, meta) -> None:
    """The reference's TcpTransport.send (tcp.py:61-65, framing :19-21): torch.save of
    the payload with its tensors moved to the CPU, one `!Q`-framed message."""
    import io
    import struct
    buf = io.BytesIO()
    torch.save({"tokens": tokens, "k": k.cpu(), "v": v.cpu(), "meta": meta}, buf)
    data = buf.getvalue()
    sock.sendall(struct.pack("!Q", len(data)))
    sock.sendall(data)


def tcp_recv_pickle(sock, device):
    """The reference's TcpTransport.recv (tcp.py:67-70, framing :24-36): read the frame
    into a bytearray in 1 MiB pieces, torch.load it, move K and V to `device`.  Only ever
    fed what tcp_send_pickle wrote in the same process (weights_only=True suffices)."""
    import io
    import struct

    def recv_n(n):
        buf = bytearray()
        while len(buf) < n:
            chunk = sock.recv(min(n - len(buf), 1 << 20))
            if not chunk:
                raise ConnectionError("peer closed during recv")
            buf.extend(chunk)
        return bytes(buf)

    (n,) = struct.unpack("!Q", recv_n(8))
    obj = torch.load(io.BytesIO(recv_n(n)), weights_only=True)
    return obj["tokens"], obj["k"].to(device), obj["v"].to(device), obj.get("meta", {})
