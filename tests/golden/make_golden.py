"""Write tests/golden/kv_path_golden.npz: small frozen cases of the KV data path.

Inputs come from numpy's PCG64 generator (stable across numpy versions and machines);
expected outputs are the CPU oracle's (oracle/ref_cpu.py), which restates the
reference's torch ops:
  append          PagedKVCache.write, index_copy_          (dispec/kv/paged_cache.py:61-68)
  copy_blocks     block copy over all layers (the data move behind CoW fork /
                  prefix-cache evict, dispec/kv/block_manager.py:119-126)
  export/import   export_contiguous / import_contiguous     (paged_cache.py:87-96)
  decode          batched paged decode attention            (dispec/engine/triton_attn.py:59-95)
  verify          multi-query attention, causal_lower_right (dispec/engine/model_runner.py:160-185)
  map             CrossModelKVMap.map with a bf16 map       (dispec/kv/transfer.py:243-283)
The RoPE tables of the map case are stored as inputs, so no libm cos/sin enters a check.
The reference ships no vector files, and it is not imported here.

Run from the repository root: python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import ref_cpu  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kv_path_golden.npz")


def bf16_normal(rng, shape, scale=1.0):
    return ref_cpu.f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


def cases(rng) -> dict:
    g = {}
    # append: 1 layer, 48 slots, KVH 2, D 32; 7 unique slots
    pool = bf16_normal(rng, (48, 2, 32))
    slots = rng.permutation(48)[:7].astype(np.int64)
    rows = bf16_normal(rng, (7, 2, 32))
    exp = pool.copy()
    ref_cpu.append(exp, slots, rows)
    g.update(append_pool=pool, append_slots=slots, append_rows=rows, append_expected=exp)

    # copy_blocks: 2 layers, 12 blocks of 4, KVH 2, D 8; chained and overlapping pairs
    bs = 4
    pool = bf16_normal(rng, (2, 12 * bs, 2, 8))
    pairs = np.array([[0, 5], [3, 7], [9, 2], [5, 11]], dtype=np.int64)
    exp = pool.copy()
    ref_cpu.copy_blocks(pool, exp, pairs.tolist(), bs)   # reads the source before the copy
    g.update(copy_pool=pool, copy_pairs=pairs, copy_block_size=np.int64(bs), copy_expected=exp)

    # export / import: 2 layers, 16 blocks of 8, KVH 2, D 16; a 23-token sequence
    bs = 8
    pool = bf16_normal(rng, (2, 16 * bs, 2, 16))
    ids = rng.permutation(16)[:3].astype(np.int64)
    g.update(xfer_pool=pool, xfer_block_ids=ids, xfer_block_size=np.int64(bs),
             xfer_export_expected=ref_cpu.export_contiguous(pool, ids, 23, bs))
    payload = bf16_normal(rng, (2, 23, 2, 16))
    exp = pool.copy()
    ref_cpu.import_contiguous(exp, ids, payload, bs)
    g.update(xfer_payload=payload, xfer_import_expected=exp)

    # decode: B 4, Hq 8, KVH 2 (G 4), D 64, block size 16, 24-block pool; ctx {1, 17, 100, 0}
    bs, nb = 16, 24
    k = bf16_normal(rng, (nb * bs, 2, 64))
    v = bf16_normal(rng, (nb * bs, 2, 64))
    q = bf16_normal(rng, (4, 8, 64))
    ctx = np.array([1, 17, 100, 0], dtype=np.int32)
    perm = rng.permutation(nb)
    bt = np.zeros((4, 7), dtype=np.int32)
    at = 0
    for b, n in enumerate(ctx):
        need = -(-int(n) // bs)
        bt[b, :need] = perm[at:at + need]
        at += need
    st = np.zeros((4, 100), dtype=np.int64)
    for b, n in enumerate(ctx):
        if n:
            st[b, :n] = ref_cpu.context_slots(bt[b], int(n), bs)
    out = ref_cpu.decode_attention(ref_cpu.bf16_to_f32(q), ref_cpu.bf16_to_f32(k),
                                   ref_cpu.bf16_to_f32(v), st, ctx, 4)
    g.update(dec_k=k, dec_v=v, dec_q=q, dec_ctx=ctx, dec_block_table=bt,
             dec_block_size=np.int64(bs), dec_expected=out)

    # verify: 2 sequences, q_len {3, 5}, ctx {20, 40}, Hq 4, KVH 2, D 64, block size 16
    nb = 6
    k = bf16_normal(rng, (nb * bs, 2, 64))
    v = bf16_normal(rng, (nb * bs, 2, 64))
    q_lens, ctxs = [3, 5], [20, 40]
    q = bf16_normal(rng, (sum(q_lens), 4, 64))
    perm = rng.permutation(nb)
    bt = np.array([[perm[0], perm[1], 0], [perm[2], perm[3], perm[4]]], dtype=np.int32)
    slot_lists = [ref_cpu.context_slots(bt[b], ctxs[b], bs) for b in range(2)]
    out = ref_cpu.mq_attention(ref_cpu.bf16_to_f32(q), ref_cpu.bf16_to_f32(k),
                               ref_cpu.bf16_to_f32(v), slot_lists, q_lens, 2)
    g.update(ver_k=k, ver_v=v, ver_q=q, ver_q_lens=np.array(q_lens, np.int32),
             ver_ctx=np.array(ctxs, np.int32), ver_block_table=bt, ver_expected=out)

    # map: 3 source layers -> 2 target layers, H 2, D 32 (kv_dim 64), T 9, k = 2 source
    # layers per target (feature order layer -> head -> dim), bf16 W ~ N(0, 1/128), bias
    L, T, H, D = 3, 9, 2, 32
    kk = bf16_normal(rng, (L, T, H, D))
    vv = bf16_normal(rng, (L, T, H, D))
    layers = np.array([[2, 0], [1, 2]], dtype=np.int64)

    def maps():
        w = [ref_cpu.round_bf16((rng.standard_normal((2 * H * D, H * D)) / np.sqrt(128))
                                .astype(np.float32)) for _ in range(2)]
        b = [ref_cpu.round_bf16(rng.standard_normal(H * D).astype(np.float32)) for _ in range(2)]
        return np.stack(w), np.stack(b)

    wk, bk = maps()
    wv, bv = maps()
    pos = np.arange(T)
    src = ref_cpu.rope_tables(pos, D, 1e6)
    tgt = ref_cpu.rope_tables(pos, D, 5e5)
    mk = [{"source_layers": tuple(layers[t]), "weight": wk[t], "bias": bk[t]} for t in range(2)]
    mv = [{"source_layers": tuple(layers[t]), "weight": wv[t], "bias": bv[t]} for t in range(2)]
    ek, ev = ref_cpu.cross_model_map_bf16(kk, vv, mk, mv, src, tgt)
    g.update(map_k=kk, map_v=vv, map_layers=layers, map_wk=wk, map_bk=bk, map_wv=wv,
             map_bv=bv, map_src_cos=src[0], map_src_sin=src[1], map_tgt_cos=tgt[0],
             map_tgt_sin=tgt[1], map_k_expected=ek, map_v_expected=ev)
    return g


def main() -> None:
    g = cases(np.random.default_rng(20261201))
    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT}: {len(g)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
