"""Seeded random shapes through every attention entry point, against the float64 oracle.

The fixed-shape tests aim at known edges; this sweep draws (deterministically, from one
seed per case) batch sizes, ragged and empty contexts, head dims, GQA groups, block sizes,
dtypes and split choices inside the documented limits, so that combinations nobody wrote
down are checked too: block-table decode (automatic split -- unsplit or balanced -- fixed
partitions, the balanced split asked for explicitly), multi-query blocks (verify rows on
16-row tiles or the balanced split, prefill chunks on the 128-row tile, explicit
partitions), shared-prefix batches, the generic kernel's shapes (fp32 caches, head dims 8,
16 and 256, GQA groups above 8) and the byte movers (append, block copy and fan-out,
export / import).  Oracle: ref_cpu.decode_attention / ref_cpu.mq_attention (the
reference's gather + repeat_kv + softmax and its per-sequence SDPA with
causal_lower_right) and the ref_cpu byte moves.  Tolerance: cosine >= 0.9999 and max-abs
<= 2e-2 for bf16 / fp16 attention outputs; fp32 outputs max-abs <= 1e-5 and cosine >=
0.999999; the byte movers bit-exact.
"""

import numpy as np
import pytest
import torch

from oracle import ref_cpu
from tests._util import (assert_attention_close, bits, cosine, f64, gen, randn,
                         random_block_tables)

pytestmark = pytest.mark.gpu
DEV = "cuda"
BALANCED = -1  # DSP_SPLIT_BALANCED


def _pool(lens, KVH, D, bs, seed, dtype, spare=4):
    NB = sum(-(-n // bs) for n in lens) + spare
    tables = random_block_tables(NB, lens, bs, seed)
    kc = randn((NB * bs, KVH, D), seed + 1, dtype)
    vc = randn((NB * bs, KVH, D), seed + 2, dtype)
    return NB, tables, kc, vc


def _table(tables, width):
    bt = torch.zeros((len(tables), max(width, 1)), dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    return bt


@pytest.mark.parametrize("case", range(48))
def test_random_decode(hip, case):
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks
    r = np.random.default_rng(1000 + case)
    D = int(r.choice([32, 64, 128]))
    KVH = int(r.choice([1, 2, 4, 8]))
    G = int(r.integers(1, 9))
    bs = int(r.choice([16, 32, 64]))
    dtype = [torch.bfloat16, torch.float16][int(r.integers(0, 2))]
    B = int(r.integers(1, 41))
    long_ctx = bool(r.integers(0, 2))
    lens = r.integers(0, 3000 if long_ctx else 600, size=B).tolist()
    max_ctx = int(max(max(lens), 1) + r.integers(0, 200))
    split = int(r.choice([0, 0, BALANCED, 64 * int(r.integers(1, 17))]))
    _, tables, kc, vc = _pool(lens, KVH, D, bs, 2000 + case, dtype)
    q = randn((B, KVH * G, D), 2100 + case, dtype)
    bt = _table(tables, -(-max_ctx // bs))
    out = paged_decode_attention_blocks(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV),
                                        torch.tensor(lens, dtype=torch.int32).to(DEV), G,
                                        block_size=bs, max_ctx=max_ctx, partition_tokens=split)
    slots = [ref_cpu.context_slots(t, n, bs) for t, n in zip(tables, lens)]
    ref = ref_cpu.decode_attention(f64(q), f64(kc), f64(vc), slots, lens, G)
    assert_attention_close(f64(out), ref, f"case {case}: D={D} KVH={KVH} G={G} bs={bs} "
                                          f"B={B} max_ctx={max_ctx} split={split} {dtype}")


@pytest.mark.parametrize("case", range(48))
def test_random_multi_query(hip, case):
    from dispec_amd.engine.hip_attn import paged_mq_attention
    r = np.random.default_rng(3000 + case)
    D = int(r.choice([64, 128])) if case % 3 else 32
    KVH = int(r.choice([1, 2, 4, 8]))
    G = int(r.integers(1, 9))
    bs = int(r.choice([16, 32, 64]))
    dtype = [torch.bfloat16, torch.float16][int(r.integers(0, 2))]
    kind = case % 3      # 0: verify rows, 1: prefill chunks, 2: mixed
    B = int(r.integers(1, (13, 5, 9)[kind]))
    if kind == 0:
        q_lens = r.integers(1, 9, size=B).tolist()
    elif kind == 1:
        q_lens = r.integers(64, 300, size=B).tolist()
    else:
        q_lens = [int(x) for x in r.choice([1, 5, 37, 150], size=B)]
    ctx = [int(ql + r.integers(0, 900)) for ql in q_lens]
    max_q = max(q_lens)
    max_ctx = max(ctx)
    balanced = kind == 0 and max_q * G <= 16 and D in (32, 64, 128) and bool(r.integers(0, 2))
    P = 0 if balanced else int(r.choice([0, 0, 128 * int(r.integers(1, 9))]))
    if P and -(-max_ctx // P) > 64:
        P = 0
    _, tables, kc, vc = _pool(ctx, KVH, D, bs, 4000 + case, dtype)
    q = randn((sum(q_lens), KVH * G, D), 4100 + case, dtype)
    bt = _table(tables, -(-max_ctx // bs))
    cu = torch.tensor([0] + list(np.cumsum(q_lens)), dtype=torch.int32)
    out = paged_mq_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), cu.to(DEV),
                             torch.tensor(ctx, dtype=torch.int32).to(DEV), G, block_size=bs,
                             max_q_len=max_q, max_ctx=max_ctx, partition_tokens=P,
                             balanced=balanced)
    slots = [ref_cpu.context_slots(t, n, bs) for t, n in zip(tables, ctx)]
    ref = ref_cpu.mq_attention(f64(q), f64(kc), f64(vc), slots, q_lens, G)
    assert_attention_close(f64(out), ref, f"case {case}: D={D} KVH={KVH} G={G} bs={bs} "
                                          f"q_lens={q_lens} P={P} balanced={balanced} {dtype}")


@pytest.mark.parametrize("case", range(24))
def test_random_shared_prefix(hip, case):
    """Sequences whose tables start with the same blocks, the shared part attended once."""
    from dispec_amd.engine.hip_attn import paged_mq_attention
    r = np.random.default_rng(5000 + case)
    D = int(r.choice([64, 128]))
    KVH = int(r.choice([1, 2, 4, 8]))
    G = int(r.integers(1, 9))
    bs = int(r.choice([16, 32, 64]))
    dtype = [torch.bfloat16, torch.float16][int(r.integers(0, 2))]
    B = int(r.integers(2, 17))
    prefix = 128 * int(r.integers(1, 9))
    shared_blocks = -(-prefix // bs) + int(r.integers(0, 3))
    q_lens = [int(x) for x in r.choice([1, 3, 5, 40], size=B)]
    suffix = [int(ql + r.integers(0, 300)) for ql in q_lens]
    ctx = [shared_blocks * bs + s for s in suffix]
    own = [-(-c // bs) - shared_blocks for c in ctx]
    NB = shared_blocks + sum(own) + 3
    perm = torch.randperm(NB, generator=gen(6000 + case)).tolist()
    tables, at = [], shared_blocks
    for n in own:
        tables.append(perm[:shared_blocks] + perm[at:at + n])
        at += n
    kc = randn((NB * bs, KVH, D), 6100 + case, dtype)
    vc = randn((NB * bs, KVH, D), 6200 + case, dtype)
    q = randn((sum(q_lens), KVH * G, D), 6300 + case, dtype)
    max_ctx = max(ctx)
    bt = _table(tables, -(-max_ctx // bs))
    cu = torch.tensor([0] + list(np.cumsum(q_lens)), dtype=torch.int32)
    out = paged_mq_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), cu.to(DEV),
                             torch.tensor(ctx, dtype=torch.int32).to(DEV), G, block_size=bs,
                             max_q_len=max(q_lens), max_ctx=max_ctx,
                             shared_prefix_tokens=prefix)
    slots = [ref_cpu.context_slots(t, n, bs) for t, n in zip(tables, ctx)]
    ref = ref_cpu.mq_attention(f64(q), f64(kc), f64(vc), slots, q_lens, G)
    assert_attention_close(f64(out), ref, f"case {case}: D={D} KVH={KVH} G={G} bs={bs} "
                                          f"B={B} prefix={prefix} q_lens={q_lens} {dtype}")


@pytest.mark.parametrize("case", range(16))
def test_random_generic_shapes(hip, case):
    """fp32 caches, head dims 8 / 16 / 256 and GQA groups above 8: the generic kernel
    (decode and multi-query alike)."""
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks, paged_mq_attention
    r = np.random.default_rng(7000 + case)
    dtype = [torch.float32, torch.bfloat16, torch.float16][case % 3]
    D = int(r.choice([8, 16, 64, 256] if dtype == torch.float32 else [8, 256]))
    KVH = int(r.choice([1, 2, 4]))
    G = int(r.choice([1, 3, 12, 16])) if case % 2 else int(r.integers(1, 9))
    bs = int(r.choice([16, 32]))
    B = int(r.integers(1, 7))
    decode = bool(case % 2)
    q_lens = [1] * B if decode else r.integers(1, 40, size=B).tolist()
    ctx = [int(ql + r.integers(0 if decode else 0, 700)) for ql in q_lens]
    if decode:
        ctx[0] = 0
    max_ctx = max(max(ctx), 1)
    P = int(r.choice([0, 128, 256]))
    _, tables, kc, vc = _pool(ctx, KVH, D, bs, 7100 + case, dtype)
    q = randn((sum(q_lens), KVH * G, D), 7200 + case, dtype)
    bt = _table(tables, -(-max_ctx // bs)).to(DEV)
    lens = torch.tensor(ctx, dtype=torch.int32).to(DEV)
    if decode:
        out = paged_decode_attention_blocks(q.to(DEV), kc.to(DEV), vc.to(DEV), bt, lens, G,
                                            block_size=bs, max_ctx=max_ctx,
                                            partition_tokens=P)
    else:
        cu = torch.tensor([0] + list(np.cumsum(q_lens)), dtype=torch.int32).to(DEV)
        out = paged_mq_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), bt, cu, lens, G,
                                 block_size=bs, max_q_len=max(q_lens), max_ctx=max_ctx,
                                 partition_tokens=P)
    slots = [ref_cpu.context_slots(t, n, bs) for t, n in zip(tables, ctx)]
    ref = (ref_cpu.decode_attention(f64(q), f64(kc), f64(vc), slots, ctx, G) if decode else
           ref_cpu.mq_attention(f64(q), f64(kc), f64(vc), slots, q_lens, G))
    what = f"case {case}: {dtype} D={D} KVH={KVH} G={G} bs={bs} q_lens={q_lens} P={P}"
    got = f64(out)
    if dtype == torch.float32:
        err = float(np.abs(got - ref).max()) if got.size else 0.0
        assert err <= 1e-5 and cosine(got, ref) >= 0.999999, f"{what}: max-abs {err:.3g}"
    else:
        assert_attention_close(got, ref, what)


@pytest.mark.parametrize("case", range(16))
def test_random_byte_movers(hip, case):
    """Append into random slots, block copies (random pairs, then one block into many),
    export of random sequences and import into others: bit-exact."""
    from dispec_amd.kv.paged_cache import PagedKVCache
    r = np.random.default_rng(8000 + case)
    dtype = [torch.bfloat16, torch.float16, torch.float32][case % 3]
    L = int(r.integers(1, 5))
    bs = int(r.choice([16, 32, 64]))
    H = int(r.choice([1, 2, 3, 8]))
    D = int(r.choice([4, 8, 40, 64, 128]))
    NB = int(r.integers(24, 80))
    c = PagedKVCache(L, NB, bs, H, D, dtype=dtype, device=DEV)
    c.key.copy_(randn(c.key.shape, 8100 + case, dtype))
    c.value.copy_(randn(c.value.shape, 8200 + case, dtype))
    kp, vp = bits(c.key), bits(c.value)
    # append
    T = int(r.integers(1, 200))
    slots = torch.randperm(c.num_slots, generator=gen(8300 + case))[:T]
    k, v = randn((T, H, D), 8400 + case, dtype), randn((T, H, D), 8500 + case, dtype)
    layer = int(r.integers(0, L))
    c.write(layer, slots.to(DEV), k.to(DEV), v.to(DEV))
    ref_cpu.append(kp[layer], slots.numpy(), bits(k))
    ref_cpu.append(vp[layer], slots.numpy(), bits(v))
    # block copies: random distinct pairs, then one source into several blocks
    ids = torch.randperm(NB, generator=gen(8600 + case)).tolist()
    n = int(r.integers(1, NB // 4))
    pairs = list(zip(ids[:n], ids[n:2 * n]))
    c.copy_blocks(pairs)
    ref_cpu.copy_blocks(kp, kp, pairs, bs)
    ref_cpu.copy_blocks(vp, vp, pairs, bs)
    fan = [(ids[2 * n], d) for d in ids[2 * n + 1:2 * n + 1 + int(r.integers(2, 12))]]
    c.copy_blocks(fan)
    ref_cpu.copy_blocks(kp, kp, fan, bs)
    ref_cpu.copy_blocks(vp, vp, fan, bs)
    assert np.array_equal(bits(c.key), kp) and np.array_equal(bits(c.value), vp)
    # export two sequences, import the first into the second's blocks
    lens = [int(r.integers(1, 4 * bs)), int(r.integers(1, 4 * bs))]
    tables = random_block_tables(NB, lens, bs, 8700 + case)
    kbuf, vbuf, cu = c.export_batch(list(zip(tables, lens)))
    for b, (t, m) in enumerate(zip(tables, lens)):
        rows = slice(L * cu[b], L * cu[b + 1])
        assert np.array_equal(bits(kbuf)[rows].reshape(L, m, H, D),
                              ref_cpu.export_contiguous(kp, t, m, bs))
    m = min(lens)
    k0 = kbuf[:L * lens[0]].view(L, lens[0], H, D)[:, :m].contiguous()
    v0 = vbuf[:L * lens[0]].view(L, lens[0], H, D)[:, :m].contiguous()
    c.import_contiguous(tables[1], k0, v0)
    ref_cpu.import_contiguous(kp, tables[1], bits(k0), bs)
    ref_cpu.import_contiguous(vp, tables[1], bits(v0), bs)
    assert np.array_equal(bits(c.key), kp) and np.array_equal(bits(c.value), vp)
    c.check_errors()
