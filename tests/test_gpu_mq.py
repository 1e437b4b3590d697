"""GPU parity of multi-query paged attention (J4) against the float64 oracle.

Verify (q_len 5, config 4's Qwen3-1.7B shape with a shared prefix), chunked prefill
(q_len 23 over 40 context tokens, as tests/test_prefill_attention.py:72-82), fresh
prefill (q_len == ctx), decode rows mixed into the same batch, several GQA groups and
head dims.  Tolerance: cosine >= 0.9999, max-abs <= 2e-2 (bf16 / fp16 outputs).
"""

import numpy as np
import pytest
import torch

from oracle import ref_cpu
from tests._util import assert_attention_close, f64, gen, randn, random_block_tables

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run(q_lens, ctx_lens, Hq, KVH, D, seed, dtype=torch.bfloat16, tables=None, NB=None,
         bs=16, P=0):
    from dispec_amd.engine.hip_attn import paged_mq_attention
    G = Hq // KVH
    if tables is None:
        NB = sum(-(-n // bs) for n in ctx_lens) + 7
        tables = random_block_tables(NB, ctx_lens, bs, seed)
    kc = randn((NB * bs, KVH, D), seed + 1, dtype)
    vc = randn((NB * bs, KVH, D), seed + 2, dtype)
    T = sum(q_lens)
    q = randn((T, Hq, D), seed + 3, dtype)
    width = max(len(t) for t in tables)
    bt = torch.zeros((len(tables), width), dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t)
    cu = torch.tensor([0] + list(np.cumsum(q_lens)), dtype=torch.int32)
    out = paged_mq_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), cu.to(DEV),
                             torch.tensor(ctx_lens, dtype=torch.int32).to(DEV), G, block_size=bs,
                             max_q_len=max(q_lens), partition_tokens=P)
    slot_lists = [ref_cpu.context_slots(t, n, bs) for t, n in zip(tables, ctx_lens)]
    ref = ref_cpu.mq_attention(f64(q), f64(kc), f64(vc), slot_lists, q_lens, G)
    return f64(out), ref


def test_verify_five_queries_shared_prefix():
    """Config-4 shape: Hq 16, KVH 8, D 128; 8 sequences share 128 prefix blocks plus a
    private copy of the partial block, with suffixes of 64..512 tokens, then a 5-query
    causal verify."""
    bs, prefix, nseq = 16, 2050, 8
    suffix = torch.randint(64, 513, (nseq,), generator=gen(40)).tolist()
    ctx = [prefix + s + 5 for s in suffix]
    shared = list(range(128))
    tables, nxt = [], 128
    for n in ctx:
        own = -(-n // bs) - 128
        tables.append(shared + list(range(nxt, nxt + own)))
        nxt += own
    out, ref = _run([5] * nseq, ctx, 16, 8, 128, 41, tables=tables, NB=nxt)
    assert_attention_close(out, ref, "verify")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_chunked_fresh_and_decode_rows_in_one_batch(dtype):
    q_lens = [23, 6, 1, 16, 1]
    ctx = [40, 6, 11, 33, 1]
    out, ref = _run(q_lens, ctx, 4, 2, 64, 50, dtype)
    assert_attention_close(out, ref, f"mixed batch {dtype}")


@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("Hq,KVH", [(16, 8), (12, 2)])
@pytest.mark.parametrize("q_lens", [[1, 1, 1], [3, 1, 2]], ids=["one-query", "three-query"])
def test_merge_of_short_query_blocks(q_lens, Hq, KVH, D):
    """Short query blocks over several key partitions: the merge's grid covers only the
    packed rows below max_q_len * G (2, 6 or 18 here, of 16-row tiles), and every row of
    every sequence still matches the oracle."""
    out, ref = _run(q_lens, [700, 1300, 260], Hq, KVH, D, 70 + D + Hq + len(q_lens), P=128)
    assert_attention_close(out, ref, f"q_lens={q_lens} D={D} Hq={Hq} KVH={KVH}")


@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("Hq,KVH", [(4, 4), (16, 8), (32, 8), (14, 2), (12, 2)])
def test_groups_and_head_dims(D, Hq, KVH):
    out, ref = _run([5, 9, 1], [300, 17, 64], Hq, KVH, D, 60 + D + Hq)
    assert_attention_close(out, ref, f"D={D} Hq={Hq} KVH={KVH}")


def test_long_prefill_many_tiles():
    out, ref = _run([300, 129], [700, 129], 32, 8, 128, 70)
    assert_attention_close(out, ref, "long prefill")


def test_bad_lengths_are_reported_and_zeroed():
    from dispec_amd.engine.hip_attn import paged_mq_attention
    kc = randn((64, 2, 64), 1).to(DEV)
    q = randn((4, 4, 64), 2).to(DEV)
    bt = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32, device=DEV)
    cu = torch.tensor([0, 3, 4], dtype=torch.int32, device=DEV)
    ctx = torch.tensor([2, 5], dtype=torch.int32, device=DEV)   # seq 0: q_len 3 > ctx 2
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = paged_mq_attention(q, kc, kc, bt, cu, ctx, 2, max_q_len=3, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 1
    assert torch.count_nonzero(out[:3]) == 0 and torch.count_nonzero(out[3]) > 0


@pytest.mark.parametrize("P", [128, 256, 640, 4096])
def test_split_k_partitions_agree(P):
    """Key partitions merged by the LSE kernel give the same result as one pass."""
    from dispec_amd.engine.hip_attn import paged_mq_attention
    q_lens, ctx = [5, 5, 40, 1], [2400, 700, 1200, 3000]
    bs, Hq, KVH, D = 16, 16, 8, 128
    NB = sum(-(-n // bs) for n in ctx) + 3
    tables = random_block_tables(NB, ctx, bs, 90)
    kc, vc = randn((NB * bs, KVH, D), 91), randn((NB * bs, KVH, D), 92)
    q = randn((sum(q_lens), Hq, D), 93)
    bt = torch.zeros((len(ctx), max(len(t) for t in tables)), dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t)
    cu = torch.tensor([0] + list(np.cumsum(q_lens)), dtype=torch.int32)
    out = paged_mq_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), cu.to(DEV),
                             torch.tensor(ctx, dtype=torch.int32).to(DEV), Hq // KVH,
                             block_size=bs, max_q_len=max(q_lens), partition_tokens=P)
    slot_lists = [ref_cpu.context_slots(t, n, bs) for t, n in zip(tables, ctx)]
    ref = ref_cpu.mq_attention(f64(q), f64(kc), f64(vc), slot_lists, q_lens, Hq // KVH)
    assert_attention_close(f64(out), ref, f"P={P}")


@pytest.mark.parametrize("q_lens", [[5, 5], [200, 200]], ids=["16-row", "128-row"])
def test_out_of_range_block_id_is_counted_and_never_read(q_lens):
    """A block id past the pool is never dereferenced and is counted; the other sequence
    of the batch (on the 16-row tiles and on the 128-row prefill tile) is unaffected."""
    from dispec_amd.engine.hip_attn import paged_mq_attention
    bs, Hq, KVH, D, NB = 16, 16, 8, 128, 40
    ctx = [300, 300]
    tables = random_block_tables(NB, ctx, bs, 95)
    kc, vc = randn((NB * bs, KVH, D), 96), randn((NB * bs, KVH, D), 97)
    q = randn((sum(q_lens), Hq, D), 98)
    bt = torch.zeros((2, max(len(t) for t in tables)), dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t)
    bt[1, 3] = 1 << 24                          # sequence 1: one block id past the pool
    cu = torch.tensor([0] + list(np.cumsum(q_lens)), dtype=torch.int32)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = paged_mq_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), cu.to(DEV),
                             torch.tensor(ctx, dtype=torch.int32).to(DEV), Hq // KVH,
                             block_size=bs, max_q_len=max(q_lens), err=err)
    torch.cuda.synchronize()
    assert int(err.item()) >= 1
    assert torch.isfinite(out).all()
    ref = ref_cpu.mq_attention(f64(q[:q_lens[0]]), f64(kc), f64(vc),
                               [ref_cpu.context_slots(tables[0], ctx[0], bs)], q_lens[:1],
                               Hq // KVH)
    assert_attention_close(f64(out[:q_lens[0]]), ref, f"good sequence, q_len {q_lens[0]}")
