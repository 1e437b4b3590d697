"""GPU parity of long query blocks (chunked and fresh prefill) against the float64 oracle.

dsp_paged_mq_attention sends batches whose longest query block has >= 128 packed rows
(q_len x G) to the 128-row prefill tile when D is 64 or 128 and blocks hold >= 16 tokens;
these cases cover that kernel: fresh prefill (q_len == ctx) and chunked prefill over a
longer context (the reference's chunked path, tests/test_prefill_attention.py:72-82),
ragged batches whose short sequences ride in the same launch, every GQA group the model
configs use, block sizes, explicit key partitions (merged by the LSE kernel), strided q
and out (views of a fused projection), fp16, and bad lengths.  Tolerance: cosine >= 0.9999
and max-abs <= 2e-2, as for every attention output.
"""

import numpy as np
import pytest
import torch

from oracle import ref_cpu
from tests._util import assert_attention_close, f64, randn, random_block_tables

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(q_lens, ctx_lens, Hq, KVH, D, seed, dtype=torch.bfloat16, bs=16):
    NB = sum(-(-n // bs) for n in ctx_lens) + 5
    tables = random_block_tables(NB, ctx_lens, bs, seed)
    kc = randn((NB * bs, KVH, D), seed + 1, dtype)
    vc = randn((NB * bs, KVH, D), seed + 2, dtype)
    q = randn((sum(q_lens), Hq, D), seed + 3, dtype)
    bt = torch.zeros((len(tables), max(len(t) for t in tables)), dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t)
    cu = torch.tensor([0] + list(np.cumsum(q_lens)), dtype=torch.int32)
    return q, kc, vc, bt, cu, tables


def _oracle(q, kc, vc, tables, q_lens, ctx_lens, G, bs):
    slots = [ref_cpu.context_slots(t, n, bs) for t, n in zip(tables, ctx_lens)]
    return ref_cpu.mq_attention(f64(q), f64(kc), f64(vc), slots, q_lens, G)


def _run(q_lens, ctx_lens, Hq, KVH, D, seed, dtype=torch.bfloat16, bs=16, P=0):
    from dispec_amd.engine.hip_attn import paged_mq_attention
    G = Hq // KVH
    q, kc, vc, bt, cu, tables = _inputs(q_lens, ctx_lens, Hq, KVH, D, seed, dtype, bs)
    out = paged_mq_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), cu.to(DEV),
                             torch.tensor(ctx_lens, dtype=torch.int32).to(DEV), G, block_size=bs,
                             max_q_len=max(q_lens), partition_tokens=P)
    return f64(out), _oracle(q, kc, vc, tables, q_lens, ctx_lens, G, bs)


@pytest.mark.parametrize("D", [64, 128])
def test_fresh_prefill_ragged_lengths(hip, D):
    """q_len == ctx; lengths straddle the 128-row tile and the 64-key chunk edges."""
    q_lens = [257, 64, 31, 129, 1]
    out, ref = _run(q_lens, q_lens, 16, 8, D, 300 + D)
    assert_attention_close(out, ref, f"fresh prefill D={D}")


@pytest.mark.parametrize("Hq,KVH", [(16, 16), (16, 8), (32, 8), (14, 2), (12, 2), (28, 4)])
def test_chunked_prefill_groups(hip, Hq, KVH):
    """A 200-token chunk over 650 cached tokens beside a short chunk and a decode row."""
    q_lens, ctx = [200, 37, 1], [650, 90, 300]
    out, ref = _run(q_lens, ctx, Hq, KVH, 128, 310 + Hq + KVH)
    assert_attention_close(out, ref, f"Hq={Hq} KVH={KVH}")


@pytest.mark.parametrize("bs", [16, 32, 64, 128])
def test_block_sizes(hip, bs):
    out, ref = _run([150, 70], [333, 70], 8, 2, 64, 320 + bs, bs=bs)
    assert_attention_close(out, ref, f"block size {bs}")


@pytest.mark.parametrize("P", [128, 256, 640])
def test_key_partitions_merge(hip, P):
    """Explicit split-K partitions: the kernel writes 16-row-tile partials, the LSE kernel
    merges them; rows whose causal range ends before a partition take no part in it."""
    out, ref = _run([300, 129], [1500, 129], 32, 8, 128, 330 + P, P=P)
    assert_attention_close(out, ref, f"P={P}")


def test_auto_partition_single_long_chunk(hip):
    """One sequence, few tiles: the heuristic splits the keys (Qwen2.5-1.5B heads)."""
    from dispec_amd import _lib
    assert _lib.lib().dsp_paged_mq_partition_tokens(1, 12, 2, 128, 256, 3000) < 3000
    out, ref = _run([256], [3000], 12, 2, 128, 340)
    assert_attention_close(out, ref, "auto partitions")


def test_fp16(hip):
    out, ref = _run([180, 40], [400, 41], 16, 4, 128, 350, dtype=torch.float16)
    assert_attention_close(out, ref, "fp16")


def test_strided_q_and_out(hip):
    """q and out as head slices of wider (T, heads, D) buffers (fused QKV projections)."""
    from dispec_amd.engine.hip_attn import paged_mq_attention
    q_lens, ctx, Hq, KVH, D = [140, 9], [260, 30], 8, 2, 128
    q, kc, vc, bt, cu, tables = _inputs(q_lens, ctx, Hq, KVH, D, 360)
    T = sum(q_lens)
    qkv = torch.zeros((T, Hq + 2 * KVH, D), dtype=torch.bfloat16)
    qkv[:, :Hq] = q
    wide = torch.full((T, Hq + 3, D), 7.0, dtype=torch.bfloat16, device=DEV)
    out = paged_mq_attention(qkv.to(DEV)[:, :Hq], kc.to(DEV), vc.to(DEV), bt.to(DEV), cu.to(DEV),
                             torch.tensor(ctx, dtype=torch.int32).to(DEV), Hq // KVH,
                             max_q_len=max(q_lens), out=wide[:, 1:Hq + 1])
    ref = _oracle(q, kc, vc, tables, q_lens, ctx, Hq // KVH, 16)
    assert_attention_close(f64(out), ref, "strided")
    assert bool((wide[:, 0] == 7).all()) and bool((wide[:, Hq + 1:] == 7).all())


def test_bad_lengths_are_reported_and_zeroed(hip):
    from dispec_amd.engine.hip_attn import paged_mq_attention
    q_lens, ctx, Hq, KVH, D = [160, 140, 20], [150, 300, 20], 8, 2, 64
    q, kc, vc, bt, cu, tables = _inputs(q_lens, [300, 300, 20], Hq, KVH, D, 370)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = paged_mq_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), cu.to(DEV),
                             torch.tensor(ctx, dtype=torch.int32).to(DEV), Hq // KVH,
                             max_q_len=max(q_lens), max_ctx=304, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 1            # sequence 0: q_len 160 > ctx 150
    assert torch.count_nonzero(out[:160]) == 0
    ref = _oracle(q[160:], kc, vc, tables[1:], q_lens[1:], ctx[1:], Hq // KVH, 16)
    assert_attention_close(f64(out[160:]), ref, "good sequences beside a bad one")
