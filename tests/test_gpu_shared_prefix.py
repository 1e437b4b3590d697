"""GPU parity of shared-prefix (cascade) multi-query attention against the float64 oracle.

dsp_paged_mq_attention_shared_prefix attends the blocks every sequence shares (copy-on-write
forks of one prompt, dispec/kv/block_manager.py:119-126; prefix-cache hits,
dispec/kv/prefix_cache.py:39-50) once for all query rows of the batch and the rest per
sequence; the oracle attends each sequence over its whole context
(ref_cpu.mq_attention, the reference's model_runner.py:160-185), so agreement shows the
split changes nothing.  Covers config 4's verify shape (q_len 5, Hq 16, KVH 8), several GQA
groups and head dims, explicit partitions, ragged and empty query blocks, block sizes, a
sequence that breaks the precondition (counted and zeroed) and argument errors.
Tolerance: cosine >= 0.9999 and max-abs <= 2e-2.
"""

import numpy as np
import pytest
import torch

from oracle import ref_cpu
from tests._util import assert_attention_close, f64, gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _setup(q_lens, suffix, shared_blocks, Hq, KVH, D, seed, bs=16, dtype=torch.bfloat16):
    """Sequences whose tables start with the same `shared_blocks` physical blocks, then
    private blocks for their own suffix tokens (ctx = shared tokens + suffix)."""
    ctx = [shared_blocks * bs + s for s in suffix]
    own = [-(-c // bs) - shared_blocks for c in ctx]
    NB = shared_blocks + sum(own) + 3
    perm = torch.randperm(NB, generator=gen(seed)).tolist()
    shared, at = perm[:shared_blocks], shared_blocks
    tables = []
    for n in own:
        tables.append(shared + perm[at:at + n])
        at += n
    kc = randn((NB * bs, KVH, D), seed + 1, dtype)
    vc = randn((NB * bs, KVH, D), seed + 2, dtype)
    q = randn((sum(q_lens), Hq, D), seed + 3, dtype)
    bt = torch.zeros((len(tables), max(len(t) for t in tables)), dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t)
    cu = torch.tensor([0] + list(np.cumsum(q_lens)), dtype=torch.int32)
    return q, kc, vc, bt, cu, tables, ctx


def _run(q_lens, suffix, shared_blocks, Hq, KVH, D, seed, prefix, P=0, bs=16,
         dtype=torch.bfloat16):
    from dispec_amd.engine.hip_attn import paged_mq_attention
    G = Hq // KVH
    q, kc, vc, bt, cu, tables, ctx = _setup(q_lens, suffix, shared_blocks, Hq, KVH, D, seed,
                                            bs, dtype)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = paged_mq_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), cu.to(DEV),
                             torch.tensor(ctx, dtype=torch.int32).to(DEV), G, block_size=bs,
                             max_q_len=max(q_lens), partition_tokens=P, err=err,
                             shared_prefix_tokens=prefix)
    torch.cuda.synchronize()
    slots = [ref_cpu.context_slots(t, n, bs) for t, n in zip(tables, ctx)]
    ref = ref_cpu.mq_attention(f64(q), f64(kc), f64(vc), slots, q_lens, G)
    return f64(out), ref, int(err.item())


def test_config4_verify_shape(hip):
    """32 forks of a 2050-token prompt (128 shared blocks; the partial block is private),
    suffixes 64..512, a 5-query verify: Qwen3-1.7B heads."""
    suffix = [2 + s + 5 for s in torch.randint(64, 513, (32,), generator=gen(500)).tolist()]
    out, ref, err = _run([5] * 32, suffix, 128, 16, 8, 128, 501, prefix=2048)
    assert err == 0
    assert_attention_close(out, ref, "config 4 shared prefix")


def test_config4_fork_decode_shape(hip):
    """The decode step of the same 32 forks (one query each) through the shared-prefix
    launch, as ModelRunner routes it: the merge covers 2 of each 16-row tile's rows."""
    suffix = [2 + s + 1 for s in torch.randint(64, 513, (32,), generator=gen(502)).tolist()]
    out, ref, err = _run([1] * 32, suffix, 128, 16, 8, 128, 503, prefix=2048)
    assert err == 0
    assert_attention_close(out, ref, "config 4 fork decode")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("Hq,KVH", [(16, 8), (32, 8), (14, 2), (12, 2)])
def test_groups_and_head_dims(hip, D, Hq, KVH):
    out, ref, err = _run([5, 3, 7, 1, 5], [40, 7, 130, 2, 64], 24, Hq, KVH, D, 510 + D + Hq,
                         prefix=384)
    assert err == 0
    assert_attention_close(out, ref, f"D={D} Hq={Hq} KVH={KVH}")


@pytest.mark.parametrize("P", [128, 256, 384])
def test_explicit_partitions(hip, P):
    out, ref, err = _run([4] * 6, [300, 5, 77, 260, 129, 16], 48, 16, 4, 128, 520 + P,
                         prefix=768, P=P)
    assert err == 0
    assert_attention_close(out, ref, f"P={P}")


def test_prefix_shorter_than_the_shared_blocks(hip):
    """Only part of the shared blocks taken as the prefix (a multiple of 128 below them)."""
    out, ref, err = _run([5] * 4, [10, 20, 30, 40], 20, 16, 8, 128, 530, prefix=256)
    assert err == 0
    assert_attention_close(out, ref, "partial prefix")


def test_ragged_and_empty_query_blocks(hip):
    """q_len 0 sequences sit between others (equal cu_q entries) and chunk-sized blocks."""
    out, ref, err = _run([5, 0, 40, 0, 1, 17], [8, 3, 60, 1, 2, 33], 16, 16, 8, 128, 540,
                         prefix=256)
    assert err == 0
    assert_attention_close(out, ref, "ragged")


@pytest.mark.parametrize("bs", [32, 64])
def test_block_sizes(hip, bs):
    out, ref, err = _run([5] * 5, [9, 40, 70, 8, 5], 512 // bs, 16, 8, 128, 550 + bs,
                         prefix=512, bs=bs)
    assert err == 0
    assert_attention_close(out, ref, f"bs={bs}")


def test_fp16(hip):
    out, ref, err = _run([5] * 4, [10, 90, 5, 33], 16, 16, 8, 128, 560, prefix=256,
                         dtype=torch.float16)
    assert err == 0
    assert_attention_close(out, ref, "fp16")


def test_precondition_violation_is_counted_and_zeroed(hip):
    """A sequence whose queries start inside the prefix (ctx - q_len < prefix_tokens)."""
    q_lens, suffix = [5, 40, 5], [20, 30, 9]     # sequence 1: ctx 286 - 40 = 246 < 256
    out, ref, err = _run(q_lens, suffix, 16, 16, 8, 128, 570, prefix=256)
    assert err == 1
    assert not np.any(out[5:45])
    keep = np.r_[0:5, 45:50]
    assert_attention_close(out[keep], ref[keep], "good sequences beside a bad one")


def test_rejects_bad_arguments(hip):
    from dispec_amd.engine.hip_attn import paged_mq_attention
    q, kc, vc, bt, cu, tables, ctx = _setup([5, 5], [10, 20], 16, 16, 8, 128, 580)
    args = (q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), cu.to(DEV),
            torch.tensor(ctx, dtype=torch.int32).to(DEV), 2)
    with pytest.raises(ValueError):        # not a multiple of 128
        paged_mq_attention(*args, max_q_len=5, shared_prefix_tokens=200)
    with pytest.raises(ValueError):        # not a multiple of the partition
        paged_mq_attention(*args, max_q_len=5, shared_prefix_tokens=256, partition_tokens=512)
    with pytest.raises(ValueError):        # the whole context
        paged_mq_attention(*args, max_q_len=5, max_ctx=256, shared_prefix_tokens=256)
    q32, kc32, vc32, bt32, cu32, _, ctx32 = _setup([5, 5], [10, 20], 16, 16, 8, 32, 590)
    with pytest.raises(ValueError):        # head_dim 32: not served by the prefix pass
        paged_mq_attention(q32.to(DEV), kc32.to(DEV), vc32.to(DEV), bt32.to(DEV), cu32.to(DEV),
                           torch.tensor(ctx32, dtype=torch.int32).to(DEV), 2, max_q_len=5,
                           shared_prefix_tokens=256)
