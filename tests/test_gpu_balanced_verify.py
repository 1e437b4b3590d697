"""GPU parity of short multi-query blocks (speculative verify) on the balanced split-K
kernel against the float64 oracle.

With partition_tokens = DSP_SPLIT_BALANCED, dsp_paged_mq_attention runs batches whose
query rows of a KV head fit one 16-row MFMA tile (max_q_len * G <= 16) on the balanced
decode kernel (what ModelRunner picks for verify batches of skewed contexts): every
wave takes an equal share of the (sequence, KV head group, 16-key unit) work, query row
i of a sequence seeing keys j <= ctx - q_len + i (the reference's native path,
dispec/engine/model_runner.py:160-185).  Covers GQA groups 1-7 with q_len * G up to 16,
head dims 32/64/128, KV head groups of 1/2/4/8 heads per workgroup, ragged and empty
query blocks, ctx == q_len, one long context among short ones (many pieces per
sequence), fp16, bad lengths (counted once, rows zeroed) and agreement with explicit key
partitions (the 16-row-tile kernel).  Tolerance: cosine >= 0.9999, max-abs <= 2e-2.
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
    bt = torch.zeros((len(tables), max(max(len(t) for t in tables), 1)), dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    cu = torch.tensor([0] + list(np.cumsum(q_lens)), dtype=torch.int32)
    return q, kc, vc, bt, cu, tables


def _run(q_lens, ctx_lens, Hq, KVH, D, seed, dtype=torch.bfloat16, P=None, bs=16):
    """P None: the balanced split; else that key partition (0: the library's choice)."""
    from dispec_amd.engine.hip_attn import paged_mq_attention
    G = Hq // KVH
    q, kc, vc, bt, cu, tables = _inputs(q_lens, ctx_lens, Hq, KVH, D, seed, dtype, bs)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = paged_mq_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), cu.to(DEV),
                             torch.tensor(ctx_lens, dtype=torch.int32).to(DEV), G,
                             block_size=bs, max_q_len=max(q_lens), partition_tokens=P or 0,
                             balanced=P is None, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    slots = [ref_cpu.context_slots(t, n, bs) for t, n in zip(tables, ctx_lens)]
    ref = ref_cpu.mq_attention(f64(q), f64(kc), f64(vc), slots, q_lens, G)
    return f64(out), ref


def test_config4_verify_of_independent_sequences():
    """Qwen3-1.7B heads (G 2): 32 sequences of 1-4k tokens, a 5-query verify (10 rows)."""
    ctx = torch.randint(1024, 4097, (32,), generator=torch.Generator().manual_seed(700))
    out, ref = _run([5] * 32, ctx.tolist(), 16, 8, 128, 701)
    assert_attention_close(out, ref, "independent verify")


@pytest.mark.parametrize("Hq,KVH,ql", [(16, 8, 5), (32, 8, 4), (14, 2, 2), (12, 2, 2),
                                       (8, 8, 16), (4, 1, 4), (8, 4, 8)])
@pytest.mark.parametrize("D", [64, 128])
def test_groups_rows_and_head_dims(Hq, KVH, ql, D):
    """q_len * G from 4 to 16 rows; KVH 8/4/2/1 put 4/4/2/1 heads in a workgroup."""
    q_lens = [ql, max(ql - 1, 1), ql, 1]
    ctx = [300, 77, 1000, 16]
    out, ref = _run(q_lens, ctx, Hq, KVH, D, 710 + Hq + ql + D)
    assert_attention_close(out, ref, f"Hq={Hq} KVH={KVH} q_len={ql} D={D}")


def test_head_dim_32():
    out, ref = _run([5, 3, 5], [200, 40, 513], 16, 8, 32, 720)
    assert_attention_close(out, ref, "D=32")


def test_ragged_empty_and_fresh_blocks():
    """Empty query blocks between others, a block as long as its context (fresh), one-key
    contexts and a context that ends on a unit boundary."""
    q_lens = [5, 0, 3, 5, 0, 1, 4]
    ctx = [5, 40, 3, 160, 9, 1, 64]
    out, ref = _run(q_lens, ctx, 16, 8, 128, 730)
    assert_attention_close(out, ref, "ragged")


def test_more_sequences_than_one_scan_block():
    """150 sequences (the merge reads each sequence's lengths out of a 64-lane scan block:
    here three blocks), ragged query blocks of 0-5 rows, contexts 5-700, and one long
    context late in the batch so that its pieces are merged from the third block."""
    g = torch.Generator().manual_seed(760)
    q_lens = torch.randint(0, 6, (150,), generator=g).tolist()
    ctx = [max(q, int(c)) for q, c in zip(q_lens, torch.randint(5, 701, (150,), generator=g))]
    ctx[140] = 6000
    q_lens[140] = 5
    out, ref = _run(q_lens, ctx, 16, 8, 128, 761)
    assert_attention_close(out, ref, "150 sequences")


def test_one_long_context_among_short_ones():
    """One 12k context beside 15 of 100-600: the long one is split over many workers and
    its pieces merged; the short ones mostly run whole."""
    ctx = [12288] + torch.randint(100, 601, (15,), generator=torch.Generator().manual_seed(740)).tolist()
    out, ref = _run([5] * 16, ctx, 16, 8, 128, 741)
    assert_attention_close(out, ref, "skewed")


def test_fp16_and_block_sizes():
    out, ref = _run([5, 5, 2], [700, 130, 2048], 16, 8, 128, 750, dtype=torch.float16)
    assert_attention_close(out, ref, "fp16")
    out, ref = _run([5, 5, 2], [700, 130, 2048], 16, 8, 128, 751, bs=64)
    assert_attention_close(out, ref, "bs=64")


@pytest.mark.parametrize("P", [0, 128, 512])
def test_agrees_with_key_partitions(P):
    """The balanced split and key partitions (16-row tiles; 0: the library's choice) both
    match the oracle and each other."""
    q_lens, ctx = [5, 5, 3, 5], [2400, 700, 1200, 3000]
    bal, ref = _run(q_lens, ctx, 16, 8, 128, 760)
    fixed, _ = _run(q_lens, ctx, 16, 8, 128, 760, P=P)
    assert_attention_close(bal, ref, "balanced")
    assert_attention_close(fixed, ref, f"P={P}")
    assert np.abs(bal - fixed).max() <= 2e-2


def test_bad_lengths_are_counted_once_and_zeroed():
    """q_len > ctx and ctx > max_ctx: each such sequence counted once, its rows zeros;
    the others (an empty query block among them) unaffected."""
    from dispec_amd.engine.hip_attn import paged_mq_attention
    q_lens, ctx = [5, 4, 0, 5, 2], [300, 3, 50, 700, 80]   # seq 1: q_len 4 > ctx 3
    Hq, KVH, D, G = 16, 8, 128, 2
    q, kc, vc, bt, cu, tables = _inputs(q_lens, ctx, Hq, KVH, D, 770)
    ctx_dev = torch.tensor(ctx, dtype=torch.int32).to(DEV)
    ctx_dev[3] = 4000                                       # seq 3: beyond max_ctx
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = paged_mq_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), cu.to(DEV),
                             ctx_dev, G, max_q_len=5, max_ctx=bt.shape[1] * 16, err=err,
                             balanced=True)
    torch.cuda.synchronize()
    assert int(err.item()) == 2
    o = f64(out)
    assert not np.any(o[5:9]) and not np.any(o[9:14])
    slots = [ref_cpu.context_slots(t, n, 16) for t, n in zip(tables, ctx)]
    ref = ref_cpu.mq_attention(f64(q), f64(kc), f64(vc), slots, q_lens, G)
    keep = np.r_[0:5, 14:16]
    assert_attention_close(o[keep], ref[keep], "good sequences beside bad ones")


def test_query_block_longer_than_max_q_len_is_counted_and_stays_in_bounds():
    """A caller passing max_q_len below a sequence's real q_len: that sequence is counted
    once, its first max_q_len query rows are zeros and its later rows untouched, the other
    sequences are right, and nothing past the workspace is written."""
    from dispec_amd import _lib
    from dispec_amd.engine.hip_attn import paged_mq_attention
    q_lens, ctx = [5, 8, 3, 5], [300, 500, 100, 2000]          # seq 1: q_len 8 > 5
    Hq, KVH, D, G, maxq = 16, 8, 128, 2, 5
    q, kc, vc, bt, cu, tables = _inputs(q_lens, ctx, Hq, KVH, D, 775)
    need = _lib.lib().dsp_paged_mq_workspace_bytes(len(ctx), Hq, KVH, D, maxq,
                                                    bt.shape[1] * 16, _lib.DSP_SPLIT_BALANCED)
    words = need // 4 + 1
    ws = torch.full((words + 4096,), 12345.0, dtype=torch.float32, device=DEV)
    out = torch.full((sum(q_lens), Hq, D), 7.0, dtype=torch.bfloat16, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    paged_mq_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), cu.to(DEV),
                       torch.tensor(ctx, dtype=torch.int32).to(DEV), G, max_q_len=maxq,
                       max_ctx=bt.shape[1] * 16, err=err, balanced=True, out=out,
                       workspace=ws[:words])
    torch.cuda.synchronize()
    assert int(err.item()) == 1
    assert bool((ws[words:] == 12345.0).all()), "workspace guard overwritten"
    o = f64(out)
    assert not np.any(o[5:10]), "rows of the first max_q_len queries must be zeros"
    assert np.all(o[10:13] == 7.0), "rows past max_q_len must be left untouched"
    slots = [ref_cpu.context_slots(t, n, 16) for t, n in zip(tables, ctx)]
    ref = ref_cpu.mq_attention(f64(q), f64(kc), f64(vc), slots, q_lens, G)
    keep = np.r_[0:5, 13:21]
    assert_attention_close(o[keep], ref[keep], "good sequences beside an over-long block")


def test_rejects_unsupported_shapes(hip):
    """The balanced split needs max_q_len * G <= 16 and excludes a shared prefix."""
    from dispec_amd.engine.hip_attn import paged_mq_attention
    q, kc, vc, bt, cu, _ = _inputs([9, 9], [100, 200], 16, 8, 128, 780)
    args = (q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), cu.to(DEV),
            torch.tensor([100, 200], dtype=torch.int32).to(DEV), 2)
    with pytest.raises(ValueError, match="no compiled kernel"):   # 9 x 2 = 18 rows
        paged_mq_attention(*args, max_q_len=9, balanced=True)
    with pytest.raises(ValueError):
        paged_mq_attention(*args, max_q_len=9, balanced=True, shared_prefix_tokens=128)


def test_workspace_covers_the_balanced_split():
    """The balanced split's workspace holds its pieces: (B * KVH + workers) slots of
    max_q_len * G rows of D + 2 floats."""
    from dispec_amd import _lib
    L = _lib.lib()
    B, Hq, KVH, D, ql, ctx = 32, 16, 8, 128, 5, 4096
    need = L.dsp_paged_mq_workspace_bytes(B, Hq, KVH, D, ql, ctx, _lib.DSP_SPLIT_BALANCED)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    workers = min(B * KVH * ctx // 16 // 4, cus * 4)
    assert need >= (B * KVH + workers) * ql * (Hq // KVH) * (D + 2) * 4
