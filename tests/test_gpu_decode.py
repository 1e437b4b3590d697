"""GPU parity of paged decode attention (J3) against the float64 oracle.

Tolerance (bf16/fp16 outputs): cosine >= 0.9999 and max-abs <= 2e-2 against the
float64 restatement of the reference's gather + repeat_kv + softmax (oracle
ref_cpu.decode_attention).  The shapes include the reference's own kernel tests
(tests/test_triton_attn.py:9-60), config 1 (Qwen2.5-0.5B shape), every GQA group 1..8,
head dims 16..128, split-K across many partitions, and the edge cases ctx = 0 / 1.
"""

import numpy as np
import pytest
import torch

from oracle import ref_cpu
from tests._util import assert_attention_close, f64, gen, randn, random_block_tables

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _slot_table(tables, lens, bs, width):
    st = torch.zeros((len(lens), width), dtype=torch.int32)
    for i, (ids, n) in enumerate(zip(tables, lens)):
        if n:
            st[i, :n] = torch.from_numpy(ref_cpu.context_slots(ids, n, bs)).to(torch.int32)
    return st


def test_reference_single_sequence_shape(hip):
    """tests/test_triton_attn.py:9-31: H=14, KVH=2, D=64, fp16, ctx=130 random slots."""
    from dispec_amd.engine.hip_attn import paged_decode_attention
    H, KVH, D, S, ctx = 14, 2, 64, 2048, 130
    q = randn((H, D), 1, torch.float16)
    kc, vc = randn((S, KVH, D), 2, torch.float16), randn((S, KVH, D), 3, torch.float16)
    slots = torch.randperm(S, generator=gen(4))[:ctx]
    out = paged_decode_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), slots.to(DEV), H // KVH)
    ref = ref_cpu.decode_attention(f64(q)[None], f64(kc), f64(vc), [slots.numpy()], [ctx], 7)[0]
    assert out.dtype == torch.float16 and out.shape == (H, D)
    assert_attention_close(f64(out), ref, "single-seq fp16")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_reference_batched_shape(hip, dtype):
    """tests/test_triton_attn.py:34-60: B=5, H=12, KVH=2, D=128, per-token slot table."""
    from dispec_amd.engine.hip_attn import batched_paged_decode_attention
    B, H, KVH, D, S = 5, 12, 2, 128, 4096
    q = randn((B, H, D), 5, dtype)
    kc, vc = randn((S, KVH, D), 6, dtype), randn((S, KVH, D), 7, dtype)
    lens = [17, 64, 130, 200, 33]
    st = torch.zeros((B, max(lens)), dtype=torch.int32)
    for i, c in enumerate(lens):
        st[i, :c] = torch.randperm(S, generator=gen(100 + i))[:c].to(torch.int32)
    out = batched_paged_decode_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), st.to(DEV),
                                         torch.tensor(lens, dtype=torch.int32).to(DEV), H // KVH)
    ref = ref_cpu.decode_attention(f64(q), f64(kc), f64(vc), st.numpy(), lens, H // KVH)
    assert_attention_close(f64(out), ref, f"batched {dtype}")


def test_config1_append_then_decode(hip):
    """Config 1: Qwen2.5-0.5B shape, pool of 256 blocks, lens {37,128,255,511}; append one
    token per sequence via slot mapping, then decode over ctx = len + 1."""
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks
    from dispec_amd.kv.paged_cache import PagedKVCache
    Hq, KVH, D, bs, NB = 14, 2, 64, 16, 256
    lens = [37, 128, 255, 511]
    c = PagedKVCache(1, NB, bs, KVH, D, device=DEV)
    c.key.copy_(randn(c.key.shape, 1001))
    c.value.copy_(randn(c.value.shape, 1002))
    perm = torch.randperm(NB, generator=gen(1003)).tolist()
    tables, at = [], 0
    for n in lens:                       # consecutive chunks of one permutation
        need = -(-(n + 1) // bs)
        tables.append(perm[at:at + need])
        at += need
    new_k, new_v = randn((4, KVH, D), 1004), randn((4, KVH, D), 1005)
    wslots = torch.tensor([ref_cpu.slots_for_positions(t, [n], bs)[0] for t, n in zip(tables, lens)])
    kp, vp = c.key[0].cpu().float().numpy().copy(), c.value[0].cpu().float().numpy().copy()
    c.write(0, wslots.to(DEV), new_k.to(DEV), new_v.to(DEV))
    ref_cpu.append(kp, wslots.numpy(), new_k.float().numpy())
    ref_cpu.append(vp, wslots.numpy(), new_v.float().numpy())
    ctx = [n + 1 for n in lens]
    q = randn((4, Hq, D), 1006)
    bt = c.block_table(tables)
    out = paged_decode_attention_blocks(q.to(DEV), c.key[0], c.value[0], bt,
                                        torch.tensor(ctx, dtype=torch.int32).to(DEV), Hq // KVH,
                                        block_size=bs, scale=1 / 8)
    st = _slot_table(tables, ctx, bs, max(ctx))
    ref = ref_cpu.decode_attention(f64(q), kp, vp, st.numpy(), ctx, Hq // KVH, 1 / 8)
    assert_attention_close(f64(out), ref, "config 1")
    c.check_errors()


@pytest.mark.parametrize("D", [16, 32, 64, 128])
@pytest.mark.parametrize("G", [1, 2, 3, 4, 5, 6, 7, 8])
def test_all_groups_and_head_dims(hip, D, G):
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks
    KVH, bs, B = 2, 16, 3
    Hq = KVH * G
    lens = [1, 70, 300]
    NB = sum(-(-n // bs) for n in lens) + 5
    tables = random_block_tables(NB, lens, bs, 7 * D + G)
    kc = randn((NB * bs, KVH, D), 11 * D + G)
    vc = randn((NB * bs, KVH, D), 13 * D + G)
    q = randn((B, Hq, D), 17 * D + G)
    bt = torch.zeros((B, max(len(t) for t in tables)), dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t)
    out = paged_decode_attention_blocks(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV),
                                        torch.tensor(lens, dtype=torch.int32).to(DEV), G)
    st = _slot_table(tables, lens, bs, max(lens))
    ref = ref_cpu.decode_attention(f64(q), f64(kc), f64(vc), st.numpy(), lens, G)
    assert_attention_close(f64(out), ref, f"D={D} G={G}")


@pytest.mark.parametrize("B,max_ctx", [(256, 512),    # one round, unsplit: the largest
                                       (257, 512),    # one pair past 2 per CU: balanced
                                       (6, 513)])     # one key past 512: balanced
def test_automatic_split_boundaries(hip, B, max_ctx):
    """The automatic split of a block-table decode runs a small launch (max_ctx <= 512, at
    most two (sequence, KV head) pairs per CU) unsplit in one launch and everything else on
    the balanced split: both sides of each boundary agree with the oracle, with contexts
    of 0 and of max_ctx among them."""
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks
    KVH, G, D, bs = 2, 7, 64, 16
    lens = torch.randint(1, max_ctx + 1, (B,), generator=gen(900 + B)).tolist()
    lens[0], lens[-1] = 0, max_ctx
    NB = sum(-(-n // bs) for n in lens) + 5
    tables = random_block_tables(NB, lens, bs, 901 + B)
    kc, vc = randn((NB * bs, KVH, D), 902 + B), randn((NB * bs, KVH, D), 903 + B)
    q = randn((B, KVH * G, D), 904 + B)
    width = -(-max_ctx // bs)
    bt = torch.zeros((B, width), dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    out = paged_decode_attention_blocks(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV),
                                        torch.tensor(lens, dtype=torch.int32).to(DEV), G,
                                        max_ctx=max_ctx)
    st = _slot_table(tables, lens, bs, max_ctx)
    ref = ref_cpu.decode_attention(f64(q), f64(kc), f64(vc), st.numpy(), lens, G)
    assert_attention_close(f64(out), ref, f"B={B} max_ctx={max_ctx}")
    assert not out[0].any()


@pytest.mark.parametrize("P", [64, 128, 512, 1024])
def test_split_k_partitions_agree(hip, P):
    """A 3000-token context split into P-token partitions and merged by the LSE combine."""
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks
    Hq, KVH, D, bs = 32, 8, 128, 16
    lens = [3000, 5, 2049]
    NB = sum(-(-n // bs) for n in lens) + 3
    tables = random_block_tables(NB, lens, bs, 200)
    kc, vc = randn((NB * bs, KVH, D), 201), randn((NB * bs, KVH, D), 202)
    q = randn((3, Hq, D), 203)
    bt = torch.zeros((3, max(len(t) for t in tables)), dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t)
    out = paged_decode_attention_blocks(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV),
                                        torch.tensor(lens, dtype=torch.int32).to(DEV), 4,
                                        partition_tokens=P)
    st = _slot_table(tables, lens, bs, max(lens))
    ref = ref_cpu.decode_attention(f64(q), f64(kc), f64(vc), st.numpy(), lens, 4)
    assert_attention_close(f64(out), ref, f"P={P}")


@pytest.mark.parametrize("D,P,ctx", [(16, 128, 33000), (32, 64, 8300), (64, 64, 4200),
                                     (128, 64, 2200)])
def test_merge_of_more_partitions_than_one_round(hip, D, P, ctx):
    """The fixed-partition merge folds 16 partitions per lane and 64 / (D/4) lane groups
    side by side per round: these contexts need more than one round (259, 130, 66 and 35
    partitions), beside a sequence that needs none."""
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks
    Hq, KVH, bs = 4, 2, 16
    lens = [ctx, 40]
    NB = sum(-(-n // bs) for n in lens) + 2
    tables = random_block_tables(NB, lens, bs, 300 + D)
    kc, vc = randn((NB * bs, KVH, D), 301 + D), randn((NB * bs, KVH, D), 302 + D)
    q = randn((2, Hq, D), 303 + D)
    bt = torch.zeros((2, max(len(t) for t in tables)), dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t)
    out = paged_decode_attention_blocks(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV),
                                        torch.tensor(lens, dtype=torch.int32).to(DEV),
                                        Hq // KVH, partition_tokens=P)
    st = _slot_table(tables, lens, bs, max(lens))
    ref = ref_cpu.decode_attention(f64(q), f64(kc), f64(vc), st.numpy(), lens, Hq // KVH)
    assert_attention_close(f64(out), ref, f"D={D} P={P}")


def test_context_zero_gives_zeros_and_bad_ctx_is_reported(hip):
    from dispec_amd import _lib
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks
    KVH, G, D, bs = 2, 2, 64, 16
    kc, vc = randn((64, KVH, D), 300).to(DEV), randn((64, KVH, D), 301).to(DEV)
    q = randn((2, KVH * G, D), 302).to(DEV)
    bt = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32).to(DEV)
    out = paged_decode_attention_blocks(q, kc, vc, bt, torch.tensor([0, 1], dtype=torch.int32).to(DEV), G)
    assert torch.count_nonzero(out[0]) == 0
    # ctx = 1 attends to exactly one key: the output is that key's value row
    expect = vc[32].repeat_interleave(G, dim=0)
    assert torch.equal(out[1], expect)
    # a context longer than the table is clamped and counted, never read past the table
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    o2 = torch.empty_like(q)
    L = _lib.lib()
    ctx = torch.tensor([40, 5], dtype=torch.int32, device=DEV)
    _lib.check(L.dsp_paged_decode(q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(),
                                  vc.data_ptr(), 64, kc.stride(0), kc.stride(1), bt.data_ptr(),
                                  bt.stride(0), bs, None, 0, ctx.data_ptr(), 2, KVH * G, KVH, D,
                                  D ** -0.5, 32, 64, None, 0, o2.data_ptr(), o2.stride(0),
                                  o2.stride(1), _lib.DSP_BF16, err.data_ptr(),
                                  _lib.stream_of(q)), "decode")
    torch.cuda.synchronize()
    assert int(err.item()) == 1


def test_invalid_arguments_raise(hip):
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks
    kc = randn((64, 2, 64), 1).to(DEV)
    q = randn((1, 4, 64), 2).to(DEV)
    bt = torch.zeros((1, 4), dtype=torch.int32, device=DEV)
    ctx = torch.ones(1, dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError):
        paged_decode_attention_blocks(q, kc, kc, bt, ctx, 3)          # 4 != 2 * 3
    with pytest.raises(ValueError):                                    # mixed dtypes
        paged_decode_attention_blocks(q.float(), kc, kc, bt, ctx, 2)
    with pytest.raises(ValueError):
        paged_decode_attention_blocks(q, kc, kc, bt, ctx, 2, block_size=12)
    big = randn((64, 2, 512), 3).to(DEV)                               # head_dim 512
    with pytest.raises(ValueError, match="no compiled kernel"):
        paged_decode_attention_blocks(randn((1, 4, 512), 4).to(DEV), big, big, bt, ctx, 2)
