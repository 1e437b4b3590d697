"""GPU parity of the generic attention kernels (fp32 caches, head_dim 8 / 256, GQA groups
above 8) against the float64 oracle.

The reference's Triton decode kernel takes any power-of-two HEAD_DIM and reads K/V as fp32
(dispec/engine/triton_attn.py:60-95); its native path attends in the model's dtype
(model_runner.py:160-185).  These shapes reach dsp_paged_decode / dsp_paged_mq_attention
through the same Python wrappers as the tuned ones.

Tolerances: fp32 caches and outputs -- max-abs <= 1e-5 and cosine >= 0.999999 against the
float64 oracle (fp32 accumulation over at most a few thousand keys of N(0, 1) data; a
bf16 rounding anywhere on the path would miss it by ~100x); bf16 / fp16 outputs -- cosine
>= 0.9999 and max-abs <= 2e-2, as for the tuned kernels.
"""

import numpy as np
import pytest
import torch

from oracle import ref_cpu
from tests._util import assert_attention_close, cosine, f64, gen, randn, random_block_tables

pytestmark = pytest.mark.gpu
DEV = "cuda"
F32_MAX_ABS = 1e-5
F32_COS_MIN = 0.999999


def _close(out, ref, dtype, what):
    if dtype == torch.float32:
        err = float(np.abs(out - ref).max()) if out.size else 0.0
        cos = cosine(out, ref)
        assert err <= F32_MAX_ABS and cos >= F32_COS_MIN, f"{what}: max-abs {err:.3g}, cos {cos}"
    else:
        assert_attention_close(out, ref, what)


def _block_tables(lens, bs, seed, NB=None):
    NB = NB or sum(-(-n // bs) for n in lens) + 5
    tables = random_block_tables(NB, lens, bs, seed)
    width = max(max(len(t) for t in tables), 1)
    bt = torch.zeros((len(lens), width), dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    return NB, tables, bt


def _decode(lens, Hq, KVH, D, dtype, seed, bs=16, partition_tokens=0):
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks
    NB, tables, bt = _block_tables(lens, bs, seed)
    kc = randn((NB * bs, KVH, D), seed + 1, dtype)
    vc = randn((NB * bs, KVH, D), seed + 2, dtype)
    q = randn((len(lens), Hq, D), seed + 3, dtype)
    out = paged_decode_attention_blocks(
        q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV),
        torch.tensor(lens, dtype=torch.int32).to(DEV), Hq // KVH, block_size=bs,
        partition_tokens=partition_tokens)
    slots = [ref_cpu.context_slots(t, n, bs) for t, n in zip(tables, lens)]
    ref = ref_cpu.decode_attention(f64(q), f64(kc), f64(vc), slots, lens, Hq // KVH)
    assert out.dtype == dtype and out.shape == q.shape
    return f64(out), ref


@pytest.mark.parametrize("D", [64, 128, 256])
def test_fp32_slot_table_reference_shape(hip, D):
    """tests/test_triton_attn.py:34-60 in fp32: B=5, H=12, KVH=2, per-token slot table."""
    from dispec_amd.engine.hip_attn import batched_paged_decode_attention
    B, H, KVH, S = 5, 12, 2, 4096
    dt = torch.float32
    q = randn((B, H, D), 5, dt)
    kc, vc = randn((S, KVH, D), 6, dt), randn((S, KVH, D), 7, dt)
    lens = [17, 64, 130, 200, 33]
    st = torch.zeros((B, max(lens)), dtype=torch.int32)
    for i, c in enumerate(lens):
        st[i, :c] = torch.randperm(S, generator=gen(100 + i))[:c].to(torch.int32)
    out = batched_paged_decode_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), st.to(DEV),
                                         torch.tensor(lens, dtype=torch.int32).to(DEV), H // KVH)
    ref = ref_cpu.decode_attention(f64(q), f64(kc), f64(vc), st.numpy(), lens, H // KVH)
    assert out.dtype == torch.float32
    _close(f64(out), ref, dt, f"fp32 slot table D={D}")


@pytest.mark.parametrize("dtype,D", [(torch.float32, 8), (torch.float32, 16),
                                     (torch.float32, 64), (torch.float32, 256),
                                     (torch.bfloat16, 8), (torch.bfloat16, 256),
                                     (torch.float16, 8), (torch.float16, 256)])
def test_decode_block_tables_split(hip, dtype, D):
    """Ragged contexts (0, 1, partition boundaries, several partitions) over 64-key
    partitions, so most rows go through the merge kernel."""
    lens = [0, 1, 63, 64, 65, 700, 1500]
    out, ref = _decode(lens, 8, 2, D, dtype, 10 + D, partition_tokens=64)
    _close(out, ref, dtype, f"decode {dtype} D={D}")
    assert not out[0].any()                     # ctx 0 writes zeros


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_automatic_partition(hip, dtype):
    """Automatic split for a long context (head_dim 256: Gemma-style heads)."""
    out, ref = _decode([4000, 100, 2500], 16, 4, 256, dtype, 20)
    _close(out, ref, dtype, f"decode auto {dtype}")


@pytest.mark.parametrize("Hq,KVH", [(16, 1), (32, 2), (48, 4)])
def test_decode_groups_above_eight(hip, Hq, KVH):
    """16 and 12 query heads per KV head: outside the tuned decode kernels' 1..8."""
    out, ref = _decode([300, 17, 1], Hq, KVH, 128, torch.bfloat16, 30 + Hq)
    _close(out, ref, torch.bfloat16, f"G={Hq // KVH}")


def test_decode_bad_block_ids_and_lengths_are_counted(hip):
    """A block id past the pool skips its keys (counted once per wave that met it); a
    context above max_ctx is clamped to it (counted once)."""
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks
    bs, KVH, D, Hq, NB = 16, 2, 256, 4, 16
    kc = randn((NB * bs, KVH, D), 40, torch.float32)
    vc = randn((NB * bs, KVH, D), 41, torch.float32)
    q = randn((2, Hq, D), 42, torch.float32)
    bt = torch.tensor([[0, 1, 999, 3], [4, 5, 6, 7]], dtype=torch.int32)
    lens = torch.tensor([64, 80], dtype=torch.int32)     # sequence 1: 80 > max_ctx 64
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = paged_decode_attention_blocks(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV),
                                        lens.to(DEV), Hq // KVH, block_size=bs, max_ctx=64,
                                        err=err)
    torch.cuda.synchronize()
    ok0 = np.r_[ref_cpu.context_slots([0, 1], 32, bs), ref_cpu.context_slots([3], 16, bs)]
    ref = ref_cpu.decode_attention(f64(q), f64(kc), f64(vc),
                                   [ok0, ref_cpu.context_slots([4, 5, 6, 7], 64, bs)],
                                   [48, 64], Hq // KVH)
    _close(f64(out), ref, torch.float32, "bad ids")
    # one clamped context + every (head, partition) wave of sequence 0 that met block 999
    assert int(err.item()) == 1 + Hq


def _mq(q_lens, ctx, Hq, KVH, D, dtype, seed, bs=16, partition_tokens=0):
    from dispec_amd.engine.hip_attn import paged_mq_attention
    NB, tables, bt = _block_tables(ctx, bs, seed)
    kc = randn((NB * bs, KVH, D), seed + 1, dtype)
    vc = randn((NB * bs, KVH, D), seed + 2, dtype)
    q = randn((sum(q_lens), Hq, D), seed + 3, dtype)
    cu = torch.tensor([0] + list(np.cumsum(q_lens)), dtype=torch.int32)
    out = paged_mq_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), cu.to(DEV),
                             torch.tensor(ctx, dtype=torch.int32).to(DEV), Hq // KVH,
                             block_size=bs, max_q_len=max(q_lens),
                             partition_tokens=partition_tokens)
    slots = [ref_cpu.context_slots(t, n, bs) for t, n in zip(tables, ctx)]
    ref = ref_cpu.mq_attention(f64(q), f64(kc), f64(vc), slots, q_lens, Hq // KVH)
    assert out.dtype == dtype
    return f64(out), ref


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("D", [8, 256])
def test_mq_verify_chunked_and_fresh(hip, dtype, D):
    """Verify rows (5 queries), a chunked-prefill block, a fresh prefill and a decode row
    in one batch, over 128-key partitions (merged)."""
    q_lens = [5, 23, 40, 1]
    ctx = [600, 300, 40, 129]
    out, ref = _mq(q_lens, ctx, 8, 2, D, dtype, 50 + D, partition_tokens=128)
    _close(out, ref, dtype, f"mq {dtype} D={D}")


@pytest.mark.parametrize("D", [64, 128])
def test_mq_fp32_tuned_head_dims(hip, D):
    """fp32 caches at the head dims the tuned kernels serve in bf16 / fp16."""
    out, ref = _mq([5, 9, 1], [300, 17, 64], 16, 8, D, torch.float32, 60 + D)
    _close(out, ref, torch.float32, f"mq fp32 D={D}")


def test_mq_bad_lengths_counted_and_zeroed(hip):
    from dispec_amd.engine.hip_attn import paged_mq_attention
    kc = randn((64, 2, 256), 1, torch.float32).to(DEV)
    q = randn((4, 4, 256), 2, torch.float32).to(DEV)
    bt = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32, device=DEV)
    cu = torch.tensor([0, 3, 4], dtype=torch.int32, device=DEV)
    ctx = torch.tensor([2, 5], dtype=torch.int32, device=DEV)   # seq 0: q_len 3 > ctx 2
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = paged_mq_attention(q, kc, kc, bt, cu, ctx, 2, max_q_len=3, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 1
    assert not out[:3].any().item()
    ref = ref_cpu.mq_attention(f64(q[3:].cpu()), f64(kc.cpu()), f64(kc.cpu()),
                               [ref_cpu.context_slots([2, 3], 5, 16)], [1], 2)
    _close(f64(out[3:]), ref, torch.float32, "good sequence")
