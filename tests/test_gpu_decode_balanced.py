"""GPU parity of the balanced split-K decode (block tables, automatic split) against the
float64 oracle (ref_cpu.decode_attention, the reference's gather + repeat_kv + softmax).

Tolerance: cosine >= 0.9999 and max-abs <= 2e-2 (bf16/fp16 outputs).  The balanced split
cuts the launch's (sequence, KV head, 16-key unit) list into equal shares, one per wave, so
the cases aim at its boundaries: ragged batches where one wave's share spans several
sequences, contexts shorter than a share, empty contexts, a single long sequence split over
many waves, block sizes 16..64 with contexts that end mid-block, every head dim and GQA
group, fp16, bad lengths and block ids, the largest batch it serves and the first it does
not, and a cache too large for 32-bit offsets.
"""

import numpy as np
import pytest
import torch

from oracle import ref_cpu
from tests._util import assert_attention_close, f64, randn, random_block_tables

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bt(tables, width=None):
    width = width or max(1, max(len(t) for t in tables))
    bt = torch.zeros((len(tables), width), dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    return bt


def _slot_table(tables, lens, bs):
    st = np.zeros((len(lens), max(1, max(lens))), dtype=np.int64)
    for i, (ids, n) in enumerate(zip(tables, lens)):
        if n:
            st[i, :n] = ref_cpu.context_slots(ids, n, bs)
    return st


def _run(lens, KVH, G, D, bs, seed, dtype=torch.bfloat16, extra_blocks=3, max_ctx=None,
         partition_tokens=None):
    """The balanced split by default (DSP_SPLIT_BALANCED: the automatic split runs small
    launches unsplit instead)."""
    from dispec_amd import _lib
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks
    if partition_tokens is None:
        partition_tokens = _lib.DSP_SPLIT_BALANCED
    B = len(lens)
    NB = sum(-(-n // bs) for n in lens) + extra_blocks
    tables = random_block_tables(NB, lens, bs, seed)
    kc = randn((NB * bs, KVH, D), seed + 1, dtype)
    vc = randn((NB * bs, KVH, D), seed + 2, dtype)
    q = randn((B, KVH * G, D), seed + 3, dtype)
    bt = _bt(tables, None if max_ctx is None else -(-max_ctx // bs))
    out = paged_decode_attention_blocks(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV),
                                        torch.tensor(lens, dtype=torch.int32).to(DEV), G,
                                        block_size=bs, max_ctx=max_ctx,
                                        partition_tokens=partition_tokens)
    ref = ref_cpu.decode_attention(f64(q), f64(kc), f64(vc), _slot_table(tables, lens, bs),
                                   lens, G)
    return out, ref


def test_ragged_batch_config2_shape(hip):
    """Config-2 head layout (12 q heads, 2 KV heads, D 128), 64 ragged contexts."""
    lens = torch.randint(1, 1500, (64,), generator=torch.Generator().manual_seed(7)).tolist()
    out, ref = _run(lens, 2, 6, 128, 16, 1000)
    assert_attention_close(f64(out), ref, "config-2 shape")


def test_shares_span_many_short_sequences(hip):
    """Contexts much shorter than one wave's share: pieces of several sequences per wave."""
    lens = [1, 2, 15, 16, 17, 31, 33, 5, 0, 64, 3, 100] * 8
    out, ref = _run(lens, 4, 4, 64, 16, 1100)
    assert_attention_close(f64(out), ref, "short contexts")


def test_single_long_sequence_split_over_many_waves(hip):
    out, ref = _run([20000], 8, 4, 128, 16, 1200)
    assert_attention_close(f64(out), ref, "one 20k sequence")


@pytest.mark.parametrize("bs", [16, 32, 64])
def test_block_sizes_and_mid_block_ends(hip, bs):
    lens = [bs * 3 + 7, 1, 2 * bs - 1, 1000 + bs // 2, 47]
    out, ref = _run(lens, 2, 3, 128, bs, 1300 + bs)
    assert_attention_close(f64(out), ref, f"block_size {bs}")


@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("G", [1, 2, 3, 4, 5, 6, 7, 8])
def test_all_groups_and_head_dims(hip, D, G):
    lens = [300, 17, 0, 1024, 555]
    out, ref = _run(lens, 2, G, D, 16, 1400 + 10 * D + G)
    assert_attention_close(f64(out), ref, f"D={D} G={G}")


@pytest.mark.parametrize("KVH,G", [(1, 8), (3, 2), (5, 3)])
def test_odd_kv_heads(hip, KVH, G):
    """Odd KV-head counts (MQA, KVH 3 and 5): segments of every head of a sequence."""
    lens = [900, 33, 0, 2000, 16]
    out, ref = _run(lens, KVH, G, 128, 16, 1450 + KVH)
    assert_attention_close(f64(out), ref, f"KVH={KVH} G={G}")


def test_strided_heads(hip):
    """Heads not adjacent in memory (a head stride larger than head_dim, slot stride larger
    than KVH * head_dim)."""
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks
    KVH, G, D, bs = 4, 2, 64, 16
    lens = [100, 300]
    NB = sum(-(-n // bs) for n in lens) + 2
    tables = random_block_tables(NB, lens, bs, 1460)
    big_k = randn((NB * bs, KVH, 2 * D), 1461)
    big_v = randn((NB * bs, KVH, 2 * D), 1462)
    kc, vc = big_k[:, :, :D], big_v[:, :, :D]            # head stride 2*D, slot stride 2*KVH*D
    q = randn((2, KVH * G, D), 1463)
    out = paged_decode_attention_blocks(q.to(DEV), big_k.to(DEV)[:, :, :D],
                                        big_v.to(DEV)[:, :, :D], _bt(tables).to(DEV),
                                        torch.tensor(lens, dtype=torch.int32).to(DEV), G)
    ref = ref_cpu.decode_attention(f64(q), f64(kc), f64(vc), _slot_table(tables, lens, bs),
                                   lens, G)
    assert_attention_close(f64(out), ref, "strided heads")


def test_fp16(hip):
    lens = [700, 33, 2048, 1]
    out, ref = _run(lens, 4, 2, 128, 16, 1500, dtype=torch.float16)
    assert out.dtype == torch.float16
    assert_attention_close(f64(out), ref, "fp16")


def test_loose_max_ctx_bound(hip):
    """max_ctx far above the real contexts (a graph-captured bucket): the split is computed
    from ctx_lens on the device, so the result is unchanged."""
    lens = [40, 900, 3]
    out, ref = _run(lens, 2, 4, 128, 16, 1600, extra_blocks=600, max_ctx=8192)
    assert_attention_close(f64(out), ref, "loose max_ctx")


def test_balanced_matches_fixed_partitions(hip):
    lens = [4096, 1, 3333, 700, 2500, 16]
    bal, ref = _run(lens, 8, 4, 128, 16, 1700)
    fixed, _ = _run(lens, 8, 4, 128, 16, 1700, partition_tokens=512)
    assert_attention_close(f64(bal), ref, "balanced")
    assert_attention_close(f64(fixed), ref, "fixed 512")
    assert_attention_close(f64(bal), f64(fixed), "balanced vs fixed")


@pytest.mark.parametrize("KVH,G,D", [(8, 4, 128), (2, 6, 128), (1, 7, 64), (4, 2, 32)])
@pytest.mark.parametrize("P", [64, 192, 512])
def test_fixed_partitions_on_head_groups(hip, KVH, G, D, P):
    """Explicit partitions on block tables: one worker of the balanced kernel per
    (sequence, group of KV heads, partition).  Contexts of 0 and 1 tokens, exact multiples
    of P, one key past a multiple, one partition short of one, and several partitions."""
    lens = [0, 1, P, P + 1, P - 16, 5 * P + 7, 3 * P, 33]
    out, ref = _run(lens, KVH, G, D, 16, 2100 + P + D, partition_tokens=P)
    assert_attention_close(f64(out), ref, f"KVH={KVH} G={G} D={D} P={P}")
    assert not out[0].any()                      # ctx 0 writes zeros


@pytest.mark.parametrize("B", [512, 513])
def test_largest_batch_and_fallback(hip, B):
    """512 sequences is the largest batch the balanced split serves; 513 falls back to
    fixed partitions.  Both agree with the oracle."""
    lens = torch.randint(0, 200, (B,), generator=torch.Generator().manual_seed(B)).tolist()
    out, ref = _run(lens, 2, 2, 64, 16, 1800 + B, partition_tokens=0)
    assert_attention_close(f64(out), ref, f"B={B}")


def _raw_decode(q, kc, vc, bt, ctx, KVH, G, bs, max_ctx, err, P=0):
    from dispec_amd import _lib
    L = _lib.lib()
    B, Hq, D = q.shape
    need = L.dsp_paged_decode_workspace_bytes(B, Hq, KVH, D, max_ctx, P)
    ws = torch.empty(need // 4 + 1, dtype=torch.float32, device=DEV)
    out = torch.full_like(q, float("nan"))
    _lib.check(L.dsp_paged_decode(q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(),
                                  vc.data_ptr(), kc.shape[0], kc.stride(0), kc.stride(1),
                                  bt.data_ptr(), bt.stride(0), bs, None, 0, ctx.data_ptr(), B,
                                  Hq, KVH, D, D ** -0.5, max_ctx, P, ws.data_ptr(),
                                  ws.numel() * 4, out.data_ptr(), out.stride(0), out.stride(1),
                                  _lib.DSP_BF16, err.data_ptr(), _lib.stream_of(q)), "decode")
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("P", [0, 64, -1])   # automatic, fixed, DSP_SPLIT_BALANCED
def test_bad_lengths_are_clamped_and_counted(hip, P):
    KVH, G, D, bs = 2, 2, 64, 16
    kc, vc = randn((64, KVH, D), 1900).to(DEV), randn((64, KVH, D), 1901).to(DEV)
    q = randn((3, KVH * G, D), 1902).to(DEV)
    bt = torch.tensor([[0, 1], [2, 3], [0, 3]], dtype=torch.int32).to(DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    ctx = torch.tensor([40, -3, 20], dtype=torch.int32, device=DEV)
    out = _raw_decode(q, kc, vc, bt, ctx, KVH, G, bs, 32, err, P)
    assert int(err.item()) == 2
    assert torch.count_nonzero(out[1]) == 0          # negative length: empty context
    tables = [[0, 1], [2, 3], [0, 3]]
    ref = ref_cpu.decode_attention(f64(q), f64(kc), f64(vc), _slot_table(tables, [32, 0, 20], bs),
                                   [32, 0, 20], G)
    assert_attention_close(f64(out), ref, "clamped")


@pytest.mark.parametrize("P", [0, 64, -1])   # automatic, fixed, DSP_SPLIT_BALANCED
def test_out_of_range_block_ids_are_counted_not_read(hip, P):
    KVH, G, D, bs = 2, 2, 64, 16
    kc, vc = randn((64, KVH, D), 2000).to(DEV), randn((64, KVH, D), 2001).to(DEV)
    q = randn((2, KVH * G, D), 2002).to(DEV)
    bt = torch.tensor([[0, 1], [2, 1 << 20]], dtype=torch.int32).to(DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    ctx = torch.tensor([20, 20], dtype=torch.int32, device=DEV)
    out = _raw_decode(q, kc, vc, bt, ctx, KVH, G, bs, 32, err, P)
    assert int(err.item()) >= 1
    assert torch.isfinite(out).all()
    ref = ref_cpu.decode_attention(f64(q[:1]), f64(kc), f64(vc), _slot_table([[0, 1]], [20], bs),
                                   [20], G)
    assert_attention_close(f64(out[:1]), ref, "good sequence beside a bad one")


def test_cache_beyond_32bit_offsets(hip):
    """A layer cache of 2^21 + 64 slots x 8 heads x 128 dims (>= 2^31 elements): the kernel
    variant with 64-bit offsets; the sequence's blocks sit at the top of the cache."""
    KVH, G, D, bs = 8, 4, 128, 16
    S = (1 << 21) + 64
    kc = torch.empty((S, KVH, D), dtype=torch.bfloat16, device=DEV)
    vc = torch.empty((S, KVH, D), dtype=torch.bfloat16, device=DEV)
    top = S // bs - 1
    tables = [[top, top - 7, 5, top - 100]]
    lens = [61]
    small_k = randn((4 * bs, KVH, D), 2100)
    small_v = randn((4 * bs, KVH, D), 2101)
    for i, blk in enumerate(tables[0]):
        kc[blk * bs:(blk + 1) * bs] = small_k[i * bs:(i + 1) * bs].to(DEV)
        vc[blk * bs:(blk + 1) * bs] = small_v[i * bs:(i + 1) * bs].to(DEV)
    q = randn((1, KVH * G, D), 2102)
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks
    out = paged_decode_attention_blocks(q.to(DEV), kc, vc, _bt(tables).to(DEV),
                                        torch.tensor(lens, dtype=torch.int32).to(DEV), G)
    # oracle on the compact copy: block i of the table is rows i*bs.. of small_k / small_v
    ref = ref_cpu.decode_attention(f64(q), f64(small_k), f64(small_v),
                                   _slot_table([[0, 1, 2, 3]], lens, bs), lens, G)
    assert_attention_close(f64(out), ref, "64-bit offsets")
    del kc, vc
    torch.cuda.empty_cache()
