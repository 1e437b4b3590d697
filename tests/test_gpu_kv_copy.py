"""GPU parity of the byte-moving kernels against the numpy oracle: bit-exact.

append (J1), slot gather, whole-sequence export (J5a) / import (J5c), block copy (J2)
and copy-on-write fork, on seeded pools, including ragged and empty sequences, partial
blocks, non-contiguous sources, rows that need narrower vectors, and out-of-range ids.
"""

import numpy as np
import pytest
import torch

from oracle import ref_cpu
from tests._util import bits, gen, randn, random_block_tables

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _cache(L, NB, bs, H, D, dtype=torch.bfloat16, seed=0):
    from dispec_amd.kv.paged_cache import PagedKVCache
    c = PagedKVCache(L, NB, bs, H, D, dtype=dtype, device=DEV)
    c.key.copy_(randn(c.key.shape, seed, dtype))
    c.value.copy_(randn(c.value.shape, seed + 1, dtype))
    return c


@pytest.mark.parametrize("H,D,dtype", [(2, 64, torch.bfloat16), (8, 128, torch.bfloat16),
                                       (2, 4, torch.float32), (3, 5, torch.float16),
                                       (2, 16, torch.float32), (16, 256, torch.bfloat16)])
def test_append_bit_exact(hip, H, D, dtype):
    # (16, 256): 8 KiB rows, more 16-byte vectors than a row's 256 lanes
    c = _cache(3, 40, 16, H, D, dtype, seed=10)
    kref, vref = bits(c.key), bits(c.value)
    T = 37
    slots = torch.randperm(c.num_slots, generator=gen(11))[:T]
    k, v = randn((T, H, D), 12, dtype), randn((T, H, D), 13, dtype)
    c.write(1, slots.to(DEV), k.to(DEV), v.to(DEV))
    ref_cpu.append(kref[1], slots.numpy(), bits(k))
    ref_cpu.append(vref[1], slots.numpy(), bits(v))
    torch.cuda.synchronize()
    assert np.array_equal(bits(c.key), kref) and np.array_equal(bits(c.value), vref)
    c.check_errors()


def test_append_from_strided_qkv_view(hip):
    """k, v as column slices of a fused qkv projection (token stride != row size)."""
    c = _cache(2, 16, 16, 2, 64, seed=20)
    kref, vref = bits(c.key), bits(c.value)
    T, qsz, kvsz = 9, 14 * 64, 2 * 64
    qkv = randn((T, qsz + 2 * kvsz), 21).to(DEV)
    k = qkv[:, qsz:qsz + kvsz].view(T, 2, 64)
    v = qkv[:, qsz + kvsz:].view(T, 2, 64)
    slots = torch.tensor([3, 200, 17, 18, 19, 100, 0, 255, 64])
    c.write(0, slots.to(DEV), k, v)
    ref_cpu.append(kref[0], slots.numpy(), bits(k))
    ref_cpu.append(vref[0], slots.numpy(), bits(v))
    assert np.array_equal(bits(c.key), kref) and np.array_equal(bits(c.value), vref)


@pytest.mark.parametrize("H,D", [(2, 64), (16, 256)])
def test_append_out_of_range_slot_is_skipped_and_reported(hip, H, D):
    c = _cache(1, 4, 16, H, D, seed=30)
    before_k, before_v = bits(c.key), bits(c.value)
    slots = torch.tensor([1, 64, 2, -1])                 # 64 == num_slots: out of range
    k, v = randn((4, H, D), 31), randn((4, H, D), 32)
    c.write(0, slots.to(DEV), k.to(DEV), v.to(DEV))
    expect_k, expect_v = before_k.copy(), before_v.copy()
    expect_k[0, 1], expect_k[0, 2] = bits(k)[0], bits(k)[2]
    expect_v[0, 1], expect_v[0, 2] = bits(v)[0], bits(v)[2]
    assert np.array_equal(bits(c.key), expect_k) and np.array_equal(bits(c.value), expect_v)
    with pytest.raises(IndexError, match="2 out-of-range"):
        c.check_errors()
    c.check_errors()  # counter was reset


@pytest.mark.parametrize("T", [16384, 16385, 20001])
def test_append_around_the_small_launch_bound(hip, T):
    """Up to 16384 rows the append's lane groups take two rows each, above it one: both
    sides of the bound, with out-of-range slots among the rows and an odd row count."""
    c = _cache(1, 1400, 16, 2, 64, seed=50)
    kref, vref = bits(c.key), bits(c.value)
    slots = torch.randperm(c.num_slots, generator=gen(51))[:T]
    bad = torch.tensor([0, T // 2, T - 1])
    slots[bad] = torch.tensor([-5, c.num_slots, c.num_slots + 100])
    k, v = randn((T, 2, 64), 52), randn((T, 2, 64), 53)
    c.write(0, slots.to(DEV), k.to(DEV), v.to(DEV))
    good = np.ones(T, bool)
    good[bad.numpy()] = False
    ref_cpu.append(kref[0], slots.numpy()[good], bits(k)[good])
    ref_cpu.append(vref[0], slots.numpy()[good], bits(v)[good])
    assert np.array_equal(bits(c.key), kref) and np.array_equal(bits(c.value), vref)
    with pytest.raises(IndexError, match="3 out-of-range"):
        c.check_errors()


def test_gather_slots_bit_exact(hip):
    c = _cache(2, 32, 16, 8, 128, seed=40)
    slots = torch.randperm(c.num_slots, generator=gen(41))[:77]
    k, v = c.gather(1, slots.to(DEV))
    assert np.array_equal(bits(k), ref_cpu.gather(bits(c.key)[1], slots.numpy()))
    assert np.array_equal(bits(v), ref_cpu.gather(bits(c.value)[1], slots.numpy()))


@pytest.mark.parametrize("lens", [[100, 1, 16, 0, 47], [4096 + 5]])
def test_export_batch_bit_exact(hip, lens):
    bs = 16
    NB = sum(-(-n // bs) for n in lens) + 9
    c = _cache(4, NB, bs, 8, 128, seed=50)
    tables = random_block_tables(NB, lens, bs, 51)
    kbuf, vbuf, cu = c.export_batch(list(zip(tables, lens)))
    kb, vb = bits(kbuf), bits(vbuf)
    kp, vp = bits(c.key), bits(c.value)
    for b, (ids, n) in enumerate(zip(tables, lens)):
        rows = slice(c.num_layers * cu[b], c.num_layers * cu[b + 1])
        shape = (c.num_layers, n, 8, 128)
        assert np.array_equal(kb[rows].reshape(shape), ref_cpu.export_contiguous(kp, ids, n, bs))
        assert np.array_equal(vb[rows].reshape(shape), ref_cpu.export_contiguous(vp, ids, n, bs))


def test_export_import_round_trip_and_untouched_rows(hip):
    bs, H, D, L = 16, 2, 64, 3
    c = _cache(L, 64, bs, H, D, seed=60)
    tables = random_block_tables(64, [70, 33], bs, 61)
    k, v = c.export_contiguous(tables[0], 70)
    assert k.shape == (L, 70, H, D)
    # import the first sequence's KV into the second sequence's blocks (first 33 tokens)
    kp, vp = bits(c.key), bits(c.value)
    c.import_contiguous(tables[1], k[:, :33].contiguous(), v[:, :33].contiguous())
    ref_cpu.import_contiguous(kp, tables[1], bits(k)[:, :33], bs)
    ref_cpu.import_contiguous(vp, tables[1], bits(v)[:, :33], bs)
    assert np.array_equal(bits(c.key), kp) and np.array_equal(bits(c.value), vp)
    k2, _ = c.export_contiguous(tables[1], 33)
    assert torch.equal(k2, k[:, :33])


def test_import_casts_like_reference(hip):
    """import_contiguous casts with .to(pool dtype) (paged_cache.py:95-96)."""
    c = _cache(2, 8, 16, 2, 8, seed=70)
    ids = [5, 2]
    kf = torch.randn((2, 20, 2, 8), generator=gen(71))
    vf = torch.randn((2, 20, 2, 8), generator=gen(72))
    c.import_contiguous(ids, kf, vf)
    k, v = c.export_contiguous(ids, 20)
    assert torch.equal(k.cpu(), kf.to(torch.bfloat16)) and torch.equal(v.cpu(), vf.to(torch.bfloat16))


def test_copy_blocks_and_cow_fork(hip):
    bs = 16
    c = _cache(3, 12, bs, 2, 64, seed=80)
    mgr = c.manager
    mgr.allocate(1, 37)                               # 3 blocks, last one holds 5 tokens
    kp, vp = bits(c.key), bits(c.value)
    child = c.cow_fork(1, 2)
    parent = mgr.block_table(1)
    assert child.block_ids[:2] == parent.block_ids[:2]
    assert child.block_ids[2] != parent.block_ids[2]
    ref_cpu.copy_blocks(kp, kp, [(parent.block_ids[2], child.block_ids[2])], bs)
    ref_cpu.copy_blocks(vp, vp, [(parent.block_ids[2], child.block_ids[2])], bs)
    assert np.array_equal(bits(c.key), kp) and np.array_equal(bits(c.value), vp)
    # both may now append without touching each other's slots
    bp, op = c.append_token(1)
    bc, oc = c.append_token(2)
    assert (bp, op) != (bc, oc) and op == oc == 5


def test_ensure_writable_unshares_a_refcount_fork(hip):
    bs = 16
    c = _cache(2, 8, bs, 2, 64, seed=90)
    mgr = c.manager
    mgr.allocate(1, 20)
    mgr.fork(1, 2)                                    # reference fork: all blocks shared
    shared = mgr.block_table(2).block_ids[1]
    kp = bits(c.key)
    blk, off = c.append_token(2)                      # must copy the shared partial block
    assert blk != shared and off == 4
    assert mgr.ref_count(shared) == 1
    ref_cpu.copy_blocks(kp, kp, [(shared, blk)], bs)
    assert np.array_equal(bits(c.key), kp)


@pytest.mark.parametrize("bs,H,D,dtype", [(32, 3, 40, torch.bfloat16),   # 7680 B blocks
                                          (16, 3, 5, torch.float16),     # 30 B rows
                                          (64, 8, 128, torch.bfloat16),  # 128 KiB blocks
                                          (16, 1, 8, torch.float32)])    # 512 B blocks
def test_copies_split_into_pieces(hip, bs, H, D, dtype):
    """The block copy and the transport kernels move a block in 4 KiB pieces (one
    workgroup each): blocks that are not a multiple of a piece, smaller than one, many
    pieces long, and rows that need narrower vectors."""
    L = 3
    lens = [5 * bs + 3, bs, 1, 2 * bs - 1]
    NB = sum(-(-n // bs) for n in lens) + 12
    c = _cache(L, NB, bs, H, D, dtype=dtype, seed=110 + bs + D)
    tables = random_block_tables(NB, lens, bs, 111)
    kp, vp = bits(c.key), bits(c.value)
    kbuf, vbuf, cu = c.export_batch(list(zip(tables, lens)))
    for b, (ids, n) in enumerate(zip(tables, lens)):
        rows = slice(L * cu[b], L * cu[b + 1])
        shape = (L, n, H, D)
        assert np.array_equal(bits(kbuf)[rows].reshape(shape), ref_cpu.export_contiguous(kp, ids, n, bs))
        assert np.array_equal(bits(vbuf)[rows].reshape(shape), ref_cpu.export_contiguous(vp, ids, n, bs))
    used = {b for t in tables for b in t}
    free = [b for b in range(NB) if b not in used]
    pairs = list(zip(tables[0][:4], free[:4]))
    c.copy_blocks_from(c, [p[0] for p in pairs], [p[1] for p in pairs])
    ref_cpu.copy_blocks(kp, kp, pairs, bs)
    ref_cpu.copy_blocks(vp, vp, pairs, bs)
    assert np.array_equal(bits(c.key), kp) and np.array_equal(bits(c.value), vp)
    # import sequence 0's payload into sequence 3's blocks (its first 2*bs - 1 tokens)
    n3 = lens[3]
    k0 = kbuf[:L * lens[0]].view(L, lens[0], H, D)[:, :n3].contiguous()
    v0 = vbuf[:L * lens[0]].view(L, lens[0], H, D)[:, :n3].contiguous()
    c.import_contiguous(tables[3], k0, v0)
    ref_cpu.import_contiguous(kp, tables[3], bits(k0), bs)
    ref_cpu.import_contiguous(vp, tables[3], bits(v0), bs)
    assert np.array_equal(bits(c.key), kp) and np.array_equal(bits(c.value), vp)
    c.check_errors()


@pytest.mark.parametrize("bs,H,D,dtype", [(16, 8, 128, torch.bfloat16),  # 32 KiB blocks
                                          (32, 3, 40, torch.bfloat16),   # 7680 B: a part piece
                                          (16, 3, 5, torch.float16),     # 30 B rows
                                          (16, 1, 8, torch.float32)])    # 512 B blocks
@pytest.mark.parametrize("n_dst", [2, 8, 13, 32])
def test_fanout_copy_of_one_block(hip, bs, H, D, dtype, n_dst):
    """copy_blocks with one source for every pair (the copy-on-write fork of one partial
    block into many children) runs dsp_kv_copy_block_fanout: bit-exact against the same
    pairs copied one by one, for group sizes around its 8 copies per workgroup."""
    L, NB = 3, 48
    c = _cache(L, NB, bs, H, D, dtype=dtype, seed=200 + n_dst + D)
    kp, vp = bits(c.key), bits(c.value)
    dst = torch.randperm(NB - 1, generator=gen(201 + n_dst))[:n_dst].add(1).tolist()
    pairs = [(0, d) for d in dst]
    c.copy_blocks(pairs)
    ref_cpu.copy_blocks(kp, kp, pairs, bs)
    ref_cpu.copy_blocks(vp, vp, pairs, bs)
    assert np.array_equal(bits(c.key), kp) and np.array_equal(bits(c.value), vp)
    c.check_errors()


def test_fanout_into_a_second_pool_and_bad_ids(hip):
    """One block of one pool into blocks of another (prefix-cache spill of a shared block);
    destination ids outside the pool are skipped and counted, through the C-ABI."""
    from dispec_amd import _lib
    src = _cache(2, 8, 16, 2, 64, seed=210)
    dst = _cache(2, 12, 16, 2, 64, seed=211)
    kd, vd = bits(dst.key), bits(dst.value)
    ids = [3, 12, 7, -1, 0, 11, 5, 9, 1, 2]            # 12 and -1 lie outside dst
    d = torch.tensor(ids, dtype=torch.int32, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    st = _lib.lib().dsp_kv_copy_block_fanout(
        src.key.data_ptr(), src.value.data_ptr(), src.layer_bytes, src.num_blocks,
        dst.key.data_ptr(), dst.value.data_ptr(), dst.layer_bytes, dst.num_blocks,
        dst.num_layers, dst.block_bytes, 6, d.data_ptr(), len(ids), err.data_ptr(),
        torch.cuda.current_stream().cuda_stream)
    assert st == 0
    torch.cuda.synchronize()
    good = [(6, i) for i in ids if 0 <= i < 12]
    ref_cpu.copy_blocks(bits(src.key), kd, good, 16)
    ref_cpu.copy_blocks(bits(src.value), vd, good, 16)
    assert np.array_equal(bits(dst.key), kd) and np.array_equal(bits(dst.value), vd)
    assert int(err.item()) == 2
    # a source id outside the pool is a host-side argument error
    st = _lib.lib().dsp_kv_copy_block_fanout(
        src.key.data_ptr(), src.value.data_ptr(), src.layer_bytes, src.num_blocks,
        dst.key.data_ptr(), dst.value.data_ptr(), dst.layer_bytes, dst.num_blocks,
        dst.num_layers, dst.block_bytes, 8, d.data_ptr(), len(ids), err.data_ptr(),
        torch.cuda.current_stream().cuda_stream)
    assert st != 0


def test_copy_blocks_out_of_range_is_reported(hip):
    from dispec_amd.kv.paged_cache import PagedKVCache
    c = _cache(2, 8, 16, 2, 64, seed=100)
    kp = bits(c.key)
    c.copy_blocks_from(c, [1, 9], [2, 3])             # 9 is outside the pool
    ref_cpu.copy_blocks(kp, kp, [(1, 2)], 16)
    assert np.array_equal(bits(c.key), kp)
    with pytest.raises(IndexError):
        c.check_errors()
    assert isinstance(c, PagedKVCache)


def test_prefix_cache_spill_copies_victims(hip):
    from dispec_amd.kv.prefix_cache import PrefixCache
    bs = 16
    c = _cache(2, 16, bs, 2, 64, seed=110)
    spill = _cache(2, 8, bs, 2, 64, seed=111)
    pc = PrefixCache(c.manager, bs).bind(c)
    t = c.manager.allocate(1, 64)
    pc.insert(list(range(64)), t.block_ids)
    c.manager.free(1)
    pc.match(list(range(32)))                         # touch the first two blocks
    victims = pc.lru_victims(2)
    assert [b for _, b in victims] == t.block_ids[2:4]
    kp = bits(c.key)
    assert pc.evict(2, spill_to=spill) == 2
    sk = bits(spill.key)
    for (key, blk) in victims:
        d = pc.spilled[key]
        assert np.array_equal(sk[:, d * bs:(d + 1) * bs], kp[:, blk * bs:(blk + 1) * bs])
    assert c.manager.num_free_blocks == 16 - 2
