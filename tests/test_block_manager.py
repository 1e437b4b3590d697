"""Host block allocator: the reference's own tests (tests/test_block_manager.py:8-57),
restated against dispec_amd's BlockManager, plus copy-on-write (CPU only)."""

import pytest

from dispec_amd.kv.block_manager import BlockManager, OutOfBlocksError


def test_allocate_and_slots():
    bm = BlockManager(num_blocks=10, block_size=4)
    table = bm.allocate(seq_id=1, num_tokens=6)
    assert len(table.block_ids) == 2 and bm.num_free_blocks == 8
    assert table.slot(4, 0) == (table.block_ids[0], 0)
    assert table.slot(4, 5) == (table.block_ids[1], 1)


def test_lifo_free_list_order_matches_reference():
    bm = BlockManager(num_blocks=5, block_size=4)
    assert bm.allocate(1, 8).block_ids == [4, 3]      # list(range(n)).pop() order
    bm.free(1)
    assert bm.allocate(2, 4).block_ids == [3]         # freed 4 then 3; 3 is popped first


def test_append_grows_blocks_only_when_full():
    bm = BlockManager(num_blocks=10, block_size=2)
    bm.allocate(seq_id=1, num_tokens=2)
    assert len(bm.block_table(1).block_ids) == 1
    blk, off = bm.append_token(1)
    assert off == 0 and len(bm.block_table(1).block_ids) == 2
    bm.append_token(1)
    assert len(bm.block_table(1).block_ids) == 2 and bm.block_table(1).num_tokens == 4


def test_free_returns_blocks():
    bm = BlockManager(num_blocks=4, block_size=4)
    bm.allocate(seq_id=1, num_tokens=16)
    assert bm.num_free_blocks == 0
    with pytest.raises(OutOfBlocksError):
        bm.allocate(seq_id=2, num_tokens=1)
    bm.free(1)
    assert bm.num_free_blocks == 4
    bm.allocate(seq_id=2, num_tokens=1)


def test_fork_is_copy_on_write_refcounted():
    bm = BlockManager(num_blocks=4, block_size=4)
    bm.allocate(seq_id=1, num_tokens=8)
    assert bm.num_free_blocks == 2
    bm.fork(parent_id=1, child_id=2)
    assert bm.num_free_blocks == 2
    bm.free(1)
    assert bm.num_free_blocks == 2
    bm.free(2)
    assert bm.num_free_blocks == 4


def test_reserve_for_tree():
    bm = BlockManager(num_blocks=10, block_size=4)
    bm.allocate(seq_id=1, num_tokens=4)
    bm.reserve(seq_id=1, num_new_tokens=5)
    assert len(bm.block_table(1).block_ids) == 3


def test_truncate_releases_trailing_blocks():
    bm = BlockManager(num_blocks=10, block_size=4)
    bm.allocate(1, 12)
    bm.truncate(1, 5)
    assert len(bm.block_table(1).block_ids) == 2 and bm.num_free_blocks == 8
    assert bm.block_table(1).num_tokens == 5


def test_allocate_with_reuse_shares_blocks():
    bm = BlockManager(num_blocks=10, block_size=4)
    t1 = bm.allocate(1, 8)
    t2 = bm.allocate(2, 10, reuse_blocks=t1.block_ids)
    assert t2.block_ids[:2] == t1.block_ids and bm.ref_count(t1.block_ids[0]) == 2
    with pytest.raises(ValueError):
        bm.allocate(2, 1)


def test_cow_fork_copies_only_the_partial_block():
    bm = BlockManager(num_blocks=10, block_size=4)
    bm.allocate(1, 10)                     # blocks: full, full, partial(2 tokens)
    parent = bm.block_table(1)
    child, pairs = bm.cow_fork(1, 2)
    assert child.block_ids[:2] == parent.block_ids[:2]
    assert pairs == [(parent.block_ids[2], child.block_ids[2])]
    assert bm.ref_count(parent.block_ids[0]) == 2 and bm.ref_count(parent.block_ids[2]) == 1
    # both append into private slots
    assert bm.append_token(1) == (parent.block_ids[2], 2)
    assert bm.append_token(2) == (child.block_ids[2], 2)
    # an aligned parent needs no copy
    bm.allocate(3, 8)
    _, pairs = bm.cow_fork(3, 4)
    assert pairs == []


def test_cow_fork_out_of_blocks():
    bm = BlockManager(num_blocks=2, block_size=4)
    bm.allocate(1, 6)
    with pytest.raises(OutOfBlocksError):
        bm.cow_fork(1, 2)
    assert not bm.has_table(2) and bm.ref_count(bm.block_table(1).block_ids[0]) == 1


def test_ensure_writable_after_refcount_fork():
    bm = BlockManager(num_blocks=10, block_size=4)
    bm.allocate(1, 6)
    bm.fork(1, 2)
    shared = bm.block_table(2).block_ids[1]
    pairs = bm.ensure_writable(2)
    assert len(pairs) == 1 and pairs[0][0] == shared
    assert bm.block_table(2).block_ids[1] == pairs[0][1] != shared
    assert bm.ref_count(shared) == 1
    assert bm.ensure_writable(2) == [] and bm.ensure_writable(1) == []
    bm.free(1)
    bm.free(2)
    assert bm.num_free_blocks == 10


def _slots_after_appends(bm, seq, n):
    return [bm.append_token(seq) for _ in range(n)]


def test_cow_fork_after_reserve_gives_private_room():
    # 20 tokens in blocks of 16, room reserved for 14 more (a third block), then a fork:
    # the partial block is copied, the reserved block is the child's own (nothing to copy)
    bm = BlockManager(num_blocks=20, block_size=16)
    bm.allocate(0, 20)
    bm.reserve(0, 14)
    parent = bm.block_table(0)
    assert len(parent.block_ids) == 3
    child, pairs = bm.cow_fork(0, 1)
    assert pairs == [(parent.block_ids[1], child.block_ids[1])]
    assert child.block_ids[0] == parent.block_ids[0]
    assert child.block_ids[2] != parent.block_ids[2]
    assert bm.ref_count(parent.block_ids[0]) == 2 and bm.ref_count(parent.block_ids[2]) == 1
    # 13 appends each: the 13th crosses into the reserved block; no slot is shared
    a = _slots_after_appends(bm, 0, 13)
    b = _slots_after_appends(bm, 1, 13)
    assert not set(a) & set(b)
    bm.free(0)
    bm.free(1)
    assert bm.num_free_blocks == 20


def test_ensure_writable_unshares_a_reserved_block():
    # a reference-style fork shares the reserved block too; ensure_writable un-shares the
    # block the next token goes into, with a copy only when it holds written tokens
    bm = BlockManager(num_blocks=20, block_size=16)
    bm.allocate(0, 32)
    bm.reserve(0, 5)
    bm.fork(0, 1)
    reserved = bm.block_table(0).block_ids[2]
    assert bm.ensure_writable(1) == []            # next token opens the reserved block
    assert bm.block_table(1).block_ids[2] != reserved
    assert bm.ref_count(reserved) == 1
    assert bm.append_token(0)[0] == reserved
    assert bm.append_token(1)[0] == bm.block_table(1).block_ids[2]
    # a partially written shared block is copied
    bm.fork(0, 2)
    pairs = bm.ensure_writable(2)
    assert pairs == [(reserved, bm.block_table(2).block_ids[2])]


def test_cow_fork_out_of_blocks_counts_reserved_room():
    bm = BlockManager(num_blocks=4, block_size=4)
    bm.allocate(0, 6)          # full + partial
    bm.reserve(0, 6)           # + 1 reserved -> 3 blocks, 1 free
    with pytest.raises(OutOfBlocksError):
        bm.cow_fork(0, 1)      # needs the partial copy and the reserved block: 2
    assert not bm.has_table(1) and bm.num_free_blocks == 1
