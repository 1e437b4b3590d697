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
