"""Prefix-cache policy: the reference's CPU tests (tests/test_prefix_cache.py:14-35)
restated against dispec_amd's PrefixCache, plus LRU victim order (CPU only)."""

from dispec_amd.kv.block_manager import BlockManager
from dispec_amd.kv.prefix_cache import PrefixCache


def test_match_returns_shared_full_blocks():
    bm = BlockManager(num_blocks=20, block_size=4)
    pc = PrefixCache(bm, block_size=4)
    t = bm.allocate(1, 8)
    pc.insert(list(range(8)), t.block_ids)
    assert len(pc) == 2
    assert pc.match(list(range(8)) + [99, 99]) == t.block_ids
    assert pc.match([100, 101, 102, 103]) == []


def test_insert_pins_blocks_and_evict_releases():
    bm = BlockManager(num_blocks=8, block_size=4)
    pc = PrefixCache(bm, block_size=4)
    t = bm.allocate(1, 8)
    pc.insert(list(range(8)), t.block_ids)
    bm.free(1)
    assert bm.num_free_blocks == 6
    assert pc.evict(2) == 2
    assert bm.num_free_blocks == 8


def test_partial_blocks_are_not_cached_and_match_stops_at_first_miss():
    bm = BlockManager(num_blocks=20, block_size=4)
    pc = PrefixCache(bm, block_size=4)
    t = bm.allocate(1, 14)
    pc.insert(list(range(14)), t.block_ids)
    assert len(pc) == 3                                  # 14 tokens = 3 full blocks
    assert pc.match([0, 1, 2, 3, 9, 9, 9, 9, 8, 9, 10, 11]) == t.block_ids[:1]
    assert pc.hits == 1 and pc.misses == 3


def test_lru_victims_oldest_first():
    bm = BlockManager(num_blocks=20, block_size=2)
    pc = PrefixCache(bm, block_size=2)
    t = bm.allocate(1, 8)
    pc.insert(list(range(8)), t.block_ids)
    pc.match(list(range(4)))                             # touches blocks 0, 1
    assert [b for _, b in pc.lru_victims(2)] == t.block_ids[2:4]
    assert pc.evict(3) == 3 and len(pc) == 1
