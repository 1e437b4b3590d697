"""Automatic prefix caching over full KV blocks (host policy).

Same policy as the reference (dispec/kv/prefix_cache.py:20-73): each *full* block is
keyed by the rolling hash h_i = hash((h_{i-1}, tokens of block i)) (:29-37); `match`
walks the keys until the first miss (:39-50); `insert` pins newly seen blocks with one
reference (:52-62); `evict` releases the least-recently-used entries (:64-70).

Addition: `evict(n, spill_to=cache)` copies the victims' K/V (every layer) into blocks
of a second pool before releasing them -- the data move of a two-tier prefix cache,
done by the block-copy kernel.  Spilled entries are kept in `spilled`.
"""

from __future__ import annotations

from dispec_amd.kv.block_manager import BlockManager


class PrefixCache:
    def __init__(self, manager: BlockManager, block_size: int):
        self.mgr = manager
        self.bs = block_size
        self._nodes: dict[int, list] = {}   # key -> [block_id, last_used]
        self._clock = 0
        self.hits = 0
        self.misses = 0
        self.spilled: dict[int, int] = {}   # key -> block id in the spill pool

    def _block_hashes(self, token_ids: list[int]) -> list[int]:
        keys, h = [], 0
        for i in range(len(token_ids) // self.bs):
            h = hash((h, tuple(token_ids[i * self.bs:(i + 1) * self.bs])))
            keys.append(h)
        return keys

    def match(self, token_ids: list[int]) -> list[int]:
        """Physical blocks of the longest cached run of this prompt's full blocks."""
        self._clock += 1
        found: list[int] = []
        for key in self._block_hashes(token_ids):
            node = self._nodes.get(key)
            if node is None:
                break
            node[1] = self._clock
            found.append(node[0])
        self.hits += len(found)
        return found

    def insert(self, token_ids: list[int], block_ids: list[int]) -> None:
        """Register a sequence's full blocks; new ones are pinned with one reference."""
        self._clock += 1
        for key, blk in zip(self._block_hashes(token_ids), block_ids):
            node = self._nodes.get(key)
            if node is None:
                self.mgr.add_ref(blk)
                self._nodes[key] = [blk, self._clock]
                self.misses += 1
            else:
                node[1] = self._clock

    def lru_victims(self, num_blocks: int) -> list[tuple[int, int]]:
        """(key, block) of the num_blocks least-recently-used entries, oldest first."""
        order = sorted(self._nodes.items(), key=lambda kv: kv[1][1])[:max(num_blocks, 0)]
        return [(key, node[0]) for key, node in order]

    def evict(self, num_blocks: int, spill_to=None) -> int:
        """Release up to num_blocks LRU entries; returns how many were evicted.

        With `spill_to` (a PagedKVCache of the same geometry) the victims' data is first
        copied into freshly allocated blocks of that pool, recorded in `spilled`.
        """
        victims = self.lru_victims(num_blocks)
        if spill_to is not None and victims:
            src = [blk for _, blk in victims]
            dst = [spill_to.manager._alloc_block() for _ in victims]
            spill_to.copy_blocks_from(self._owner_cache(), src, dst)
            for (key, _), d in zip(victims, dst):
                self.spilled[key] = d
        for key, blk in victims:
            del self._nodes[key]
            self.mgr.release(blk)
        return len(victims)

    def bind(self, cache) -> "PrefixCache":
        """Attach the PagedKVCache whose pool this cache's block ids index."""
        self._cache = cache
        return self

    def _owner_cache(self):
        cache = getattr(self, "_cache", None)
        if cache is None:
            raise ValueError("evict(spill_to=...) needs the source pool: call bind(cache) first")
        return cache

    def __len__(self) -> int:
        return len(self._nodes)
