"""PrefixCache against an independent model, over seeded random serving traffic (CPU).

The model keys each cached block by the whole token prefix it ends (a tuple), not by a
hash, and keeps (block, last use, insertion order) per key.  Prompts are drawn so that
many share leading blocks and some share a block's tokens after different earlier
blocks.  Each step either serves a prompt -- `match`, then a sequence allocated with the
matched blocks leading it, `insert` of its full blocks, the sequence freed -- or evicts a
few entries.  After each step the cache agrees with the model on:

  * the blocks `match` returns (the longest run of the prompt's leading full blocks that
    are cached) and the hit / miss counters;
  * the victims of `evict`: least recently used first, ties in insertion order (the
    reference sorts its insertion-ordered dict by last use, a stable sort:
    dispec/kv/prefix_cache.py:64-70);
  * the pins: every cached block holds exactly one reference per key in the block manager.

A cache that keys a block by its own tokens only (no chain through the earlier blocks)
fails the comparison.
"""

import random

import pytest

from dispec_amd.kv.block_manager import BlockManager, OutOfBlocksError
from dispec_amd.kv.prefix_cache import PrefixCache

BS, NB = 4, 96


class Model:
    def __init__(self):
        self.nodes: dict[tuple, list] = {}   # prefix -> [block, last_use, insertion index]
        self.clock = self.order = self.hits = self.misses = 0

    def keys(self, prompt):
        return [tuple(prompt[:(i + 1) * BS]) for i in range(len(prompt) // BS)]

    def match(self, prompt):
        self.clock += 1
        out = []
        for key in self.keys(prompt):
            node = self.nodes.get(key)
            if node is None:
                break
            node[1] = self.clock
            out.append(node[0])
        self.hits += len(out)
        return out

    def insert(self, prompt, blocks):
        self.clock += 1
        for key, blk in zip(self.keys(prompt), blocks):
            node = self.nodes.get(key)
            if node is None:
                self.order += 1
                self.nodes[key] = [blk, self.clock, self.order]
                self.misses += 1
            else:
                node[1] = self.clock

    def evict(self, n):
        victims = sorted(self.nodes.items(), key=lambda kv: (kv[1][1], kv[1][2]))[:n]
        for key, _ in victims:
            del self.nodes[key]
        return sorted(node[0] for _, node in victims)


def _prompt(rng, pool):
    if pool and rng.random() < 0.7:                  # extend or cut a previous prompt
        base = rng.choice(pool)
        cut = rng.randint(0, len(base))
        p = base[:cut] + [rng.randrange(6) for _ in range(rng.randint(0, 3 * BS))]
        if rng.random() < 0.2 and len(p) >= 2 * BS:  # same later block, different earlier one
            p[0] = (p[0] + 1) % 6
    else:
        p = [rng.randrange(6) for _ in range(rng.randint(1, 4 * BS))]
    pool.append(p)
    return p or [0]


def _traffic(seed, cache_cls=PrefixCache, steps=400):
    rng = random.Random(seed)
    mgr = BlockManager(NB, BS)
    cache, model = cache_cls(mgr, BS), Model()
    pool, sid = [], 0
    stats = {"full": 0, "evict": 0}
    for _ in range(steps):
        if rng.random() < 0.85:
            prompt = _prompt(rng, pool)
            got, want = cache.match(prompt), model.match(prompt)
            assert got == want, f"match {got} != {want}"
            try:
                table = mgr.allocate(sid, len(prompt), reuse_blocks=got)
            except OutOfBlocksError:                 # pool full of pinned blocks: evict
                n = rng.randint(1, 8)
                k = min(n, len(cache))
                assert sorted(b for _, b in cache.lru_victims(n)) == model.evict(n)
                assert cache.evict(n) == k
                stats["full"] += 1
                continue
            cache.insert(prompt, table.block_ids)
            model.insert(prompt, table.block_ids)
            mgr.free(sid)
            sid += 1
        else:
            n = rng.randint(1, 6)
            victims = sorted(b for _, b in cache.lru_victims(n))
            assert victims == model.evict(n), "evict order"
            cache.evict(n)
            stats["evict"] += 1
        assert (cache.hits, cache.misses) == (model.hits, model.misses)
        assert len(cache) == len(model.nodes)
        pins: dict[int, int] = {}
        for blk, _, _ in model.nodes.values():
            pins[blk] = pins.get(blk, 0) + 1
        assert {b: mgr.ref_count(b) for b in range(NB) if mgr.ref_count(b)} == pins
    return cache, model, stats


@pytest.mark.parametrize("seed", range(5))
def test_random_traffic_agrees_with_the_model(seed):
    cache, model, stats = _traffic(seed)
    assert model.hits > 50 and model.misses > 50     # the traffic shared prefixes
    assert stats["full"] > 0 and stats["evict"] > 10  # and filled the pool


class _UnchainedKeys(PrefixCache):
    def _block_hashes(self, token_ids):
        return [hash(tuple(token_ids[i * self.bs:(i + 1) * self.bs]))
                for i in range(len(token_ids) // self.bs)]


def test_unchained_block_keys_fail_the_comparison():
    with pytest.raises(AssertionError):
        for seed in range(5):
            _traffic(seed, _UnchainedKeys)
