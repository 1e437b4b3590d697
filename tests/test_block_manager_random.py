"""Seeded random operation sequences on BlockManager against a shadow model of the blocks'
contents (CPU).

Every step applies one operation a serving loop performs -- allocate (sometimes adopting a
live sequence's full blocks, as a prefix-cache hit does), append one token (after
`ensure_writable`, applying the copy pair it returns), refcount `fork`, `cow_fork` (applying
its copy pairs), `reserve`, `truncate`, `free`, and a pin / unpin of a block -- to the
manager and to a model that stores a token value per (block, offset).  After each step:

  * every block is free exactly once or referenced, never both, and the free list plus the
    referenced blocks are the whole pool;
  * each block's reference count equals the number of block-table entries naming it plus
    the pins the test holds on it;
  * every live sequence has room for its tokens and reads back exactly the token values it
    wrote (through `BlockTable.slot`), whatever the other sequences wrote: copy-on-write
    keeps forks from seeing each other's appends;
  * a manager call that raises OutOfBlocksError has changed nothing (an append is two
    calls: `ensure_writable`, whose private copy stays, then `append_token`).

Three managers with a planted slip each (no un-sharing before a write, a block never
returned to the pool, a fork that shares the partially filled block) fail these checks.
"""

import random

import pytest

from dispec_amd.kv.block_manager import BlockManager, OutOfBlocksError

BS, NB = 4, 24


class Shadow:
    def __init__(self, seed: int, manager=BlockManager):
        self.rng = random.Random(seed)
        self.mgr = manager(NB, BS)
        self.out_of_blocks = 0
        self.shared_seen = False
        self.data: dict[int, list] = {}     # block -> BS token values (None: never written)
        self.expect: dict[int, list] = {}   # seq -> its tokens
        self.pins: dict[int, int] = {}      # block -> pins held by the test
        self.next_sid = 0
        self.next_val = 0

    # -- helpers -------------------------------------------------------------------------
    def val(self):
        self.next_val += 1
        return self.next_val

    def write(self, sid: int, pos: int, v) -> None:
        blk, off = self.mgr.block_table(sid).slot(BS, pos)
        self.data.setdefault(blk, [None] * BS)[off] = v

    def copy(self, pairs) -> None:
        for src, dst in pairs:
            self.data[dst] = list(self.data.get(src, [None] * BS))

    def call(self, fn, *args):
        """One manager call; one that raises OutOfBlocksError must have changed nothing."""
        before = self.snapshot()
        try:
            return fn(*args)
        except OutOfBlocksError:
            assert self.snapshot() == before, f"{fn.__name__} changed state before failing"
            raise

    def snapshot(self):
        tables = {s: (list(self.mgr.block_table(s).block_ids), self.mgr.block_table(s).num_tokens)
                  for s in self.expect}
        return tables, list(self.mgr._free), dict(self.mgr._ref_count)

    # -- invariants -------------------------------------------------------------------------
    def check(self) -> None:
        mgr = self.mgr
        free = mgr._free
        assert len(set(free)) == len(free), "a block is on the free list twice"
        uses: dict[int, int] = {}
        for sid in self.expect:
            for blk in mgr.block_table(sid).block_ids:
                uses[blk] = uses.get(blk, 0) + 1
        for blk, n in self.pins.items():
            uses[blk] = uses.get(blk, 0) + n
        assert set(free).isdisjoint(uses), "a referenced block is on the free list"
        assert set(free) | set(uses) == set(range(NB)), "blocks leaked"
        assert {b: mgr.ref_count(b) for b in uses} == uses, "reference counts drifted"
        self.shared_seen |= any(n > 1 for n in uses.values())
        for sid, toks in self.expect.items():
            table = mgr.block_table(sid)
            assert table.num_tokens == len(toks)
            assert len(table.block_ids) * BS >= len(toks)
            got = []
            for pos in range(len(toks)):
                blk, off = table.slot(BS, pos)
                got.append(self.data.get(blk, [None] * BS)[off])
            assert got == toks, f"seq {sid} reads {got}, wrote {toks}"

    # -- operations -------------------------------------------------------------------------
    def op_allocate(self):
        sid = self.next_sid
        n = self.rng.randint(1, 3 * BS + 1)
        reuse, prefix = [], []
        live = [s for s in self.expect if self.mgr.block_table(s).num_tokens >= BS]
        if live and self.rng.random() < 0.4:          # prefix-cache hit: adopt full blocks
            src = self.rng.choice(live)
            k = self.rng.randint(1, self.mgr.block_table(src).num_tokens // BS)
            reuse = self.mgr.block_table(src).block_ids[:k]
            prefix = self.expect[src][:k * BS]
            n = max(n, k * BS + self.rng.randint(0, BS))
        self.call(self.mgr.allocate, sid, n, reuse)
        self.next_sid += 1
        toks = list(prefix) + [self.val() for _ in range(n - len(prefix))]
        self.expect[sid] = toks
        for pos in range(len(prefix), n):              # the prefill writes its own tokens
            self.write(sid, pos, toks[pos])

    def op_append(self, sid):
        # two calls, each all-or-nothing: a private copy of the block the token goes into
        # (kept even if the append then finds the pool empty), then the append
        self.copy(self.call(self.mgr.ensure_writable, sid))
        pos = self.mgr.block_table(sid).num_tokens
        self.call(self.mgr.append_token, sid)
        v = self.val()
        self.write(sid, pos, v)
        self.expect[sid].append(v)

    def op_fork(self, sid):
        child = self.next_sid
        self.call(self.mgr.fork, sid, child)
        self.next_sid += 1
        self.expect[child] = list(self.expect[sid])

    def raw_append(self, sid):
        """Append without ensure_writable: only where the block the token goes into is
        known to be this sequence's alone."""
        pos = self.mgr.block_table(sid).num_tokens
        self.call(self.mgr.append_token, sid)
        v = self.val()
        self.write(sid, pos, v)
        self.expect[sid].append(v)

    def op_cow_fork(self, sid):
        table = self.mgr.block_table(sid)
        i = table.num_tokens // BS
        # the block the parent's next token goes into exists and is the parent's alone
        tail_private = i < len(table.block_ids) and self.mgr.ref_count(table.block_ids[i]) == 1
        child = self.next_sid
        _, pairs = self.call(self.mgr.cow_fork, sid, child)
        self.next_sid += 1
        self.copy(pairs)
        self.expect[child] = list(self.expect[sid])
        if tail_private:
            # cow_fork's promise: parent and child append at once without touching each
            # other's slots -- no ensure_writable in between
            self.raw_append(sid)
            self.raw_append(child)

    def op_reserve(self, sid):
        self.call(self.mgr.reserve, sid, self.rng.randint(1, 2 * BS))

    def op_truncate(self, sid):
        n = self.rng.randint(0, len(self.expect[sid]))
        self.mgr.truncate(sid, n)
        del self.expect[sid][n:]

    def op_free(self, sid):
        self.mgr.free(sid)
        del self.expect[sid]

    def op_pin(self, sid):
        ids = self.mgr.block_table(sid).block_ids
        if ids:
            blk = self.rng.choice(ids)
            self.mgr.add_ref(blk)
            self.pins[blk] = self.pins.get(blk, 0) + 1

    def op_unpin(self, _sid):
        if self.pins:
            blk = self.rng.choice(sorted(self.pins))
            self.mgr.release(blk)
            self.pins[blk] -= 1
            if not self.pins[blk]:
                del self.pins[blk]

    def step(self) -> str:
        ops = ["allocate", "append", "append", "append", "fork", "cow_fork", "reserve",
               "truncate", "free", "pin", "unpin"]
        name = self.rng.choice(ops) if self.expect else "allocate"
        sid = self.rng.choice(sorted(self.expect)) if self.expect else None
        try:
            getattr(self, "op_" + name)() if name == "allocate" else getattr(self, "op_" + name)(sid)
        except OutOfBlocksError:
            self.out_of_blocks += 1
            if self.expect and self.rng.random() < 0.5:   # make room for the next steps
                self.op_free(self.rng.choice(sorted(self.expect)))
        return name


def _run(seed, manager=BlockManager, steps=600):
    sh = Shadow(seed, manager)
    counts: dict[str, int] = {}
    for _ in range(steps):
        name = sh.step()
        counts[name] = counts.get(name, 0) + 1
        sh.check()
    return sh, counts


@pytest.mark.parametrize("seed", range(6))
def test_random_operations_keep_every_sequence_intact(seed):
    sh, counts = _run(seed)
    # every operation ran many times, the pool ran dry and blocks were shared
    assert all(counts.get(op, 0) > 10 for op in ("allocate", "append", "fork", "cow_fork",
                                                  "reserve", "truncate", "free"))
    assert sh.out_of_blocks > 0 and sh.shared_seen


class _NoUnshare(BlockManager):
    def ensure_writable(self, seq_id):
        return []


class _Leaky(BlockManager):
    def _drop(self, blk):
        n = self._ref_count[blk] - 1
        if n:
            self._ref_count[blk] = n
        else:
            del self._ref_count[blk]        # never back on the free list


class _SharesPartial(BlockManager):
    def cow_fork(self, parent_id, child_id):
        return self.fork(parent_id, child_id), []


@pytest.mark.parametrize("manager", [_NoUnshare, _Leaky, _SharesPartial],
                         ids=["no-unshare", "leak", "shared-partial"])
def test_planted_manager_slips_fail_the_checks(manager):
    with pytest.raises(AssertionError):
        for seed in range(6):
            _run(seed, manager)


def test_a_planted_slip_is_caught():
    """The checks notice a copy-on-write slip: parent and refcount-forked child both
    append without ensure_writable, so the parent's next token lands in the slot of the
    shared partial block that already holds the child's."""
    sh = Shadow(99)
    sh.mgr.allocate(0, BS + 2)                       # one full block and a partial one
    sh.next_sid = 1
    sh.expect[0] = [sh.val() for _ in range(BS + 2)]
    for pos, v in enumerate(sh.expect[0]):
        sh.write(0, pos, v)
    sh.op_fork(0)                                    # child 1 shares both blocks
    pos = sh.mgr.block_table(1).num_tokens           # append without ensure_writable
    sh.mgr.append_token(1)
    v = sh.val()
    sh.write(1, pos, v)
    sh.expect[1].append(v)
    sh.check()                                       # still consistent: parent unaffected
    pos = sh.mgr.block_table(0).num_tokens           # the parent skips it too
    sh.mgr.append_token(0)
    v = sh.val()
    sh.write(0, pos, v)
    sh.expect[0].append(v)
    with pytest.raises(AssertionError, match="seq 1 reads"):
        sh.check()
