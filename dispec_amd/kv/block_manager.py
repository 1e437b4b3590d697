"""Host-side paged-KV block allocator (no tensors).

Same contract as the reference allocator (dispec/kv/block_manager.py:34-152): a LIFO
free list of physical block ids, per-block reference counts, and per-sequence block
tables.  `fork` shares every block by refcount exactly as the reference does
(:119-126).  Two additions make copy-on-write real instead of refcount-only:

  * `cow_fork` shares the parent's full blocks but gives the child its own copy of the
    parent's partially filled last block, returning the (src, dst) block pair.
  * `ensure_writable` is called before a sequence writes into its last block; if that
    block is shared it is replaced by a private block and the (src, dst) pair returned.

The returned pairs are what `PagedKVCache.copy_blocks` moves on the GPU.  Without them a
forked parent and child would both write the next token into the same shared slot
(append_token allocates only when num_tokens % block_size == 0, :98-106).
"""

from __future__ import annotations

from dataclasses import dataclass, field


class OutOfBlocksError(RuntimeError):
    """The block pool is exhausted (reference: dispec/kv/block_manager.py:18-19)."""


@dataclass
class BlockTable:
    """Ordered physical blocks of one sequence and its logical token count."""

    block_ids: list[int] = field(default_factory=list)
    num_tokens: int = 0

    def slot(self, block_size: int, token_pos: int) -> tuple[int, int]:
        """(physical block, offset) of a logical token position (block_manager.py:29-31)."""
        return self.block_ids[token_pos // block_size], token_pos % block_size


class BlockManager:
    def __init__(self, num_blocks: int, block_size: int):
        if num_blocks < 0 or block_size <= 0:
            raise ValueError(f"bad pool geometry: {num_blocks} blocks of {block_size}")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self._free: list[int] = list(range(num_blocks))   # pop() from the end: LIFO
        self._ref_count: dict[int, int] = {}
        self._tables: dict[int, BlockTable] = {}

    # -- introspection ------------------------------------------------------------
    @property
    def num_free_blocks(self) -> int:
        return len(self._free)

    def blocks_needed(self, num_tokens: int) -> int:
        return -(-num_tokens // self.block_size)

    def has_table(self, seq_id: int) -> bool:
        return seq_id in self._tables

    def block_table(self, seq_id: int) -> BlockTable:
        return self._tables[seq_id]

    def ref_count(self, block_id: int) -> int:
        return self._ref_count.get(block_id, 0)

    # -- allocation ---------------------------------------------------------------
    def _alloc_block(self) -> int:
        if not self._free:
            raise OutOfBlocksError("block pool exhausted")
        blk = self._free.pop()
        self._ref_count[blk] = 1
        return blk

    def _drop(self, blk: int) -> None:
        n = self._ref_count[blk] - 1
        if n:
            self._ref_count[blk] = n
        else:
            del self._ref_count[blk]
            self._free.append(blk)

    def allocate(self, seq_id: int, num_tokens: int,
                 reuse_blocks: list[int] | None = None) -> BlockTable:
        """New sequence with room for num_tokens; `reuse_blocks` lead it, shared."""
        if seq_id in self._tables:
            raise ValueError(f"seq {seq_id} already allocated")
        reuse = list(reuse_blocks or [])
        fresh = self.blocks_needed(num_tokens) - len(reuse)
        if fresh > self.num_free_blocks:
            raise OutOfBlocksError(f"need {fresh} blocks, have {self.num_free_blocks}")
        for blk in reuse:
            self._ref_count[blk] += 1
        table = BlockTable(reuse + [self._alloc_block() for _ in range(fresh)], num_tokens)
        self._tables[seq_id] = table
        return table

    def add_ref(self, block_id: int) -> None:
        self._ref_count[block_id] += 1

    def release(self, block_id: int) -> None:
        self._drop(block_id)

    def append_token(self, seq_id: int) -> tuple[int, int]:
        """Room for one more token; returns its (block, offset)."""
        table = self._tables[seq_id]
        if table.num_tokens % self.block_size == 0:
            table.block_ids.append(self._alloc_block())
        slot = table.slot(self.block_size, table.num_tokens)
        table.num_tokens += 1
        return slot

    def reserve(self, seq_id: int, num_new_tokens: int) -> None:
        """Make sure num_new_tokens more tokens fit (speculative verify, trees)."""
        table = self._tables[seq_id]
        room = len(table.block_ids) * self.block_size - table.num_tokens
        if num_new_tokens > room:
            extra = self.blocks_needed(num_new_tokens - room)
            if extra > self.num_free_blocks:
                raise OutOfBlocksError(f"reserve needs {extra}, have {self.num_free_blocks}")
            table.block_ids.extend(self._alloc_block() for _ in range(extra))

    # -- sharing --------------------------------------------------------------------
    def fork(self, parent_id: int, child_id: int) -> BlockTable:
        """Child shares every parent block by refcount (reference semantics)."""
        parent = self._tables[parent_id]
        for blk in parent.block_ids:
            self._ref_count[blk] += 1
        child = BlockTable(list(parent.block_ids), parent.num_tokens)
        self._tables[child_id] = child
        return child

    def cow_fork(self, parent_id: int, child_id: int) -> tuple[BlockTable, list[tuple[int, int]]]:
        """Fork that gives the child private copies of every block it may still write.

        Blocks holding only already-written tokens are shared by refcount.  The parent's
        partially filled block is copied for the child, and the (src, dst) pair whose data
        must be moved is returned.  Blocks past the written tokens (room made by `reserve`)
        hold no data yet, so the child gets fresh private blocks for them with nothing to
        copy.  Parent and child can then append without touching each other's slots.
        """
        if child_id in self._tables:
            raise ValueError(f"seq {child_id} already allocated")
        parent = self._tables[parent_id]
        written = parent.num_tokens // self.block_size   # blocks holding only written tokens
        private = len(parent.block_ids) - written          # partial block + reserved room
        if private > self.num_free_blocks:
            raise OutOfBlocksError(f"cow_fork needs {private}, have {self.num_free_blocks}")
        ids = list(parent.block_ids[:written])
        for blk in ids:
            self._ref_count[blk] += 1
        copies: list[tuple[int, int]] = []
        for i in range(written, len(parent.block_ids)):
            new = self._alloc_block()
            if i * self.block_size < parent.num_tokens:      # the partial block: copy it
                copies.append((parent.block_ids[i], new))
            ids.append(new)
        child = BlockTable(ids, parent.num_tokens)
        self._tables[child_id] = child
        return child, copies

    def ensure_writable(self, seq_id: int) -> list[tuple[int, int]]:
        """Give the sequence a private copy of the block its next token goes into.

        Call before writing the next token.  When that block exists (partially filled, or
        reserved ahead) and is shared, it is replaced by a private block.  Returns the
        (src, dst) pair to copy when the block holds written tokens; [] when the block is
        already private, does not exist yet (append_token allocates it) or holds none of
        this sequence's tokens.
        """
        table = self._tables[seq_id]
        i = table.num_tokens // self.block_size
        if i >= len(table.block_ids):
            return []
        blk = table.block_ids[i]
        if self._ref_count[blk] == 1:
            return []
        new = self._alloc_block()
        self._drop(blk)
        table.block_ids[i] = new
        return [(blk, new)] if table.num_tokens % self.block_size else []

    def truncate(self, seq_id: int, num_tokens: int) -> None:
        """Roll back to num_tokens tokens, releasing trailing blocks (spec rejection)."""
        table = self._tables[seq_id]
        keep = self.blocks_needed(num_tokens)
        for blk in table.block_ids[keep:]:
            self._drop(blk)
        table.block_ids = table.block_ids[:keep]
        table.num_tokens = num_tokens

    def free(self, seq_id: int) -> None:
        table = self._tables.pop(seq_id, None)
        if table is None:
            return
        for blk in table.block_ids:
            self._drop(blk)
