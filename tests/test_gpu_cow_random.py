"""Seeded random operation sequences on a PagedKVCache on the GPU: the block manager's
copy-on-write pairs applied by the block-copy kernels, token rows written by the append
kernel, and every live sequence read back bit-exact.

The operations and the CPU model are tests/test_block_manager_random.py's; here each
token value also becomes K and V rows in the GPU pool (every layer, every KV head: bf16
bit patterns derived from the value, never NaN or Inf), written with `PagedKVCache.write`
(dsp_kv_append), and each copy pair the manager returns is moved with
`PagedKVCache.copy_blocks` (dsp_kv_copy_blocks, or dsp_kv_copy_block_fanout when one block
is forked into several children at once -- an operation added here).  Every few steps all
live sequences' context rows are gathered from the pool and compared with the rows their
token values give.
"""

import numpy as np
import pytest
import torch

from dispec_amd.kv.block_manager import OutOfBlocksError
from tests.test_block_manager_random import BS, NB, Shadow

pytestmark = pytest.mark.gpu
DEV = "cuda"
L, KVH, D = 2, 2, 8


def _rows(values, kind: int) -> torch.Tensor:
    """(len(values), L, KVH, D) bf16 rows of the given token values, as bit patterns below
    0x7f00 (finite)."""
    v = np.asarray(values, dtype=np.int64)[:, None, None, None]
    layer = np.arange(L)[None, :, None, None]
    head = np.arange(KVH)[None, None, :, None]
    dim = np.arange(D)[None, None, None, :]
    bits = (v * 2654435761 + layer * 40503 + head * 9973 + dim * 131 + kind * 7919) % 0x7f00
    return torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16)


class GpuShadow(Shadow):
    def __init__(self, seed: int):
        super().__init__(seed)
        from dispec_amd.kv.paged_cache import PagedKVCache
        self.fanouts = 0
        self.cache = PagedKVCache(L, NB, BS, KVH, D, dtype=torch.bfloat16, device=DEV)
        self.mgr = self.cache.manager
        self.pending: dict[int, int] = {}     # slot -> token value, not yet on the GPU

    def write(self, sid, pos, v):
        super().write(sid, pos, v)
        blk, off = self.mgr.block_table(sid).slot(BS, pos)
        self.pending[blk * BS + off] = v

    def flush(self):
        if not self.pending:
            return
        slots = torch.tensor(sorted(self.pending), dtype=torch.int64, device=DEV)
        vals = [self.pending[s] for s in sorted(self.pending)]
        k, v = _rows(vals, 0).to(DEV), _rows(vals, 1).to(DEV)
        for layer in range(L):
            self.cache.write(layer, slots, k[:, layer], v[:, layer])
        self.pending.clear()

    def copy(self, pairs):
        pairs = list(pairs)
        if pairs:
            self.flush()                      # the copies read what was written before
            self.cache.copy_blocks(pairs)
        super().copy(pairs)

    def op_fanout(self, sid):
        """Fork one parent into 2-4 children with cow_fork and move every copy in one call
        (the source block is the same for all: the fan-out kernel)."""
        pairs = []
        try:
            for _ in range(self.rng.randint(2, 4)):
                child = self.next_sid
                _, p = self.call(self.mgr.cow_fork, sid, child)
                self.next_sid += 1
                pairs += p
                self.expect[child] = list(self.expect[sid])
        finally:                              # children forked before a failure get theirs
            self.copy(pairs)
            self.fanouts += len(pairs) > 1

    def step(self):
        if self.expect and self.rng.random() < 0.08:
            try:
                self.op_fanout(self.rng.choice(sorted(self.expect)))
            except OutOfBlocksError:
                self.out_of_blocks += 1
            return "fanout"
        return super().step()

    def check_gpu(self):
        self.flush()
        torch.cuda.synchronize()
        self.cache.check_errors()
        for sid, toks in self.expect.items():
            if not toks:
                continue
            slots = self.cache.context_slots(self.mgr.block_table(sid).block_ids, len(toks))
            want_k, want_v = _rows(toks, 0), _rows(toks, 1)
            for layer in range(L):
                k, v = self.cache.gather(layer, slots)
                assert torch.equal(k.cpu().view(torch.int16), want_k[:, layer].view(torch.int16)), \
                    f"seq {sid} layer {layer}: K rows differ"
                assert torch.equal(v.cpu().view(torch.int16), want_v[:, layer].view(torch.int16)), \
                    f"seq {sid} layer {layer}: V rows differ"


@pytest.mark.parametrize("seed", range(3))
def test_random_copy_on_write_traffic_on_the_gpu(seed):
    sh = GpuShadow(100 + seed)
    for i in range(300):
        sh.step()
        sh.check()
        if i % 25 == 24:
            sh.check_gpu()
    sh.check_gpu()
    assert sh.shared_seen and sh.out_of_blocks > 0 and sh.fanouts > 0


class _SkipsGpuCopies(GpuShadow):
    def copy(self, pairs):
        Shadow.copy(self, pairs)              # the model copies, the pool does not


def test_a_skipped_block_copy_is_caught():
    sh = _SkipsGpuCopies(100)
    with pytest.raises(AssertionError, match="rows differ"):
        for i in range(300):
            sh.step()
            sh.check()
            if i % 25 == 24:
                sh.check_gpu()
        sh.check_gpu()
