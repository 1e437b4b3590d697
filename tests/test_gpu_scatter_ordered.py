"""dsp_kv_scatter_ordered (the import scatter in destination-block order) against
dsp_kv_scatter (sequence order) through the C ABI (GPU).

Seeded random geometries: 1-5 layers, rows of 2 to 2048 bytes (every vector width of the
copy: 16, 8, 4, 2 and 1 byte), blocks of 4-32 tokens, 1-6 sequences whose lengths include
zero and partial last blocks, tables that name most of the pool (the ordered kernel) or
a small part of it (the library falls back to the sequence-order kernel), sometimes a
block id outside the pool.  Both pools must match byte for byte over their whole extent
(rows no table names untouched by both) and both error counts must agree.  A block named
by two table entries is written from the later entry alone (the header's rule), checked
against the reference's import_contiguous (paged_cache.py:92-96) run sequence by sequence
on every row the later entry covers.
"""

import random

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _geometry(seed):
    rng = random.Random(seed)
    row_bytes = rng.choice((2048, 512, 24, 8, 4, 2, 6, 1))
    bs = rng.choice((4, 8, 16, 32))
    L = rng.randint(1, 5)
    lens = [rng.choice((0, rng.randint(1, 4 * bs), rng.randint(1, 12 * bs))) for _ in range(rng.randint(1, 6))]
    need = sum(-(-t // bs) for t in lens)
    dense = rng.random() < 0.7
    NB = max(need, 1) + (rng.randint(0, need // 3 + 1) if dense else 3 * need + rng.randint(4, 40))
    return rng, row_bytes, bs, L, lens, NB


def _run(entry, pool_k, pool_v, L, NB, bs, row_bytes, table, cu, lens, kb, vb, owner):
    from dispec_amd import _lib
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    args = [pool_k.data_ptr(), pool_v.data_ptr(), L, NB * bs * row_bytes, NB, row_bytes, bs,
            table.data_ptr(), table.stride(0), cu.data_ptr(), len(lens), max(lens + [0]),
            kb.data_ptr(), vb.data_ptr()]
    if entry == "ordered":
        args.append(owner.data_ptr())
    args += [err.data_ptr(), _lib.stream_of(pool_k)]
    fn = _lib.lib().dsp_kv_scatter_ordered if entry == "ordered" else _lib.lib().dsp_kv_scatter
    assert fn(*args) == 0
    torch.cuda.synchronize()
    return int(err.item())


@pytest.mark.parametrize("seed", range(24))
def test_ordered_scatter_equals_sequence_order_scatter(seed):
    rng, row_bytes, bs, L, lens, NB = _geometry(seed)
    g = torch.Generator().manual_seed(900 + seed)
    need = [-(-t // bs) for t in lens]
    width = max(need + [1])
    perm = torch.randperm(NB, generator=g)[:sum(need)].tolist()
    table = np.zeros((len(lens), width), dtype=np.int32)
    it = iter(perm)
    for b, n in enumerate(need):
        for j in range(n):
            table[b, j] = next(it)
    bad = sum(need) > 0 and rng.random() < 0.3
    if bad:
        b = next(i for i, n in enumerate(need) if n)
        table[b, rng.randrange(need[b])] = NB + rng.randint(0, 5)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    rows = L * int(cu[-1])
    kb = torch.randint(0, 256, (max(rows, 1), row_bytes), generator=g, dtype=torch.uint8).to(DEV)
    vb = torch.randint(0, 256, (max(rows, 1), row_bytes), generator=g, dtype=torch.uint8).to(DEV)
    base_k = torch.randint(0, 256, (L, NB * bs, row_bytes), generator=g, dtype=torch.uint8)
    base_v = torch.randint(0, 256, (L, NB * bs, row_bytes), generator=g, dtype=torch.uint8)
    table_d = torch.from_numpy(table).to(DEV)
    cu_d = torch.from_numpy(cu).to(DEV)
    owner = torch.empty(NB, dtype=torch.int32, device=DEV)
    out = {}
    for entry in ("sequence", "ordered"):
        pk, pv = base_k.to(DEV), base_v.to(DEV)
        errs = _run(entry, pk, pv, L, NB, bs, row_bytes, table_d, cu_d, lens, kb, vb, owner)
        out[entry] = (pk.cpu(), pv.cpu(), errs)
    case = f"seed={seed} row_bytes={row_bytes} bs={bs} L={L} lens={lens} NB={NB} bad={bad}"
    assert torch.equal(out["ordered"][0], out["sequence"][0]), case
    assert torch.equal(out["ordered"][1], out["sequence"][1]), case
    assert out["ordered"][2] == out["sequence"][2] == int(bad), case
    if sum(lens):
        assert not torch.equal(out["ordered"][0], base_k), case   # something was written


def test_a_block_named_twice_takes_the_later_entry():
    """Two sequences whose tables share blocks (the tables name every block of a small
    pool, so the ordered kernel runs): a shared block ends with the later entry's rows --
    those of a sequential import -- and, past a partial later entry, with the rows the pool
    held; every other block with its own sequence's rows."""
    L, bs, row_bytes = 2, 16, 64
    lens = [3 * bs, 2 * bs + 5]
    NB = 4
    table = np.array([[0, 1, 2], [3, 1, 0]], dtype=np.int32)   # block 1 named by (0,1), (1,1)
    cu = np.array([0, lens[0], lens[0] + lens[1]], dtype=np.int64)
    g = torch.Generator().manual_seed(77)
    rows = L * int(cu[-1])
    kb = torch.randint(0, 256, (rows, row_bytes), generator=g, dtype=torch.uint8)
    vb = torch.randint(0, 256, (rows, row_bytes), generator=g, dtype=torch.uint8)
    pool = torch.randint(0, 256, (2, L, NB * bs, row_bytes), generator=g, dtype=torch.uint8)
    # sequential import, sequence by sequence (the later table entry wins)
    want = pool.clone()
    for b, T in enumerate(lens):
        for l in range(L):
            for t in range(T):
                slot = int(table[b, t // bs]) * bs + t % bs
                src = L * int(cu[b]) + l * T + t
                want[0, l, slot] = kb[src]
                want[1, l, slot] = vb[src]
    pk, pv = pool[0].clone().to(DEV), pool[1].clone().to(DEV)
    owner = torch.empty(NB, dtype=torch.int32, device=DEV)
    # block 0 is named by (0, 0) and by (1, 2), a row-partial last block: the later entry
    # writes its 5 rows and the other 11 keep the pool's (a sequential import would leave
    # the first sequence's there), so block 0 is compared on its own below
    errs = _run("ordered", pk, pv, L, NB, bs, row_bytes, torch.from_numpy(table).to(DEV),
                torch.from_numpy(cu).to(DEV), lens, kb.to(DEV), vb.to(DEV), owner)
    assert errs == 0
    got_k, got_v = pk.cpu(), pv.cpu()
    for blk in (1, 2, 3):
        sl = slice(blk * bs, (blk + 1) * bs)
        assert torch.equal(got_k[:, sl], want[0][:, sl]), blk
        assert torch.equal(got_v[:, sl], want[1][:, sl]), blk
    # block 0: the later entry's 5 rows over the untouched pool rows past them
    sl = slice(0, 5)
    assert torch.equal(got_k[:, sl], want[0][:, sl]) and torch.equal(got_v[:, sl], want[1][:, sl])
    rest = slice(5, bs)
    assert torch.equal(got_k[:, rest], pool[0][:, rest]) and torch.equal(got_v[:, rest], pool[1][:, rest])
