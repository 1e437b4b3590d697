"""HipGraphDecoder: graph replays against the eager ModelRunner, step by step.

Mirrors the reference's graph tests (tests/test_cuda_graph.py:16-55,
tests/test_qwen3.py:132-156): teacher-forced decode over 40 steps that cross 16-token
block boundaries, each step's graph logits compared with the eager path's.  Here the
graph body IS the eager forward, so with the same block-table width (the split-K grid
depends on it) a replay must equal an eager forward bit for bit; against the eager
forward at its own width, and against the float32 CPU oracle, the bar is the
reference's cosine >= 0.999.  Every replay is followed by eager work and a host sync
before the next replay, and every replay is checked.

Two caches hold identical contents: the graph writes one, the eager runner the other,
both with the same new rows in the same slots.
"""

import copy

import pytest
import torch

from oracle import ref_torch
from tests.toy_lm import toy_lm

pytestmark = pytest.mark.gpu
DEV = "cuda"
BS = 16
BLOCKS_PER_SEQ = 8          # 128 tokens per sequence


def _setup(family="qwen3", num_seqs=4):
    from dispec_amd.engine.model_runner import ModelRunner
    from dispec_amd.kv.paged_cache import PagedKVCache
    base = toy_lm(family).to(torch.bfloat16)
    cpu = copy.deepcopy(base).float()
    gm = base.to(DEV)
    runner = ModelRunner(gm, attn_backend="hip")
    nblk = num_seqs * BLOCKS_PER_SEQ + 3
    caches = [PagedKVCache.for_model(gm.config, nblk, BS, torch.bfloat16, DEV) for _ in range(2)]
    # sequence s owns blocks in a scrambled order, so block ids are not positions
    perm = torch.randperm(nblk, generator=torch.Generator().manual_seed(3)).tolist()
    tables = [perm[s * BLOCKS_PER_SEQ:(s + 1) * BLOCKS_PER_SEQ] for s in range(num_seqs)]
    return runner, caches, tables, cpu


def _slot(table, pos):
    return table[pos // BS] * BS + pos % BS


def _prefill(runner, caches, tables, prompts):
    from dispec_amd.engine.model_runner import SeqMeta
    toks, pos, slots, meta = [], [], [], []
    for t, p in zip(tables, prompts):
        toks += p
        pos += list(range(len(p)))
        slots += [_slot(t, i) for i in range(len(p))]
        meta.append(SeqMeta(t, len(p), len(p)))
    args = [torch.tensor(x, device=DEV) for x in (toks, pos, slots)]
    for c in caches:
        runner.forward(*args, meta, c)


def _eager(runner, cache, toks, cur, tables, width=None):
    """One eager decode step; `width` pins the block-table width (and so the split-K grid)."""
    from dispec_amd.engine.model_runner import SeqMeta
    meta = [SeqMeta(t[:width] if width else t, 1, c + 1) for t, c in zip(tables, cur)]
    h = runner.forward(torch.tensor(toks, device=DEV), torch.tensor(cur, device=DEV),
                       torch.tensor([_slot(t, c) for t, c in zip(tables, cur)], device=DEV),
                       meta, cache)
    return runner.logits(h)


@pytest.mark.parametrize("family", ["qwen3", "qwen2"])
def test_batched_replays_equal_eager_bitwise(family):
    from dispec_amd.engine.hip_graph import HipGraphDecoder
    from dispec_amd.engine.model_runner import SeqMeta
    runner, (cg, ce), tables, _ = _setup(family, num_seqs=3)
    g = torch.Generator().manual_seed(11)
    lens = [5, 30, 47]
    prompts = [torch.randint(0, 128, (n,), generator=g).tolist() for n in lens]
    _prefill(runner, (cg, ce), tables, prompts)
    graph = HipGraphDecoder(runner, cg, buckets=(32, 64, 128))
    toks, cur = [p[-1] for p in prompts], list(lens)
    seen = set()
    for step in range(40):                       # max ctx 48 -> 87: buckets 64 then 128
        meta = [SeqMeta(t, 1, c + 1) for t, c in zip(tables, cur)]
        glog = graph.decode_batch(toks, cur, [_slot(t, c) for t, c in zip(tables, cur)], meta)
        glog = glog.float().cpu()
        bucket = graph._bucket(max(cur) + 1)
        seen.add(bucket)
        elog = _eager(runner, ce, toks, cur, tables, width=bucket // BS).float().cpu()
        assert torch.equal(glog, elog), f"step {step}, bucket {bucket}: replay != eager"
        toks, cur = elog.argmax(-1).tolist(), [c + 1 for c in cur]
    assert seen == {64, 128}
    assert torch.equal(cg.key, ce.key) and torch.equal(cg.value, ce.value)
    cg.check_errors()
    ce.check_errors()


def test_reference_signature_batch1_against_eager_and_oracle():
    """decode(token, position, write_slot, ctx_slots) as the reference's test drives it:
    ctx_slots from cache.context_slots on the device, 40 steps over block boundaries."""
    from dispec_amd.engine.hip_graph import HipGraphDecoder
    runner, (cg, ce), tables, cpu = _setup("qwen3", num_seqs=1)
    table = tables[0]
    ids = torch.randint(0, 128, (9,), generator=torch.Generator().manual_seed(5)).tolist()
    _prefill(runner, (cg, ce), tables, [ids])
    graph = HipGraphDecoder(runner, cg, buckets=(64,))
    graph.capture()                              # with live data in the cache
    cfg = cpu.config
    shape = (cfg.num_hidden_layers, cg.num_slots, cfg.num_key_value_heads, cfg.head_dim)
    okey, oval = torch.zeros(shape), torch.zeros(shape)
    n = len(ids)
    ref_torch.native_forward(cpu, torch.tensor(ids), torch.arange(n),
                             torch.tensor([_slot(table, i) for i in range(n)]),
                             [(table, n, n)], okey, oval, BS)
    nxt, cur = ids[-1], n
    for step in range(40):
        cslots = cg.context_slots(table, cur + 1)
        glog = graph.decode(nxt, cur, _slot(table, cur), cslots).float().cpu()[0]
        elog = _eager(runner, ce, [nxt], [cur], [table], width=64 // BS).float().cpu()[0]
        assert torch.equal(glog, elog), f"step {step}: replay != eager"
        h = ref_torch.native_forward(cpu, torch.tensor([nxt]), torch.tensor([cur]),
                                     torch.tensor([_slot(table, cur)]),
                                     [(table, 1, cur + 1)], okey, oval, BS)
        olog = cpu.lm_head(h)[0].float()
        c = torch.nn.functional.cosine_similarity(glog, olog, dim=0).item()
        assert c >= 0.999, f"step {step}, ctx {cur + 1}: cosine {c:.5f} vs oracle"
        nxt, cur = int(elog.argmax()), cur + 1
    cg.check_errors()


def test_device_tokens_and_default_width_eager():
    """Greedy decode fed by the previous replay's device argmax (no host read of the
    token), against the eager runner at its own block-table width."""
    from dispec_amd.engine.hip_graph import HipGraphDecoder
    from dispec_amd.engine.model_runner import SeqMeta
    runner, (cg, ce), tables, _ = _setup("qwen3", num_seqs=4)
    g = torch.Generator().manual_seed(21)
    lens = [3, 17, 16, 40]
    prompts = [torch.randint(0, 128, (n,), generator=g).tolist() for n in lens]
    _prefill(runner, (cg, ce), tables, prompts)
    graph = HipGraphDecoder(runner, cg, buckets=(128,))
    tok_dev = torch.tensor([p[-1] for p in prompts], device=DEV)
    toks, cur = [p[-1] for p in prompts], list(lens)
    for step in range(24):
        meta = [SeqMeta(t, 1, c + 1) for t, c in zip(tables, cur)]
        pos_dev = torch.tensor(cur, device=DEV)
        glog = graph.decode_batch(tok_dev, pos_dev, [_slot(t, c) for t, c in zip(tables, cur)],
                                  meta)
        tok_dev = glog.argmax(-1)                # stays on the device
        elog = _eager(runner, ce, toks, cur, tables).float().cpu()
        c = torch.nn.functional.cosine_similarity(glog.float().cpu(), elog, dim=-1).min().item()
        assert c >= 0.999, f"step {step}: cosine {c:.5f}"
        got = tok_dev.cpu().tolist()
        want = elog.argmax(-1).tolist()
        if got != want:                          # a bf16 near-tie: continue both on eager's
            tok_dev = torch.tensor(want, device=DEV)
        toks, cur = want, [c + 1 for c in cur]
    torch.testing.assert_close(cg.key, ce.key, rtol=2e-2, atol=5e-2)


def test_capture_leaves_live_cache_untouched():
    from dispec_amd.engine.hip_graph import HipGraphDecoder
    runner, (cg, _), tables, _ = _setup("qwen3", num_seqs=2)
    _prefill(runner, (cg,), tables, [[1, 2, 3, 4, 5], list(range(20, 60))])
    k0, v0 = cg.key.clone(), cg.value.clone()
    graph = HipGraphDecoder(runner, cg, buckets=(32, 128))
    graph.capture(batch_sizes=(1, 2))
    torch.cuda.synchronize()
    assert torch.equal(cg.key, k0) and torch.equal(cg.value, v0)
    cg.check_errors()                            # warm-up's skipped rows were not kept
    assert sorted(graph._g) == [(1, 32), (1, 128), (2, 32), (2, 128)]


def test_rejects_prefill_rows_and_long_contexts():
    from dispec_amd.engine.hip_graph import HipGraphDecoder
    from dispec_amd.engine.model_runner import SeqMeta
    runner, (cg, _), tables, _ = _setup("qwen3", num_seqs=1)
    graph = HipGraphDecoder(runner, cg, buckets=(32,))
    assert graph.can_handle(32) and not graph.can_handle(33)
    with pytest.raises(ValueError, match="decode only"):
        graph.decode_batch([1, 2], [0, 1], [0, 1], [SeqMeta(tables[0], 2, 2)])
    with pytest.raises(ValueError, match="largest bucket"):
        graph.decode_batch([1], [40], [_slot(tables[0], 40)], [SeqMeta(tables[0], 1, 41)])
    with pytest.raises(ValueError, match="blocks"):
        graph.decode_batch([1], [40], [0], [SeqMeta(tables[0][:1], 1, 20)])


def test_random_subsets_and_batch_sizes_replay_equal_eager_bitwise():
    """Each step a random subset of 6 sequences decodes (batch sizes 1-6 in any order, so
    graphs are captured on demand and replayed out of order across sizes and context
    buckets); every replay equals the eager forward at the same width bit for bit, and the
    two caches stay identical."""
    import random

    from dispec_amd.engine.hip_graph import HipGraphDecoder
    from dispec_amd.engine.model_runner import SeqMeta
    runner, (cg, ce), tables, _ = _setup("qwen3", num_seqs=6)
    rng = random.Random(21)
    g = torch.Generator().manual_seed(22)
    lens = [rng.randint(3, 60) for _ in range(6)]
    prompts = [torch.randint(0, 128, (n,), generator=g).tolist() for n in lens]
    _prefill(runner, (cg, ce), tables, prompts)
    graph = HipGraphDecoder(runner, cg, buckets=(32, 64, 128))
    nxt, cur = [p[-1] for p in prompts], list(lens)
    sizes, buckets = set(), set()
    for step in range(45):
        live = [s for s in range(6) if cur[s] + 1 <= BLOCKS_PER_SEQ * BS]
        pick = sorted(rng.sample(live, k=rng.randint(1, len(live))))
        toks = [nxt[s] for s in pick]
        pos = [cur[s] for s in pick]
        tabs = [tables[s] for s in pick]
        meta = [SeqMeta(t, 1, c + 1) for t, c in zip(tabs, pos)]
        glog = graph.decode_batch(toks, pos, [_slot(t, c) for t, c in zip(tabs, pos)], meta)
        glog = glog.float().cpu()
        bucket = graph._bucket(max(pos) + 1)
        elog = _eager(runner, ce, toks, pos, tabs, width=bucket // BS).float().cpu()
        assert torch.equal(glog, elog), f"step {step}, batch {pick}, bucket {bucket}"
        sizes.add(len(pick))
        buckets.add(bucket)
        for s, t in zip(pick, elog.argmax(-1).tolist()):
            nxt[s], cur[s] = t, cur[s] + 1
    assert len(sizes) >= 5 and len(buckets) >= 2, (sizes, buckets)
    torch.cuda.synchronize()
    assert torch.equal(cg.key, ce.key) and torch.equal(cg.value, ce.value)
    cg.check_errors()
    ce.check_errors()
