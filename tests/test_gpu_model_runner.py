"""ModelRunner(attn_backend="hip") end to end against the oracle's native forward.

Mirrors the reference's backend test (tests/test_triton_attn.py:63-97: per-step logits
cosine >= 0.999 against the native path over 30 decode steps crossing block boundaries)
and its prefill tests (tests/test_prefill_attention.py:72-101: chunked prefill equals
one prefill; a decode row mixed with a fresh prefill equals the separate runs).  The
model is a tiny random Qwen2/Qwen3 in bf16 on the GPU; the oracle runs the reference's
native torch path on the CPU in float32 with the same (bf16-rounded) weights.
"""

import copy

import pytest
import torch

from oracle import ref_torch
from tests.toy_lm import toy_lm

pytestmark = pytest.mark.gpu
DEV = "cuda"
FAMILIES = ("qwen3", "qwen2")


def _pair(family, dtype=torch.bfloat16):
    base = toy_lm(family).to(dtype)
    ref = copy.deepcopy(base).float()          # same rounded weights, fp32 math
    return base.to(DEV), ref


class _Both:
    """Drive the HIP runner and the CPU oracle through identical cache operations."""

    def __init__(self, gpu_model, cpu_model, num_blocks=64, bs=16, dtype=torch.bfloat16,
                 backend="hip", fuse=False):
        from dispec_amd.engine.model_runner import ModelRunner
        from dispec_amd.kv.paged_cache import PagedKVCache
        self.runner = ModelRunner(gpu_model, attn_backend=backend, fuse=fuse)
        self.cache = PagedKVCache.for_model(gpu_model.config, num_blocks, bs, dtype, DEV)
        cfg = cpu_model.config
        shape = (cfg.num_hidden_layers, num_blocks * bs, cfg.num_key_value_heads, cfg.head_dim)
        self.key, self.value = torch.zeros(shape), torch.zeros(shape)
        self.cpu_model, self.bs = cpu_model, bs

    def forward(self, rows):
        """rows: (seq_id, token_ids, start_pos); returns (hip logits, oracle logits)."""
        from dispec_amd.engine.model_runner import SeqMeta
        mgr = self.cache.manager
        tokens, positions, slots, meta, omet = [], [], [], [], []
        for sid, ids, start in rows:
            if not mgr.has_table(sid):
                mgr.allocate(sid, start + len(ids))
            else:
                for _ in ids:
                    mgr.append_token(sid)
            table = mgr.block_table(sid)
            table.num_tokens = start + len(ids)
            pos = list(range(start, start + len(ids)))
            tokens += ids
            positions += pos
            slots += [table.block_ids[p // self.bs] * self.bs + p % self.bs for p in pos]
            meta.append(SeqMeta(list(table.block_ids), len(ids), start + len(ids)))
            omet.append((list(table.block_ids), len(ids), start + len(ids)))
        t, p, s = torch.tensor(tokens), torch.tensor(positions), torch.tensor(slots)
        h = self.runner.forward(t.to(DEV), p.to(DEV), s.to(DEV), meta, self.cache)
        got = self.runner.logits(h).float().cpu()
        hr = ref_torch.native_forward(self.cpu_model, t, p, s, omet, self.key, self.value, self.bs)
        self.cache.check_errors()
        return got, self.cpu_model.lm_head(hr).float()


def _cos(a, b):
    return torch.nn.functional.cosine_similarity(a, b, dim=-1)


@pytest.mark.parametrize("family", sorted(FAMILIES))
def test_prefill_then_decode_matches_native(family):
    gm, cm = _pair(family)
    both = _Both(gm, cm)
    ids = torch.randint(0, 128, (37,), generator=torch.Generator().manual_seed(6)).tolist()
    got, ref = both.forward([(1, ids, 0)])
    assert _cos(got, ref).min() >= 0.999
    nxt, cur = int(ref[-1].argmax()), len(ids)
    for step in range(30):                                  # crosses two block boundaries
        got, ref = both.forward([(1, [nxt], cur)])
        c = _cos(got[0], ref[0]).item()
        assert c >= 0.999, f"step {step}, ctx {cur + 1}: cosine {c:.5f}"
        nxt, cur = int(ref[0].argmax()), cur + 1


@pytest.mark.parametrize("family", sorted(FAMILIES))
def test_fp32_model_end_to_end(family):
    """An fp32 model on the HIP path: the fp32 prologue and the generic attention kernel
    (the MFMA kernels serve bf16 / fp16), against the oracle's fp32 native forward --
    prefill, 20 decode steps and a chunked continuation; logits cosine >= 0.99999."""
    gm, cm = _pair(family, torch.float32)
    both = _Both(gm, cm, dtype=torch.float32)
    assert not both.runner._tuned_attention
    ids = torch.randint(0, 128, (37,), generator=torch.Generator().manual_seed(16)).tolist()
    got, ref = both.forward([(1, ids, 0)])
    assert _cos(got, ref).min() >= 0.99999
    nxt, cur = int(ref[-1].argmax()), len(ids)
    for step in range(20):
        got, ref = both.forward([(1, [nxt], cur)])
        c = _cos(got[0], ref[0]).item()
        assert c >= 0.99999, f"fp32 step {step}: cosine {c:.7f}"
        nxt, cur = int(ref[0].argmax()), cur + 1
    more = torch.randint(0, 128, (9,), generator=torch.Generator().manual_seed(17)).tolist()
    got, ref = both.forward([(1, more, cur)])
    assert _cos(got, ref).min() >= 0.99999


@pytest.mark.parametrize("family", sorted(FAMILIES))
def test_chunked_prefill_and_mixed_batch(family):
    gm, cm = _pair(family)
    both = _Both(gm, cm)
    a = torch.randint(0, 128, (40,), generator=torch.Generator().manual_seed(1)).tolist()
    b = torch.randint(0, 128, (13,), generator=torch.Generator().manual_seed(2)).tolist()
    got, ref = both.forward([(1, a[:17], 0)])
    assert _cos(got, ref).min() >= 0.999
    got, ref = both.forward([(1, a[17:], 17)])                # q_len 23 over 40 of context
    assert _cos(got, ref).min() >= 0.999
    got, ref = both.forward([(1, [a[-1]], 40), (2, b, 0)])    # decode row + fresh prefill
    assert _cos(got, ref).min() >= 0.999


def test_batched_decode_many_sequences():
    gm, cm = _pair("qwen3")
    both = _Both(gm, cm, num_blocks=128)
    g = torch.Generator().manual_seed(9)
    lens = [5, 16, 33, 70, 1]
    prompts = [torch.randint(0, 128, (n,), generator=g).tolist() for n in lens]
    for sid, p in enumerate(prompts):
        both.forward([(sid, p, 0)])
    cur = list(lens)
    toks = [p[-1] for p in prompts]
    for _ in range(20):
        got, ref = both.forward([(sid, [toks[sid]], cur[sid]) for sid in range(len(lens))])
        assert _cos(got, ref).min() >= 0.999
        toks = ref.argmax(-1).tolist()
        cur = [c + 1 for c in cur]


def test_verify_of_forked_sequences_uses_the_shared_prefix():
    """Speculative verify after copy-on-write forks of one 640-token prompt (40 shared
    blocks, block_manager.py:119-126): the runner finds the shared blocks and attends them
    once for the batch (dsp_paged_mq_attention_shared_prefix); logits match the native
    path sequence by sequence."""
    from dispec_amd.engine.model_runner import SeqMeta
    gm, cm = _pair("qwen3")
    both = _Both(gm, cm, num_blocks=96)
    g = torch.Generator().manual_seed(12)
    prompt = torch.randint(0, 128, (640,), generator=g).tolist()
    both.forward([(0, prompt, 0)])
    for child in range(1, 5):
        _, copies = both.cache.manager.cow_fork(0, child)
        assert copies == []                      # block-aligned prompt: every block shared
    drafts = [torch.randint(0, 128, (5,), generator=g).tolist() for _ in range(5)]
    got, ref = both.forward([(sid, drafts[sid], 640) for sid in range(5)])
    assert _cos(got, ref).min() >= 0.999
    mgr = both.cache.manager
    meta = [SeqMeta(list(mgr.block_table(s).block_ids), 5, 645) for s in range(5)]
    assert both.runner._batch(meta, both.cache).shared_prefix == 640


def test_decode_of_forked_sequences_uses_the_shared_prefix():
    """Decode steps of five copy-on-write forks of one 640-token prompt: each step is a
    q_len 1 batch whose 40 leading blocks are shared, which the runner attends once for the
    batch instead of the per-sequence decode kernel.  Twenty steps cross a block boundary
    of the private suffixes; logits match the native path at every step."""
    from dispec_amd.engine.model_runner import SeqMeta
    gm, cm = _pair("qwen3")
    both = _Both(gm, cm, num_blocks=96)
    g = torch.Generator().manual_seed(13)
    prompt = torch.randint(0, 128, (640,), generator=g).tolist()
    got, ref = both.forward([(0, prompt, 0)])
    for child in range(1, 5):
        both.cache.manager.cow_fork(0, child)
    toks = torch.randint(0, 128, (5,), generator=g).tolist()   # diverging first tokens
    cur = 640
    mgr = both.cache.manager
    for step in range(20):
        got, ref = both.forward([(sid, [toks[sid]], cur) for sid in range(5)])
        c = _cos(got, ref).min().item()
        assert c >= 0.999, f"step {step}, ctx {cur + 1}: cosine {c:.5f}"
        meta = [SeqMeta(list(mgr.block_table(s).block_ids), 1, cur + 1) for s in range(5)]
        batch = both.runner._batch(meta, both.cache)
        assert batch.decode and batch.shared_prefix == 640
        toks = ref.argmax(-1).tolist()
        cur += 1


@pytest.mark.parametrize("family", sorted(FAMILIES))
def test_verify_of_skewed_sequences_uses_the_balanced_split(family):
    """A 5-token verify over sequences of 600, 20, 45 and 9 tokens (independent prompts,
    no shared blocks): the runner picks the balanced split-K kernel (its keys per resident
    workgroup are far below the fixed split's partition) and the logits match the native
    path sequence by sequence."""
    from dispec_amd.engine.model_runner import SeqMeta
    gm, cm = _pair(family)
    both = _Both(gm, cm, num_blocks=96)
    g = torch.Generator().manual_seed(14)
    lens = [600, 20, 45, 9]
    for sid, n in enumerate(lens):
        both.forward([(sid, torch.randint(0, 128, (n,), generator=g).tolist(), 0)])
    drafts = [torch.randint(0, 128, (5,), generator=g).tolist() for _ in lens]
    got, ref = both.forward([(sid, drafts[sid], n) for sid, n in enumerate(lens)])
    assert _cos(got, ref).min() >= 0.999
    mgr = both.cache.manager
    meta = [SeqMeta(list(mgr.block_table(s).block_ids), 5, n + 5) for s, n in enumerate(lens)]
    batch = both.runner._batch(meta, both.cache)
    assert batch.balanced and not batch.shared_prefix and not batch.decode


@pytest.mark.parametrize("backend,fuse", [("native", False), ("native", True), ("hip", True)])
@pytest.mark.parametrize("family", sorted(FAMILIES))
def test_other_backend_and_fused_projections(family, backend, fuse):
    """attn_backend="native" (the reference's per-sequence torch SDPA over the gathered
    context, kept as a peer of "hip") and fuse=True (one GEMM for q/k/v and one for
    gate/up, model_runner.py:93-118) against the oracle's native forward: a prefill, 12
    decode steps across a block boundary, and a decode row beside a fresh prefill."""
    gm, cm = _pair(family)
    both = _Both(gm, cm, backend=backend, fuse=fuse)
    assert both.runner.fused == fuse and both.runner.attn_backend == backend
    ids = torch.randint(0, 128, (27,), generator=torch.Generator().manual_seed(18)).tolist()
    got, ref = both.forward([(1, ids, 0)])
    assert _cos(got, ref).min() >= 0.999
    nxt, cur = int(ref[-1].argmax()), len(ids)
    for step in range(12):
        got, ref = both.forward([(1, [nxt], cur)])
        c = _cos(got[0], ref[0]).item()
        assert c >= 0.999, f"{backend} fuse={fuse} step {step}: cosine {c:.5f}"
        nxt, cur = int(ref[0].argmax()), cur + 1
    b = torch.randint(0, 128, (11,), generator=torch.Generator().manual_seed(19)).tolist()
    got, ref = both.forward([(1, [nxt], cur), (2, b, 0)])
    assert _cos(got, ref).min() >= 0.999
