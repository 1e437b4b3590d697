"""Host-side detection of a shared prefix in ModelRunner (no GPU): the leading blocks that
every sequence's table holds and every query sees, rounded down to a multiple of 128
tokens, and the cases where the shared-prefix kernels are not used."""

from types import SimpleNamespace

import torch

from dispec_amd.engine.model_runner import ModelRunner, SeqMeta


def _runner(head_dim=128):
    return SimpleNamespace(shared_prefix_min_seqs=4, shared_prefix_min_tokens=512,
                           head_dim=head_dim, _tuned_attention=True)


def _detect(tables, q_lens, ctx, bs=16, head_dim=128):
    meta = [SeqMeta(t, q, c) for t, q, c in zip(tables, q_lens, ctx)]
    width = max(len(t) for t in tables)
    table = torch.zeros((len(tables), width), dtype=torch.int32)
    for i, t in enumerate(tables):
        table[i, :len(t)] = torch.tensor(t)
    return ModelRunner._shared_prefix(_runner(head_dim), meta, table, bs)


def _forks(n_seq, shared_blocks, own_blocks):
    shared = list(range(shared_blocks))
    return [shared + list(range(1000 + 10 * s, 1000 + 10 * s + own_blocks)) for s in range(n_seq)]


def test_forks_of_one_prompt():
    # config 4: 2050-token prompt, 128 full blocks shared, private partial block
    tables = _forks(8, 128, 3)
    assert _detect(tables, [5] * 8, [2050 + 40 + 5] * 8) == 2048
    # their decode steps (q_len 1) as well
    assert _detect(tables, [1] * 8, [2050 + 41] * 8) == 2048


def test_rounded_down_to_128_and_limited_by_the_queries():
    tables = _forks(4, 40, 2)                                  # 640 shared tokens
    assert _detect(tables, [5] * 4, [680] * 4) == 640
    # a long query block that starts inside the shared blocks limits what all rows see:
    # 900 - 300 = 600 tokens = 37 full blocks -> 592 -> 512
    tables = _forks(4, 50, 8)
    assert _detect(tables, [5, 5, 300, 5], [900] * 4) == 512
    tables = _forks(4, 38, 2)                                  # 608 shared -> 512
    assert _detect(tables, [5] * 4, [640] * 4) == 512


def test_not_used():
    tables = _forks(3, 128, 2)                                 # too few sequences
    assert _detect(tables, [5] * 3, [2100] * 3) == 0
    tables = _forks(6, 20, 2)                                  # 320 tokens: too short
    assert _detect(tables, [5] * 6, [350] * 6) == 0
    tables = _forks(6, 128, 2)
    tables[3][0] = 999                                         # first block differs
    assert _detect(tables, [5] * 6, [2100] * 6) == 0
    tables = _forks(6, 128, 2)
    tables[2][50] = 999                                        # diverges after 50 blocks
    assert _detect(tables, [5] * 6, [2100] * 6) == 768         # 50 blocks = 800 tokens
    assert _detect(_forks(6, 128, 2), [5] * 6, [2100] * 6, head_dim=32) == 0


def test_fp32_models_do_not_take_the_shared_prefix():
    """The shared-prefix kernel serves bf16 / fp16; an fp32 runner attends per sequence."""
    tables = [list(range(130)) + [200 + i] for i in range(8)]
    meta = [SeqMeta(t, 5, 2050 + 40 + 5) for t in tables]
    table = torch.tensor(tables, dtype=torch.int32)
    r = _runner()
    r._tuned_attention = False
    assert ModelRunner._shared_prefix(r, meta, table, 16) == 0
