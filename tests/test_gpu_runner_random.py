"""ModelRunner(attn_backend="hip") under seeded random serving traffic against the oracle's
native forward (GPU).

Each step serves one batch drawn at random, as a continuous-batching scheduler would form
it: new sequences arriving with a prefill chunk of 5-100 tokens beside live sequences that
decode one token or verify five (speculative drafts), in any mix.  The runner routes each
batch itself, and the test records the routes its batches took and requires all four: the
decode kernel (all-decode batches), the balanced split (short query blocks over skewed
contexts), the 16-row multi-query tiles and the 128-row prefill tile (a chunk of >= 64
tokens: 128 packed rows at this model's 2 query heads per KV head).  Every row's logits
must match the oracle's float32 native forward on the same cache contents (cosine >= 0.999:
the reference backend test's bar, tests/test_triton_attn.py:63-97).
"""

import random

import pytest

from tests.test_gpu_model_runner import FAMILIES, _Both, _cos, _pair

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("family", sorted(FAMILIES))
def test_random_batches_match_the_native_forward(family):
    rng = random.Random(7000 + len(family))
    gpu_model, cpu_model = _pair(family)
    both = _Both(gpu_model, cpu_model, num_blocks=200)
    vocab = gpu_model.config.vocab_size
    G = both.runner.kv_groups
    routes, batch_of = set(), both.runner._batch

    def recorded(seq_meta, cache):
        b = batch_of(seq_meta, cache)
        routes.add("decode" if b.decode else "balanced" if b.balanced
                   else "prefill-tile" if b.max_q_len * G >= 128 else "multi-query")
        return b

    both.runner._batch = recorded
    lengths: dict[int, int] = {}
    next_sid, kinds = 0, set()
    for _ in range(20):
        rows = []
        if not lengths or rng.random() < 0.35:                 # arrivals
            for _ in range(rng.randint(1, 2)):
                n = rng.randint(5, 100)
                rows.append((next_sid, [rng.randrange(vocab) for _ in range(n)], 0))
                lengths[next_sid] = n
                next_sid += 1
                kinds.add("prefill")
        live = [s for s in sorted(lengths) if s not in {r[0] for r in rows}]
        for sid in rng.sample(live, k=min(len(live), rng.randint(1, 5))):
            q = rng.choice((1, 1, 5))
            rows.append((sid, [rng.randrange(vocab) for _ in range(q)], lengths[sid]))
            lengths[sid] += q
            kinds.add("decode" if q == 1 else "verify")
        rng.shuffle(rows)
        got, ref = both.forward(rows)
        cos = _cos(got, ref)
        assert float(cos.min()) >= 0.999, (family, [r[0] for r in rows], cos.min())
    assert kinds == {"prefill", "decode", "verify"}
    assert routes == {"decode", "balanced", "multi-query", "prefill-tile"}, routes
