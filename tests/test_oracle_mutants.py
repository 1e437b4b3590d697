"""The oracle's pins catch plausible slips (CPU only).

Each mutant below is the oracle module itself with one edit applied to its source text
-- the kind of slip a restatement can make: a query head served by the wrong KV head, a
dropped softmax scale, scores taken against V instead of K, a softmax normalised over
the wrong axis, a causal mask one key short, a slot computed from the wrong block index,
an append that writes its rows in the wrong order, a block copy run backwards, an export
that walks the block table backwards, a RoPE frequency or rotation sign wrong, a map's
design row in the wrong feature order, its bias or its residual's GELU dropped, the
attention prologue's norm weight left out or k normalised with q's weight, the bf16 map's
GEMM result not rounded before its bias, its keys mapped without stripping RoPE, its
values rotated.
The edited module is executed in a fresh namespace and run through the same kinds of
checks tests/test_oracle.py pins the real oracle with: torch's SDPA (with enable_gqa and
causal_lower_right), `index_copy_` and advanced indexing (the routines the reference path
calls), transformers' Qwen3 rotary and RMSNorm modules, the reference's known answers (slot math,
tests/test_block_manager.py:8-15; the map's feature order, tests/test_kv_transfer.py:89-100)
and hand-built ones (a block copy, a quarter-turn rotation).  Every mutant must fail at least one check, and the
unedited source must pass all of them, so the checks are shown to tell a right
restatement from a wrong one.
"""

import inspect
import types

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch.nn.attention.bias import causal_lower_right

from oracle import ref_cpu, ref_torch
from tests._util import gen

_SOURCE = inspect.getsource(ref_cpu)

# (name, text in the oracle's source, replacement, occurrences to edit)
MUTANTS = [
    ("kv head h % KVH instead of h // G",
     "np.repeat(np.asarray(k_cache[slots], dtype=np.float64), kv_groups, axis=1)",
     "np.tile(np.asarray(k_cache[slots], dtype=np.float64), (1, kv_groups, 1))", 2),
    ("decode scale dropped", "[:, :, 0] * scale  # (Hq, n)", "[:, :, 0]  # (Hq, n)", 1),
    ("decode scores against V", "np.matmul(k.transpose(1, 0, 2), q[b][:, :, None])",
     "np.matmul(v.transpose(1, 0, 2), q[b][:, :, None])", 1),
    ("decode softmax over the heads", "p /= p.sum(axis=1, keepdims=True)",
     "p /= p.sum(axis=0, keepdims=True)", 1),
    ("causal mask one key short", "<= np.arange(q_len)[:, None] + past",
     "< np.arange(q_len)[:, None] + past", 1),
    ("multi-query scale dropped", "k.transpose(1, 2, 0)) * scale",
     "k.transpose(1, 2, 0))", 1),
    ("slot from the position, not its block", "return bt[p // block_size] * block_size + p % block_size",
     "return bt[p % len(bt)] * block_size + p % block_size", 1),
    ("append rows in reverse order", "    pool_layer[slots] = rows\n",
     "    pool_layer[slots] = rows[::-1]\n", 1),
    ("block copy run backwards", "src_pool[:, s * block_size:(s + 1) * block_size]",
     "src_pool[:, d * block_size:(d + 1) * block_size]", 1),
    ("export walks the table backwards",
     "np.ascontiguousarray(pool[:, context_slots(block_ids, seq_len, block_size)])",
     "np.ascontiguousarray(pool[:, context_slots(block_ids[::-1], seq_len, block_size)])", 1),
    ("rope frequency exponent halved", ".astype(np.float32) / head_dim))",
     ".astype(np.float32) / (2 * head_dim)))", 1),
    ("rotate-half sign flipped", "np.concatenate([-x[..., h:], x[..., :h]], axis=-1)",
     "np.concatenate([x[..., h:], -x[..., :h]], axis=-1)", 1),
    ("design row dims before heads", "np.ascontiguousarray(sel.transpose(1, 0, 2, 3))",
     "np.ascontiguousarray(sel.transpose(1, 0, 3, 2))", 1),
    ("map bias dropped", "    y = y + np.asarray(bias, np.float64)\n", "    y = y\n", 1),
    ("residual GELU dropped", "y = y + _gelu(x @ down_w.T + down_b) @ up_w.T",
     "y = y + (x @ down_w.T + down_b) @ up_w.T", 1),
    ("norm weight left out",
     "return round_bf16(bf16_to_f32(w_bits) * round_bf16((x * inv).astype(np.float32)))",
     "return round_bf16(round_bf16((x * inv).astype(np.float32)))", 1),
    ("k normalised with q's weight", "rms_norm_bf16(k_bits, kw_bits, eps)",
     "rms_norm_bf16(k_bits, qw_bits, eps)", 1),
    ("map GEMM not rounded before the bias",
     'y = round_bf16((x @ np.asarray(m["weight"], np.float64)).astype(np.float32))',
     'y = (x @ np.asarray(m["weight"], np.float64)).astype(np.float32)', 1),
    ("keys mapped without stripping RoPE",
     "content = f32_to_bf16(strip_rope(bf16_to_f32(k_bits), *source_rope))",
     "content = np.asarray(k_bits, dtype=np.uint16)", 1),
    ("values rotated too", "run(vals, value_maps, None)", "run(vals, value_maps, target_rope)", 1),
]


def _module(source: str) -> types.ModuleType:
    mod = types.ModuleType("ref_cpu_variant")
    exec(compile(source, "ref_cpu_variant", "exec"), mod.__dict__)
    return mod


def _decode_agrees(m) -> bool:
    Hq, KVH, D, S = 14, 2, 32, 256
    q = torch.randn((3, Hq, D), generator=gen(70), dtype=torch.float64)
    kc = torch.randn((S, KVH, D), generator=gen(71), dtype=torch.float64)
    vc = torch.randn((S, KVH, D), generator=gen(72), dtype=torch.float64)
    lens = [1, 90, 41]
    st = torch.zeros((3, 90), dtype=torch.long)
    for i, n in enumerate(lens):
        st[i, :n] = torch.randperm(S, generator=gen(73 + i))[:n]
    ours = m.decode_attention(q.numpy(), kc.numpy(), vc.numpy(), st.numpy(), lens, Hq // KVH)
    for b, n in enumerate(lens):
        s = st[b, :n]
        lib = F.scaled_dot_product_attention(q[b][None, :, None], kc[s].transpose(0, 1)[None],
                                             vc[s].transpose(0, 1)[None], enable_gqa=True)
        if not np.allclose(ours[b], lib[0, :, 0].numpy(), atol=1e-10):
            return False
    return True


def _mq_agrees(m) -> bool:
    for q_len, ctx in ((5, 19), (3, 3), (1, 12)):
        g = gen(80 + q_len * 31 + ctx)
        q = torch.randn(1, 4, q_len, 16, generator=g, dtype=torch.float64)
        k = torch.randn(1, 2, ctx, 16, generator=g, dtype=torch.float64)
        v = torch.randn(1, 2, ctx, 16, generator=g, dtype=torch.float64)
        lib = F.scaled_dot_product_attention(q, k, v, attn_mask=causal_lower_right(q_len, ctx),
                                             enable_gqa=True)
        ours = m.mq_attention(q[0].permute(1, 0, 2).numpy(), k[0].permute(1, 0, 2).numpy(),
                              v[0].permute(1, 0, 2).numpy(), [np.arange(ctx)], [q_len], 2)
        if not np.allclose(ours, lib[0].permute(1, 0, 2).numpy(), atol=1e-10):
            return False
    return True


def _slots_agree(m) -> bool:
    # tests/test_block_manager.py:8-15: bs=4, token 0 -> (block 0, 0), token 5 -> (block 1, 1)
    ids = [7, 3, 9]
    return (int(m.slots_for_positions(ids, [0], 4)[0]) == 7 * 4 + 0 and
            int(m.slots_for_positions(ids, [5], 4)[0]) == 3 * 4 + 1 and
            int(m.slots_for_positions(ids, [10], 4)[0]) == 9 * 4 + 2)


def _u16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _byte_moves_agree(m) -> bool:
    key = torch.randn((3, 96, 2, 4), generator=gen(90)).to(torch.bfloat16)
    slots = torch.randperm(96, generator=gen(91))[:13]
    rows = torch.randn((13, 2, 4), generator=gen(92)).to(torch.bfloat16)
    ours = _u16(key).copy()
    m.append(ours[1], slots.numpy(), _u16(rows))
    theirs = key.clone()
    theirs[1].index_copy_(0, slots, rows)
    if not np.array_equal(ours, _u16(theirs)):
        return False
    ids, n = [5, 0, 2], 37
    tslots = ref_torch.context_slots(ids, n, 16)
    if not np.array_equal(m.export_contiguous(_u16(key), ids, n, 16), _u16(key[:, tslots])):
        return False
    # hand-built known answer: L = 2, 6 blocks of 2 slots, rows numbered in order
    pool = np.arange(2 * 6 * 2, dtype=np.uint16).reshape(2, 6 * 2, 1, 1)
    m.copy_blocks(pool, pool, [(0, 5), (3, 1)], 2)
    return (pool[0, 10:12].ravel().tolist() == [0, 1] and
            pool[1, 10:12].ravel().tolist() == [12, 13] and
            pool[0, 2:4].ravel().tolist() == [6, 7] and pool[0, 0:2].ravel().tolist() == [0, 1])


def _rope_agrees(m) -> bool:
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding
    cfg = Qwen3Config(hidden_size=64, num_attention_heads=4, num_key_value_heads=2,
                      head_dim=16, rope_theta=1e6, num_hidden_layers=1, vocab_size=16)
    pos = torch.arange(200)
    cos, sin = Qwen3RotaryEmbedding(cfg)(torch.zeros(1, 1), pos[None])
    ours_c, ours_s = m.rope_tables(pos.numpy(), 16, 1e6)
    if not (np.allclose(ours_c, cos[0].numpy(), atol=2e-6) and
            np.allclose(ours_s, sin[0].numpy(), atol=2e-6)):
        return False
    # a quarter turn maps the halves (x1, x2) to (-x2, x1)
    y = m.apply_rope(np.array([[[[1, 2, 3, 4]]]], np.float32), np.zeros((1, 4), np.float32),
                     np.ones((1, 4), np.float32))
    return y.ravel().tolist() == [-3, -4, 1, 2]


def _map_agrees(m) -> bool:
    g = np.random.default_rng(12)
    src = g.standard_normal((3, 5, 2, 4))
    x = m.design_rows(src, (2, 0))
    # tests/test_kv_transfer.py:89-100: a row is the source layers in map order, each
    # layer's heads then dims
    if not all(np.array_equal(x[t], np.concatenate([src[2, t].ravel(), src[0, t].ravel()]))
               for t in range(5)):
        return False
    W, b = g.standard_normal((16, 8)), g.standard_normal(8)
    down_w, down_b, up_w = g.standard_normal((3, 16)), g.standard_normal(3), g.standard_normal((8, 3))
    got = m.layer_map_apply(x, W, b, residual=(down_w, down_b, up_w))
    xt = torch.from_numpy(x)
    expect = F.linear(xt, torch.from_numpy(W).T, torch.from_numpy(b)) + F.linear(
        F.gelu(F.linear(xt, torch.from_numpy(down_w), torch.from_numpy(down_b))),
        torch.from_numpy(up_w))
    return np.allclose(got, expect.numpy())


def _prologue_agrees(m) -> bool:
    """transformers' Qwen3RMSNorm, the rotate-half RoPE and index_copy_ as torch bf16 ops
    (model_runner.py:142-148), elementwise within one bf16 ulp, >= 99.9 % identical."""
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm
    g = gen(60)
    T, Hq, KVH, D = 5, 4, 2, 64
    q = torch.randn((T, Hq, D), generator=g).to(torch.bfloat16)
    k = torch.randn((T, KVH, D), generator=g).to(torch.bfloat16)
    v = torch.randn((T, KVH, D), generator=g).to(torch.bfloat16)
    wq = (1 + 0.3 * torch.randn(D, generator=g)).to(torch.bfloat16)
    wk = (1 + 0.3 * torch.randn(D, generator=g)).to(torch.bfloat16)
    cos_f, sin_f = ref_cpu.rope_tables(np.arange(100, 100 + T), D, 1e6)
    cos, sin = torch.from_numpy(cos_f).to(torch.bfloat16), torch.from_numpy(sin_f).to(torch.bfloat16)
    qn, kn = Qwen3RMSNorm(D, eps=1e-6).to(torch.bfloat16), Qwen3RMSNorm(D, eps=1e-6).to(torch.bfloat16)
    qn.weight.data.copy_(wq)
    kn.weight.data.copy_(wk)

    def rope(x):
        x1, x2 = x.chunk(2, dim=-1)
        return x * cos.unsqueeze(1) + torch.cat((-x2, x1), dim=-1) * sin.unsqueeze(1)

    slots = torch.tensor([7, 0, 12, 3, 9])
    kpool = torch.randn((16, KVH, D), generator=gen(61)).to(torch.bfloat16)
    vpool = torch.randn((16, KVH, D), generator=gen(62)).to(torch.bfloat16)
    with torch.no_grad():
        tq, tk = rope(qn(q)), rope(kn(k))
        tkp = kpool.clone()
        tkp.index_copy_(0, slots, tk)
    ok, ov = _u16(kpool), _u16(vpool)
    oq = m.qk_norm_rope_append(_u16(q), _u16(k), _u16(v), _u16(wq), _u16(wk), 1e-6, _u16(cos),
                               _u16(sin), slots.numpy(), ok, ov)
    for got, want in ((oq, _u16(tq)), (ok, _u16(tkp))):
        err = np.abs(ref_cpu.bf16_to_f32(got) - ref_cpu.bf16_to_f32(want))
        ulp = np.abs(ref_cpu.bf16_to_f32(want)) * 2.0 ** -7 + 1e-30
        if float((got == want).mean()) < 0.999 or not (err <= ulp).all():
            return False
    return True


def _bf16_map_agrees(m) -> bool:
    g = gen(64)
    L, T, H, D = 3, 11, 2, 8
    k = torch.randn((L, T, H, D), generator=g).to(torch.bfloat16)
    v = torch.randn((L, T, H, D), generator=g).to(torch.bfloat16)
    # identity maps between models with the same RoPE: values come back bit for bit, keys
    # within the two roundings of strip -> bf16 -> apply (each element mixes with its
    # partner half a head away, so the bound scales with the larger of the two)
    cos, sin = ref_cpu.rope_tables(np.arange(40, 40 + T), D, 1e4)
    eye = {"weight": np.eye(H * D), "bias": np.zeros(H * D)}
    maps = [dict(eye, source_layers=(i,)) for i in range(L)]
    km, vm = m.cross_model_map_bf16(_u16(k), _u16(v), maps, maps, (cos, sin), (cos, sin))
    if not np.array_equal(vm, _u16(v)):
        return False
    kf = k.float().numpy()
    mag = np.maximum(np.abs(kf), np.abs(np.roll(kf, D // 2, axis=-1)))
    if not (np.abs(ref_cpu.bf16_to_f32(km) - kf) <= mag * 2.0 ** -6 + 1e-6).all():
        return False
    # a random bf16 map: exact GEMM rounded to bf16, then the bias added in bf16
    # (transfer.py:104-112 as torch bf16 ops)
    W = torch.randn((2 * H * D, H * D), generator=g).to(torch.bfloat16)
    b = torch.randn((H * D,), generator=g).to(torch.bfloat16)
    mm = [{"source_layers": (2, 0), "weight": W.float().numpy(), "bias": b.float().numpy()}]
    ones, zeros = np.ones((T, D), np.float32), np.zeros((T, D), np.float32)
    _, vm = m.cross_model_map_bf16(_u16(k), _u16(v), mm, mm, (ones, zeros), (ones, zeros))
    x = v[[2, 0]].permute(1, 0, 2, 3).reshape(T, -1)
    y = (x.double() @ W.double()).float().to(torch.bfloat16) + b
    return np.array_equal(vm[0], _u16(y.view(T, H, D)))


def _passes_all(m) -> bool:
    checks = (_decode_agrees, _mq_agrees, _slots_agree, _byte_moves_agree, _rope_agrees,
              _map_agrees, _prologue_agrees, _bf16_map_agrees)
    for check in checks:
        try:
            if not check(m):
                return False
        except (ValueError, IndexError):  # a mutant may also fail loudly
            return False
    return True


def test_unedited_oracle_passes_every_check():
    assert _passes_all(_module(_SOURCE))


@pytest.mark.parametrize("name,old,new,count", MUTANTS, ids=[m[0] for m in MUTANTS])
def test_each_slip_fails_a_check(name, old, new, count):
    assert _SOURCE.count(old) == count, f"the oracle's source no longer holds {old!r}"
    mutant = _module(_SOURCE.replace(old, new))
    assert not _passes_all(mutant), f"no check tells the oracle from its mutant: {name}"
