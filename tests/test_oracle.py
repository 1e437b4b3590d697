"""Pins the CPU oracle before anything is checked against it (CPU only).

Each oracle function is checked against something other than its own formula: torch
library routines the reference itself calls (index_copy_, advanced indexing, index_put,
SDPA with enable_gqa / causal_lower_right), known answers from the reference's tests,
closed forms, and brute force on tiny inputs.  A plausible slip in the oracle -- a wrong
head mapping, a dropped scale, a transposed operand, a shifted causal mask -- fails at
least one test here.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch.nn.attention.bias import causal_lower_right

from oracle import ref_cpu, ref_torch
from tests._util import gen


# ---------------------------------------------------------------------- bf16 helpers
def test_bf16_rounding_matches_torch():
    x = torch.cat([torch.randn(100_000, generator=gen(1)) * 10,
                   torch.tensor([0.0, -0.0, 1e-40, 3.0e38, float("inf"), -float("inf"),
                                 1.00390625, 1.01171875, 65504.0])])  # incl. ties
    ours = ref_cpu.f32_to_bf16(x.numpy())
    theirs = x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    back = ref_cpu.bf16_to_f32(theirs)
    assert np.array_equal(back, x.to(torch.bfloat16).float().numpy())
    assert np.isnan(ref_cpu.bf16_to_f32(ref_cpu.f32_to_bf16(np.array([np.nan], np.float32))))


# ------------------------------------------------------------------------ slot math
def test_slot_math_known_answers():
    # tests/test_block_manager.py:8-15: bs=4, token 0 -> (block0, 0), token 5 -> (block1, 1)
    ids = [7, 3]
    assert ref_cpu.slots_for_positions(ids, [0], 4)[0] == 7 * 4 + 0
    assert ref_cpu.slots_for_positions(ids, [5], 4)[0] == 3 * 4 + 1
    # brute force walk of a block table
    ids = [9, 0, 4, 2]
    walk = [b * 16 + o for b in ids for o in range(16)][:50]
    assert ref_cpu.context_slots(ids, 50, 16).tolist() == walk
    assert ref_torch.context_slots(ids, 50, 16).tolist() == walk


# ------------------------------------------------------------------------ byte moves
def _pool(L, S, H, D, seed):
    return torch.randn((L, S, H, D), generator=gen(seed)).to(torch.bfloat16)


def _u16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_append_matches_index_copy_and_leaves_other_rows():
    key = _pool(2, 64, 2, 8, 1)
    slots = torch.randperm(64, generator=gen(2))[:11]
    k = torch.randn((11, 2, 8), generator=gen(3)).to(torch.bfloat16)
    ours = _u16(key).copy()
    ref_cpu.append(ours[1], slots.numpy(), _u16(k))
    theirs = key.clone()
    theirs[1].index_copy_(0, slots, k)
    assert np.array_equal(ours, _u16(theirs))
    untouched = np.setdiff1d(np.arange(64), slots.numpy())
    assert np.array_equal(ours[1][untouched], _u16(key)[1][untouched])
    assert np.array_equal(ours[0], _u16(key)[0])
    with pytest.raises(IndexError):
        ref_cpu.append(ours[0], [64], _u16(k)[:1])


def test_gather_export_import_match_torch_indexing():
    key = _pool(3, 80, 2, 4, 4)
    ids, n = [4, 0, 2], 37
    slots = ref_torch.context_slots(ids, n, 16)
    assert np.array_equal(ref_cpu.gather(_u16(key)[2], slots.numpy()), _u16(key[2][slots]))
    exp = ref_cpu.export_contiguous(_u16(key), ids, n, 16)
    assert exp.shape == (3, n, 2, 4)
    assert np.array_equal(exp, _u16(key[:, slots].contiguous()))
    # import == index_put, and export(import(x)) == x
    x = torch.randn((3, n, 2, 4), generator=gen(5)).to(torch.bfloat16)
    ours = _u16(key).copy()
    ref_cpu.import_contiguous(ours, [1, 3, 4], _u16(x), 16)
    theirs = key.clone()
    theirs[:, ref_torch.context_slots([1, 3, 4], n, 16)] = x
    assert np.array_equal(ours, _u16(theirs))
    assert np.array_equal(ref_cpu.export_contiguous(ours, [1, 3, 4], n, 16), _u16(x))


def test_copy_blocks_known_answer():
    pool = np.arange(2 * 6 * 4, dtype=np.uint16).reshape(2, 6 * 2, 2, 1)  # L=2, 6 blocks of bs=2
    ref_cpu.copy_blocks(pool, pool, [(0, 5), (3, 1)], 2)
    # block 5 of each layer now holds block 0's rows, block 1 holds block 3's
    assert pool[0, 10:12].ravel().tolist() == [0, 1, 2, 3]
    assert pool[1, 10:12].ravel().tolist() == [24, 25, 26, 27]
    assert pool[0, 2:4].ravel().tolist() == [12, 13, 14, 15]
    assert pool[0, 0:2].ravel().tolist() == [0, 1, 2, 3]


# ------------------------------------------------------------------------- attention
def test_decode_matches_sdpa_with_gqa_and_reference_brute_force():
    Hq, KVH, D, S = 14, 2, 64, 512
    q = torch.randn((3, Hq, D), generator=gen(10), dtype=torch.float64)
    kc = torch.randn((S, KVH, D), generator=gen(11), dtype=torch.float64)
    vc = torch.randn((S, KVH, D), generator=gen(12), dtype=torch.float64)
    lens = [1, 130, 77]
    st = torch.zeros((3, 130), dtype=torch.long)
    for i, n in enumerate(lens):
        st[i, :n] = torch.randperm(S, generator=gen(20 + i))[:n]
    ours = ref_cpu.decode_attention(q.numpy(), kc.numpy(), vc.numpy(), st.numpy(), lens, 7)
    for b, n in enumerate(lens):
        s = st[b, :n]
        lib = F.scaled_dot_product_attention(q[b][None, :, None], kc[s].transpose(0, 1)[None],
                                             vc[s].transpose(0, 1)[None], enable_gqa=True)
        assert np.allclose(ours[b], lib[0, :, 0].numpy(), atol=1e-12)
        # reference test's brute force (tests/test_triton_attn.py:24-27)
        ki = kc[s].repeat_interleave(7, dim=1).permute(1, 0, 2)
        vi = vc[s].repeat_interleave(7, dim=1).permute(1, 0, 2)
        sc = (q[b][:, None, :] * ki).sum(-1) * D ** -0.5
        assert np.allclose(ours[b], (sc.softmax(-1)[:, :, None] * vi).sum(1).numpy(), atol=1e-12)
    # the graph decoder's repeat_kv + SDPA form agrees too (cuda_graph.py:72-76)
    rk = ref_torch.decode_repeat_kv_sdpa(q, kc, vc, [st[b, :n] for b, n in enumerate(lens)], 7)
    assert np.allclose(ours, rk.numpy(), atol=1e-12)


def test_decode_closed_forms():
    D = 8
    rng = np.random.default_rng(0)
    v = rng.standard_normal((10, 2, D))
    k = np.tile(rng.standard_normal((1, 2, D)), (10, 1, 1))   # all keys equal
    q = rng.standard_normal((1, 4, D))
    out = ref_cpu.decode_attention(q, k, v, [np.arange(10)], [10], 2)
    assert np.allclose(out[0, 0], v[:, 0].mean(0)) and np.allclose(out[0, 3], v[:, 1].mean(0))
    # one key aligned with a huge query dominates: output = that key's value row
    k = rng.standard_normal((10, 2, D)) * 0.01
    k[6, 1] = 1.0
    q = np.zeros((1, 4, D))
    q[0, 2:] = 1e4
    out = ref_cpu.decode_attention(q, k, v, [np.arange(10)], [10], 2)
    assert np.allclose(out[0, 2], v[6, 1]) and np.allclose(out[0, 3], v[6, 1])
    # heads 0..1 read KV head 0, heads 2..3 KV head 1 (h // G, not h % KVH)
    assert not np.allclose(out[0, 2], out[0, 0])
    # context of one token: the value row itself
    out = ref_cpu.decode_attention(rng.standard_normal((1, 4, D)), k, v, [np.array([3])], [1], 2)
    assert np.allclose(out[0, 1], v[3, 0]) and np.allclose(out[0, 2], v[3, 1])
    # ctx 0 -> zeros (kernel convention)
    assert not ref_cpu.decode_attention(q, k, v, [np.array([], int)], [0], 2).any()


@pytest.mark.parametrize("q_len,ctx_len", [(6, 6), (1, 11), (4, 11), (9, 17), (16, 33)])
def test_causal_lower_right_mask(q_len, ctx_len):
    """Same shapes as tests/test_prefill_attention.py:58-69."""
    mask = ref_cpu.causal_lower_right_mask(q_len, ctx_len)
    past = ctx_len - q_len
    brute = np.array([[j <= i + past for j in range(ctx_len)] for i in range(q_len)])
    assert np.array_equal(mask, brute)
    g = gen(q_len * 100 + ctx_len)
    q = torch.randn(1, 4, q_len, 8, generator=g, dtype=torch.float64)
    k = torch.randn(1, 2, ctx_len, 8, generator=g, dtype=torch.float64)
    v = torch.randn(1, 2, ctx_len, 8, generator=g, dtype=torch.float64)
    lib = F.scaled_dot_product_attention(q, k, v, attn_mask=causal_lower_right(q_len, ctx_len),
                                         enable_gqa=True)
    ours = ref_cpu.mq_attention(q[0].permute(1, 0, 2).numpy(), k[0].permute(1, 0, 2).numpy(),
                                v[0].permute(1, 0, 2).numpy(), [np.arange(ctx_len)], [q_len], 2)
    assert np.allclose(ours, lib[0].permute(1, 0, 2).numpy(), atol=1e-12)


def test_mq_reduces_to_decode_and_to_plain_causal():
    rng = np.random.default_rng(3)
    k, v = rng.standard_normal((40, 2, 16)), rng.standard_normal((40, 2, 16))
    q = rng.standard_normal((1, 6, 16))
    slots = rng.permutation(40)[:23]
    mq = ref_cpu.mq_attention(q, k, v, [slots], [1], 3)
    dec = ref_cpu.decode_attention(q, k, v, [slots], [23], 3)
    assert np.allclose(mq, dec)
    # q_len == ctx: ordinary causal attention (SDPA is_causal, library routine)
    q = rng.standard_normal((23, 6, 16))
    mq = ref_cpu.mq_attention(q, k, v, [slots], [23], 3)
    qt = torch.from_numpy(q).permute(1, 0, 2)[None]
    kt = torch.from_numpy(k[slots]).permute(1, 0, 2)[None].repeat_interleave(3, 1)
    vt = torch.from_numpy(v[slots]).permute(1, 0, 2)[None].repeat_interleave(3, 1)
    lib = F.scaled_dot_product_attention(qt, kt, vt, is_causal=True)
    assert np.allclose(mq, lib[0].permute(1, 0, 2).numpy())
    # packed multi-sequence equals per-sequence calls
    s2 = rng.permutation(40)[:9]
    q2 = rng.standard_normal((5 + 2, 6, 16))
    both = ref_cpu.mq_attention(q2, k, v, [slots, s2], [5, 2], 3)
    assert np.allclose(both[:5], ref_cpu.mq_attention(q2[:5], k, v, [slots], [5], 3))
    assert np.allclose(both[5:], ref_cpu.mq_attention(q2[5:], k, v, [s2], [2], 3))


def test_native_attention_restatement_matches_oracle():
    rng = np.random.default_rng(4)
    k = torch.from_numpy(rng.standard_normal((64, 2, 8)))
    v = torch.from_numpy(rng.standard_normal((64, 2, 8)))
    q = torch.from_numpy(rng.standard_normal((5 + 1, 4, 8)))
    s1, s2 = torch.randperm(64, generator=gen(1))[:20], torch.randperm(64, generator=gen(2))[:9]
    lib = ref_torch.native_attention(q, k, v, [s1, s2], [5, 1])
    ours = ref_cpu.mq_attention(q.numpy(), k.numpy(), v.numpy(), [s1.numpy(), s2.numpy()], [5, 1], 2)
    assert np.allclose(lib.numpy(), ours)


# ------------------------------------------------------------------------------ RoPE
def test_rope_tables_match_transformers_rotary_module():
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding
    cfg = Qwen3Config(hidden_size=64, num_attention_heads=4, num_key_value_heads=2,
                      head_dim=16, rope_theta=1e6, num_hidden_layers=1, vocab_size=16)
    rot = Qwen3RotaryEmbedding(cfg)
    pos = torch.arange(300)
    cos, sin = rot(torch.zeros(1, 1), pos[None])
    ours_c, ours_s = ref_cpu.rope_tables(pos.numpy(), 16, 1e6)
    assert np.allclose(ours_c, cos[0].numpy(), atol=2e-6)
    assert np.allclose(ours_s, sin[0].numpy(), atol=2e-6)


def test_rope_strip_inverts_apply_and_rotates_halves():
    cos, sin = ref_cpu.rope_tables(np.arange(37), 16, 1e6)
    x = np.random.default_rng(5).standard_normal((2, 37, 2, 16)).astype(np.float32)
    assert np.allclose(ref_cpu.strip_rope(ref_cpu.apply_rope(x, cos, sin), cos, sin), x, atol=1e-5)
    # position 0 is the identity; a quarter turn maps (x1, x2) -> (-x2, x1)
    c = np.zeros((1, 4), np.float32)
    s = np.ones((1, 4), np.float32)
    y = ref_cpu.apply_rope(np.array([[[[1, 2, 3, 4]]]], np.float32), c, s)
    assert y.ravel().tolist() == [-3, -4, 1, 2]
    assert np.allclose(ref_cpu.apply_rope(x[:, :1], cos[:1], sin[:1]), x[:, :1])


# ------------------------------------------------------------------------- the map
def test_layer_map_feature_order_known_answer():
    """tests/test_kv_transfer.py:89-100: row = concat over source layers (map order) of
    heads then dims."""
    g = np.random.default_rng(3)
    src = g.standard_normal((3, 5, 2, 4))
    W, b = g.standard_normal((16, 8)), g.standard_normal(8)
    x = ref_cpu.design_rows(src, (2, 0))
    for t in range(5):
        assert np.array_equal(x[t], np.concatenate([src[2, t].ravel(), src[0, t].ravel()]))
    y = ref_cpu.layer_map_apply(x, W, b)
    assert np.allclose(y[1], np.concatenate([src[2, 1].ravel(), src[0, 1].ravel()]) @ W + b)


def test_layer_map_factored_and_residual_forms():
    g = np.random.default_rng(4)
    left, right = g.standard_normal((16, 3)), g.standard_normal((3, 8))
    bias, x = g.standard_normal(8), g.standard_normal((6, 16))
    assert np.allclose(ref_cpu.layer_map_apply(x, factors=(left, right), bias=bias),
                       ref_cpu.layer_map_apply(x, left @ right, bias))
    down_w, down_b, up_w = g.standard_normal((3, 16)), g.standard_normal(3), g.standard_normal((8, 3))
    W = g.standard_normal((16, 8))
    got = ref_cpu.layer_map_apply(x, W, bias, residual=(down_w, down_b, up_w))
    xt = torch.from_numpy(x)
    expect = xt @ torch.from_numpy(W) + torch.from_numpy(bias) + F.gelu(
        xt @ torch.from_numpy(down_w).T + torch.from_numpy(down_b)) @ torch.from_numpy(up_w).T
    assert np.allclose(got, expect.numpy())
    assert np.allclose(ref_cpu.layer_map_apply(x, W, bias, residual=(down_w, down_b, 0 * up_w)),
                       x @ W + bias)


def test_bf16_map_identity_reproduces_input_and_matches_torch_rounding():
    g = gen(8)
    L, T, H, D = 3, 11, 2, 8
    k = torch.randn((L, T, H, D), generator=g).to(torch.bfloat16)
    v = torch.randn((L, T, H, D), generator=g).to(torch.bfloat16)
    eye = {"weight": np.eye(H * D), "bias": np.zeros(H * D)}
    maps = [dict(eye, source_layers=(i,)) for i in range(L)]
    ones, zeros = np.ones((T, D), np.float32), np.zeros((T, D), np.float32)
    km, vm = ref_cpu.cross_model_map_bf16(_u16(k), _u16(v), maps, maps, (ones, zeros), (ones, zeros))
    assert np.array_equal(km, _u16(k)) and np.array_equal(vm, _u16(v))
    # a random bf16 map: same roundings as the torch bf16 ops of transfer.py:104-112
    W = torch.randn((2 * H * D, H * D), generator=g).to(torch.bfloat16)
    b = torch.randn((H * D,), generator=g).to(torch.bfloat16)
    m = [{"source_layers": (2, 0), "weight": W.float().numpy(), "bias": b.float().numpy()}]
    _, vm = ref_cpu.cross_model_map_bf16(_u16(k), _u16(v), m, m, (ones, zeros), (ones, zeros))
    x = v[[2, 0]].permute(1, 0, 2, 3).reshape(T, -1)
    y = (x.double() @ W.double()).float().to(torch.bfloat16) + b     # exact GEMM, bf16 add
    assert np.array_equal(vm[0], _u16(y.view(T, H, D)))


def _prologue_inputs(T=5, Hq=4, KVH=2, D=64, seed=50):
    g = gen(seed)
    q = torch.randn((T, Hq, D), generator=g).to(torch.bfloat16)
    k = torch.randn((T, KVH, D), generator=g).to(torch.bfloat16)
    v = torch.randn((T, KVH, D), generator=g).to(torch.bfloat16)
    wq = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    wk = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    pos = torch.arange(100, 100 + T)
    cos_f, sin_f = ref_cpu.rope_tables(pos.numpy(), D, 1e6)
    cos = torch.from_numpy(cos_f).to(torch.bfloat16)
    sin = torch.from_numpy(sin_f).to(torch.bfloat16)
    return q, k, v, wq, wk, cos, sin


def test_prologue_matches_torch_ops():
    """qk_norm_rope_append == transformers' Qwen3RMSNorm + the runner's _apply_rope +
    index_copy_, run as torch bf16 ops (model_runner.py:142-148).  The variance is an fp32
    reduction whose summation order differs, so a rare element may round the other way."""
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm
    q, k, v, wq, wk, cos, sin = _prologue_inputs()
    T, Hq, D = q.shape
    qn, kn = Qwen3RMSNorm(D, eps=1e-6).to(torch.bfloat16), Qwen3RMSNorm(D, eps=1e-6).to(torch.bfloat16)
    qn.weight.data.copy_(wq)
    kn.weight.data.copy_(wk)

    def rope(x):
        x1, x2 = x.chunk(2, dim=-1)
        return x * cos.unsqueeze(1) + torch.cat((-x2, x1), dim=-1) * sin.unsqueeze(1)

    slots = torch.tensor([7, 0, 12, 3, 9])
    kpool = torch.randn((16, 2, D), generator=gen(51)).to(torch.bfloat16)
    vpool = torch.randn((16, 2, D), generator=gen(52)).to(torch.bfloat16)
    with torch.no_grad():
        tq, tk = rope(qn(q)), rope(kn(k))
        tkp, tvp = kpool.clone(), vpool.clone()
        tkp.index_copy_(0, slots, tk)
        tvp.index_copy_(0, slots, v)
    ok, ov = _u16(kpool), _u16(vpool)
    oq = ref_cpu.qk_norm_rope_append(_u16(q), _u16(k), _u16(v), _u16(wq), _u16(wk), 1e-6,
                                     _u16(cos), _u16(sin), slots.numpy(), ok, ov)
    for got, want in ((oq, _u16(tq)), (ok, _u16(tkp))):
        same = float((got == want).mean())
        err = np.abs(ref_cpu.bf16_to_f32(got) - ref_cpu.bf16_to_f32(want))
        ulp = np.abs(ref_cpu.bf16_to_f32(want)) * 2.0 ** -7 + 1e-30
        assert same >= 0.999 and (err <= ulp).all(), f"identical {same:.4f}"
    assert np.array_equal(ov, _u16(tvp))

    # no norm (Qwen2): rope only; unit weights and zero angle: normalise only
    ok2, ov2 = _u16(kpool), _u16(vpool)
    oq2 = ref_cpu.qk_norm_rope_append(_u16(q), _u16(k), _u16(v), None, None, 1e-6, _u16(cos),
                                      _u16(sin), slots.numpy(), ok2, ov2)
    assert np.array_equal(oq2, _u16(rope(q)))
    ones = _u16(torch.ones(D, dtype=torch.bfloat16))
    c0, s0 = _u16(torch.ones((T, D), dtype=torch.bfloat16)), _u16(torch.zeros((T, D), dtype=torch.bfloat16))
    oq3 = ref_cpu.qk_norm_rope_append(_u16(q), _u16(k), _u16(v), ones, ones, 1e-6, c0, s0,
                                      slots.numpy(), _u16(kpool), _u16(vpool))
    x = q.float().numpy()
    want = x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6)
    assert np.allclose(ref_cpu.bf16_to_f32(oq3), want, rtol=2 ** -7, atol=1e-6)
