"""GPU parity of the cross-model map (J5b) and the RoPE kernel against the oracle.

Tolerance for the map (north_star leaves it unstated), per element: the map rounds to bf16
at the reference's points -- x @ W, then + b, then (keys) the fp32 re-rotation -- and the
kernel's fp32 accumulation differs from the oracle's float64 only in summation order, so
an output may differ from the oracle's restatement of that sequence
(oracle.ref_cpu.cross_model_map_bf16) by at most the rounding gaps of its own chain: two
bf16 gaps at |x @ W|, two at |x @ W| + |b|, and for keys those of the rotated partner
element and of the rotated value (tests/_util.bf16_chain_bound).  A near-zero output
therefore gets a bound at the magnitude of the intermediates that cancelled into it, not
at the whole tensor's.  At least 99 % of outputs must also be bit-identical.  RoPE alone
(fp32 elementwise) is bit-exact.
"""

import numpy as np
import pytest
import torch

from oracle import ref_cpu
from tests._util import (assert_bf16_within, bf16_chain_bound, bits, fp32_dot_slack, gen,
                         randn)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _affine_bound(src_f32, maps, T, H, D):
    """Per-element bound of y = bf16(bf16(x @ W) + b) for every target layer of `maps`:
    stages |x @ W| and |x @ W| + |b| (float64 magnitudes of the oracle's design rows)."""
    out = np.empty((len(maps), T, H, D))
    for t, m in enumerate(maps):
        x = ref_cpu.design_rows(src_f32, m["source_layers"]).astype(np.float64)
        a = np.abs(x @ np.asarray(m["weight"], np.float64))
        out[t] = bf16_chain_bound(a, a + np.abs(np.asarray(m["bias"], np.float64))).reshape(T, H, D)
    return out


def _affine_magnitude(src_f32, maps, T, H, D):
    out = np.empty((len(maps), T, H, D))
    for t, m in enumerate(maps):
        x = ref_cpu.design_rows(src_f32, m["source_layers"]).astype(np.float64)
        out[t] = (np.abs(x) @ np.abs(np.asarray(m["weight"], np.float64))
                  + np.abs(np.asarray(m["bias"], np.float64))).reshape(T, H, D)
    return out


def _rotated_bound(pre_bound, pre_mag, cos, sin):
    """The bound after y = bf16(x*cos + rotate_half(x)*sin): each input's error weighted by
    its table entry, plus two gaps at the rotated value's magnitude."""
    D = pre_bound.shape[-1]
    c, s_ = np.abs(cos)[None, :, None, :], np.abs(sin)[None, :, None, :]
    partner = lambda a: np.roll(a, D // 2, axis=-1)  # noqa: E731  (d <-> d +- D/2)
    mag = pre_mag * c + partner(pre_mag) * s_
    return pre_bound * c + partner(pre_bound) * s_ + bf16_chain_bound(mag)


def _maps(n_src, n_tgt, kv_dim, k, seed, scale=None, layer_fn=None):
    g = gen(seed)
    out = []
    for t in range(n_tgt):
        layers = layer_fn(t) if layer_fn else sorted(torch.randperm(n_src, generator=g)[:k].tolist())
        w = torch.randn((len(layers) * kv_dim, kv_dim), generator=g)
        if scale:
            w = w * scale
        out.append({"source_layers": tuple(layers), "weight": w.to(torch.bfloat16),
                    "bias": torch.randn(kv_dim, generator=g).to(torch.bfloat16)})
    return out


def _to_layer_maps(maps):
    from dispec_amd.kv.transfer import LayerMap
    return [LayerMap(m["source_layers"], m["bias"], weight=m["weight"]).to(DEV, torch.bfloat16)
            for m in maps]


def _np_maps(maps):
    return [{"source_layers": m["source_layers"], "weight": m["weight"].float().numpy(),
             "bias": m["bias"].float().numpy()} for m in maps]


def _cfg(n_layers, heads, head_dim):
    from types import SimpleNamespace
    return SimpleNamespace(num_hidden_layers=n_layers, num_key_value_heads=heads,
                           head_dim=head_dim, hidden_size=16, num_attention_heads=4,
                           vocab_size=100, _name_or_path="org/m")


def _check_map(L_src, L_tgt, H, D, T, k, seed):
    """CrossModelKVMap.map with RoPE strip / re-apply against the oracle's bf16 chain."""
    from dispec_amd.kv.transfer import CrossModelKVMap
    kv = H * D
    maps_k = _maps(L_src, L_tgt, kv, k, 100 + seed, scale=kv ** -0.5)
    maps_v = _maps(L_src, L_tgt, kv, k, 200 + seed, scale=kv ** -0.5)
    kmap = CrossModelKVMap(_to_layer_maps(maps_k), _to_layer_maps(maps_v), _cfg(L_src, H, D),
                           _cfg(L_tgt, H, D))
    kk, vv = randn((L_src, T, H, D), 1 + seed), randn((L_src, T, H, D), 2 + seed)
    src_rope = ref_cpu.rope_tables(np.arange(T), D, 1e6)
    tgt_rope = ref_cpu.rope_tables(np.arange(T), D, 5e5)
    t = lambda a: torch.from_numpy(a).to(DEV)  # noqa: E731
    got_k, got_v = kmap.map(kk.to(DEV), vv.to(DEV), (t(src_rope[0]), t(src_rope[1])),
                            (t(tgt_rope[0]), t(tgt_rope[1])))
    ref_k, ref_v = ref_cpu.cross_model_map_bf16(bits(kk), bits(vv), _np_maps(maps_k),
                                                _np_maps(maps_v), src_rope, tgt_rope)
    assert got_k.shape == (L_tgt, T, H, D) and got_k.dtype == torch.bfloat16
    src_v = ref_cpu.bf16_to_f32(bits(vv))
    assert_bf16_within(bits(got_v), ref_v, _affine_bound(src_v, _np_maps(maps_v), T, H, D),
                       "values")
    content = ref_cpu.round_bf16(ref_cpu.strip_rope(ref_cpu.bf16_to_f32(bits(kk)), *src_rope))
    kb = _rotated_bound(_affine_bound(content, _np_maps(maps_k), T, H, D),
                        _affine_magnitude(content, _np_maps(maps_k), T, H, D), *tgt_rope)
    assert_bf16_within(bits(got_k), ref_k, kb, "keys")


@pytest.mark.parametrize("L_src,L_tgt,H,D,T,k", [(3, 4, 2, 4, 5, 2), (4, 3, 2, 64, 37, 2),
                                                  (3, 2, 8, 128, 300, 1)])
def test_map_matches_bf16_oracle_with_rope(L_src, L_tgt, H, D, T, k):
    _check_map(L_src, L_tgt, H, D, T, k, D)


@pytest.mark.parametrize("case", range(12))
def test_map_random_shapes(case):
    """Seeded random geometries: layer counts, heads, head dims (RoPE halves of 2..64),
    token counts across the tile edges, 1-3 source layers per target row; the last cases
    are large enough for the 256 x 256 direct-to-LDS kernel (>= 128 tiles)."""
    r = np.random.default_rng(9000 + case)
    if case >= 10:
        H, D, T, k = 8, 128, (8192, 8448)[case - 10], 1
        L_src, L_tgt = 1, 1
    else:
        H = int(r.choice([1, 2, 4, 8]))
        D = int(r.choice([4, 8, 32, 64, 128]))
        T = int(r.integers(1, 700))
        k = int(r.integers(1, 4))
        L_src, L_tgt = int(r.integers(k, 6)), int(r.integers(1, 6))
    _check_map(L_src, L_tgt, H, D, T, k, 900 + case)


def test_config5_shape_layer_selection():
    """Config 5 geometry on a shortened sequence: 28 -> 36 layers, target i reads source
    round(i*27/35), 1024 x 1024 bf16 maps ~N(0, 1/1024)."""
    from dispec_amd.kv.transfer import CrossModelKVMap
    L_src, L_tgt, H, D, T = 28, 36, 8, 128, 128
    pick = lambda i: [int(round(i * 27 / 35))]  # noqa: E731
    assert [pick(i)[0] for i in range(L_tgt)][:9] == [0, 1, 2, 2, 3, 4, 5, 5, 6]
    maps = _maps(L_src, L_tgt, H * D, 1, 5, scale=1 / 32, layer_fn=pick)
    kmap = CrossModelKVMap(_to_layer_maps(maps), _to_layer_maps(maps), _cfg(L_src, H, D),
                           _cfg(L_tgt, H, D))
    kk, vv = randn((L_src, T, H, D), 6), randn((L_src, T, H, D), 7)
    ident = (torch.ones(T, D, device=DEV), torch.zeros(T, D, device=DEV))
    got_k, got_v = kmap.map(kk.to(DEV), vv.to(DEV), ident, ident)
    ones, zeros = np.ones((T, D), np.float32), np.zeros((T, D), np.float32)
    ref_k, ref_v = ref_cpu.cross_model_map_bf16(bits(kk), bits(vv), _np_maps(maps),
                                                _np_maps(maps), (ones, zeros), (ones, zeros))
    for got, src, ref, what in ((got_v, vv, ref_v, "values"), (got_k, kk, ref_k, "keys")):
        bound = _affine_bound(ref_cpu.bf16_to_f32(bits(src)), _np_maps(maps), T, H, D)
        assert_bf16_within(bits(got), ref, bound, what)


def test_identity_map_reproduces_raw_kv():
    """tests/test_kv_transfer.py:234-252: an identity map returns its input exactly."""
    from dispec_amd.kv.transfer import CrossModelKVMap, LayerMap
    L, H, D, T = 3, 2, 64, 41
    eye = lambda i: LayerMap((i,), torch.zeros(H * D), weight=torch.eye(H * D))  # noqa: E731
    kmap = CrossModelKVMap([eye(i) for i in range(L)], [eye(i) for i in range(L)],
                           _cfg(L, H, D), _cfg(L, H, D)).to(DEV, torch.bfloat16)
    kk, vv = randn((L, T, H, D), 8).to(DEV), randn((L, T, H, D), 9).to(DEV)
    ident = (torch.ones(T, D, device=DEV), torch.zeros(T, D, device=DEV))
    gk, gv = kmap.map(kk, vv, ident, ident)
    assert torch.equal(gk, kk) and torch.equal(gv, vv)


def _stage(got, expect, *stages, carry=0.0, what=""):
    """One rounding stage: the kernel's output against the oracle applied to the kernel's
    own input, per element within its chain bound."""
    assert_bf16_within(bits(got), ref_cpu.f32_to_bf16(np.asarray(expect, np.float32)),
                       bf16_chain_bound(*stages, carry=carry), what)


def test_factored_and_residual_forms():
    """The low-rank form bf16(bf16(bf16(x @ L) @ R) + b) and the residual form
    bf16(y + bf16(bf16(gelu(bf16(x @ dw^T + db))) @ up^T)), checked stage by stage: each
    GEMM launch against the oracle's rounding of the same stage applied to the kernel's own
    input, every element within the bound of that stage's roundings (two bf16 gaps at each
    value rounded, plus fp32 summation-order slack), so a near-zero output is held to its
    own intermediates' magnitudes; and the whole map (LayerMap.apply) bit-identical to the
    stages run one after the other."""
    from dispec_amd.kv.transfer import LayerMap, _gemm
    g = gen(4)
    K, N, r, hidden, T = 128, 64, 16, 24, 77
    left, right = torch.randn(K, r, generator=g) / 8, torch.randn(r, N, generator=g) / 4
    bias = torch.randn(N, generator=g)
    x = torch.randn(T, K, generator=g).to(torch.bfloat16)
    xg = x.to(DEV)
    xd = x.double().numpy()
    rnd = ref_cpu.round_bf16
    f64 = lambda t: t.double().cpu().numpy()  # noqa: E731

    fac = LayerMap((0,), bias, factors=(left, right)).to(DEV, torch.bfloat16)
    got = fac.apply(xg)
    lb, rb, bb = f64(fac.factors[0]), f64(fac.factors[1]), f64(fac.bias)
    mid = _gemm(xg, [0], K, K, T, fac._lt, torch.empty((T, r), dtype=torch.bfloat16, device=DEV))
    sl = fp32_dot_slack(np.abs(xd), np.abs(lb))
    _stage(mid, rnd(xd @ lb), np.abs(xd @ lb) + sl, carry=sl, what="x @ L")
    md = f64(mid)
    sl = fp32_dot_slack(np.abs(md), np.abs(rb))
    a = np.abs(md @ rb) + sl
    _stage(got, rnd(rnd(md @ rb) + bb), a, a + np.abs(bb), carry=sl, what="(x @ L) @ R + b")
    two = _gemm(mid, [0], r, r, T, fac._rt, torch.empty((T, N), dtype=torch.bfloat16, device=DEV),
                fac._b, bias_mode=1)
    assert torch.equal(got, two), "factored apply differs from its two GEMMs"

    dw, db, uw = torch.randn(hidden, K, generator=g) / 8, torch.randn(hidden, generator=g), \
        torch.randn(N, hidden, generator=g) / 4
    W = torch.randn(K, N, generator=g) / 8
    res = LayerMap((0,), bias, weight=W, residual=(dw, db, uw)).to(DEV, torch.bfloat16)
    got = res.apply(xg)
    plain = res.apply(xg, use_residual=False)     # use_residual=False: the plain affine map
    Wb, dwb, dbb, uwb = (f64(t) for t in (res.weight, *res.residual))
    a = np.abs(xd @ Wb) + fp32_dot_slack(np.abs(xd), np.abs(Wb))
    _stage(plain, rnd(rnd(xd @ Wb) + bb), a, a + np.abs(bb),
           carry=fp32_dot_slack(np.abs(xd), np.abs(Wb)), what="x @ W + b")
    h = _gemm(xg, [0], K, K, T, res._down[0], torch.empty((T, hidden), dtype=torch.bfloat16,
                                                           device=DEV),
              res._down[1], bias_mode=2, act=1)
    pre = xd @ dwb.T + dbb
    sl = fp32_dot_slack(np.abs(xd), np.abs(dwb.T))
    e_pre = bf16_chain_bound(np.abs(pre) + sl, carry=sl)
    act = ref_cpu._gelu(rnd(pre))
    _stage(h, rnd(act), np.abs(act) + 1.13 * e_pre, carry=1.13 * e_pre, what="gelu(x @ dw^T + db)")
    hd, yd = f64(h), f64(plain)
    s_r = hd @ uwb.T
    sl = fp32_dot_slack(np.abs(hd), np.abs(uwb.T))
    a = np.abs(s_r) + sl
    _stage(got, rnd(yd + rnd(s_r)), a, np.abs(yd) + a, carry=sl, what="y + up(h)")
    both = _gemm(h, [0], hidden, hidden, T, res._up, plain.clone(), accumulate=True)
    assert torch.equal(got, both), "residual apply differs from its GEMMs"


@pytest.mark.parametrize("in_dtype", [torch.float32, torch.bfloat16])
def test_rope_kernel_bit_exact(in_dtype):
    from dispec_amd.kv.transfer import apply_rope, strip_rope
    L, T, H, D = 2, 37, 2, 16
    cos, sin = ref_cpu.rope_tables(np.arange(T), D, 1e6)
    x = randn((L, T, H, D), 11, in_dtype)
    c, s = torch.from_numpy(cos).to(DEV), torch.from_numpy(sin).to(DEV)
    xs = x.float().numpy()
    assert np.array_equal(strip_rope(x.to(DEV), c, s).cpu().numpy(), ref_cpu.strip_rope(xs, cos, sin))
    assert np.array_equal(apply_rope(x.to(DEV), c, s).cpu().numpy(), ref_cpu.apply_rope(xs, cos, sin))
    back = strip_rope(apply_rope(x.to(DEV), c, s), c, s).cpu()
    torch.testing.assert_close(back, x.float(), atol=1e-5, rtol=1e-5)


def test_escalation_export_map_import_round_trip():
    """map_prefix with an identity map returns the source's own exported KV, and it
    imports into a second pool bit-exactly (tests/test_kv_transfer.py:234-252)."""
    from dispec_amd.engine.model_runner import ModelRunner, SeqMeta
    from dispec_amd.kv.paged_cache import PagedKVCache
    from dispec_amd.kv.transfer import CrossModelKVMap, LayerMap
    from dispec_amd.workers.escalation import map_prefix
    from tests.toy_lm import toy_lm
    model = toy_lm("qwen3").to(torch.bfloat16).to(DEV)
    cfg = model.config
    runner = ModelRunner(model)
    cache = PagedKVCache.for_model(cfg, 32, 16, torch.bfloat16, DEV)
    ids = torch.randint(0, 128, (37,), generator=gen(6)).tolist()
    table = cache.manager.allocate(1, 37)
    table.num_tokens = 37
    runner.forward(torch.tensor(ids, device=DEV), torch.arange(37, device=DEV),
                   cache.context_slots(table.block_ids, 37),
                   [SeqMeta(table.block_ids, 37, 37)], cache)
    kvd = cfg.num_key_value_heads * cfg.head_dim
    eye = lambda i: LayerMap((i,), torch.zeros(kvd), weight=torch.eye(kvd))  # noqa: E731
    kmap = CrossModelKVMap([eye(i) for i in range(cfg.num_hidden_layers)],
                           [eye(i) for i in range(cfg.num_hidden_layers)], cfg, cfg
                           ).to(DEV, torch.bfloat16)
    raw = cache.export_contiguous(table.block_ids, 36)
    mk, mv = map_prefix(runner, cache, table.block_ids, 37, kmap, runner)
    assert torch.equal(mv, raw[1])
    # keys went through strip (bf16) then apply: equal within one bf16 rounding
    torch.testing.assert_close(mk.float(), raw[0].float(), atol=0.05, rtol=0.02)
    other = PagedKVCache.for_model(cfg, 16, 16, torch.bfloat16, DEV)
    t2 = other.manager.allocate(5, 36)
    other.import_contiguous(t2.block_ids, mk, mv)
    back = other.export_contiguous(t2.block_ids, 36)
    assert torch.equal(back[0], mk) and torch.equal(back[1], mv)


def test_admitted_prefix_reproduces_the_prefill():
    """A model's own KV for n-1 prompt tokens, raw and through an identity map, admitted
    with admit_prefix (the check and import of the reference scheduler's admission), then
    the last prompt token forwarded alone: its logits equal a plain prefill's
    (tests/test_kv_transfer.py:234-252, the identity-injection gate).  In bf16 the one-row
    and 37-row projections round differently, so the bar is cosine, not 1e-4."""
    from dispec_amd.engine.model_runner import ModelRunner, SeqMeta
    from dispec_amd.kv.paged_cache import PagedKVCache
    from dispec_amd.kv.transfer import CrossModelKVMap, LayerMap
    from dispec_amd.workers.escalation import admit_prefix, map_prefix
    from tests.toy_lm import toy_lm
    model = toy_lm("qwen3").to(torch.bfloat16).to(DEV)
    cfg = model.config
    runner = ModelRunner(model)
    cache = PagedKVCache.for_model(cfg, 32, 16, torch.bfloat16, DEV)
    n = 37
    ids = torch.randint(0, 128, (n,), generator=gen(16)).tolist()

    def prefill(sid):
        table = cache.manager.allocate(sid, n)
        h = runner.forward(torch.tensor(ids, device=DEV), torch.arange(n, device=DEV),
                           cache.context_slots(table.block_ids, n),
                           [SeqMeta(table.block_ids, n, n)], cache)
        return table, runner.logits(h[-1:]).float()[0]

    src, plain = prefill(1)
    kvd = cfg.num_key_value_heads * cfg.head_dim
    eye = lambda i: LayerMap((i,), torch.zeros(kvd), weight=torch.eye(kvd))  # noqa: E731
    kmap = CrossModelKVMap([eye(i) for i in range(cfg.num_hidden_layers)],
                           [eye(i) for i in range(cfg.num_hidden_layers)], cfg, cfg
                           ).to(DEV, torch.bfloat16)
    raw = cache.export_contiguous(src.block_ids, n - 1)
    mapped = map_prefix(runner, cache, src.block_ids, n, kmap, runner)
    for sid, prefix in ((2, raw), (3, mapped)):
        table = admit_prefix(cache, sid, ids, prefix)
        assert table.num_tokens == n - 1
        assert torch.equal(cache.export_contiguous(table.block_ids, n - 1)[1], prefix[1])
        slot = cache.context_slots(table.block_ids, n)[-1:]
        table.num_tokens = n
        h = runner.forward(torch.tensor(ids[-1:], device=DEV), torch.tensor([n - 1], device=DEV),
                           slot, [SeqMeta(table.block_ids, 1, n)], cache)
        got = runner.logits(h[-1:]).float()[0]
        cosine = torch.nn.functional.cosine_similarity(got, plain, dim=0).item()
        assert cosine >= 0.999, (sid, cosine)
        assert int(got.argmax()) == int(plain.argmax())
        cache.manager.free(sid)
    with pytest.raises(ValueError, match="fewer than all"):
        admit_prefix(cache, 4, ids[:-1], raw)


@pytest.mark.parametrize("B,M,N,bias_mode,act,accum", [
    (4, 2053, 1000, 1, 0, False),   # 9 x 4 x 4 = 144 tiles: ragged M and N, x @ W + b
    (4, 2053, 1000, 2, 1, False),   # F.linear + gelu (residual down projection)
    (4, 2053, 1000, 0, 0, True),    # no bias, accumulate (residual up projection)
    (40, 100, 1024, 2, 1, True),    # 160 tiles of mostly clamped rows
    (4, 2053, 996, 0, 0, True),     # N % 8 = 4 and 1992-byte rows: C chunks partial, unaligned
])
def test_large_tile_gemm_path(B, M, N, bias_mode, act, accum):
    """Problems of >= 128 output tiles of 256 x 256 take the direct-to-LDS kernel.  A design
    row of two source layers (two K segments, in map order 2, 0), against the float64
    oracle with the reference's rounding sequence, and bit-identical to the small-tile
    kernel, which takes the first problem of the batch on its own (too few tiles)."""
    from dispec_amd.kv.transfer import _gemm
    g = gen(300 + M + bias_mode)
    L, seg, layers = 3, 1024, (2, 0)
    K = seg * len(layers)
    src = torch.randn((B, L, M, seg), generator=g).to(torch.bfloat16)
    bt = (torch.randn((N, K), generator=g) / 40).to(torch.bfloat16)
    bias = torch.randn(N, generator=g).to(torch.bfloat16)
    c0 = torch.randn((B, M, N), generator=g).to(torch.bfloat16)
    offs = [lay * M * seg for lay in layers]
    a_d, bt_d, bias_d = src.to(DEV), bt.to(DEV), bias.to(DEV)
    out = c0.to(DEV)
    _gemm(a_d, offs, seg, seg, M, bt_d, out, bias_d if bias_mode else None, bias_mode, act,
          accum, batch=B, a_batch_stride=L * M * seg, c_batch_stride=M * N)
    one = c0[:1].to(DEV)
    _gemm(a_d, offs, seg, seg, M, bt_d, one, bias_d if bias_mode else None, bias_mode, act,
          accum, batch=1, a_batch_stride=L * M * seg, c_batch_stride=M * N)
    assert torch.equal(out[:1], one), "large- and small-tile kernels differ"
    x = np.concatenate([src[:, lay].double().numpy() for lay in layers], axis=-1)
    acc = x @ bt.double().numpy().T
    rb, b = ref_cpu.round_bf16, bias.double().numpy()
    y = rb(rb(acc) + b) if bias_mode == 1 else rb(acc + b) if bias_mode == 2 else rb(acc)
    # magnitudes rounded at each step of the chain, for the per-element bound
    stages = [np.abs(acc)] + ([np.abs(acc) + np.abs(b)] if bias_mode == 1 else [])
    if bias_mode == 2:
        stages = [np.abs(acc) + np.abs(b)]
    if act:  # the oracle's exact-erf gelu, vectorised (scipy's erf) for 8M outputs
        from scipy.special import erf
        yd = y.astype(np.float64)
        y = rb(0.5 * yd * (1.0 + erf(yd / np.sqrt(2.0))))
        stages.append(np.abs(yd) * 1.13)
    if accum:
        stages.append(np.abs(c0.double().numpy()) + np.abs(stages[-1]) * 1.13)
        y = rb(c0.double().numpy() + y)
    assert_bf16_within(bits(out.cpu()), ref_cpu.f32_to_bf16(y.astype(np.float32)),
                       bf16_chain_bound(*stages, lipschitz=1.13),
                       f"B={B} M={M} N={N} bias={bias_mode} act={act} accum={accum}")


# ------------------------------------------- fused target RoPE + pool scatter (J5b + J5c)
def _pool_pair(L, NB, bs, H, D, seed):
    from dispec_amd.kv.paged_cache import PagedKVCache
    caches = [PagedKVCache(L, NB, bs, H, D, device=DEV) for _ in range(2)]
    g = torch.Generator(device=DEV).manual_seed(seed)
    for pool in (caches[0].key, caches[0].value):
        pool.normal_(generator=g)
    caches[1].key.copy_(caches[0].key)
    caches[1].value.copy_(caches[0].value)
    return caches


@pytest.mark.parametrize("D,rope,bad_block", [(128, True, False), (128, False, False),
                                              (64, True, False), (128, True, True)])
def test_gemm_to_pool_equals_gemm_rope_scatter(D, rope, bad_block):
    """dsp_kv_map_gemm_to_pool against dsp_kv_map_gemm -> dsp_kv_rope -> dsp_kv_scatter on
    the same inputs: 3 requests of 1000 tokens (ragged against the 256-row tiles and the
    16-token blocks), a design row of two source layers, random block placement; every
    pool byte must match (rows outside the requests' blocks untouched by both)."""
    from dispec_amd import _lib
    from dispec_amd.kv.transfer import LayerMap, _gemm, _rope
    R, Ls, T, bs = 3, 3, 1000, 16
    H = 1024 // D
    kv = H * D
    g = gen(900 + D + int(rope) + 2 * int(bad_block))
    src = torch.randn((R, Ls, T, kv), generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn((2 * kv, kv), generator=g) / 45).to(torch.bfloat16)
    b = torch.randn(kv, generator=g).to(torch.bfloat16)
    m = LayerMap((2, 0), b, weight=w).to(DEV, torch.bfloat16)
    cos, sin = (torch.from_numpy(a).to(DEV) for a in ref_cpu.rope_tables(np.arange(T), D, 1e6))
    NB = R * (-(-T // bs)) + 11
    ref_c, got_c = _pool_pair(2, NB, bs, H, D, 77)
    perm = torch.randperm(NB, generator=g)[:R * (-(-T // bs))].view(R, -1).to(torch.int32)
    if bad_block:
        perm[1, 5] = NB + 3                       # outside the pool: skipped and counted
    table = perm.to(DEV)
    offs = [2 * T * kv, 0]
    # reference: dense GEMM, RoPE pass, import scatter into layer 1 (K plane)
    dense = torch.empty((R, T, kv), dtype=torch.bfloat16, device=DEV)
    m.apply_into(src, offs, kv, kv, T, dense, batch=R, a_batch_stride=Ls * T * kv,
                 c_batch_stride=T * kv)
    if rope:
        for r in range(R):
            _rope(dense[r].view(1, T, H, D), cos, sin, +1, out=dense[r].view(1, T, H, D))
    err_ref = torch.zeros(1, dtype=torch.int32, device=DEV)
    cu = torch.arange(0, (R + 1) * T, T, dtype=torch.int64, device=DEV)
    layer = ref_c.key[1]
    _lib.check(_lib.lib().dsp_kv_scatter(
        layer.data_ptr(), layer.data_ptr(), 1, ref_c.layer_bytes, ref_c.num_blocks,
        ref_c.row_bytes, bs, table.data_ptr(), table.stride(0), cu.data_ptr(), R, T,
        dense.data_ptr(), dense.data_ptr(), err_ref.data_ptr(), _lib.stream_of(dense)), "scatter")
    # fused
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    assert m.apply_to_pool(src, offs, kv, kv, T, got_c.key[1], table, bs,
                           (cos, sin) if rope else None, batch=R,
                           a_batch_stride=Ls * T * kv, err=err)
    torch.cuda.synchronize()
    assert torch.equal(got_c.key.view(torch.int16), ref_c.key.view(torch.int16))
    assert torch.equal(got_c.value.view(torch.int16), ref_c.value.view(torch.int16))
    assert (int(err.item()) > 0) == bad_block and (int(err_ref.item()) > 0) == bad_block


@pytest.mark.parametrize("form", ["dense", "residual", "factored-128", "factored-96"])
def test_map_into_equals_map_then_import(form, monkeypatch):
    """CrossModelKVMap.map_into (fused GEMM -> pool per target layer) leaves the target cache
    bit-identical to map() followed by import_contiguous (config-5 layer selection at a
    small size).  A map with a trained residual takes the unfused path per layer; low-rank
    maps take the fused launch for their second factor when the rank is a multiple of 64
    (128) and the unfused path otherwise (96) -- deciding before the first factor's GEMM,
    so no GEMM runs twice (counted)."""
    from dispec_amd.kv import transfer
    from dispec_amd.kv.transfer import CrossModelKVMap, LayerMap
    L_src, L_tgt, H, D, T = 6, 8, 8, 128, 300
    kv = H * D
    pick = lambda i: [int(round(i * (L_src - 1) / (L_tgt - 1)))]  # noqa: E731
    maps = _maps(L_src, L_tgt, kv, 1, 31, scale=1 / 32, layer_fn=pick)
    rank = int(form.split("-")[1]) if form.startswith("factored") else 0

    def layer_maps():
        out = []
        for i, mm in enumerate(maps):
            if rank:
                g = gen(40 + i)
                lm = LayerMap(mm["source_layers"], mm["bias"],
                              factors=(torch.randn(kv, rank, generator=g) / 32,
                                       torch.randn(rank, kv, generator=g) / rank ** 0.5))
            else:
                lm = LayerMap(mm["source_layers"], mm["bias"], weight=mm["weight"])
            if form == "residual":
                g = gen(32)
                lm.residual = (torch.randn(64, kv, generator=g) / 32, torch.randn(64, generator=g),
                               torch.randn(kv, 64, generator=g) / 8)
            out.append(lm.to(DEV, torch.bfloat16))
        return out

    kmap = CrossModelKVMap(layer_maps(), layer_maps(), _cfg(L_src, H, D), _cfg(L_tgt, H, D))
    kk, vv = randn((L_src, T, H, D), 33).to(DEV), randn((L_src, T, H, D), 34).to(DEV)
    t = lambda a: torch.from_numpy(a).to(DEV)  # noqa: E731
    src_rope = tuple(t(a) for a in ref_cpu.rope_tables(np.arange(T), D, 1e6))
    tgt_rope = tuple(t(a) for a in ref_cpu.rope_tables(np.arange(T), D, 5e5))
    ref_c, got_c = _pool_pair(L_tgt, 64, 16, H, D, 35)
    ids = torch.randperm(64, generator=gen(36))[:-(-T // 16)].tolist()
    mk, mv = kmap.map(kk, vv, src_rope, tgt_rope)
    ref_c.import_contiguous(ids, mk, mv)
    gemms = []
    real_gemm = transfer._gemm
    monkeypatch.setattr(transfer, "_gemm", lambda *a, **k: gemms.append(1) or real_gemm(*a, **k))
    kmap.map_into(kk, vv, src_rope, tgt_rope, got_c, ids)
    torch.cuda.synchronize()
    got_c.check_errors()
    assert torch.equal(got_c.key.view(torch.int16), ref_c.key.view(torch.int16))
    assert torch.equal(got_c.value.view(torch.int16), ref_c.value.view(torch.int16))
    per_map = {"dense": 0, "residual": 3, "factored-128": 1, "factored-96": 2}[form]
    assert len(gemms) == 2 * L_tgt * per_map, (form, len(gemms))
