"""Parity at the benchmark configurations' own sizes (GPU).

Each case runs the HIP path on one layer (attention) or all layers (byte movers, map) of a
benchmark configuration at full size, with the benchmark's shapes and random block
placement, and checks it against the oracle:

  config 3  16 x 32768 contexts, Qwen3-4B heads (32 q / 8 KV, D 128): the automatic
            (balanced) split -- at this size each worker covers 256 units and each
            segment spans 8 workers -- and the literal fixed 512-token partitions + LSE,
            each against ref_cpu.decode_attention in float64, sequence by sequence, all
            32 heads (cosine >= 0.9999, max-abs <= 2e-2);
  config 2  64 x U[512, 4096] contexts, Qwen2.5-1.5B heads (12 / 2, D 128), pool 1.25x
            the tokens, seeded as the benchmark seeds it;
  config 5  the gather of 8 requests x 4096 tokens x 28 layers and the scatter of 36
            target layers into a Qwen3-4B-layout pool, bit-exact against the oracle's
            export/import for every request (and every untouched pool row), and the
            batched map GEMM at T = 4096 for three target layers of two requests, within
            the per-element bf16 rounding-chain bound.

The reference's bar for its own kernel is a direct comparison at the served shape
(tests/test_triton_attn.py:34-60).
"""

import numpy as np
import pytest
import torch

from oracle import ref_cpu
from tests._util import assert_attention_close, assert_bf16_within, bf16_chain_bound, bits, f64

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _device_randn(shape, seed, dtype=torch.bfloat16):
    g = torch.Generator(device=DEV).manual_seed(seed)
    t = torch.empty(shape, dtype=dtype, device=DEV)
    for i in range(shape[0]):               # chunked: no full-size fp32 temporary
        t[i].normal_(generator=g)
    return t


def _check_decode_per_sequence(outs, q, kc, vc, tables, lens, G, bs, label):
    """Each output in `outs` against the float64 oracle, one sequence at a time (the
    oracle reads only that sequence's gathered rows)."""
    for b, n in enumerate(lens):
        slots = torch.as_tensor(ref_cpu.context_slots(tables[b], n, bs), device=DEV)
        kb, vb = f64(kc[slots]), f64(vc[slots])
        ref = ref_cpu.decode_attention(f64(q[b:b + 1]), kb, vb, [np.arange(n)], [n], G)
        for name, out in outs.items():
            assert_attention_close(f64(out[b:b + 1]), ref, f"{label} {name}, sequence {b}")


# ------------------------------------------------------------------------------ config 3
@pytest.fixture(scope="module")
def config3():
    B, ctx, Hq, KVH, D, bs = 16, 32768, 32, 8, 128, 16
    nb = ctx // bs
    NB = B * nb + 64
    kc = _device_randn((NB * bs, KVH, D), 3301)
    vc = _device_randn((NB * bs, KVH, D), 3302)
    perm = torch.randperm(NB, generator=torch.Generator().manual_seed(3303))[:B * nb]
    tables = perm.view(B, nb).tolist()
    bt = perm.view(B, nb).to(torch.int32).to(DEV)
    q = torch.randn((B, Hq, D), generator=torch.Generator().manual_seed(3304)).to(torch.bfloat16)
    yield dict(B=B, ctx=ctx, Hq=Hq, KVH=KVH, D=D, bs=bs, kc=kc, vc=vc, tables=tables, bt=bt,
               q=q.to(DEV))
    del kc, vc
    torch.cuda.empty_cache()


def test_config3_headline_batch_full_size(config3):
    """The headline launch exactly as benchmarked (automatic split, max_ctx 32768) and the
    configuration's literal fixed 512-token partitions, 16 x 32768 keys each."""
    from dispec_amd import _lib
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks
    c = config3
    G = c["Hq"] // c["KVH"]
    lens = [c["ctx"]] * c["B"]
    ctx_lens = torch.tensor(lens, dtype=torch.int32, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    outs = {}
    for name, P in (("balanced", 0), ("fixed-512", 512)):
        outs[name] = paged_decode_attention_blocks(
            c["q"], c["kc"], c["vc"], c["bt"], ctx_lens, G, block_size=c["bs"],
            max_ctx=c["ctx"], partition_tokens=P, err=err)
    torch.cuda.synchronize()
    # the automatic split at this shape is the balanced kernel (the benchmark's route)
    L = _lib.lib()
    assert L.dsp_paged_decode_workspace_bytes(16, 32, 8, 128, 32768, 0) != \
        L.dsp_paged_decode_workspace_bytes(16, 32, 8, 128, 32768, 512)
    assert int(err.item()) == 0, "a launch met a bad block id or a clamped length"
    _check_decode_per_sequence(outs, c["q"], c["kc"], c["vc"], c["tables"], lens, G,
                               c["bs"], "config 3")


# ------------------------------------------------------------------------------ config 2
def test_config2_batch_full_size():
    """64 contexts ~U[512, 4096] (the benchmark's seed), blocks scattered over a pool of
    1.25x the tokens; the automatic split."""
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks
    Hq, KVH, D, bs, B = 12, 2, 128, 16, 64
    gcpu = torch.Generator().manual_seed(2001)
    ctx = torch.randint(512, 4097, (B,), generator=gcpu)
    need = [-(-int(n) // bs) for n in ctx]
    NB = int(sum(need) * 1.25)
    kc = _device_randn((NB * bs, KVH, D), 2002)
    vc = _device_randn((NB * bs, KVH, D), 2003)
    perm = torch.randperm(NB, generator=gcpu).tolist()
    tables, at = [], 0
    for n in need:
        tables.append(perm[at:at + n])
        at += n
    bt = torch.zeros((B, max(need)), dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    q = torch.randn((B, Hq, D), generator=torch.Generator().manual_seed(2004)).to(torch.bfloat16)
    lens = ctx.tolist()
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = paged_decode_attention_blocks(q.to(DEV), kc, vc, bt.to(DEV),
                                        ctx.to(torch.int32).to(DEV), Hq // KVH, block_size=bs,
                                        max_ctx=int(ctx.max()), err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0, "the launch met a bad block id or a clamped length"
    _check_decode_per_sequence({"automatic": out}, q, kc, vc, tables, lens, Hq // KVH, bs,
                               "config 2")


# ------------------------------------------------------------------------------ config 5
C5 = dict(Ls=28, Lt=36, KVH=8, D=128, bs=16, R=8, T=4096)


@pytest.fixture(scope="module")
def config5_gathered():
    """Config 5's source pool, its 8 x 4096-token gather (the benchmark's call), and the
    block tables."""
    from dispec_amd.kv.paged_cache import PagedKVCache
    c = C5
    nb = c["R"] * c["T"] // c["bs"]
    NB = int(nb * 1.25)
    src = PagedKVCache(c["Ls"], NB, c["bs"], c["KVH"], c["D"], device=DEV)
    src.key.copy_(_device_randn(src.key.shape, 5001))
    src.value.copy_(_device_randn(src.value.shape, 5002))
    gcpu = torch.Generator().manual_seed(5003)
    perm = torch.randperm(NB, generator=gcpu)[:nb].view(c["R"], c["T"] // c["bs"])
    cu = torch.arange(0, (c["R"] + 1) * c["T"], c["T"], dtype=torch.int64, device=DEV)
    rows = c["Ls"] * c["R"] * c["T"]
    kbuf = torch.empty((rows, c["KVH"], c["D"]), dtype=torch.bfloat16, device=DEV)
    vbuf = torch.empty_like(kbuf)
    src.gather_into(perm.to(torch.int32).to(DEV), cu, c["T"], kbuf, vbuf)
    torch.cuda.synchronize()
    src.check_errors()
    yield dict(src=src, tables=perm.tolist(), kbuf=kbuf, vbuf=vbuf, cu=cu, NB=NB, gcpu=gcpu)
    del src, kbuf, vbuf
    torch.cuda.empty_cache()


def test_config5_gather_every_request_bit_exact(config5_gathered):
    x = config5_gathered
    c = C5
    per = c["Ls"] * c["T"]
    for pool, buf in ((x["src"].key, x["kbuf"]), (x["src"].value, x["vbuf"])):
        host_pool = bits(pool)                                   # (Ls, S, KVH, D) uint16
        host_buf = bits(buf)
        for b, ids in enumerate(x["tables"]):
            ref = ref_cpu.export_contiguous(host_pool, ids, c["T"], c["bs"])
            got = host_buf[b * per:(b + 1) * per].reshape(ref.shape)
            assert np.array_equal(got, ref), f"gather of request {b} differs"


def test_config5_scatter_into_target_pool_bit_exact(config5_gathered):
    """36 target layers of 8 requests (random rows) into a randomly placed 36-layer pool
    whose other rows hold random data: every request's rows and every untouched row."""
    from dispec_amd.kv.paged_cache import PagedKVCache
    x = config5_gathered
    c = C5
    tgt = PagedKVCache(c["Lt"], x["NB"], c["bs"], c["KVH"], c["D"], device=DEV)
    tgt.key.copy_(_device_randn(tgt.key.shape, 5011))
    tgt.value.copy_(_device_randn(tgt.value.shape, 5012))
    nb = c["R"] * c["T"] // c["bs"]
    perm = torch.randperm(x["NB"], generator=x["gcpu"])[:nb].view(c["R"], c["T"] // c["bs"])
    rows = c["Lt"] * c["R"] * c["T"]
    per = c["Lt"] * c["T"]
    kb = _device_randn((rows, c["KVH"], c["D"]), 5013)
    vb = _device_randn((rows, c["KVH"], c["D"]), 5014)
    before = {"K": bits(tgt.key), "V": bits(tgt.value)}
    tgt.scatter_from(perm.to(torch.int32).to(DEV), x["cu"], c["T"], kb, vb)
    torch.cuda.synchronize()
    for name, pool, buf in (("K", tgt.key, kb), ("V", tgt.value, vb)):
        expect = before.pop(name)
        host_buf = bits(buf)
        for b, ids in enumerate(perm.tolist()):
            chunk = host_buf[b * per:(b + 1) * per].reshape(c["Lt"], c["T"], c["KVH"], c["D"])
            ref_cpu.import_contiguous(expect, ids, chunk, c["bs"])
        assert np.array_equal(bits(pool), expect), f"{name} scatter differs from the oracle"
        del expect, host_buf
    del kb, vb
    tgt.check_errors()
    del tgt
    torch.cuda.empty_cache()


def test_config5_map_full_length(config5_gathered):
    """The benchmark's batched map call (one launch per target layer and K|V, the 8 requests
    as the GEMM batch, M = 4096 rows each) with a seeded bias, for target layers 0, 17 and
    35, checked for requests 0 and 7 against the oracle's bf16 rounding sequence."""
    from dispec_amd.kv.transfer import LayerMap
    x = config5_gathered
    c = C5
    kv = c["KVH"] * c["D"]
    g = torch.Generator().manual_seed(5021)
    targets = (0, 17, 35)
    maps = []
    for i in targets:
        w = (torch.randn((kv, kv), generator=g) / 32).to(torch.bfloat16)
        bias = torch.randn(kv, generator=g).to(torch.bfloat16)
        maps.append(dict(source_layers=(int(round(i * 27 / 35)),), weight=w, bias=bias))
    R, T, Ls = c["R"], c["T"], c["Ls"]
    for buf in (x["kbuf"], x["vbuf"]):
        out = torch.empty((R, len(targets), T, kv), dtype=torch.bfloat16, device=DEV)
        for j, m in enumerate(maps):
            lm = LayerMap(m["source_layers"], m["bias"], weight=m["weight"]).to(DEV, torch.bfloat16)
            lm.apply_into(buf, [m["source_layers"][0] * T * kv], kv, kv, T, out[:, j],
                          batch=R, a_batch_stride=Ls * T * kv,
                          c_batch_stride=len(targets) * T * kv)
        torch.cuda.synchronize()
        host_out = bits(out)
        np_maps = [dict(source_layers=m["source_layers"], weight=m["weight"].float().numpy(),
                        bias=m["bias"].float().numpy()) for m in maps]
        ident = (np.ones((T, c["D"]), np.float32), np.zeros((T, c["D"]), np.float32))
        for b in (0, R - 1):
            src_bits = bits(buf[b * Ls * T:(b + 1) * Ls * T]).reshape(Ls, T, c["KVH"], c["D"])
            _, ref = ref_cpu.cross_model_map_bf16(src_bits, src_bits, [], np_maps, ident, ident)
            src = ref_cpu.bf16_to_f32(src_bits)
            for j, m in enumerate(np_maps):
                xrow = ref_cpu.design_rows(src, m["source_layers"]).astype(np.float64)
                a = np.abs(xrow @ m["weight"].astype(np.float64))
                bound = bf16_chain_bound(a, a + np.abs(m["bias"].astype(np.float64)))
                assert_bf16_within(host_out[b, j], ref[j].reshape(T, kv), bound,
                                   f"request {b}, target layer {targets[j]}")
