"""Golden fixtures (tests/golden/kv_path_golden.npz, written by tests/golden/make_golden.py).

CPU: the oracle regenerates every fixture from the same seed (integer and bf16 results bit
for bit; float64 attention to 1e-12; the bf16 map, whose float64 GEMM may sum in another
order under another BLAS, to 1 bf16 ulp with >= 99.9 % of outputs identical), and the
fixtures satisfy the closed forms they contain (ctx 1 -> the value row, ctx 0 -> zeros,
export followed by import is the identity).
GPU: the HIP path on the fixtures' inputs against their stored outputs -- copies bit-exact,
attention within cosine >= 0.9999 / max-abs <= 2e-2, the map within 2 bf16 ulp with >= 99 %
identical.
"""

import os
import sys

import numpy as np
import pytest
import torch

from oracle import ref_cpu
from tests._util import assert_attention_close

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "kv_path_golden.npz")
sys.path.insert(0, os.path.join(HERE, "golden"))
DEV = "cuda"


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _map_close(got_bits, ref_bits, max_ulp, min_exact):
    got, ref = ref_cpu.bf16_to_f32(got_bits), ref_cpu.bf16_to_f32(ref_bits)
    exact = float((got_bits == ref_bits).mean())
    bound = max_ulp * 2.0 ** -7 * float(np.abs(ref).max())
    err = float(np.abs(got - ref).max())
    assert err <= bound and exact >= min_exact, f"max err {err:.3g} > {bound:.3g} or exact {exact:.4f}"


# ------------------------------------------------------------------------------ CPU


def test_oracle_regenerates_the_fixtures(golden):
    import make_golden
    fresh = make_golden.cases(np.random.default_rng(20261201))
    assert set(fresh) == set(golden)
    for name, want in golden.items():
        got = fresh[name]
        assert got.shape == want.shape and got.dtype == want.dtype, name
        if name.startswith("map_") and name.endswith("_expected"):
            _map_close(got, want, max_ulp=1, min_exact=0.999)
        elif want.dtype == np.float64:
            assert np.allclose(got, want, rtol=1e-12, atol=1e-12), name
        elif name.startswith("map_") and want.dtype == np.float32:
            assert np.allclose(got, want, rtol=0, atol=2e-7), name       # libm cos/sin
        else:
            assert np.array_equal(got, want), name


def test_fixture_closed_forms(golden):
    # decode, ctx 1: the single key's value row for each of the G query heads of a KV head
    bt, bs = golden["dec_block_table"], int(golden["dec_block_size"])
    v = ref_cpu.bf16_to_f32(golden["dec_v"])
    slot = int(ref_cpu.context_slots(bt[0], 1, bs)[0])
    assert np.allclose(golden["dec_expected"][0], np.repeat(v[slot], 4, axis=0), atol=1e-12)
    # decode, ctx 0: zeros
    assert not golden["dec_expected"][3].any()
    # verify: the last query of each sequence sees its whole context -> equals decode
    k, vv = ref_cpu.bf16_to_f32(golden["ver_k"]), ref_cpu.bf16_to_f32(golden["ver_v"])
    q = ref_cpu.bf16_to_f32(golden["ver_q"])
    bt2 = golden["ver_block_table"]
    for b, last in ((0, 2), (1, 7)):
        n = int(golden["ver_ctx"][b])
        st = ref_cpu.context_slots(bt2[b], n, 16)[None]
        dec = ref_cpu.decode_attention(q[last][None], k, vv, st, [n], 2)
        assert np.allclose(golden["ver_expected"][last], dec[0], atol=1e-12)
    # export then import of the exported rows leaves the pool as it was
    pool = golden["xfer_pool"].copy()
    ref_cpu.import_contiguous(pool, golden["xfer_block_ids"], golden["xfer_export_expected"],
                              int(golden["xfer_block_size"]))
    assert np.array_equal(pool, golden["xfer_pool"])


# ------------------------------------------------------------------------------ GPU


def _t(a):
    """bf16 bit patterns (uint16) -> a bf16 tensor on the GPU."""
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(DEV)


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _cache(pool_bits, block_size):
    """A PagedKVCache whose K and V pools both hold pool_bits ([L, S, KVH, D] or [S, KVH, D])."""
    from dispec_amd.kv.paged_cache import PagedKVCache
    p = pool_bits if pool_bits.ndim == 4 else pool_bits[None]
    L, S, KVH, D = p.shape
    c = PagedKVCache(L, S // block_size, block_size, KVH, D, dtype=torch.bfloat16, device=DEV)
    c.key.copy_(_t(p))
    c.value.copy_(_t(p))
    return c


@pytest.mark.gpu
def test_gpu_append_is_bit_exact(golden, hip):
    c = _cache(golden["append_pool"], 16)
    rows = _t(golden["append_rows"])
    c.write(0, torch.from_numpy(golden["append_slots"]).to(DEV), rows, rows)
    torch.cuda.synchronize()
    c.check_errors()
    assert np.array_equal(_bits(c.key[0]), golden["append_expected"])
    assert np.array_equal(_bits(c.value[0]), golden["append_expected"])


@pytest.mark.gpu
def test_gpu_block_copy_is_bit_exact(golden, hip):
    bs = int(golden["copy_block_size"])
    src, dst = _cache(golden["copy_pool"], bs), _cache(golden["copy_pool"], bs)
    pairs = golden["copy_pairs"]
    dst.copy_blocks_from(src, pairs[:, 0].tolist(), pairs[:, 1].tolist())
    torch.cuda.synchronize()
    dst.check_errors()
    assert np.array_equal(_bits(dst.key), golden["copy_expected"])
    assert np.array_equal(_bits(dst.value), golden["copy_expected"])


@pytest.mark.gpu
def test_gpu_export_and_import_are_bit_exact(golden, hip):
    bs = int(golden["xfer_block_size"])
    ids = golden["xfer_block_ids"].tolist()
    c = _cache(golden["xfer_pool"], bs)
    k, v = c.export_contiguous(ids, 23)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(k), golden["xfer_export_expected"])
    assert np.array_equal(_bits(v), golden["xfer_export_expected"])
    payload = _t(golden["xfer_payload"])
    c.import_contiguous(ids, payload, payload)
    torch.cuda.synchronize()
    c.check_errors()
    assert np.array_equal(_bits(c.key), golden["xfer_import_expected"])
    assert np.array_equal(_bits(c.value), golden["xfer_import_expected"])


@pytest.mark.gpu
@pytest.mark.parametrize("partition_tokens", [0, 64])
def test_gpu_decode_matches_fixture(golden, hip, partition_tokens):
    from dispec_amd.engine.hip_attn import paged_decode_attention_blocks
    out = paged_decode_attention_blocks(
        _t(golden["dec_q"]), _t(golden["dec_k"]), _t(golden["dec_v"]),
        torch.from_numpy(golden["dec_block_table"]).to(DEV),
        torch.from_numpy(golden["dec_ctx"]).to(DEV), 4,
        block_size=int(golden["dec_block_size"]), partition_tokens=partition_tokens)
    assert_attention_close(out.double().cpu().numpy(), golden["dec_expected"],
                           f"decode golden, partition_tokens={partition_tokens}")


@pytest.mark.gpu
def test_gpu_verify_matches_fixture(golden, hip):
    from dispec_amd.engine.hip_attn import paged_mq_attention
    q_lens = golden["ver_q_lens"]
    cu_q = torch.tensor([0, int(q_lens[0]), int(q_lens.sum())], dtype=torch.int32, device=DEV)
    out = paged_mq_attention(_t(golden["ver_q"]), _t(golden["ver_k"]), _t(golden["ver_v"]),
                             torch.from_numpy(golden["ver_block_table"]).to(DEV), cu_q,
                             torch.from_numpy(golden["ver_ctx"]).to(DEV), 2, block_size=16)
    assert_attention_close(out.double().cpu().numpy(), golden["ver_expected"], "verify golden")


@pytest.mark.gpu
def test_gpu_map_matches_fixture(golden, hip):
    from types import SimpleNamespace

    from dispec_amd.kv.transfer import CrossModelKVMap, LayerMap

    def cfg(n):
        return SimpleNamespace(num_hidden_layers=n, num_key_value_heads=2, head_dim=32,
                               hidden_size=16, num_attention_heads=4, vocab_size=100,
                               _name_or_path="org/m")

    def maps(w, b):
        return [LayerMap(tuple(golden["map_layers"][t].tolist()),
                         torch.from_numpy(b[t]).to(torch.bfloat16),
                         weight=torch.from_numpy(w[t]).to(torch.bfloat16)).to(DEV, torch.bfloat16)
                for t in range(2)]

    kmap = CrossModelKVMap(maps(golden["map_wk"], golden["map_bk"]),
                           maps(golden["map_wv"], golden["map_bv"]), cfg(3), cfg(2))
    t = lambda a: torch.from_numpy(a).to(DEV)  # noqa: E731
    got_k, got_v = kmap.map(_t(golden["map_k"]), _t(golden["map_v"]),
                            (t(golden["map_src_cos"]), t(golden["map_src_sin"])),
                            (t(golden["map_tgt_cos"]), t(golden["map_tgt_sin"])))
    _map_close(_bits(got_v), golden["map_v_expected"], max_ulp=2, min_exact=0.99)
    _map_close(_bits(got_k), golden["map_k_expected"], max_ulp=2, min_exact=0.99)
