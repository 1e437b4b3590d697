"""The map GEMM's kernels on seeded random problems (GPU): the two GEMM kernels against
each other, and the fused map-into-pool launch against the unfused chain.

`dsp_kv_map_gemm` runs problems of at least 128 output tiles of 256 x 256 on the
direct-to-LDS kernel (256 x 256 tiles, its C tile staged through LDS with swizzled 256-byte
rows before the stores) and smaller ones on the 128 x 128 kernel.  Both accumulate every
output over K in 32-wide MFMA steps in increasing k and round in the same epilogue order,
so they must agree bit for bit.  Each case here draws a batch large enough for the first
(B problems, >= 128 tiles together) and runs every one of its problems again on its own,
small enough for the second (< 128 tiles), then compares all B outputs bit for bit:
ragged M and N (partial tiles, C rows whose last 16-byte chunk is partial), design rows of
1-3 source layers in random order (K segments), every bias mode, gelu and accumulation.
The float64 oracle bound for the same kernels is tests/test_gpu_map.py's
test_large_tile_gemm_path.
"""

import random

import numpy as np
import pytest
import torch

from tests._util import bits

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _tiles(M, N, size):
    return -(-M // size) * -(-N // size)


def _case(seed):
    rng = random.Random(seed)
    M, N = rng.randint(300, 3000), rng.randint(200, 1100)
    one = _tiles(M, N, 256)
    B = -(-128 // one) + rng.randint(0, 2)
    L = 3
    layers = rng.sample(range(L), rng.randint(1, 3))
    seg = rng.choice((64, 128, 256, 512))
    while True:
        bias_mode, act, accum = rng.randrange(3), rng.randrange(2), rng.randrange(2)
        if not (bias_mode == 1 and act == 1 and accum == 1):   # a form the large kernel leaves
            return M, N, B, L, layers, seg, bias_mode, act, accum


@pytest.mark.parametrize("seed", range(12))
def test_large_and_small_tile_kernels_agree_bitwise(seed):
    from dispec_amd.kv.transfer import _gemm
    M, N, B, L, layers, seg, bias_mode, act, accum = _case(seed)
    assert B * _tiles(M, N, 256) >= 128 > _tiles(M, N, 256), "batch on the large kernel only"
    K = seg * len(layers)
    g = torch.Generator().manual_seed(5000 + seed)
    src = torch.randn((B, L, M, seg), generator=g).to(torch.bfloat16).to(DEV)
    bt = (torch.randn((N, K), generator=g) / (4 * K ** 0.5)).to(torch.bfloat16).to(DEV)
    bias = torch.randn(N, generator=g).to(torch.bfloat16).to(DEV) if bias_mode else None
    c0 = torch.randn((B, M, N), generator=g).to(torch.bfloat16).to(DEV)
    offs = [lay * M * seg for lay in layers]
    out = c0.clone()
    _gemm(src, offs, seg, seg, M, bt, out, bias, bias_mode, act, bool(accum), batch=B,
          a_batch_stride=L * M * seg, c_batch_stride=M * N)
    for z in range(B):
        single = c0[z:z + 1].clone()
        _gemm(src[z], offs, seg, seg, M, bt, single, bias, bias_mode, act, bool(accum))
        assert np.array_equal(bits(out[z:z + 1]), bits(single)), \
            f"problem {z} of M={M} N={N} B={B} layers={layers} seg={seg} bias={bias_mode} " \
            f"act={act} accum={accum}"
    assert torch.isfinite(out.float()).all()


def _pool_case(seed):
    rng = random.Random(seed)
    D = rng.choice((64, 128))
    H = rng.choice((2, 4, 8))
    layers = tuple(rng.sample(range(3), rng.randint(1, 2)))
    return (rng.randint(1, 4), rng.randint(40, 1500), D, H, layers, rng.random() < 0.7,
            rng.choice((16, 32)), rng.random() < 0.3)


@pytest.mark.parametrize("seed", range(10))
def test_fused_map_into_pool_equals_gemm_rope_scatter(seed):
    """dsp_kv_map_gemm_to_pool (the large-tile kernel with the target RoPE and the pool
    scatter in its epilogue, whatever the problem size) against dsp_kv_map_gemm ->
    dsp_kv_rope -> dsp_kv_scatter on seeded random shapes: 1-4 requests of 40-1500 tokens
    (ragged against the 256-row tiles and the blocks), 2-8 heads of 64 or 128 dims, design
    rows of one or two source layers, RoPE on or off, 16- or 32-token blocks, sometimes a
    block id outside the pool (skipped and counted).  Every pool byte must match."""
    from dispec_amd import _lib
    from dispec_amd.kv.transfer import LayerMap, _rope
    from oracle import ref_cpu
    from tests.test_gpu_map import _pool_pair
    R, T, D, H, layers, rope, bs, bad_block = _pool_case(seed)
    Ls, kv = 3, H * D
    g = torch.Generator().manual_seed(7000 + seed)
    src = torch.randn((R, Ls, T, kv), generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn((len(layers) * kv, kv), generator=g) / (2 * kv ** 0.5)).to(torch.bfloat16)
    b = torch.randn(kv, generator=g).to(torch.bfloat16)
    m = LayerMap(layers, b, weight=w).to(DEV, torch.bfloat16)
    cos, sin = (torch.from_numpy(a).to(DEV) for a in ref_cpu.rope_tables(np.arange(T), D, 1e6))
    per_req = -(-T // bs)
    NB = R * per_req + 7
    ref_c, got_c = _pool_pair(2, NB, bs, H, D, 100 + seed)
    perm = torch.randperm(NB, generator=g)[:R * per_req].view(R, -1).to(torch.int32)
    if bad_block:
        perm[R - 1, per_req // 2] = NB + 1
    table = perm.to(DEV)
    offs = [lay * T * kv for lay in layers]
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
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    assert m.apply_to_pool(src, offs, kv, kv, T, got_c.key[1], table, bs,
                           (cos, sin) if rope else None, batch=R,
                           a_batch_stride=Ls * T * kv, err=err)
    torch.cuda.synchronize()
    case = f"R={R} T={T} D={D} H={H} layers={layers} rope={rope} bs={bs} bad={bad_block}"
    assert torch.equal(got_c.key.view(torch.int16), ref_c.key.view(torch.int16)), case
    assert torch.equal(got_c.value.view(torch.int16), ref_c.value.view(torch.int16)), case
    assert (int(err.item()) > 0) == bad_block and (int(err_ref.item()) > 0) == bad_block, case
