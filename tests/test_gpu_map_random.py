"""The map GEMM's two kernels against each other on seeded random problems (GPU).

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
