"""The per-element bf16 bound the map parity tests use (tests/_util.bf16_chain_bound), on the
CPU: an fp32 evaluation of the map's rounding chain in another summation order stays inside
it, and plausible kernel mistakes fall outside it."""

import numpy as np
import pytest

from oracle import ref_cpu
from tests._util import assert_bf16_within, bf16_chain_bound, bf16_spacing


def _chain(x, w, b, dtype, order=None):
    """bf16(bf16(x @ W) + b) with the GEMM in `dtype`; `order` permutes the K sum."""
    if order is not None:
        x, w = x[:, order], w[order]
    acc = (x.astype(dtype) @ w.astype(dtype)).astype(np.float32)
    return ref_cpu.f32_to_bf16(ref_cpu.round_bf16(ref_cpu.round_bf16(acc) + b.astype(np.float32)))


def _case(seed, T=512, K=1024, N=256):
    rng = np.random.default_rng(seed)
    x = ref_cpu.round_bf16(rng.standard_normal((T, K)).astype(np.float32)).astype(np.float64)
    w = ref_cpu.round_bf16((rng.standard_normal((K, N)) / 32).astype(np.float32)).astype(np.float64)
    # biases near -x@W for a quarter of the columns: heavy cancellation into near-zero outputs
    b = ref_cpu.round_bf16(rng.standard_normal(N).astype(np.float32)).astype(np.float64)
    b[: N // 4] = ref_cpu.round_bf16(-(x[0] @ w)[: N // 4].astype(np.float32))
    a = np.abs(x @ w)
    return x, w, b, bf16_chain_bound(a, a + np.abs(b))


def test_spacing_known_answers():
    assert bf16_spacing(1.0) == 2 ** -7 and bf16_spacing(1.99) == 2 ** -7
    assert bf16_spacing(2.0) == 2 ** -6 and bf16_spacing(-0.25) == 2 ** -9
    assert bf16_spacing(0.0) == 0.0


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_fp32_in_another_order_stays_inside(seed):
    x, w, b, bound = _case(seed)
    ref = _chain(x, w, b, np.float64)
    perm = np.random.default_rng(seed + 10).permutation(x.shape[1])
    got = _chain(x, w, b, np.float32, order=perm)
    assert_bf16_within(got, ref, bound, "fp32, permuted K")


@pytest.mark.parametrize("mistake", ["bias dropped", "bias of the next column",
                                     "one K term dropped", "no rounding of x@W",
                                     "transposed weight block"])
def test_plausible_mistakes_fall_outside(mistake):
    x, w, b, bound = _case(5)
    ref = _chain(x, w, b, np.float64)
    if mistake == "bias dropped":
        got = _chain(x, w, np.zeros_like(b), np.float64)
    elif mistake == "bias of the next column":
        got = _chain(x, w, np.roll(b, 1), np.float64)
    elif mistake == "one K term dropped":
        got = _chain(x[:, 1:], w[1:], b, np.float64)
    elif mistake == "no rounding of x@W":
        got = ref_cpu.f32_to_bf16((x @ w + b).astype(np.float32))
    else:
        w2 = w.copy()
        w2[:256, :256] = w[:256, :256].T
        got = _chain(x, w2, b, np.float64)
    with pytest.raises(AssertionError):
        assert_bf16_within(got, ref, bound, mistake)
