"""Shared helpers for the tests: seeded inputs and comparisons."""

from __future__ import annotations

import numpy as np
import torch

# Attention tolerance stated by the task for bf16 outputs.
COS_MIN = 0.9999
MAX_ABS = 2e-2


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def randn(shape, seed: int, dtype=torch.bfloat16, device="cpu") -> torch.Tensor:
    """~N(0,1) generated on the CPU in float32, cast, then moved (identical bytes everywhere)."""
    return torch.randn(shape, generator=gen(seed)).to(dtype).to(device)


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw bit patterns of a 2-byte tensor as uint16 (or 4-byte as uint32)."""
    t = t.detach().cpu().contiguous()
    if t.element_size() == 2:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.element_size() == 4:
        return t.view(torch.int32).numpy().view(np.uint32)
    raise TypeError(t.dtype)


def f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().to(torch.float64).numpy()


def cosine(a: np.ndarray, b: np.ndarray) -> float:
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    if na == 0 and nb == 0:
        return 1.0
    return float(a @ b / (na * nb))


def assert_attention_close(got, ref, what=""):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    cos = cosine(got, ref)
    err = float(np.abs(got - ref).max()) if got.size else 0.0
    assert cos >= COS_MIN and err <= MAX_ABS, f"{what}: cosine {cos:.6f}, max-abs {err:.4g}"


def random_block_tables(num_blocks: int, lens, block_size: int, seed: int) -> list[list[int]]:
    """Disjoint block lists for sequences of the given lengths, from a seeded permutation."""
    perm = torch.randperm(num_blocks, generator=gen(seed)).tolist()
    tables, at = [], 0
    for n in lens:
        need = -(-n // block_size)
        tables.append(perm[at:at + need])
        at += need
    assert at <= num_blocks, "pool too small for the requested lengths"
    return tables


# ------------------------------------------------------------ bf16 rounding-chain bounds
def bf16_spacing(x) -> np.ndarray:
    """Gap between adjacent bf16 values at magnitude |x| (8 significand bits): 2^(e-7)
    for |x| in [2^e, 2^(e+1)); 0 where x == 0."""
    m = np.abs(np.asarray(x, np.float64))
    e = np.floor(np.log2(np.where(m > 0, m, 1.0)))
    return np.where(m > 0, np.exp2(e - 7), 0.0)


def bf16_chain_bound(*stages, lipschitz: float = 1.0, carry=0.0) -> np.ndarray:
    """Per-element bound on |got - ref| for two evaluations of one chain of bf16 roundings
    whose exact inputs agree up to fp32 accumulation order.

    `stages` are (upper bounds of) the magnitudes of the value rounded at each step, in
    order.  Two roundings of values that differ by e land at most e + one gap apart, and
    the gap at the next binade up is twice the gap at |x|, so each step adds 2 gaps at its
    magnitude; `lipschitz` bounds how much a step between roundings (e.g. gelu, |f'| <
    1.13) can amplify the error carried into it.  `carry` is an error already present
    before the first rounding (fp32 accumulation order, or an earlier chain's bound
    pushed through a matrix product).
    """
    bound = np.asarray(carry, np.float64)
    for m in stages:
        bound = lipschitz * bound + 2.0 * bf16_spacing(np.asarray(m, np.float64) * (1 + 2 ** -7))
    return bound


def fp32_dot_slack(abs_a, abs_b) -> np.ndarray:
    """Bound on how far two fp32 evaluations of a @ b (any summation order) can differ:
    2 * K * 2^-24 * (|a| @ |b|) for an inner dimension K (Higham's gamma_K, twice)."""
    abs_a, abs_b = np.asarray(abs_a, np.float64), np.asarray(abs_b, np.float64)
    return 2.0 * abs_a.shape[-1] * 2.0 ** -24 * (abs_a @ abs_b)


def assert_bf16_within(got_bits, ref_bits, bound, what, min_exact: float = 0.99) -> None:
    """Every element within its own `bound` of the reference, and at least `min_exact` of
    the elements bit-identical (a differing bit pattern is a rounding-boundary case)."""
    from oracle import ref_cpu
    got_bits, ref_bits = np.asarray(got_bits, np.uint16), np.asarray(ref_bits, np.uint16)
    got = ref_cpu.bf16_to_f32(got_bits).astype(np.float64)
    ref = ref_cpu.bf16_to_f32(ref_bits).astype(np.float64)
    err = np.abs(got - ref)
    bound = np.broadcast_to(np.asarray(bound, np.float64), err.shape)
    over = err > bound
    exact = float((got_bits == ref_bits).mean()) if got.size else 1.0
    if over.any():
        i = np.unravel_index(int(np.argmax(err - bound)), err.shape)
        raise AssertionError(f"{what}: {int(over.sum())} elements outside their bound; worst "
                             f"at {i}: got {got[i]:.6g} ref {ref[i]:.6g} bound {bound[i]:.3g}")
    assert exact >= min_exact, f"{what}: only {exact:.4f} of outputs bit-identical"
