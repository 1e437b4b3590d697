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
