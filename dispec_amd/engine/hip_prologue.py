"""The attention prologue of a decoder layer on one HIP kernel.

`qk_norm_rope_append` replaces the sequence ModelRunner._attention runs between the
q/k/v projections and attention (dispec/engine/model_runner.py:142-148): Qwen3's
per-head q_norm / k_norm, RoPE on q and k (the runner's `_apply_rope`, rotate-half
convention), and `cache.write(layer, slots, k, v)`.  One launch (dsp_qk_norm_rope_append)
instead of ~25 torch kernels; rounding points are those of the torch ops.
"""

from __future__ import annotations

import torch

from dispec_amd import _lib


def _rms_weight(norm):
    if norm is None:
        return None, 0.0
    eps = getattr(norm, "variance_epsilon", getattr(norm, "eps", None))
    if eps is None:
        raise ValueError(f"{type(norm).__name__}: no epsilon attribute (variance_epsilon / eps)")
    return norm.weight, float(eps)


def qk_norm_rope_append(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor,
                        sin: torch.Tensor, slots: torch.Tensor, cache, layer_idx: int,
                        q_norm=None, k_norm=None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Normalise (optional) and rotate q and k, append k and v to `cache` layer `layer_idx`
    at `slots`, and return the rotated q.

    q: (T, Hq, D), k and v: (T, KVH, D) -- strided views of a fused QKV output are fine as
    long as head_dim is contiguous; cos, sin: (T, D) in the model dtype; slots: (T,) int.
    q_norm / k_norm: the layer's RMSNorm modules (Qwen3) or None (Qwen2).
    """
    _lib.require_gpu(q, k, v, cos, sin, slots)
    if q.dim() != 3 or k.dim() != 3 or v.shape != k.shape or q.shape[0] != k.shape[0]:
        raise ValueError(f"expected q (T, Hq, D), k and v (T, KVH, D); got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")
    T, Hq, D = q.shape
    KVH = k.shape[1]
    if k.shape[2] != D or (KVH, D) != tuple(cache.key.shape[2:]):
        raise ValueError(f"head layout {KVH}x{D} does not match the cache {tuple(cache.key.shape[2:])}")
    if (q_norm is None) != (k_norm is None):
        raise ValueError("q_norm and k_norm come together")
    dt = q.dtype
    if dt not in (torch.bfloat16, torch.float16, torch.float32) or k.dtype != dt \
            or v.dtype != dt or cache.key.dtype != dt:
        raise ValueError(f"q/k/v/cache dtypes {q.dtype}/{k.dtype}/{v.dtype}/{cache.key.dtype}: "
                         "the prologue kernel takes bf16, fp16 or fp32, all the same")
    for t in (q, k, v):
        if t.stride(2) != 1:
            raise ValueError("head_dim must be contiguous in q, k and v")
    cos = cos.to(dt).contiguous()
    sin = sin.to(dt).contiguous()
    if cos.shape != (T, D) or sin.shape != (T, D):
        raise ValueError(f"cos/sin must be (T, D) = ({T}, {D}); got {tuple(cos.shape)}")
    qw, eps = _rms_weight(q_norm)
    kw, _ = _rms_weight(k_norm)
    if qw is not None:
        qw = qw.to(dt).contiguous()
        kw = kw.to(dt).contiguous()
    slots = cache._as_slots(slots.reshape(-1), q.device)
    if slots.numel() != T:
        raise ValueError(f"{slots.numel()} slots for {T} tokens")
    if out is None:
        out = torch.empty((T, Hq, D), dtype=dt, device=q.device)
    kl, vl = cache.key[layer_idx], cache.value[layer_idx]
    _lib.check(_lib.calls().dsp_qk_norm_rope_append(
        q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
        v.data_ptr(), v.stride(0), v.stride(1), _lib.ptr(qw), _lib.ptr(kw), eps,
        cos.data_ptr(), sin.data_ptr(), cos.stride(0), slots.data_ptr(), T, Hq, KVH, D,
        out.data_ptr(), out.stride(0), out.stride(1), kl.data_ptr(), vl.data_ptr(),
        kl.shape[0], kl.stride(0), kl.stride(1), _lib.dtype_code(dt), cache._err.data_ptr(),
        _lib.stream_of(q)), "dsp_qk_norm_rope_append")
    cache._after()
    return out
