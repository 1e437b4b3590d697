"""GPU parity of the fused attention prologue (dsp_qk_norm_rope_append) against the oracle
(ref_cpu.qk_norm_rope_append: the reference's q_norm / k_norm, rotate-half RoPE and
cache.write, dispec/engine/model_runner.py:142-148, with torch's rounding points).

Bar: v rows and untouched pool rows bit-exact; q and k >= 99.9 % bit-identical, and every
element within 2 ulp (bf16 or fp16) at the magnitude of its row.  The only freedom is the
summation order of the fp32 variance and rsqrt's last bit, which can move a normalised value
by one ulp; RoPE's sum x*cos + rot(x)*sin cancels for some elements, so that ulp is bounded
at the row's scale (the rotation preserves the row's norm), not at the near-zero output.
"""

import numpy as np
import pytest
import torch

from oracle import ref_cpu
from tests._util import bits, gen

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _close(got, want, dtype, what):
    if dtype == torch.bfloat16:
        g, w = ref_cpu.bf16_to_f32(got), ref_cpu.bf16_to_f32(want)
        unit = 2.0 ** -7
    else:
        g = got.view(np.float16).astype(np.float32)
        w = want.view(np.float16).astype(np.float32)
        unit = 2.0 ** -10
    bound = 2 * unit * np.abs(w).max(axis=-1, keepdims=True)   # 2 ulp at the row's scale
    same = float((got == want).mean())
    bad = int((np.abs(g - w) > bound).sum())
    assert same >= 0.999 and bad == 0, f"{what}: identical {same:.5f}, {bad} beyond 2 row ulp"


def _f16_oracle(q, k, v, wq, wk, eps, cos, sin, slots, kp, vp):
    """fp16 restatement: the same steps with fp16 rounding (numpy float16 is IEEE binary16,
    round to nearest even)."""
    r = lambda x: np.asarray(x, np.float32).astype(np.float16).astype(np.float32)  # noqa: E731
    qf, kf = q.float().numpy(), k.float().numpy()
    if wq is not None:
        def norm(x, w):
            var = np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32)
            inv = (np.float32(1) / np.sqrt(var + np.float32(eps))).astype(np.float32)
            return r(w.float().numpy() * r(x * inv))
        qf, kf = norm(qf, wq), norm(kf, wk)
    c, s = cos.float().numpy()[:, None], sin.float().numpy()[:, None]

    def rope(x):
        h = x.shape[-1] // 2
        rot = np.concatenate([-x[..., h:], x[..., :h]], -1)
        return r(r(x * c) + r(rot * s))
    qo, ko = rope(qf), rope(kf)
    kp[slots.numpy()] = ko.astype(np.float16)
    vp[slots.numpy()] = v.numpy()
    return qo.astype(np.float16)


def _setup(T, Hq, KVH, D, dtype, norm, seed, fused_qkv=False, num_slots=64):
    from dispec_amd.kv.paged_cache import PagedKVCache
    g = gen(seed)
    if fused_qkv:   # strided views of one (T, (Hq + 2 KVH) * D) projection output
        qkv = torch.randn((T, (Hq + 2 * KVH) * D), generator=g).to(dtype)
        q, k, v = qkv.split([Hq * D, KVH * D, KVH * D], dim=-1)
        q, k, v = q.view(T, Hq, D), k.view(T, KVH, D), v.view(T, KVH, D)
    else:
        q = torch.randn((T, Hq, D), generator=g).to(dtype)
        k = torch.randn((T, KVH, D), generator=g).to(dtype)
        v = torch.randn((T, KVH, D), generator=g).to(dtype)
    wq = (1 + 0.2 * torch.randn(D, generator=g)).to(dtype) if norm else None
    wk = (1 + 0.2 * torch.randn(D, generator=g)).to(dtype) if norm else None
    cf, sf = ref_cpu.rope_tables(np.arange(37, 37 + T), D, 1e6)
    cos, sin = torch.from_numpy(cf).to(dtype), torch.from_numpy(sf).to(dtype)
    slots = torch.randperm(num_slots, generator=g)[:T]
    cache = PagedKVCache(1, num_slots // 16, 16, KVH, D, dtype=dtype, device=DEV)
    kp0 = torch.randn(cache.key.shape, generator=g).to(dtype)
    vp0 = torch.randn(cache.value.shape, generator=g).to(dtype)
    cache.key.copy_(kp0)
    cache.value.copy_(vp0)
    return q, k, v, wq, wk, cos, sin, slots, cache, kp0[0], vp0[0]


class _Norm:
    def __init__(self, w, eps):
        self.weight, self.variance_epsilon = w, eps


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("norm", [True, False])
@pytest.mark.parametrize("fused_qkv", [False, True])
def test_prologue_bf16(hip, D, norm, fused_qkv):
    from dispec_amd.engine.hip_prologue import qk_norm_rope_append
    T, Hq, KVH = 13, 8, 2
    q, k, v, wq, wk, cos, sin, slots, cache, kp0, vp0 = _setup(T, Hq, KVH, D, torch.bfloat16,
                                                               norm, 60 + D, fused_qkv)
    out = qk_norm_rope_append(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV),
                              slots.to(DEV), cache, 0,
                              _Norm(wq.to(DEV), 1e-6) if norm else None,
                              _Norm(wk.to(DEV), 1e-6) if norm else None)
    torch.cuda.synchronize()
    cache.check_errors()
    kp, vp = bits(kp0), bits(vp0)
    oq = ref_cpu.qk_norm_rope_append(bits(q), bits(k), bits(v), bits(wq) if norm else None,
                                     bits(wk) if norm else None, 1e-6, bits(cos), bits(sin),
                                     slots.numpy(), kp, vp)
    _close(bits(out), oq, torch.bfloat16, "q")
    _close(bits(cache.key[0]), kp, torch.bfloat16, "k pool")
    assert np.array_equal(bits(cache.value[0]), vp), "v pool"


def test_prologue_fp16_and_qwen3_shape(hip):
    """fp16, and Qwen3-4B's head layout (32 q heads, 8 KV heads, head_dim 128) on a batch
    of 64 decode tokens."""
    from dispec_amd.engine.hip_prologue import qk_norm_rope_append
    T, Hq, KVH, D = 64, 32, 8, 128
    q, k, v, wq, wk, cos, sin, slots, cache, kp0, vp0 = _setup(T, Hq, KVH, D, torch.float16,
                                                               True, 71, num_slots=128)
    out = qk_norm_rope_append(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV),
                              slots.to(DEV), cache, 0, _Norm(wq.to(DEV), 1e-6),
                              _Norm(wk.to(DEV), 1e-6))
    torch.cuda.synchronize()
    kp = kp0.numpy().copy()
    vp = vp0.numpy().copy()
    oq = _f16_oracle(q, k, v, wq, wk, 1e-6, cos, sin, slots, kp, vp)
    _close(bits(out), oq.view(np.uint16), torch.float16, "q fp16")
    _close(bits(cache.key[0]), kp.view(np.uint16), torch.float16, "k pool fp16")
    assert np.array_equal(bits(cache.value[0]), vp.view(np.uint16))


def test_prologue_bad_slot_is_counted_and_skipped(hip):
    from dispec_amd.engine.hip_prologue import qk_norm_rope_append
    T, Hq, KVH, D = 3, 4, 2, 64
    q, k, v, wq, wk, cos, sin, _, cache, kp0, vp0 = _setup(T, Hq, KVH, D, torch.bfloat16, True, 80)
    slots = torch.tensor([5, 1 << 40, 9])
    qk_norm_rope_append(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV),
                        slots.to(DEV), cache, 0, _Norm(wq.to(DEV), 1e-6), _Norm(wk.to(DEV), 1e-6))
    torch.cuda.synchronize()
    with pytest.raises(IndexError):
        cache.check_errors()
    got_v = bits(cache.value[0])
    want_v = bits(vp0).copy()
    want_v[[5, 9]] = bits(v)[[0, 2]]
    assert np.array_equal(got_v, want_v), "only the in-range tokens are written"


def test_prologue_rejects_bad_arguments(hip):
    from dispec_amd.engine.hip_prologue import qk_norm_rope_append
    q, k, v, wq, wk, cos, sin, slots, cache, _, _ = _setup(4, 4, 2, 64, torch.bfloat16, True, 90)
    d = lambda t: t.to(DEV)  # noqa: E731
    with pytest.raises(ValueError):   # q_norm without k_norm
        qk_norm_rope_append(d(q), d(k), d(v), d(cos), d(sin), d(slots), cache, 0,
                            _Norm(d(wq), 1e-6), None)
    with pytest.raises(ValueError):   # cos of the wrong length
        qk_norm_rope_append(d(q), d(k), d(v), d(cos[:3]), d(sin[:3]), d(slots), cache, 0)
    with pytest.raises(RuntimeError):  # CPU tensors: no CPU path
        qk_norm_rope_append(q, k, v, cos, sin, slots, cache, 0)


@pytest.mark.parametrize("D", [64, 128, 256])
def test_prologue_fp32(hip, D):
    """fp32 models: the same steps with fp32 rounding only (numpy float32, one rounding per
    op as torch's fp32 ops); bound 4 fp32 ulp at the row's scale (the variance's summation
    order and rsqrt's last bits), v rows and untouched pool rows bit-exact."""
    from dispec_amd.engine.hip_prologue import qk_norm_rope_append
    T, Hq, KVH = 9, 8, 2
    dt = torch.float32
    q, k, v, wq, wk, cos, sin, slots, cache, kp0, vp0 = _setup(T, Hq, KVH, D, dt, True, 95 + D)
    out = qk_norm_rope_append(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV),
                              slots.to(DEV), cache, 0, _Norm(wq.to(DEV), 1e-6),
                              _Norm(wk.to(DEV), 1e-6))
    torch.cuda.synchronize()
    f = np.float32

    def norm(x, w):
        var = np.mean(x * x, axis=-1, keepdims=True, dtype=f)
        inv = (f(1) / np.sqrt(var + f(1e-6))).astype(f)
        return (w * (x * inv)).astype(f)

    c, s = cos.numpy()[:, None], sin.numpy()[:, None]

    def rope(x):
        h = x.shape[-1] // 2
        rot = np.concatenate([-x[..., h:], x[..., :h]], -1)
        return (x * c + rot * s).astype(f)
    qo = rope(norm(q.numpy(), wq.numpy()))
    ko = rope(norm(k.numpy(), wk.numpy()))
    kp, vp = kp0.numpy().copy(), vp0.numpy().copy()
    kp[slots.numpy()] = ko
    vp[slots.numpy()] = v.numpy()
    for got, want, what in ((out.cpu().numpy(), qo, "q"), (cache.key[0].cpu().numpy(), kp, "k")):
        bound = 4 * 2.0 ** -23 * np.abs(want).max(axis=-1, keepdims=True)
        worst = float((np.abs(got - want) - bound).max())
        assert worst <= 0, f"{what} fp32 D={D}: {worst:.3g} beyond 4 row ulp"
    assert np.array_equal(cache.value[0].cpu().numpy(), vp), "v pool"
