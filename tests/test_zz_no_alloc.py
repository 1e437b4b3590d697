"""dsp_paged_decode_noalloc (the decode entry point that allocates nothing: its split-K
workspace is the library's fixed per-device scratch array) against dsp_paged_decode with a
caller workspace, through the C ABI, on two calls in a row -- the second smaller, so it
runs over what the first left in the scratch.  Both run the same kernels and split, so the
outputs must be bit-identical; each is also checked against the float64 oracle at the
attention tolerance.  A launch whose workspace exceeds the scratch is refused up front."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import ref_cpu
from tests._util import assert_attention_close, f64, randn, random_block_tables

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(lens, Hq, KVH, D, seed, bs=16):
    NB = sum(-(-n // bs) for n in lens) + 4
    tables = random_block_tables(NB, lens, bs, seed)
    kc = randn((NB * bs, KVH, D), seed + 1)
    vc = randn((NB * bs, KVH, D), seed + 2)
    q = randn((len(lens), Hq, D), seed + 3)
    bt = torch.zeros((len(lens), max(len(t) for t in tables)), dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    return dict(q=q, kc=kc, vc=vc, bt=bt, tables=tables, lens=lens, Hq=Hq, KVH=KVH, D=D,
                bs=bs)


def _call(c, P, noalloc):
    from dispec_amd import _lib
    L = _lib.lib()
    q, kc, vc, bt = (c[k].to(DEV) for k in ("q", "kc", "vc", "bt"))
    ctx = torch.tensor(c["lens"], dtype=torch.int32, device=DEV)
    out = torch.full_like(q, float("nan"))
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    B, Hq, KVH, D = len(c["lens"]), c["Hq"], c["KVH"], c["D"]
    max_ctx = bt.shape[1] * c["bs"]
    stream = torch.cuda.current_stream().cuda_stream
    head = (q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(), kc.shape[0],
            kc.stride(0), kc.stride(1), bt.data_ptr(), bt.stride(0), c["bs"], None, 0,
            ctx.data_ptr(), B, Hq, KVH, D, D ** -0.5, max_ctx, P)
    tail = (out.data_ptr(), out.stride(0), out.stride(1), _lib.DSP_BF16, err.data_ptr(), stream)
    if noalloc:
        st = L.dsp_paged_decode_noalloc(*head, *tail)
    else:
        need = L.dsp_paged_decode_workspace_bytes(B, Hq, KVH, D, max_ctx, P)
        ws = torch.empty(need // 4 + 1, dtype=torch.float32, device=DEV)
        st = L.dsp_paged_decode(*head, ws.data_ptr(), ws.numel() * 4, *tail)
    assert st == 0, _lib.error_string(st)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    return out


@pytest.mark.parametrize("P", [0, 512], ids=["automatic", "fixed-512"])
def test_noalloc_matches_the_workspace_entry_point_twice(P):
    first = _case([4000, 17, 1500, 3333, 64, 2900, 1, 4096], 32, 8, 128, 9100)
    second = _case([700, 33, 1200], 16, 8, 128, 9200)           # smaller, other heads
    for c in (first, second):
        ref_out = _call(c, P, noalloc=False)
        got = _call(c, P, noalloc=True)
        assert torch.equal(got.view(torch.int16), ref_out.view(torch.int16)), \
            "no-allocation output differs from the workspace entry point"
        st = np.zeros((len(c["lens"]), max(c["lens"])), dtype=np.int64)
        for i, (t, n) in enumerate(zip(c["tables"], c["lens"])):
            st[i, :n] = ref_cpu.context_slots(t, n, c["bs"])
        ref = ref_cpu.decode_attention(f64(c["q"]), f64(c["kc"]), f64(c["vc"]), st, c["lens"],
                                       c["Hq"] // c["KVH"])
        assert_attention_close(f64(got), ref, f"no-alloc P={P}")


def test_noalloc_refuses_a_launch_beyond_its_scratch():
    from dispec_amd import _lib
    L = _lib.lib()
    # 64 sequences x 32 heads x 64 partitions of 512 keys: 68 MB of workspace
    B, Hq, KVH, D, max_ctx, P = 64, 32, 8, 128, 32768, 512
    need = L.dsp_paged_decode_workspace_bytes(B, Hq, KVH, D, max_ctx, P)
    assert need > _lib.DSP_NOALLOC_SCRATCH_BYTES
    dummy = torch.zeros(16, dtype=torch.bfloat16, device=DEV)
    ctx = torch.zeros(B, dtype=torch.int32, device=DEV)
    bt = torch.zeros((B, max_ctx // 16), dtype=torch.int32, device=DEV)
    st = L.dsp_paged_decode_noalloc(
        dummy.data_ptr(), Hq * D, D, dummy.data_ptr(), dummy.data_ptr(), 16, KVH * D, D,
        bt.data_ptr(), bt.stride(0), 16, None, 0, ctx.data_ptr(), B, Hq, KVH, D, 0.1, max_ctx,
        P, dummy.data_ptr(), Hq * D, D, _lib.DSP_BF16, None,
        torch.cuda.current_stream().cuda_stream)
    assert st == _lib.DSP_ESCRATCH
    assert "no-allocation" in _lib.error_string(st)
