"""dsp_paged_decode_noalloc (the decode entry point that allocates nothing: its split-K
workspace is the library's fixed per-device scratch array) against dsp_paged_decode with a
caller workspace, through the C ABI, on two calls in a row -- the second smaller, so it
runs over what the first left in the scratch.  Both run the same kernels and split, so the
outputs must be bit-identical; each is also checked against the float64 oracle at the
attention tolerance.  A launch whose workspace exceeds the scratch is refused up front.

The first test captures the process's first no-allocation call in a HIP graph: that call
is where the library looks up its per-device scratch address, and graph capture is the
use the entry point exists for.  No other test file calls it, so this holds both when this
file runs alone and when it runs after the rest of the suite."""

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


class _Launch:
    """One decode problem's device tensors, callable through either entry point."""

    def __init__(self, c, P):
        self.c, self.P = c, P
        self.q, self.kc, self.vc, self.bt = (c[k].to(DEV) for k in ("q", "kc", "vc", "bt"))
        self.ctx = torch.tensor(c["lens"], dtype=torch.int32, device=DEV)
        self.out = torch.full_like(self.q, float("nan"))
        self.err = torch.zeros(1, dtype=torch.int32, device=DEV)
        self.B, self.Hq, self.KVH, self.D = len(c["lens"]), c["Hq"], c["KVH"], c["D"]
        self.max_ctx = self.bt.shape[1] * c["bs"]

    def __call__(self, noalloc, stream=None):
        from dispec_amd import _lib
        L = _lib.lib()
        q, kc, out = self.q, self.kc, self.out
        stream = torch.cuda.current_stream().cuda_stream if stream is None else stream
        head = (q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), self.vc.data_ptr(),
                kc.shape[0], kc.stride(0), kc.stride(1), self.bt.data_ptr(), self.bt.stride(0),
                self.c["bs"], None, 0, self.ctx.data_ptr(), self.B, self.Hq, self.KVH, self.D,
                self.D ** -0.5, self.max_ctx, self.P)
        tail = (out.data_ptr(), out.stride(0), out.stride(1), _lib.DSP_BF16,
                self.err.data_ptr(), stream)
        if noalloc:
            st = L.dsp_paged_decode_noalloc(*head, *tail)
        else:
            need = L.dsp_paged_decode_workspace_bytes(self.B, self.Hq, self.KVH, self.D,
                                                      self.max_ctx, self.P)
            self.ws = torch.empty(need // 4 + 1, dtype=torch.float32, device=DEV)
            st = L.dsp_paged_decode(*head, self.ws.data_ptr(), self.ws.numel() * 4, *tail)
        assert st == 0, _lib.error_string(st)
        return st


def _call(c, P, noalloc):
    launch = _Launch(c, P)
    launch(noalloc)
    torch.cuda.synchronize()
    assert int(launch.err.item()) == 0
    return launch.out


def test_first_noalloc_call_inside_a_graph_capture():
    """The process's first no-allocation call is captured into a HIP graph; the graph
    replays four times, with eager launches writing the same output buffer in between,
    and every replay is bit-identical to the workspace entry point run eagerly."""
    c = _case([3000, 45, 2048, 700, 1, 4096], 32, 8, 128, 9300)
    expect = _call(c, 0, noalloc=False).clone()
    launch = _Launch(c, 0)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch(noalloc=True)
    torch.cuda.synchronize()
    other = _case([100, 900], 16, 8, 128, 9400)
    for i in range(4):
        launch.out.fill_(float("nan"))
        _call(other, 0, noalloc=True)          # eager use of the scratch between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(launch.out.view(torch.int16), expect.view(torch.int16)), \
            f"replay {i} differs from the eager workspace entry point"
    assert int(launch.err.item()) == 0
    del graph


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
