"""The TCP transport with GPU payloads: a sequence exported from one paged cache (J5a
gather), sent over a socket pair through pinned staging in pieces, received into GPU
memory and imported into another cache at other blocks (J5c scatter) arrives bit for bit
-- the handoff of the reference's disaggregated workers (dispec/workers/disaggregated.py:
45-61 over dispec/transport/tcp.py:61-70).  The payload spans several 32 MiB pieces so
the overlapped copy pipeline runs in both directions."""

import socket
import threading

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("T", [5000, 1])
def test_export_send_recv_import_is_exact(hip, T):
    from dispec_amd.kv.paged_cache import PagedKVCache
    from dispec_amd.transport.base import KVPayload
    from dispec_amd.transport.tcp import TcpTransport
    L, KVH, D, bs = 4, 8, 128, 16
    nb = -(-T // bs) + 4
    g = torch.Generator().manual_seed(700 + T)
    src = PagedKVCache(L, nb, bs, KVH, D, device=DEV)
    dst = PagedKVCache(L, nb, bs, KVH, D, device=DEV)
    src.key.copy_(torch.randn(src.key.shape, generator=g).to(torch.bfloat16))
    src.value.copy_(torch.randn(src.value.shape, generator=g).to(torch.bfloat16))
    need = -(-T // bs)
    src_ids = torch.randperm(nb, generator=g)[:need].tolist()
    dst_ids = torch.randperm(nb, generator=g)[:need].tolist()
    tokens = torch.randint(0, 150_000, (T,), generator=g).tolist()
    a, b = socket.socketpair()
    tx, rx = TcpTransport(a, DEV), TcpTransport(b, DEV)
    p = KVPayload.export(src, src_ids, tokens, request_id="req-1", first_token=42)
    th = threading.Thread(target=tx.send, args=(p,))
    th.start()
    got = rx.recv()
    th.join()
    assert got.k.is_cuda and got.tokens == tokens
    assert got.meta == {"request_id": "req-1", "first_token": 42}
    assert torch.equal(got.k, p.k) and torch.equal(got.v, p.v)
    got.import_into(dst, dst_ids)
    torch.cuda.synchronize()
    dst.check_errors()
    k2, v2 = dst.export_contiguous(dst_ids, T)
    assert torch.equal(k2, p.k) and torch.equal(v2, p.v)
    tx.close()
    rx.close()
