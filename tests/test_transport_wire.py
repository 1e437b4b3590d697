"""The KV wire format and the TCP transport on CPU tensors (no GPU).

Round trips over a socket pair (the reference's TcpTransport contract,
dispec/transport/tcp.py:38-73: `send(payload)` on one end, `recv()` on the other gives
the same tokens, K, V and metadata), the byte layout of a message (known answer), and
the error cases: a foreign or truncated stream, metadata that is not JSON, a length
that disagrees with the header.
"""

import json
import socket
import struct
import threading

import pytest
import torch

from dispec_amd.transport import wire
from dispec_amd.transport.base import KVPayload
from dispec_amd.transport.tcp import TcpTransport


def _pair():
    a, b = socket.socketpair()
    return TcpTransport(a, device="cpu"), TcpTransport(b, device="cpu")


def _payload(L, T, H, D, dtype=torch.bfloat16, seed=0, **meta):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn((L, T, H, D), generator=g).to(dtype)
    v = torch.randn((L, T, H, D), generator=g).to(dtype)
    toks = torch.randint(0, 150_000, (T,), generator=g).tolist()
    return KVPayload(toks, k, v, dict(meta))


def _roundtrip(p):
    tx, rx = _pair()
    t = threading.Thread(target=tx.send, args=(p,))
    t.start()
    got = rx.recv()
    t.join()
    tx.close()
    rx.close()
    return got


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_roundtrip_is_exact(dtype):
    p = _payload(3, 37, 2, 64, dtype, seed=1, request_id="r-17", first_token=9, ok=True)
    got = _roundtrip(p)
    assert got.tokens == p.tokens and got.meta == p.meta
    assert got.k.dtype == dtype and got.k.shape == p.k.shape
    assert torch.equal(got.k.view(torch.uint8), p.k.view(torch.uint8))
    assert torch.equal(got.v.view(torch.uint8), p.v.view(torch.uint8))


def test_empty_and_large_payloads():
    got = _roundtrip(_payload(2, 0, 2, 64))
    assert got.tokens == [] and got.k.shape == (2, 0, 2, 64)
    p = _payload(4, 2000, 8, 128, seed=2)            # 16 MB per tensor: many socket writes
    got = _roundtrip(p)
    assert torch.equal(got.k.view(torch.uint8), p.k.view(torch.uint8))
    assert torch.equal(got.v.view(torch.uint8), p.v.view(torch.uint8))


def test_byte_layout_known_answer():
    k = torch.arange(2 * 3 * 1 * 4, dtype=torch.float32).view(2, 3, 1, 4)
    v = -k
    meta = wire.encode_meta({"a": 1})
    lay = wire.layout_of(k, v, [5, 6, 7], meta)
    prefix = wire.pack_prefix(lay, [5, 6, 7], meta)
    assert lay.body_offset == 256 and len(prefix) == 256
    assert lay.total == 256 + 2 * 24 * 4
    assert prefix[:4] == b"DSKV"
    assert struct.unpack_from("<HHIIIIII", prefix, 4) == (1, 3, 2, 3, 1, 4, len(meta), 0)
    assert struct.unpack_from("<3q", prefix, 32) == (5, 6, 7)
    assert json.loads(prefix[56:56 + len(meta)]) == {"a": 1}
    assert not any(prefix[56 + len(meta):])
    assert wire.parse_header(prefix) == lay
    assert wire.parse_prefix(lay, prefix) == ([5, 6, 7], {"a": 1})


def test_errors():
    with pytest.raises(TypeError):
        wire.encode_meta({"t": torch.zeros(1)})
    with pytest.raises(ValueError):
        wire.parse_header(b"XXXX" + bytes(28))
    with pytest.raises(ValueError):            # token count and K rows disagree
        wire.layout_of(torch.zeros(1, 3, 1, 4), torch.zeros(1, 3, 1, 4), [1, 2], b"")
    # a peer that closes mid-message
    a, b = socket.socketpair()
    rx = TcpTransport(b, device="cpu")
    p = _payload(1, 4, 1, 8)
    meta = wire.encode_meta({})
    lay = wire.layout_of(p.k, p.v, p.tokens, meta)
    a.sendall(struct.pack("!Q", lay.total) + wire.pack_prefix(lay, p.tokens, meta) + b"\0" * 10)
    a.close()
    with pytest.raises(ConnectionError):
        rx.recv()
    rx.close()
    # a length that disagrees with the header
    a, b = socket.socketpair()
    rx = TcpTransport(b, device="cpu")
    a.sendall(struct.pack("!Q", lay.total + 1) + wire.pack_prefix(lay, p.tokens, meta))
    with pytest.raises(ValueError):
        rx.recv()
    a.close()
    rx.close()


def test_reference_pickle_path_restatement_roundtrips():
    """The oracle's restatement of the reference's pickle framing (timed beside the wire
    format in bench.py's CPU-baseline leg) returns what it was given."""
    from oracle import ref_torch
    p = _payload(2, 9, 2, 16, seed=3)
    a, b = socket.socketpair()
    t = threading.Thread(target=ref_torch.tcp_send_pickle, args=(a, p.tokens, p.k, p.v, {"x": 1}))
    t.start()
    toks, k, v, meta = ref_torch.tcp_recv_pickle(b, "cpu")
    t.join()
    a.close()
    b.close()
    assert toks == p.tokens and meta == {"x": 1}
    assert torch.equal(k, p.k) and torch.equal(v, p.v)
