"""TCP transport with the raw wire format (reference: dispec/transport/tcp.py:38-73).

Same constructor, `connect` / `listen`, `send` / `recv` / `close` as the reference's
TcpTransport and the same length-prefixed framing; the body is `wire`'s header + raw
tensor bytes instead of a `torch.save` pickle.  A GPU payload leaves through pinned host
memory in 32 MiB pieces: the device-to-host copy of the next piece runs while the current
one is on the socket, and the receiver reads straight into pinned memory and copies each
piece to the GPU while the next arrives.  CPU payloads are sent from and received into the
tensors' own memory.  Nothing on the receiving side unpickles.
"""

from __future__ import annotations

import socket
import struct

import torch

from dispec_amd.transport import wire
from dispec_amd.transport.base import KVPayload, Transport

CHUNK = 32 << 20   # bytes per pipelined piece


def _recv_exact(sock: socket.socket, view: memoryview) -> None:
    got, n = 0, len(view)
    while got < n:
        r = sock.recv_into(view[got:], n - got)
        if r == 0:
            raise ConnectionError("peer closed during recv")
        got += r


def _recv_n(sock: socket.socket, n: int) -> bytes:
    buf = bytearray(n)
    _recv_exact(sock, memoryview(buf))
    return bytes(buf)


def _as_bytes(t: torch.Tensor) -> torch.Tensor:
    """A contiguous tensor's memory as a flat uint8 tensor (no copy)."""
    return t.reshape(-1).view(torch.uint8)


class TcpTransport(Transport):
    def __init__(self, sock: socket.socket, device: str = "cuda"):
        self._sock = sock
        self.device = device if torch.cuda.is_available() else "cpu"
        self._stage: torch.Tensor | None = None    # 2 x CHUNK pinned bytes, made on first use

    @classmethod
    def connect(cls, host: str, port: int, device: str = "cuda") -> "TcpTransport":
        s = socket.create_connection((host, port))
        s.setsockopt(socket.IPPROTO_TCP, socket.TCP_NODELAY, 1)
        return cls(s, device)

    @classmethod
    def listen(cls, host: str, port: int, device: str = "cuda") -> "TcpTransport":
        srv = socket.socket(socket.AF_INET, socket.SOCK_STREAM)
        srv.setsockopt(socket.SOL_SOCKET, socket.SO_REUSEADDR, 1)
        srv.bind((host, port))
        srv.listen(1)
        conn, _ = srv.accept()
        conn.setsockopt(socket.IPPROTO_TCP, socket.TCP_NODELAY, 1)
        srv.close()
        return cls(conn, device)

    # -- staging -------------------------------------------------------------------------
    def _halves(self) -> tuple[torch.Tensor, torch.Tensor]:
        if self._stage is None:
            self._stage = torch.empty(2 * CHUNK, dtype=torch.uint8, pin_memory=True)
        return self._stage[:CHUNK], self._stage[CHUNK:]

    # -- send ----------------------------------------------------------------------------
    def send(self, payload: KVPayload) -> None:
        meta = wire.encode_meta(payload.meta)
        k, v = payload.k.contiguous(), payload.v.contiguous()
        lay = wire.layout_of(k, v, list(payload.tokens), meta)
        self._sock.sendall(struct.pack("!Q", lay.total))
        self._sock.sendall(wire.pack_prefix(lay, list(payload.tokens), meta))
        self._send_tensor(k)
        self._send_tensor(v)

    def _send_tensor(self, t: torch.Tensor) -> None:
        src = _as_bytes(t)
        n = src.numel()
        if n == 0:
            return
        if not t.is_cuda:
            self._sock.sendall(memoryview(src.numpy()))
            return
        halves = self._halves()
        events = [torch.cuda.Event(), torch.cuda.Event()]
        pieces = [(off, min(CHUNK, n - off)) for off in range(0, n, CHUNK)]

        def stage(i):
            off, m = pieces[i]
            halves[i % 2][:m].copy_(src[off:off + m], non_blocking=True)
            events[i % 2].record()

        stage(0)
        for i, (_, m) in enumerate(pieces):
            if i + 1 < len(pieces):
                stage(i + 1)          # its half was sent (synchronously) in iteration i - 1
            events[i % 2].synchronize()
            self._sock.sendall(memoryview(halves[i % 2][:m].numpy()))

    # -- recv ----------------------------------------------------------------------------
    def recv(self) -> KVPayload:
        (total,) = struct.unpack("!Q", _recv_n(self._sock, 8))
        head = _recv_n(self._sock, wire.HEADER.size)
        lay = wire.parse_header(head)
        if lay.total != total:
            raise ValueError(f"KV message of {total} bytes, its header describes {lay.total}")
        prefix = head + _recv_n(self._sock, lay.body_offset - wire.HEADER.size)
        tokens, meta = wire.parse_prefix(lay, prefix)
        k = torch.empty(lay.shape, dtype=lay.dtype, device=self.device)
        v = torch.empty(lay.shape, dtype=lay.dtype, device=self.device)
        self._recv_tensor(k)
        self._recv_tensor(v)
        return KVPayload(tokens, k, v, meta)

    def _recv_tensor(self, t: torch.Tensor) -> None:
        dst = _as_bytes(t)
        n = dst.numel()
        if n == 0:
            return
        if not t.is_cuda:
            _recv_exact(self._sock, memoryview(dst.numpy()))
            return
        halves = self._halves()
        events = [torch.cuda.Event(), torch.cuda.Event()]
        used = [False, False]
        for i, off in enumerate(range(0, n, CHUNK)):
            m = min(CHUNK, n - off)
            h = i % 2
            if used[h]:
                events[h].synchronize()   # the copy out of this half two pieces ago is done
            _recv_exact(self._sock, memoryview(halves[h][:m].numpy()))
            dst[off:off + m].copy_(halves[h][:m], non_blocking=True)
            events[h].record()
            used[h] = True
        for h in (0, 1):                  # the staging halves are reused by the next call
            if used[h]:
                events[h].synchronize()

    def close(self) -> None:
        self._sock.close()
