"""Wire format of a KVPayload: a fixed header, the tokens, JSON metadata and the raw K/V
bytes -- replacing the reference's `torch.save` pickle of the payload
(dispec/transport/tcp.py:61-70).

Message body (little-endian), one per payload:

    offset 0   header, 32 bytes:  magic b"DSKV", u16 version (1), u16 dtype code
                                  (1 bf16, 2 fp16, 3 fp32), u32 layers, u32 tokens,
                                  u32 kv_heads, u32 head_dim, u32 meta bytes, u32 0
    32         tokens             int64 x tokens
               meta               UTF-8 JSON object, `meta bytes` long
               padding            zeros up to the next multiple of 256
    body_off   K                  layers x tokens x kv_heads x head_dim elements, the
                                  KVPayload layout (reference transport/base.py:24-44)
               V                  the same

On the socket each body is framed by its length as a big-endian u64, as the reference
frames its pickles (tcp.py:19-36).  The receiver learns every size from the header
before reading the tensors, so it can read them straight into pinned memory and copy them
to the GPU while the rest arrives; nothing is unpickled (the metadata is JSON: a receiver
executes no code from the wire).
"""

from __future__ import annotations

import json
import struct
from dataclasses import dataclass

import torch

MAGIC = b"DSKV"
VERSION = 1
HEADER = struct.Struct("<4sHHIIIIII")
ALIGN = 256
_CODES = {torch.bfloat16: 1, torch.float16: 2, torch.float32: 3}
_DTYPES = {v: k for k, v in _CODES.items()}


@dataclass(frozen=True)
class Layout:
    """Sizes and offsets of one message body."""

    dtype: torch.dtype
    layers: int
    tokens: int
    kv_heads: int
    head_dim: int
    meta_bytes: int

    @property
    def shape(self) -> tuple[int, int, int, int]:
        return (self.layers, self.tokens, self.kv_heads, self.head_dim)

    @property
    def tensor_bytes(self) -> int:
        n = self.layers * self.tokens * self.kv_heads * self.head_dim
        return n * torch.empty((), dtype=self.dtype).element_size()

    @property
    def body_offset(self) -> int:
        end = HEADER.size + 8 * self.tokens + self.meta_bytes
        return -(-end // ALIGN) * ALIGN

    @property
    def total(self) -> int:
        return self.body_offset + 2 * self.tensor_bytes


def layout_of(k: torch.Tensor, v: torch.Tensor, tokens: list[int], meta_json: bytes) -> Layout:
    if k.dim() != 4 or v.shape != k.shape or v.dtype != k.dtype:
        raise ValueError(f"k and v must be equal (layers, tokens, kv_heads, head_dim) tensors; "
                         f"got {tuple(k.shape)} {k.dtype} and {tuple(v.shape)} {v.dtype}")
    if k.dtype not in _CODES:
        raise ValueError(f"unsupported payload dtype {k.dtype}")
    if k.shape[1] != len(tokens):
        raise ValueError(f"payload has {k.shape[1]} token rows for {len(tokens)} tokens")
    return Layout(k.dtype, *k.shape, len(meta_json))


def encode_meta(meta: dict) -> bytes:
    """JSON metadata (request id, first decoded token, ...).  Values must be JSON types."""
    try:
        return json.dumps(meta, separators=(",", ":")).encode()
    except TypeError as e:
        raise TypeError(f"KVPayload.meta must hold JSON values to go on the wire: {e}") from None


def pack_prefix(lay: Layout, tokens: list[int], meta_json: bytes) -> bytes:
    """Header, tokens, metadata and padding: the body's first `body_offset` bytes."""
    head = HEADER.pack(MAGIC, VERSION, _CODES[lay.dtype], lay.layers, lay.tokens,
                       lay.kv_heads, lay.head_dim, lay.meta_bytes, 0)
    toks = struct.pack(f"<{lay.tokens}q", *tokens)
    out = head + toks + meta_json
    return out + bytes(lay.body_offset - len(out))


def parse_header(buf: bytes) -> Layout:
    magic, ver, code, L, T, H, D, meta_bytes, _ = HEADER.unpack(buf[:HEADER.size])
    if magic != MAGIC:
        raise ValueError("not a dispec_amd KV message (bad magic)")
    if ver != VERSION:
        raise ValueError(f"KV message version {ver}; this build reads version {VERSION}")
    if code not in _DTYPES:
        raise ValueError(f"KV message dtype code {code} unknown")
    return Layout(_DTYPES[code], L, T, H, D, meta_bytes)


def parse_prefix(lay: Layout, buf: bytes) -> tuple[list[int], dict]:
    """Tokens and metadata from the body's first `body_offset` bytes."""
    toks = list(struct.unpack_from(f"<{lay.tokens}q", buf, HEADER.size))
    off = HEADER.size + 8 * lay.tokens
    meta = json.loads(bytes(buf[off:off + lay.meta_bytes]).decode()) if lay.meta_bytes else {}
    return toks, meta
