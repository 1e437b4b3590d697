"""The KV payload moved between workers (reference: dispec/transport/base.py:24-59).

k, v are (num_layers, seq_len, num_kv_heads, head_dim) contiguous tensors -- the layout
PagedKVCache.export_contiguous produces with the block-table gather kernel and
import_contiguous consumes with the scatter kernel, so a payload is portable across
workers whose block pools differ.  The channels themselves (CUDA IPC queue, TCP) are
outside this package.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from dataclasses import dataclass, field

import torch


@dataclass
class KVPayload:
    tokens: list[int]
    k: torch.Tensor
    v: torch.Tensor
    meta: dict = field(default_factory=dict)

    @property
    def seq_len(self) -> int:
        return len(self.tokens)

    def nbytes(self) -> int:
        return self.k.numel() * self.k.element_size() * 2

    @classmethod
    def export(cls, cache, block_ids: list[int], tokens: list[int], **meta) -> "KVPayload":
        """Gather a sequence's KV for its tokens out of a paged cache."""
        k, v = cache.export_contiguous(block_ids, len(tokens))
        return cls(list(tokens), k, v, dict(meta))

    def import_into(self, cache, block_ids: list[int]) -> None:
        """Scatter this payload into a sequence's blocks of another cache."""
        cache.import_contiguous(block_ids, self.k, self.v)


class Transport(ABC):
    """A one-directional channel that moves a KVPayload from sender to receiver."""

    @abstractmethod
    def send(self, payload: KVPayload) -> None:
        ...

    @abstractmethod
    def recv(self) -> KVPayload:
        ...

    def close(self) -> None:
        pass
