"""HipIpcTransport's host-side checks (CPU only): the region size limit and GPU-only sends."""

import pytest
import torch


def test_region_limit_and_payload_checks():
    from dispec_amd.transport.base import KVPayload
    from dispec_amd.transport.ipc import MAX_REGION_BYTES, HipIpcTransport, alloc_region
    with pytest.raises(ValueError, match="IPC region"):
        alloc_region(MAX_REGION_BYTES + 1)
    tr = HipIpcTransport(HipIpcTransport.make_queue())
    cpu = torch.zeros(2, 3, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU payloads only"):
        tr.send(KVPayload([1, 2, 3], cpu, cpu))
