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


def test_release_gives_up_on_a_silent_receiver():
    """A receiver that never acknowledges (it died with the mapping open) makes release()
    raise after its timeout, naming how many payloads are outstanding, instead of hanging."""
    from dispec_amd.transport.ipc import HipIpcTransport
    msgs, acks = HipIpcTransport.make_queues()
    tr = HipIpcTransport(msgs, acks)
    tr._inflight[1] = ((), None)
    tr._inflight[2] = ((), None)
    acks.put(2)
    with pytest.raises(TimeoutError, match="1 sent payloads still unacknowledged"):
        tr.release(timeout=0.5)
    assert list(tr._inflight) == [1]
    acks.put(1)
    tr.release(timeout=5)
    assert tr.in_flight == 0


def test_an_exported_region_dropped_unsent_is_freed():
    """The transport holds exported regions weakly: once the payload's tensors (which keep
    their region alive) are gone, the region is released, not kept until the transport
    dies."""
    import gc

    from dispec_amd.transport.ipc import HipIpcTransport, _DeviceMemory
    freed = []
    tr = HipIpcTransport(HipIpcTransport.make_queue())
    mem = _DeviceMemory(0x1000, 4096, 0, freed.append)   # release records, frees nothing
    tr._exported[0x1000] = mem
    assert len(tr._exported) == 1
    del mem
    gc.collect()
    assert freed == [0x1000] and len(tr._exported) == 0
