"""Same-node hand-off of a KVPayload to another process through HIP IPC handles (GPU).

The reference moves a prefill worker's exported KV to the decode worker on the same GPU by
putting CUDA tensors on a torch.multiprocessing queue (dispec/transport/cuda_ipc.py:20-48,
used by dispec/workers/disaggregated.py:37-75: prefill_export -> send -> recv ->
decode_from_kv's import_contiguous).  Here the sender's gather kernel writes the payload
into shareable regions (HipIpcTransport.export), a second process -- started fresh by
tests/conftest.py before this process touched the GPU -- maps them by handle, scatters them
into its own randomly placed blocks with the import kernel and re-exports them; what it
reads back must equal the oracle's export of the sender's pool bit for bit.
"""

import numpy as np
import pytest
import torch

from oracle import ref_cpu
from tests._util import bits

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _source(L, NB, bs, KVH, D, T, seed):
    from dispec_amd.kv.paged_cache import PagedKVCache
    cache = PagedKVCache(L, NB, bs, KVH, D, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(seed)
    for pool in (cache.key, cache.value):
        for layer in range(L):
            pool[layer].normal_(generator=g)
    ids = torch.randperm(NB, generator=torch.Generator().manual_seed(seed + 1))[:-(-T // bs)]
    return cache, ids.tolist()


def _hand_off(ipc_peer, cache, ids, T, report, seed, copy_path=False, **meta):
    from dispec_amd.transport.base import KVPayload
    from dispec_amd.transport.ipc import HipIpcTransport
    tr = HipIpcTransport(ipc_peer["msg"], ipc_peer["ack"])
    ipc_peer["cmd"].put(dict(layers=cache.num_layers, num_blocks=cache.num_blocks + 7,
                             block_size=cache.block_size, kv_heads=cache.num_kv_heads,
                             head_dim=cache.head_dim, seed=seed, report=report))
    tokens = list(range(1000, 1000 + T))
    if copy_path:   # an ordinary torch payload: sent through one copy into a region
        payload = KVPayload.export(cache, ids, tokens, **meta)
    else:           # gathered straight into shareable regions
        payload = tr.export(cache, ids, tokens, **meta)
    tr.send(payload)
    res = ipc_peer["res"].get(timeout=180)
    assert res["ok"], res.get("error")
    tr.release()                 # waits for the peer's acknowledgement
    assert tr.in_flight == 0
    assert res["tokens"] == T and res["meta"] == meta
    assert tuple(res["shape"]) == (cache.num_layers, T, cache.num_kv_heads, cache.head_dim)
    return res["result"]


@pytest.mark.parametrize("copy_path", [False, True], ids=["exported-region", "torch-tensor"])
def test_small_ragged_payload_bit_exact(ipc_peer, copy_path):
    """3 layers, 8 KV heads of 128, 300 tokens (the last block partial)."""
    cache, ids = _source(3, 40, 16, 8, 128, 300, 8100)
    k, v = _hand_off(ipc_peer, cache, ids, 300, "bytes", 8200, copy_path, request_id=7)
    for got, pool in ((k, cache.key), (v, cache.value)):
        ref = ref_cpu.export_contiguous(bits(pool), ids, 300, 16)
        assert np.array_equal(got.view(np.uint16), ref)


def _row_checksums(a: np.ndarray) -> np.ndarray:
    """The peer's per-(layer, token) checksum: sum of int32 word * (index + 1) in int64."""
    L, T = a.shape[0], a.shape[1]
    words = np.ascontiguousarray(a).view(np.int32).reshape(L, T, -1).astype(np.int64)
    return (words * np.arange(1, words.shape[-1] + 1, dtype=np.int64)).sum(axis=-1)


def test_config5_request_payload(ipc_peer):
    """One config-5 request: Qwen3-1.7B geometry (28 layers, 8 KV heads of 128), 4096
    tokens -- 235 MB each of K and V in one region apiece -- checked per layer against
    the oracle's export of the sender's pool, row by row: a position-weighted checksum of
    each (layer, token) row's words, so a row landing in another row's place (the error a
    scatter through the wrong block makes) fails at that row."""
    cache, ids = _source(28, 300, 16, 8, 128, 4096, 8300)
    k_sums, v_sums = _hand_off(ipc_peer, cache, ids, 4096, "checksum", 8400, request_id=1,
                               first_token=42)
    for got, pool in ((k_sums, cache.key), (v_sums, cache.value)):
        ref = _row_checksums(ref_cpu.export_contiguous(bits(pool), ids, 4096, 16))
        assert got.shape == (28, 4096)
        bad = np.argwhere(got != ref)
        assert bad.size == 0, f"{len(bad)} rows differ, first (layer, token) {bad[0].tolist()}"
