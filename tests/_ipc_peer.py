"""Receiving end of the HIP IPC hand-off tests (tests/test_gpu_ipc.py).

Runs in its own process, started by tests/conftest.py with the multiprocessing "spawn"
context right after collection, before the test process touches the GPU: a fresh
interpreter, never a fork or an exec of a process that has a GPU context.  For each command
it builds its own paged cache, receives one payload through HipIpcTransport, scatters it
into randomly placed blocks of its cache with the import kernel, re-exports those blocks
with the gather kernel and reports what it read back (bytes for small payloads, per-layer
position-weighted checksums of every row for large ones).
"""

from __future__ import annotations


def _row_checksums(t):
    """One int64 per (layer, token) row: sum over the row's int32 words of word * (i + 1).
    Compared position by position, a moved, swapped or reordered row or word shows."""
    import torch
    L, T = t.shape[0], t.shape[1]
    words = t.contiguous().view(torch.int32).reshape(L, T, -1).to(torch.int64)
    weight = torch.arange(1, words.shape[-1] + 1, dtype=torch.int64, device=t.device)
    return (words * weight).sum(dim=-1).cpu().numpy()


def serve(cmd_q, res_q, msg_q, ack_q) -> None:
    import torch
    torch.cuda.set_device(0)
    from dispec_amd.kv.paged_cache import PagedKVCache
    from dispec_amd.transport.ipc import HipIpcTransport
    tr = HipIpcTransport(msg_q, ack_q)
    while True:
        cmd = cmd_q.get()
        if cmd is None:
            return
        try:
            cache = PagedKVCache(cmd["layers"], cmd["num_blocks"], cmd["block_size"],
                                 cmd["kv_heads"], cmd["head_dim"], dtype=torch.bfloat16)
            payload = tr.recv()
            T = payload.seq_len
            need = -(-T // cmd["block_size"])
            gen = torch.Generator().manual_seed(cmd["seed"])
            ids = torch.randperm(cmd["num_blocks"], generator=gen)[:need].tolist()
            shape = tuple(payload.k.shape)
            payload.import_into(cache, ids)
            tr.done(payload)                          # mapping closed, sender acknowledged
            k, v = cache.export_contiguous(ids, T)    # this process's own copy
            torch.cuda.synchronize()
            if cmd["report"] == "bytes":
                out = (k.view(torch.int16).cpu().numpy(), v.view(torch.int16).cpu().numpy())
            else:
                out = (_row_checksums(k), _row_checksums(v))
            res_q.put({"ok": True, "shape": shape, "tokens": len(payload.tokens),
                       "meta": payload.meta, "result": out})
            del cache, k, v
            torch.cuda.empty_cache()
        except Exception as e:   # reported to the test, which fails with it
            res_q.put({"ok": False, "error": f"{type(e).__name__}: {e}"})
