"""Escalation helpers: hand a prompt's KV from a small model to a large one.

Same contract as the reference (dispec/workers/escalation.py:28-77): only n-1 prompt
tokens are transferred -- the last prompt token is forwarded by the target itself to
produce the logits of the first output token.  The export is the block-table gather
kernel, the map runs on the MFMA map GEMM and the fp32 RoPE kernel.

The reference hands the mapped KV to its scheduler (`escalate` ->
`add_request(prefix_kv=...)`), which checks it (scheduler.py:103-112) and scatters it
into the request's blocks at admission (:161-170).  The scheduler is not part of this
package, so `admit_prefix` is that admission step on its own: the same check and
messages, then the import, leaving the block table holding the covered tokens.
"""

from __future__ import annotations

import torch

from dispec_amd.engine.model_runner import ModelRunner, SeqMeta
from dispec_amd.kv.block_manager import BlockTable
from dispec_amd.kv.paged_cache import PagedKVCache
from dispec_amd.kv.transfer import CrossModelKVMap, rope_tables


def map_prefix(source_runner: ModelRunner, source_cache: PagedKVCache, block_ids: list[int],
               n_tokens: int, kv_map: CrossModelKVMap, target_runner: ModelRunner,
               use_residual: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    """(k, v) of shape (target_layers, n_tokens - 1, H, D): the first n-1 tokens of a
    source sequence mapped into the target's layout (escalation.py:28-47)."""
    covered = n_tokens - 1
    k, v = source_cache.export_contiguous(block_ids, covered)
    at = torch.arange(covered, device=k.device)
    return kv_map.map(k, v, rope_tables(source_runner.rotary_emb, at),
                      rope_tables(target_runner.rotary_emb, at), use_residual)


@torch.inference_mode()
def prefill_and_map(source_runner: ModelRunner, source_cache: PagedKVCache, sid: int,
                    prompt_ids: list[int], kv_map: CrossModelKVMap, target_runner: ModelRunner,
                    use_residual: bool = True):
    """Prefill the prompt on the source model, return its KV mapped for the target, and
    free the source sequence (escalation.py:50-69)."""
    n = len(prompt_ids)
    table = source_cache.manager.allocate(sid, n)
    dev = source_runner.device
    slots = source_cache.context_slots(table.block_ids, n)
    table.num_tokens = n
    source_runner.forward(torch.tensor(prompt_ids, device=dev), torch.arange(n, device=dev),
                          slots, [SeqMeta(table.block_ids, n, n)], source_cache)
    try:
        return map_prefix(source_runner, source_cache, table.block_ids, n, kv_map,
                          target_runner, use_residual)
    finally:
        source_cache.manager.free(sid)


def admit_prefix(target_cache: PagedKVCache, seq_id: int, prompt_ids: list[int],
                 mapped_kv) -> BlockTable:
    """Admit sequence `seq_id` to the target cache with transferred KV.

    Checks `mapped_kv` against the cache layout and the prompt (ValueError with the
    reference scheduler's messages, before any block is taken), allocates the prompt's
    blocks, scatters the KV into them and sets the table's token count to the tokens it
    covers; the caller forwards the remaining prompt tokens (normally the last one).
    """
    n = len(prompt_ids)
    target_cache.check_prefix_kv(mapped_kv, n)
    table = target_cache.manager.allocate(seq_id, n)
    try:
        table.num_tokens = target_cache.admit_prefix(table.block_ids, mapped_kv, n)
    except BaseException:
        target_cache.manager.free(seq_id)
        raise
    return table
