"""Admission of transferred prefix KV (reference dispec/sched/scheduler.py:103-112).

The reference's scheduler checks a request's `prefix_kv` before admitting it: both
tensors must have this cache's layout (L, T, KVH, D) and T must cover at least one and
fewer than all of the prompt's tokens.  Its own test (tests/test_kv_transfer.py:185-194)
matches the two messages by "fewer than all" and "cache layout".  These run on the host:
the check reads only the cache's geometry and rejects before any block is taken or any
kernel launched.
"""

from types import SimpleNamespace

import pytest
import torch

from dispec_amd.kv.block_manager import BlockManager
from dispec_amd.kv.paged_cache import PagedKVCache, check_prefix_coverage, check_prefix_kv

L, KVH, D = 3, 2, 16


def geometry():
    return SimpleNamespace(num_layers=L, num_kv_heads=KVH, head_dim=D)


def kv(shape):
    return torch.zeros(shape), torch.zeros(shape)


def test_whole_prompt_is_rejected_with_the_reference_message():
    n = 20
    with pytest.raises(ValueError, match="fewer than all") as e:
        check_prefix_kv(geometry(), kv((L, n, KVH, D)), n)
    assert str(e.value) == ("prefix_kv covers 20 tokens of a 20-token prompt; it must cover "
                            "at least one and fewer than all of them")


def test_wrong_layout_is_rejected_with_the_reference_message():
    n = 20
    bad = (L, n - 1, KVH, D // 2)
    with pytest.raises(ValueError, match="cache layout") as e:
        check_prefix_kv(geometry(), kv(bad), n)
    assert str(e.value) == (f"prefix_kv shapes {bad}/{bad} do not match this model's cache "
                            f"layout {(L, n - 1, KVH, D)}")


@pytest.mark.parametrize("k_shape,v_shape", [
    ((L + 1, 5, KVH, D), (L + 1, 5, KVH, D)),    # another model's layer count
    ((L, 5, KVH + 1, D), (L, 5, KVH + 1, D)),    # another head count
    ((L, 5, KVH, D), (L, 4, KVH, D)),            # V covers other tokens than K
    ((L, 5, KVH, D), (L, 5, KVH, D, 1)),         # an extra dimension
])
def test_any_shape_mismatch_is_a_layout_error(k_shape, v_shape):
    with pytest.raises(ValueError, match="cache layout"):
        check_prefix_kv(geometry(), (torch.zeros(k_shape), torch.zeros(v_shape)), 20)


@pytest.mark.parametrize("covered,prompt_len,ok", [
    (0, 20, False), (1, 20, True), (19, 20, True), (20, 20, False), (21, 20, False),
    (1, 1, False), (1, 2, True),
])
def test_coverage_bounds(covered, prompt_len, ok):
    if ok:
        check_prefix_kv(geometry(), kv((L, covered, KVH, D)), prompt_len)
        check_prefix_coverage(covered, prompt_len)
    else:
        with pytest.raises(ValueError, match="at least one and fewer than all"):
            check_prefix_kv(geometry(), kv((L, covered, KVH, D)), prompt_len)


def test_cache_method_and_admission_reject_before_taking_blocks():
    """PagedKVCache.check_prefix_kv is the same check; admit_prefix (via the escalation
    helper) raises before the allocator gives out a block."""
    from dispec_amd.workers.escalation import admit_prefix
    fake = SimpleNamespace(num_layers=L, num_kv_heads=KVH, head_dim=D,
                           manager=BlockManager(8, 16))
    fake.check_prefix_kv = lambda p, n: PagedKVCache.check_prefix_kv(fake, p, n)
    with pytest.raises(ValueError, match="fewer than all"):
        admit_prefix(fake, 1, list(range(20)), kv((L, 20, KVH, D)))
    with pytest.raises(ValueError, match="cache layout"):
        admit_prefix(fake, 1, list(range(20)), kv((L, 19, KVH, D + 1)))
    assert fake.manager.num_free_blocks == 8 and not fake.manager.has_table(1)


def test_map_into_checks_coverage_before_touching_the_gpu():
    from dispec_amd.kv.transfer import CrossModelKVMap, LayerMap
    cfg = SimpleNamespace(num_hidden_layers=1, num_key_value_heads=KVH, head_dim=D,
                          hidden_size=32, num_attention_heads=4, vocab_size=8,
                          _name_or_path="m")
    eye = LayerMap((0,), torch.zeros(KVH * D), weight=torch.eye(KVH * D))
    kmap = CrossModelKVMap([eye], [eye], cfg, cfg)
    k = torch.zeros((1, 20, KVH, D))
    with pytest.raises(ValueError, match="covers 20 tokens of a 20-token prompt"):
        kmap.map_into(k, k, (None, None), (None, None), None, [], prompt_len=20)
