"""Host-side choice between fixed key partitions and the balanced split-K kernel for
short query blocks (ModelRunner._prefer_balanced), no GPU: the balanced split for verify
batches whose contexts are skewed (the longest sequence's partitions would run as a
tail), fixed partitions for contexts of similar length, and never for shapes the
balanced kernel does not serve.  The library assumes 256 CUs without a GPU."""

from types import SimpleNamespace

import pytest

from dispec_amd.engine.model_runner import ModelRunner, SeqMeta


@pytest.fixture(scope="module", autouse=True)
def _built():
    from dispec_amd import _lib
    if not _lib.LIB_PATH.exists():
        from dispec_amd.build import build
        build()


def _prefer(ctx, q_len=5, Hq=16, KVH=8, D=128, bs=16):
    r = SimpleNamespace(num_heads=Hq, num_kv_heads=KVH, head_dim=D, kv_groups=Hq // KVH,
                        balanced_key_fraction=0.6, _cus=256, _tuned_attention=True)
    meta = [SeqMeta([], q_len, c) for c in ctx]
    max_ctx = -(-max(ctx) // bs) * bs
    return ModelRunner._prefer_balanced(r, meta, q_len, max_ctx, bs)


def test_skewed_verify_batches_take_the_balanced_split():
    assert _prefer([32768] + [512] * 15)          # measured 44 vs 93 us
    assert _prefer([16384] + [1000] * 31)         # 51 vs 95 us
    assert _prefer([30000, 200, 15000, 100, 28000, 9000, 22000, 500])   # 114 vs 133 us


def test_similar_lengths_keep_fixed_partitions():
    assert not _prefer([2560] * 32)               # 84 vs 88 us
    assert not _prefer([8192] * 16)               # 105 vs 111 us
    assert not _prefer([1152] * 128)              # 138 vs 180 us
    assert not _prefer([2304] * 64)               # 153 vs 159 us


def test_shapes_the_balanced_kernel_does_not_serve():
    assert not _prefer([32768] + [512] * 15, q_len=9)          # 18 rows per KV head
    assert not _prefer([32768] + [512] * 15, Hq=32, KVH=8)     # 5 x 4 = 20 rows
    assert not _prefer([32768] + [16] * 600)                   # B > 512
    assert not _prefer([32768] + [512] * 15, bs=8)
    assert not _prefer([32768] + [512] * 15, D=256)
