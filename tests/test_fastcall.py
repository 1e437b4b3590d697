"""The METH_FASTCALL bindings (dispec_amd._fastcall) against the ctypes functions: same
arguments, same status codes, on calls the library answers on the host (argument checks and
empty launches), so no GPU is needed."""

import ctypes

import pytest

from dispec_amd import _lib

FAST = pytest.importorskip("dispec_amd._fastcall")


def _both(name):
    return getattr(_lib.lib(), name), getattr(_lib.calls(), name)


def test_fast_names_are_bound_to_the_fast_module():
    calls = _lib.calls()
    for name in _lib.FAST_CALLS:
        assert getattr(calls, name) is getattr(FAST, name)
    # every other entry point stays the ctypes function
    assert isinstance(calls.dsp_kv_gather, ctypes._CFuncPtr)


@pytest.mark.parametrize("name", _lib.FAST_CALLS)
def test_fast_signatures_equal_the_ctypes_argtypes(name):
    """The type letters the fast module converts each argument with are the ctypes
    argtypes of the same entry point, position by position (an int32 / int64 swap at any
    position would otherwise reach the kernels as a wrong value)."""
    assert FAST.SIGNATURES[name] == _lib.type_letters(_lib.SIGNATURES[name][1])
    assert name in _lib.calls().fast_bound


def test_a_stale_fast_signature_falls_back_to_ctypes(monkeypatch):
    name = "dsp_kv_append"
    sig = FAST.SIGNATURES[name]
    monkeypatch.setitem(FAST.SIGNATURES, name, sig[:8] + ("i" if sig[8] == "q" else "q") + sig[9:])
    calls = _lib._Calls(_lib.lib())
    assert name not in calls.fast_bound
    assert isinstance(getattr(calls, name), ctypes._CFuncPtr)
    assert getattr(calls, "dsp_paged_decode") is FAST.dsp_paged_decode


@pytest.mark.parametrize("name", _lib.FAST_CALLS)
def test_wrong_argument_count_and_type_raise(name):
    fn = getattr(_lib.calls(), name)
    n = len(_lib.SIGNATURES[name][1])
    with pytest.raises(TypeError, match="takes"):
        fn(*([0] * (n - 1)))
    with pytest.raises(TypeError, match="argument 0"):
        fn("not a pointer", *([0] * (n - 1)))


def test_append_statuses_match():
    slow, fast = _both("dsp_kv_append")
    p = 4096  # any non-null address: the calls below return before touching memory
    ok = (p, p, 16, 128, p, p, 128, p, 0, 128, None, None)        # no tokens
    bad = (None, p, 16, 128, p, p, 128, p, 4, 128, None, None)    # null pool
    assert slow(*ok) == fast(*ok) == _lib.DSP_OK
    assert slow(*bad) == fast(*bad) == _lib.DSP_EINVAL


def test_decode_statuses_match():
    slow, fast = _both("dsp_paged_decode")
    p = 4096

    def args(B, Hq, KVH, dtype=_lib.DSP_BF16):
        return (p, 1024, 128, p, p, 4096, 256, 128, p, 64, 16, None, 0, p, B, Hq, KVH, 128,
                0.088, 1024, 0, None, 0, p, 1024, 128, dtype, None, None)

    assert slow(*args(0, 8, 2)) == fast(*args(0, 8, 2)) == _lib.DSP_OK       # empty batch
    assert slow(*args(-1, 8, 2)) == fast(*args(-1, 8, 2)) == _lib.DSP_EINVAL
    assert slow(*args(2, 8, 3)) == fast(*args(2, 8, 3)) == _lib.DSP_EINVAL   # 8 % 3 != 0
    assert slow(*args(2, 8, 2, 7)) == fast(*args(2, 8, 2, 7)) == _lib.DSP_EUNSUPPORTED


def test_multi_query_statuses_match():
    p = 4096
    head = (p, 1024, 128, p, p, 4096, 256, 128, p, 64, 16, p, p)
    for name, extra in (("dsp_paged_mq_attention", ()),
                        ("dsp_paged_mq_attention_shared_prefix", (512,))):
        slow, fast = _both(name)
        for B, st in ((0, _lib.DSP_OK), (-3, _lib.DSP_EINVAL)):
            a = head + (B, 8, 2, 128, 0.088, 5, 1024) + extra + (0, None, 0, p, 1024, 128,
                                                               _lib.DSP_BF16, None, None)
            assert slow(*a) == fast(*a) == st, (name, B)


def test_prologue_statuses_match():
    slow, fast = _both("dsp_qk_norm_rope_append")
    p = 4096

    def args(T, D):
        return (p, 1024, 128, p, 256, 128, p, 256, 128, None, None, 1e-6, p, p, 128, p, T,
                8, 2, D, p, 1024, 128, p, p, 4096, 256, 128, _lib.DSP_BF16, None, None)

    assert slow(*args(0, 128)) == fast(*args(0, 128)) == _lib.DSP_OK
    assert slow(*args(3, 48)) == fast(*args(3, 48)) == _lib.DSP_EUNSUPPORTED
