"""The C-ABI library loads and exports every symbol include/dispec_hip.h declares.

CPU only: no kernel is launched.  Host-side argument checks that return before any HIP
call are exercised through the ABI as well.
"""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _declared() -> set[str]:
    text = (ROOT / "include" / "dispec_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"^\s*(?:const\s+)?[\w]+\*?\s+\*?(dsp_\w+)\s*\(", text, flags=re.M))


@pytest.fixture(scope="module")
def lib():
    from dispec_amd import _lib
    if not _lib.LIB_PATH.exists():
        from dispec_amd.build import build
        build()
    return _lib.lib()


def test_header_declares_the_expected_entry_points():
    names = _declared()
    for n in ("dsp_kv_append", "dsp_kv_copy_blocks", "dsp_kv_gather", "dsp_kv_scatter",
              "dsp_kv_gather_slots", "dsp_paged_decode", "dsp_paged_decode_workspace_bytes",
              "dsp_error_string"):
        assert n in names, n


def test_library_exports_every_declared_symbol(lib):
    from dispec_amd import _lib
    names = _declared()
    raw = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in names if not hasattr(raw, n)]
    assert not missing, missing
    assert set(_lib.SIGNATURES) == names, "ctypes prototypes out of sync with the header"


def _header_prototypes() -> dict[str, tuple[str, list[str]]]:
    """name -> (return type, parameter types) of every dsp_* declaration, types with the
    parameter names dropped and whitespace normalised ('const int32_t*', 'float', ...)."""
    text = (ROOT / "include" / "dispec_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for ret, name, params in re.findall(
            r"^\s*((?:const\s+)?\w+\s*\*?)\s*(dsp_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.M):
        types = []
        for p in params.split(","):
            p = " ".join(p.replace("*", "* ").split())
            if p != "void":
                types.append(re.sub(r"\s+\w+$", "", p).replace(" *", "*"))
        out[name] = (ret.replace(" ", ""), types)
    return out


def test_ctypes_prototypes_match_header_types():
    """Every argument's ctypes type has the width and kind of the header's C type: a
    pointer for a pointer, c_int64 for int64_t, c_int32 for int32_t / int, c_size_t for
    size_t, c_float for float.  ctypes passes whatever it is told, so an int32 / int64 swap
    here would reach the kernels as a wrong value with no error."""
    from dispec_amd import _lib
    scalar = {"int64_t": ctypes.c_int64, "int32_t": ctypes.c_int32, "int": ctypes.c_int32,
              "size_t": ctypes.c_size_t, "float": ctypes.c_float}
    protos = _header_prototypes()
    assert set(protos) == set(_lib.SIGNATURES)
    for name, (ret, params) in protos.items():
        restype, argtypes = _lib.SIGNATURES[name]
        want_ret = ctypes.c_char_p if ret == "constchar*" else scalar[ret]
        assert restype is want_ret, (name, ret, restype)
        assert len(argtypes) == len(params), (name, len(argtypes), len(params))
        for i, (c_type, ct) in enumerate(zip(params, argtypes)):
            if c_type.endswith("*") or c_type == "dsp_stream_t":   # dsp_stream_t: void*
                ok = ct is ctypes.c_void_p or (
                    c_type.replace("const ", "") == "int64_t*" and ct is _lib._I64P)
            else:
                ok = ct is scalar[c_type]
            assert ok, f"{name} argument {i}: header {c_type!r}, ctypes {ct.__name__}"


def test_status_strings_and_version(lib):
    from dispec_amd import _lib
    assert lib.dsp_version() >= 1
    assert _lib.error_string(0) == "ok"
    assert "invalid argument" in _lib.error_string(_lib.DSP_EINVAL)
    assert "no compiled kernel" in _lib.error_string(_lib.DSP_EUNSUPPORTED)


def test_host_argument_checks_reject_before_launch(lib):
    from dispec_amd import _lib
    # null pools
    assert lib.dsp_kv_append(None, None, 10, 16, None, None, 16, None, 1, 16, None, None) == \
        _lib.DSP_EINVAL
    # empty work is a no-op success even with no device
    fake = ctypes.c_void_p(0x1000)
    assert lib.dsp_kv_append(fake, fake, 10, 16, fake, fake, 16, None, 0, 16, None, None) == 0
    # decode: head_dim 512 has no kernel; a non-power-of-two block size is invalid
    args = dict(B=1, Hq=18, KVH=2, D=512)
    st = lib.dsp_paged_decode(fake, 64 * 18, 64, fake, fake, 64, 128, 64, fake, 4, 16, None, 0,
                              fake, args["B"], args["Hq"], args["KVH"], args["D"], 0.125, 64, 0,
                              None, 0, fake, 64 * 18, 64, _lib.DSP_BF16, None, None)
    assert st == _lib.DSP_EUNSUPPORTED
    st = lib.dsp_paged_decode(fake, 64 * 4, 64, fake, fake, 64, 128, 64, fake, 4, 12, None, 0,
                              fake, 1, 4, 2, 64, 0.125, 48, 0, None, 0, fake, 256, 64,
                              _lib.DSP_BF16, None, None)
    assert st == _lib.DSP_EINVAL


def test_partition_and_workspace_sizing(lib):
    # Qwen3-4B long-context shape: 16 x 32768, KVH 8 -> 1024-token partitions (4096 WGs)
    assert lib.dsp_paged_decode_partition_tokens(16, 8, 128, 32768) == 1024
    # few workgroups: halved until the launch has >= 512 (or the 128-token floor)
    assert lib.dsp_paged_decode_partition_tokens(1, 8, 128, 32768) == 512
    assert lib.dsp_paged_decode_partition_tokens(1, 1, 64, 1000) == 128
    # head_dim 16 stays on the VALU kernel's sizing (power-of-two multiple of 128, <= 512)
    assert lib.dsp_paged_decode_partition_tokens(16, 8, 16, 32768) == 512
    # multi-query, long query blocks (128-row tiles; 256 CUs assumed without a GPU):
    # 96 tiles fill one round of 512 resident tiles with 5 partitions of 1664 keys
    assert lib.dsp_paged_mq_partition_tokens(2, 12, 2, 128, 512, 8192) == 1664
    assert lib.dsp_paged_mq_partition_tokens(4, 32, 8, 128, 512, 4096) == 4096  # 512 tiles
    assert lib.dsp_paged_mq_partition_tokens(2, 16, 4, 64, 1024, 4096) == 1024  # 4 per CU
    # short ones (verify) on 16-row tiles, three resident per CU: 256 tiles of ~2.6k keys
    # fill one round in 3 partitions; 512 tiles of 704 keys stay whole (a split would need
    # a second round and the merge)
    assert lib.dsp_paged_mq_partition_tokens(32, 16, 8, 128, 5, 2688) == 896
    assert lib.dsp_paged_mq_partition_tokens(64, 16, 8, 128, 5, 704) == 768
    assert lib.dsp_paged_mq_partition_tokens(8, 16, 8, 128, 5, 2560) == 384
    # multi-query workspace: 0 sizes the partition the launch picks; DSP_SPLIT_BALANCED the
    # balanced split's pieces, (B*KVH + worker waves) slots of max_q_len * G rows
    from dispec_amd import _lib
    P = lib.dsp_paged_mq_partition_tokens(32, 16, 8, 128, 5, 2688)
    assert lib.dsp_paged_mq_workspace_bytes(32, 16, 8, 128, 5, 2688, 0) == \
        lib.dsp_paged_mq_workspace_bytes(32, 16, 8, 128, 5, 2688, P) == 32 * 8 * 3 * 16 * 130 * 4
    assert lib.dsp_paged_mq_workspace_bytes(32, 16, 8, 128, 5, 2688, _lib.DSP_SPLIT_BALANCED) == \
        (32 * 8 + 1024) * 10 * 130 * 4
    # more than 16 query rows per KV head: no balanced split, no workspace for it
    assert lib.dsp_paged_mq_workspace_bytes(32, 16, 8, 128, 9, 2688, _lib.DSP_SPLIT_BALANCED) == 0
    assert lib.dsp_paged_decode_workspace_bytes(16, 32, 8, 128, 32768, 512) == 16 * 32 * 64 * 130 * 4
    assert lib.dsp_paged_decode_workspace_bytes(4, 14, 2, 64, 500, 512) == 0   # one partition
    # automatic split: room for the balanced split (B*KVH + waves slots of G rows) and for
    # the fixed partitions a slot-table launch of the same shape picks.  Without a GPU the
    # library assumes 256 CUs: one worker wave per SIMD, 256 * 4 = 1024 waves.
    fixed = 16 * 32 * 32 * 130 * 4                  # 1024-token partitions
    balanced = (16 * 8 + 1024) * 4 * 130 * 4
    assert lib.dsp_paged_decode_workspace_bytes(16, 32, 8, 128, 32768, 0) == max(fixed, balanced)
    assert lib.dsp_paged_decode_workspace_bytes(512, 32, 8, 128, 4096, 0) >= \
        (512 * 8 + 1024) * 4 * 130 * 4
    # a small launch: at least 4 units of 16 keys per wave -> 4*2*ceil(500/16)/4 = 64 waves
    assert lib.dsp_paged_decode_workspace_bytes(4, 14, 2, 64, 500, 0) == (4 * 2 + 64) * 7 * 66 * 4
    # the balanced split asked for explicitly: its workspace alone
    assert lib.dsp_paged_decode_workspace_bytes(4, 14, 2, 64, 500, _lib.DSP_SPLIT_BALANCED) == \
        (4 * 2 + 64) * 7 * 66 * 4
    # its unit scans add 64 sequences' 16-key unit counts in 32-bit lanes: contexts up to
    # 2^29 - 16 tokens, none beyond (the automatic split then takes fixed partitions)
    bal = _lib.DSP_SPLIT_BALANCED
    assert lib.dsp_paged_decode_workspace_bytes(1, 2, 1, 64, (1 << 29) - 16, bal) > 0
    assert lib.dsp_paged_decode_workspace_bytes(1, 2, 1, 64, (1 << 29) - 15, bal) == 0
    assert lib.dsp_paged_mq_workspace_bytes(1, 2, 1, 64, 5, (1 << 29) - 15, bal) == 0
    assert lib.dsp_paged_decode_workspace_bytes(1, 2, 1, 64, (1 << 29) - 15, 0) > 0
    assert lib.dsp_paged_decode_workspace_bytes(4, 14, 2, 64, 500, -2) == 0
    assert lib.dsp_paged_decode_workspace_bytes(4, 14, 3, 64, 500, 0) == 0     # 14 % 3 != 0
    # head_dim 256 (generic kernel): 1024-token partitions halved while the launch has fewer
    # than 1024 (sequence, KV head, partition) triples; one partition needs no workspace
    assert lib.dsp_paged_decode_partition_tokens(16, 8, 256, 32768) == 1024
    assert lib.dsp_paged_decode_partition_tokens(1, 2, 256, 4096) == 64
    assert lib.dsp_paged_decode_workspace_bytes(16, 32, 8, 256, 32768, 0) == 16 * 32 * 32 * 258 * 4
    assert lib.dsp_paged_decode_workspace_bytes(1, 4, 2, 256, 64, 0) == 0
    assert lib.dsp_paged_decode_partition_tokens(1, 2, 512, 4096) == 0          # no D=512 kernel
