"""ctypes binding of libdispec_hip.so (the C ABI in include/dispec_hip.h).

This is the only place Python touches the native library.  Every entry point takes raw
device pointers, sizes and a hipStream_t; the helpers here turn torch tensors into those
arguments and status codes into the exceptions the reference raises for the same misuse
(ValueError for bad shapes and arguments, RuntimeError for launch failures).

There is no fallback: if the library is missing or fails to load, `lib()` raises, and so
does every kernel wrapper built on it.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libdispec_hip.so"

DSP_BF16, DSP_F16, DSP_F32 = 0, 1, 2
DSP_OK, DSP_EINVAL, DSP_EALIGN, DSP_EUNSUPPORTED, DSP_EWORKSPACE = 0, -1, -2, -3, -4
DSP_ESCRATCH = -5
DSP_NOALLOC_SCRATCH_BYTES = 32 << 20   # fixed workspace of dsp_paged_decode_noalloc
DSP_SPLIT_BALANCED = -1   # partition_tokens of dsp_paged_mq_attention: balanced split-K

# (name, restype, argtypes) for every symbol the header declares.
_P = c_void_p
_I64P = POINTER(c_int64)
SIGNATURES: dict[str, tuple] = {
    "dsp_error_string": (c_char_p, [c_int]),
    "dsp_version": (c_int, []),
    "dsp_kv_append": (c_int, [_P, _P, c_int64, c_int64, _P, _P, c_int64, _P, c_int64, c_int64,
                              _P, _P]),
    "dsp_kv_gather_slots": (c_int, [_P, _P, c_int64, c_int64, _P, c_int64, c_int64, _P, _P,
                                    c_int64, _P, _P]),
    "dsp_kv_copy_blocks": (c_int, [_P, _P, c_int64, c_int64, _P, _P, c_int64, c_int64, c_int64,
                                   c_int64, _P, _P, c_int64, _P, _P]),
    "dsp_kv_copy_block_fanout": (c_int, [_P, _P, c_int64, c_int64, _P, _P, c_int64, c_int64,
                                         c_int64, c_int64, c_int32, _P, c_int64, _P, _P]),
    "dsp_kv_gather": (c_int, [_P, _P, c_int64, c_int64, c_int64, c_int64, c_int32, _P, c_int64,
                              _P, c_int32, c_int64, _P, _P, _P, _P]),
    "dsp_kv_scatter": (c_int, [_P, _P, c_int64, c_int64, c_int64, c_int64, c_int32, _P, c_int64,
                               _P, c_int32, c_int64, _P, _P, _P, _P]),
    "dsp_kv_scatter_ordered": (c_int, [_P, _P, c_int64, c_int64, c_int64, c_int64, c_int32, _P,
                                       c_int64, _P, c_int32, c_int64, _P, _P, _P, _P, _P]),
    "dsp_paged_decode_workspace_bytes": (c_size_t, [c_int32, c_int32, c_int32, c_int32, c_int32,
                                                      c_int32]),
    "dsp_paged_decode_partition_tokens": (c_int, [c_int32, c_int32, c_int32, c_int32]),
    "dsp_paged_decode": (c_int, [_P, c_int64, c_int64, _P, _P, c_int64, c_int64, c_int64,
                                 _P, c_int64, c_int32, _P, c_int64, _P, c_int32, c_int32,
                                 c_int32, c_int32, c_float, c_int32, c_int32, _P, c_size_t,
                                 _P, c_int64, c_int64, c_int32, _P, _P]),
    "dsp_paged_decode_noalloc": (c_int, [_P, c_int64, c_int64, _P, _P, c_int64, c_int64,
                                         c_int64, _P, c_int64, c_int32, _P, c_int64, _P,
                                         c_int32, c_int32, c_int32, c_int32, c_float, c_int32,
                                         c_int32, _P, c_int64, c_int64, c_int32, _P, _P]),
    "dsp_paged_mq_partition_tokens": (c_int, [c_int32] * 6),
    "dsp_paged_mq_workspace_bytes": (c_size_t, [c_int32, c_int32, c_int32, c_int32, c_int32,
                                                c_int32, c_int32]),
    "dsp_paged_mq_attention": (c_int, [_P, c_int64, c_int64, _P, _P, c_int64, c_int64, c_int64,
                                       _P, c_int64, c_int32, _P, _P, c_int32, c_int32, c_int32,
                                       c_int32, c_float, c_int32, c_int32, c_int32, _P, c_size_t,
                                       _P, c_int64, c_int64, c_int32, _P, _P]),
    "dsp_paged_mq_shared_prefix_partition_tokens": (c_int, [c_int32] * 7),
    "dsp_paged_mq_attention_shared_prefix": (
        c_int, [_P, c_int64, c_int64, _P, _P, c_int64, c_int64, c_int64, _P, c_int64, c_int32,
                _P, _P, c_int32, c_int32, c_int32, c_int32, c_float, c_int32, c_int32, c_int32,
                c_int32, _P, c_size_t, _P, c_int64, c_int64, c_int32, _P, _P]),
    "dsp_kv_map_gemm": (c_int, [_P, _I64P, c_int32, c_int64, c_int64, _P, c_int64, _P, c_int64,
                                c_int64, c_int64, c_int64, c_int32, c_int64, c_int64, _P, c_int32,
                                c_int32, c_int32, c_int32, _P]),
    "dsp_kv_map_gemm_to_pool": (c_int, [_P, _I64P, c_int32, c_int64, c_int64, _P, c_int64, _P,
                                        c_int64, c_int64, _P, c_int64, c_int32, c_int64, c_int64,
                                        c_int64, c_int32, c_int64, _P, _P, _P, c_int32, c_int32,
                                        _P, _P]),
    "dsp_kv_rope": (c_int, [_P, c_int64, _P, c_int64, c_int64, c_int64, c_int64, c_int64, _P, _P,
                            c_int32, c_int32, c_int32, _P]),
    "dsp_qk_norm_rope_append": (c_int, [_P, c_int64, c_int64, _P, c_int64, c_int64, _P, c_int64,
                                        c_int64, _P, _P, c_float, _P, _P, c_int64, _P, c_int64,
                                        c_int32, c_int32, c_int32, _P, c_int64, c_int64, _P, _P,
                                        c_int64, c_int64, c_int64, c_int32, _P, _P]),
}

_LIB: ctypes.CDLL | None = None
_CALLS = None

# Entry points a decode step calls once per layer: dispec_amd._fastcall (csrc/fastcall.c)
# binds them with METH_FASTCALL functions that take the same arguments as the ctypes
# functions and skip ctypes' per-argument conversion (~4-5 us a call).
FAST_CALLS = ("dsp_paged_decode", "dsp_kv_append", "dsp_paged_mq_attention",
              "dsp_paged_mq_attention_shared_prefix", "dsp_qk_norm_rope_append")


class HipLibraryError(RuntimeError):
    """libdispec_hip.so is missing or does not export the expected ABI."""


def lib() -> ctypes.CDLL:
    """Load libdispec_hip.so once and bind every symbol of the header."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = Path(os.environ.get("DISPEC_HIP_LIB", LIB_PATH))
    if not path.exists():
        raise HipLibraryError(
            f"{path} is not built; run `python -m dispec_amd.build` (hipcc, gfx950) first")
    try:
        handle = ctypes.CDLL(str(path))
    except OSError as e:  # pragma: no cover - depends on the machine
        raise HipLibraryError(f"cannot load {path}: {e}") from e
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name, None)
        if fn is None:
            raise HipLibraryError(f"{path} does not export {name}")
        fn.restype = restype
        fn.argtypes = argtypes
    _LIB = handle
    return handle


# ctypes argument type -> the type letter dispec_amd._fastcall converts it with
_TYPE_LETTERS = {c_void_p: "P", c_int64: "q", c_int32: "i", c_size_t: "z", c_float: "f"}


def type_letters(argtypes) -> str:
    """The fast binding's signature string for a list of ctypes argtypes ('?' for a type
    the fast binding does not convert)."""
    return "".join(_TYPE_LETTERS.get(t, "?") for t in argtypes)


class _Calls:
    """Attribute access to the library's entry points: the fast binding where there is one
    and its argument types equal the ctypes argtypes, the ctypes function otherwise (same
    arguments, same int status)."""

    def __init__(self, handle: ctypes.CDLL):
        fast = None
        try:
            from dispec_amd import _fastcall as fast
        except ImportError:
            fast = None
        fast_sigs = getattr(fast, "SIGNATURES", {}) if fast is not None else {}
        self.fast_bound: list[str] = []
        for name, (_, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            if name in FAST_CALLS and fast_sigs.get(name) == type_letters(argtypes):
                fast.bind(name, ctypes.cast(fn, c_void_p).value)
                fn = getattr(fast, name)
                self.fast_bound.append(name)
            setattr(self, name, fn)


def calls() -> _Calls:
    """The entry points to call (see _Calls); loads the library on first use."""
    global _CALLS
    if _CALLS is None:
        _CALLS = _Calls(lib())
    return _CALLS


def error_string(status: int) -> str:
    return lib().dsp_error_string(status).decode()


def check(status: int, what: str) -> None:
    """Map a C-ABI status to the exception the reference raises for the same misuse."""
    if status == DSP_OK:
        return
    msg = f"{what}: {error_string(status)} (status {status})"
    if status < 0:
        raise ValueError(msg)
    raise RuntimeError(msg)


_DTYPE_CODES: dict = {}


def dtype_code(dtype) -> int:
    if not _DTYPE_CODES:
        import torch
        _DTYPE_CODES.update({torch.bfloat16: DSP_BF16, torch.float16: DSP_F16,
                             torch.float32: DSP_F32})
    code = _DTYPE_CODES.get(dtype)
    if code is None:
        raise ValueError(f"unsupported dtype {dtype}")
    return code


def ptr(t) -> int | None:
    """Device address of a tensor (None for a missing optional tensor)."""
    return None if t is None else t.data_ptr()


def stream_of(t) -> int:
    """hipStream_t of torch's current stream on the tensor's device."""
    import torch
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is not None:  # the handle itself, without building a torch Stream object
        return raw(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def require_gpu(*tensors) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "dispec_amd kernels run on the GPU only (tensor on "
                f"{t.device}); there is no CPU path")
