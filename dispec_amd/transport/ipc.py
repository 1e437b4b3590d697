"""Same-node KV hand-off between processes through HIP IPC memory handles (zero copy).

Drop-in for the reference's CudaIpcTransport (dispec/transport/cuda_ipc.py:20-48): the same
`make_queue`, `send`, `recv`, `send_sentinel` and `release`, and the same contract -- the
receiving process maps the sender's device memory instead of receiving a copy.  What
differs is where the shared memory comes from:

  * The reference puts torch CUDA tensors on a torch.multiprocessing queue, which shares
    the caching allocator's whole segment behind each tensor.  Such a segment can be far
    larger than the payload (a freed 77 GB pool split into a 470 MB payload still shares
    the 77 GB), and this platform maps shared allocations reliably only below 2 GiB.
  * Here a payload lives in regions of its own: one `hipMalloc` per K and per V, each
    below 2 GiB (`MAX_REGION_BYTES`), shared by a 64-byte `hipIpcGetMemHandle` handle on
    a plain multiprocessing queue.  `export` runs the block-table gather kernel
    (dsp_kv_gather, the J5a kernel) straight into those regions, and the receiver's
    `KVPayload.import_into` runs the scatter kernel (J5c) straight out of the mapped
    memory: the hand-off itself moves no bytes.

Lifetime: the sender keeps a region until the receiver says it is done with it.  With an
acknowledgement queue (`make_queues`), `recv_into` / `done` on the receiving side close the
mapping and acknowledge, and the sender frees acknowledged regions on its next call (or
`release`).  Without one, the sender keeps every region until `release()`, as the
reference keeps its in-flight tensors.  The sender synchronises its stream before a send,
so the receiver never maps a half-written payload; the receiver synchronises before it
closes a mapping.

GPU only: the regions are device memory of the current device (torch's).
"""

from __future__ import annotations

import ctypes
import itertools
import queue as _queue
import time
import weakref

import torch

from dispec_amd.transport.base import KVPayload, Transport

MAX_REGION_BYTES = (2 << 30) - (2 << 20)   # one shared allocation stays below 2 GiB
_HANDLE_BYTES = 64
_LAZY_ENABLE_PEER_ACCESS = 1               # hipIpcMemLazyEnablePeerAccess
_DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


class _IpcHandle(ctypes.Structure):
    # unsigned bytes: a c_char array would read back only up to its first zero byte
    _fields_ = [("reserved", ctypes.c_ubyte * _HANDLE_BYTES)]


_HIP = None


def _hip():
    """The HIP runtime torch loaded into this process (one runtime per process: the library
    is found by path in the process's own mappings, so ctypes gets the same instance)."""
    global _HIP
    if _HIP is not None:
        return _HIP
    if not torch.cuda.is_available():
        raise RuntimeError("HIP IPC needs a GPU; there is no CPU path")
    torch.cuda.init()
    path = None
    with open("/proc/self/maps") as f:
        for line in f:
            if "libamdhip64.so" in line:
                path = line.split()[-1]
                break
    lib = ctypes.CDLL(path or "libamdhip64.so.7")
    P, VP = ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)
    for name, args in (("hipMalloc", [VP, ctypes.c_size_t]), ("hipFree", [P]),
                       ("hipIpcGetMemHandle", [ctypes.POINTER(_IpcHandle), P]),
                       ("hipIpcOpenMemHandle", [VP, _IpcHandle, ctypes.c_uint]),
                       ("hipIpcCloseMemHandle", [P])):
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = ctypes.c_int, args
    lib.hipGetErrorString.restype = ctypes.c_char_p
    lib.hipGetErrorString.argtypes = [ctypes.c_int]
    _HIP = lib
    return lib


def _check(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what} failed: {_hip().hipGetErrorString(status).decode()} "
                           f"(hipError {status})")


class _DeviceMemory:
    """Device memory this object owns (a hipMalloc'd region, or a region of another
    process mapped by handle), released when the last tensor viewing it is gone."""

    def __init__(self, ptr: int, nbytes: int, device: int, release):
        self.ptr, self.nbytes, self.device = ptr, nbytes, device
        self._release = release

    def tensor(self, dtype: torch.dtype, shape: tuple[int, ...], offset: int = 0) -> torch.Tensor:
        """A torch view of [offset, offset + numel * itemsize) that keeps this memory alive."""
        n = 1
        for s in shape:
            n *= s
        nbytes = n * torch.empty((), dtype=dtype).element_size()
        if offset < 0 or offset + nbytes > self.nbytes:
            raise ValueError(f"view of {nbytes} bytes at {offset} outside a {self.nbytes}-byte region")
        owner = self

        class _View:   # __cuda_array_interface__ carrier; the tensor holds it, it holds owner
            __cuda_array_interface__ = {"shape": (nbytes,), "typestr": "|u1",
                                        "data": (self.ptr + offset, False), "version": 2,
                                        "strides": None}
            keep = owner

        raw = torch.as_tensor(_View(), device=f"cuda:{self.device}")
        return raw.view(dtype).view(shape)

    def __del__(self):
        release, self._release = self._release, None
        if release is not None:
            try:
                release(self.ptr)
            except Exception:   # interpreter shutdown: the process exit reclaims it
                pass


def alloc_region(nbytes: int, device: int | None = None) -> _DeviceMemory:
    """A shareable device region of nbytes (< MAX_REGION_BYTES) on `device`."""
    if not 0 < nbytes <= MAX_REGION_BYTES:
        raise ValueError(f"an IPC region holds 1..{MAX_REGION_BYTES} bytes, asked {nbytes}; "
                         "split the payload (e.g. fewer requests per hand-off)")
    lib = _hip()
    dev = torch.cuda.current_device() if device is None else device
    ptr = ctypes.c_void_p()
    with torch.cuda.device(dev):
        _check(lib.hipMalloc(ctypes.byref(ptr), nbytes), "hipMalloc")
    return _DeviceMemory(ptr.value, nbytes, dev, lambda p: lib.hipFree(ctypes.c_void_p(p)))


def _handle_of(mem: _DeviceMemory) -> bytes:
    h = _IpcHandle()
    with torch.cuda.device(mem.device):
        _check(_hip().hipIpcGetMemHandle(ctypes.byref(h), ctypes.c_void_p(mem.ptr)),
               "hipIpcGetMemHandle")
    return bytes(bytearray(h.reserved))


def _open(handle: bytes, nbytes: int, device: int) -> _DeviceMemory:
    lib = _hip()
    h = _IpcHandle()
    if len(handle) != _HANDLE_BYTES:
        raise ValueError(f"an IPC handle has {_HANDLE_BYTES} bytes, got {len(handle)}")
    ctypes.memmove(h.reserved, handle, _HANDLE_BYTES)
    ptr = ctypes.c_void_p()
    with torch.cuda.device(device):
        _check(lib.hipIpcOpenMemHandle(ctypes.byref(ptr), h, _LAZY_ENABLE_PEER_ACCESS),
               "hipIpcOpenMemHandle")
    return _DeviceMemory(ptr.value, nbytes, device,
                         lambda p: lib.hipIpcCloseMemHandle(ctypes.c_void_p(p)))


class HipIpcTransport(Transport):
    """One direction of a same-node hand-off: `send` on one process, `recv` on the other.

    queue: a multiprocessing queue from `make_queue` / `make_queues` (spawn context), shared
    by both ends.  acks: the optional acknowledgement queue of `make_queues`.
    """

    _ids = itertools.count(1)

    def __init__(self, queue, acks=None):
        self._q = queue
        self._acks = acks
        self._inflight: dict[int, tuple] = {}   # sender: id -> regions kept alive
        # sender: data_ptr -> the exported region behind it, held weakly: the payload's
        # tensors keep a region alive, so one exported and dropped unsent frees itself
        self._exported: weakref.WeakValueDictionary = weakref.WeakValueDictionary()
        self._mapped: dict[int, int] = {}       # receiver: id(payload) -> message id

    @staticmethod
    def make_queue(ctx=None):
        """A queue for the hand-off messages (handles and metadata only)."""
        ctx = ctx or torch.multiprocessing.get_context("spawn")
        return ctx.Queue()

    @staticmethod
    def make_queues(ctx=None):
        """(messages, acknowledgements): with acknowledgements the sender frees a payload's
        regions as soon as the receiver is done with them."""
        ctx = ctx or torch.multiprocessing.get_context("spawn")
        return ctx.Queue(), ctx.Queue()

    # -- sending side ---------------------------------------------------------------------
    def export(self, cache, block_ids: list[int], tokens: list[int], **meta) -> KVPayload:
        """Gather a sequence's KV straight into fresh shareable regions (one gather kernel
        launch over all layers) and return it as a payload ready for `send`."""
        L, T = cache.num_layers, len(tokens)
        shape = (L, T, cache.num_kv_heads, cache.head_dim)
        nbytes = L * T * cache.row_bytes
        kmem, vmem = alloc_region(nbytes), alloc_region(nbytes)
        k, v = kmem.tensor(cache.dtype, shape), vmem.tensor(cache.dtype, shape)
        cache._check_blocks(block_ids, T)
        table = cache.block_table([block_ids])
        cu = torch.tensor([0, T], dtype=torch.long).to(cache.key.device)
        flat = (L * T, cache.num_kv_heads, cache.head_dim)
        cache.gather_into(table, cu, T, k.view(flat), v.view(flat))
        cache.check_errors()
        self._exported[k.data_ptr()] = kmem
        self._exported[v.data_ptr()] = vmem
        return KVPayload(list(tokens), k, v, dict(meta))

    def send(self, payload: KVPayload) -> None:
        self._collect_acks(timeout=None)
        msg_id = next(self._ids)
        keep, parts = [], {}
        for name, t in (("k", payload.k), ("v", payload.v)):
            if not t.is_cuda:
                raise RuntimeError("HipIpcTransport sends GPU payloads only")
            t = t.contiguous()
            nbytes = t.numel() * t.element_size()
            mem = self._exported.pop(t.data_ptr(), None)
            if mem is None or mem.nbytes != nbytes:
                # not an exported region: one device copy into a fresh one
                mem = alloc_region(nbytes, t.device.index)
                mem.tensor(torch.uint8, (nbytes,)).copy_(t.reshape(-1).view(torch.uint8))
            keep.append(mem)
            parts[name] = {"handle": _handle_of(mem), "nbytes": nbytes}
        torch.cuda.current_stream().synchronize()    # the receiver maps finished bytes
        self._inflight[msg_id] = (tuple(keep), payload)
        self._q.put({"id": msg_id, "tokens": list(payload.tokens), "meta": dict(payload.meta),
                     "dtype": str(payload.k.dtype).replace("torch.", ""),
                     "shape": tuple(payload.k.shape), "device": payload.k.device.index,
                     "k": parts["k"], "v": parts["v"]})

    def send_sentinel(self) -> None:
        self._q.put(None)

    def _collect_acks(self, timeout: float | None) -> None:
        """Free the regions of acknowledged payloads: those already acknowledged when
        timeout is None, otherwise waiting up to `timeout` seconds for all of them."""
        if self._acks is None:
            return
        deadline = None if timeout is None else time.monotonic() + timeout
        while self._inflight:
            try:
                if deadline is None:
                    msg_id = self._acks.get(block=False)
                else:
                    msg_id = self._acks.get(timeout=max(0.0, deadline - time.monotonic()))
            except _queue.Empty:
                return
            self._inflight.pop(msg_id, None)

    def release(self, timeout: float = 120.0) -> None:
        """Drop every sent payload's regions (reference semantics: call once the consumer
        has mapped them).  With acknowledgements this waits up to `timeout` seconds for the
        outstanding ones and raises TimeoutError, keeping the unacknowledged regions, if
        the receiver has not answered by then (it may have died with the mappings open)."""
        if self._acks is not None:
            self._collect_acks(timeout=timeout)
            if self._inflight:
                raise TimeoutError(f"{len(self._inflight)} sent payloads still unacknowledged "
                                   f"after {timeout:g} s; their regions are kept until "
                                   "release() succeeds or this transport is dropped")
        self._inflight.clear()

    @property
    def in_flight(self) -> int:
        self._collect_acks(timeout=None)
        return len(self._inflight)

    # -- receiving side -------------------------------------------------------------------
    def recv(self) -> KVPayload | None:
        """The next payload, its K and V viewing the sender's memory (None at the sentinel)."""
        msg = self._q.get()
        if msg is None:
            return None
        dtype = _DTYPES[msg["dtype"]]
        dev = torch.cuda.current_device()
        k = _open(msg["k"]["handle"], msg["k"]["nbytes"], dev).tensor(dtype, msg["shape"])
        v = _open(msg["v"]["handle"], msg["v"]["nbytes"], dev).tensor(dtype, msg["shape"])
        payload = KVPayload(msg["tokens"], k, v, msg["meta"])
        self._mapped[id(payload)] = msg["id"]
        return payload

    def done(self, payload: KVPayload) -> None:
        """The receiver is finished with `payload`: wait for the work that reads it, drop
        its mapping and acknowledge, so the sender can free the regions."""
        msg_id = self._mapped.pop(id(payload), None)
        torch.cuda.current_stream().synchronize()
        payload.k = payload.v = None           # the mapping closes with the last view
        if msg_id is not None and self._acks is not None:
            self._acks.put(msg_id)

    def recv_into(self, cache, block_ids_for) -> KVPayload | None:
        """recv, scatter into `cache` (block_ids_for(payload) -> the blocks to fill), done.
        Returns the payload (K/V dropped), or None at the sentinel."""
        payload = self.recv()
        if payload is None:
            return None
        payload.import_into(cache, block_ids_for(payload))
        self.done(payload)
        return payload

