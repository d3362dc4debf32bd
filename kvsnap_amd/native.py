"""Loading ``_native/libkvsnap_hip.so`` and the helpers every launch shares.

* ``resolve_cuda_library`` finds the library without loading it or touching
  the GPU (the reference's lookup contract, ``kvsnap/connector/dataplane.py:
  12-25``, with its ``KVSNAP_CUDA_LIBRARY`` override first).
* ``kernel_library`` loads it once per path, types every kernel entry point
  (``include/kvsnap_kernels.h``) and refuses another kernel ABI.
* ``HostStaging`` holds the small pinned buffers that launch tables cross the
  host link in (see its docstring for why torch's pinned copies are not used).

There is no fallback anywhere: without the library every copy path raises.
"""
from __future__ import annotations

import ctypes as C
from contextlib import contextmanager
import os
from pathlib import Path
import threading

from .pool import declare

NATIVE = Path(__file__).resolve().parent / "_native"
HIP_LIBRARY_NAME = "libkvsnap_hip.so"
KERNEL_ABI_VERSION = 2


def resolve_cuda_library(library=None):
    """The C-ABI library's path, without loading it or touching the GPU.

    Order: the argument, ``KVSNAP_CUDA_LIBRARY`` (the reference's variable),
    ``KVSNAP_HIP_LIBRARY``, then ``kvsnap_amd/_native/libkvsnap_hip.so``.
    """
    for candidate in (library, os.environ.get("KVSNAP_CUDA_LIBRARY"), os.environ.get("KVSNAP_HIP_LIBRARY")):
        if candidate:
            return Path(candidate)
    return NATIVE / HIP_LIBRARY_NAME


#: "result <- arguments" per kernel entry point; "stream" is a hipStream_t as an integer.
KERNEL_SIGNATURES = {
    "kvsnap_cuda_error": "str <-",
    "kvsnap_kernels_abi_version": "int <-",
    "kvsnap_kernels_init": "int <- int",
    "kvsnap_restore_blocks": "int <- ptr ptr i64 ptr ptr ptr ptr i64 i64 int stream",
    "kvsnap_restore_blocks_checked": "int <- ptr ptr i64 ptr ptr ptr ptr i64 int ptr stream",
    "kvsnap_gather_blocks_checked": "int <- ptr ptr i64 ptr ptr ptr ptr i64 ptr i64 int ptr stream",
    "kvsnap_gather_crc32c_fits": "int <- u64",
    "kvsnap_gather_crc32c": "int <- ptr i64 ptr ptr u64 ptr i64 ptr stream",
    "kvsnap_restore_checked_crc32c": "int <- ptr i64 ptr ptr i64 u64 ptr stream",
    "kvsnap_gather_blocks": "int <- ptr i64 ptr ptr ptr ptr i64 i64 ptr i64 int stream",
    "kvsnap_scatter_blocks": "int <- ptr i64 ptr i64 ptr ptr ptr ptr i64 i64 int stream",
    "kvsnap_gather_to_records": "int <- ptr ptr i64 ptr ptr ptr ptr i64 i64 int stream",
    "kvsnap_copy_to_device": "int <- ptr ptr size stream",
    "kvsnap_copy_to_host": "int <- ptr ptr size stream",
    "kvsnap_zero_regions": "int <- ptr ptr ptr i64 stream",
    "kvsnap_synth_decode": "int <- ptr ptr ptr i64 ptr i64 i64 ptr int stream",
    "kvsnap_synth_fill": "int <- u64 int ptr ptr ptr ptr i64 i64 i64 stream",
    "kvsnap_crc32c_workspace_bytes": "size <- u64 i64",
    "kvsnap_crc32c_records": "int <- ptr u64 u64 i64 u32 ptr ptr size stream",
    "kvsnap_crc32c_records_noalloc": "int <- ptr u64 u64 i64 u32 ptr stream",
    "kvsnap_sha256_records": "int <- ptr u64 u64 i64 ptr stream",
    "kvsnap_sha256_blocks": "u64 <- u64",
    "kvsnap_sha256_records_range": "int <- ptr u64 u64 i64 u64 u64 ptr ptr stream",
    "kvsnap_sha256_ranges": "int <- int ptr ptr ptr ptr ptr ptr ptr ptr stream",
    "kvsnap_sha_round_probe": "int <- u32 int ptr stream",
    "kvsnap_read_probe": "int <- ptr u64 ptr stream",
    "kvsnap_copy_probe": "int <- ptr ptr u64 stream",
    "kvsnap_stream_create": "int <- int size*",
    "kvsnap_stream_destroy": "int <- stream",
    "kvsnap_hold_stream": "int <- stream int",
}

_loaded = {}
_load_lock = threading.Lock()


def kernel_library(library=None):
    """The loaded HIP library with its kernel entry points typed; raises if it is not built."""
    path = resolve_cuda_library(library)
    key = str(path)
    with _load_lock:
        lib = _loaded.get(key)
        if lib is None:
            if not path.is_file():
                raise RuntimeError(f"HIP dataplane library not built ({path}); run python -m kvsnap_amd.build")
            lib = C.CDLL(key)
            for name, signature in KERNEL_SIGNATURES.items():
                declare(lib, name, signature)
            version = lib.kvsnap_kernels_abi_version()
            if version != KERNEL_ABI_VERSION:
                raise RuntimeError(f"unsupported kvsnap HIP kernel ABI {version}; rebuild the library")
            _loaded[key] = lib
    return lib


def check(lib, rc):
    """``rc`` of a kernel entry point, or RuntimeError with the library's message if it is negative."""
    if rc < 0:
        raise RuntimeError(lib.kvsnap_cuda_error().decode())
    return rc


def drain(torch, stream):
    """Wait for the work queued on ``stream`` so far, on an event no other thread holds.

    HIP holds a query of an event while another thread synchronizes on that
    same event object (a scheduler thread polling a load's ``progress`` events
    stalled for the whole 21 ms restore while the loader thread waited on the
    last of them).  So the thread that queued the launches waits on an event
    of its own, recorded after them, and the published events are only ever
    queried.
    """
    own = torch.cuda.Event()
    own.record(stream)
    own.synchronize()


class HostStaging:
    """Pinned host buffers for the tables a launch reads (block ids, record addresses) and for the few
    results a launch hands back, reused from call to call.

    A table crosses the host link with the library's own copy
    (``kvsnap_copy_to_device``) on the stream the launch runs on, never with
    torch's ``non_blocking`` copies: for those, torch's pinned allocator
    records an event on the current stream and queries it when the pinned
    tensor is freed.  The data plane's streams are its own and are destroyed
    at ``close``; a pinned tensor outliving them (held by a traceback, say)
    would have its events queried on destroyed streams when it is finally
    freed, which crashed a test process in the HIP runtime.  Here nothing is
    recorded: a borrowed buffer goes back to the free list when the caller's
    ``with`` block ends, which callers place after the stream has drained.
    """

    GRAIN = 64 << 10

    def __init__(self, torch):
        self._torch = torch
        self._lock = threading.Lock()
        self._free = []

    @contextmanager
    def borrow(self, nbytes):
        """A pinned uint8 tensor of at least ``nbytes`` bytes, all the caller's until the block ends."""
        size = max(self.GRAIN, -(-nbytes // self.GRAIN) * self.GRAIN)
        with self._lock:
            fits = [b for b in self._free if b.numel() >= size]
            buffer = min(fits, key=lambda b: b.numel()) if fits else None
            if buffer is not None:
                self._free.remove(buffer)
        if buffer is None:
            buffer = self._torch.empty(size, dtype=self._torch.uint8, pin_memory=True)
        try:
            yield buffer
        finally:
            with self._lock:
                self._free.append(buffer)

    def upload_int64(self, buffer, values, device, stream, lib):
        """``values`` as a new int64 device tensor, copied from ``buffer`` on ``stream``."""
        import numpy as np
        torch = self._torch
        n = len(values)
        if n:
            buffer.numpy()[:8 * n].view(np.int64)[:] = values
        with torch.cuda.stream(stream):
            table = torch.empty(max(n, 1), dtype=torch.int64, device=device)[:n]
        if n:
            check(lib, lib.kvsnap_copy_to_device(table.data_ptr(), buffer.data_ptr(), 8 * n, stream.cuda_stream))
        return table
