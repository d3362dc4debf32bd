"""CPU oracle for the KV snapshot dataplane -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only to check results.  ``kvsnap_amd`` never
imports, links or calls anything here: its paths run on the HIP library and
fail loudly without it.

Contents and what pins each function (paths relative to the simon-jd/kvsnap
tree):

===========================  =====================================  ===========================================
function                     restates                               pinned by
===========================  =====================================  ===========================================
crc32c / crc32c_bitwise      csrc/dataplane/io.cpp:16-47            the reference's known-answer vectors
                                                                    (io_test.cpp:9-10, test_native_io.py:99-103),
                                                                    the compiled reference io.cpp (oracle/_ref),
                                                                    bitwise == SSE4.2, split/extend property
sha256                       hashlib at volatile.py:151,            FIPS 180-4 test vectors; hashlib (OpenSSL)
                             store.py:622                           as a library oracle
gather / scatter             dataplane.py:388-437,                  torch strided views of the reference's own
                             copy_kernel.py:25-40,                  Qwen3-8B fixture (test_scatter_gather.py:
                             test_scatter_gather.py:71-76           137-158, 181-229), brute force on the four
                                                                    stride permutations (:291-317)
zero_tail                    dataplane.py:262-272                   the expected bytes of test_scatter_gather.py
                                                                    :197-204 and :299-308
register_layout              dataplane.py:221-249                   test_kv_layout.py:60-80 accept/reject cases and
                                                                    the fixture's shape/stride/bytes (:181-185)
copy_left / early report     vllm.py:67, 649-679                    test_failure_policy.py:180-206 scenarios
blob header                  store/common.py:10-11, blobs.py:94-108 struct "<8sIQI8s" parsed independently as in
                                                                    test_native_io.py:188-195
dedup                        volatile.py:254-279, store.py:616-627  invariants: equal bytes <=> equal id
fill_span (synthetic input)  none (bench input)                     torch's float->bf16 rounding, moments of N(0,1)
===========================  =====================================  ===========================================
"""
from __future__ import annotations

import ctypes as C
import hashlib
import os
import struct
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "_build" / "liboracle.so"

_lib = None


def build(force: bool = False) -> Path:
    """Compile oracle.c with gcc into oracle/_build/liboracle.so."""
    if LIBRARY.is_file() and not force:
        return LIBRARY
    LIBRARY.parent.mkdir(parents=True, exist_ok=True)
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = ["gcc", "-std=c11", "-O3", "-fPIC", "-shared", "-pthread", "-Wall", "-Wextra", "-Werror",
           str(HERE / "oracle.c"), "-o", str(tmp)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    os.replace(tmp, LIBRARY)
    return LIBRARY


def lib():
    global _lib
    if _lib is None:
        if not LIBRARY.is_file():
            build()
        handle = C.CDLL(str(LIBRARY))
        sig = {
            "oracle_crc32c_bitwise": ([C.c_void_p, C.c_size_t, C.c_uint32], C.c_uint32),
            "oracle_crc32c": ([C.c_void_p, C.c_size_t, C.c_uint32], C.c_uint32),
            "oracle_sha256": ([C.c_void_p, C.c_size_t, C.c_void_p], None),
            "oracle_sha256_select": ([C.c_int], None),
            "oracle_gather": ([C.c_size_t, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                               C.c_size_t, C.c_void_p, C.c_size_t], None),
            "oracle_scatter": ([C.c_size_t, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                C.c_void_p, C.c_size_t], None),
            "oracle_zero_tail": ([C.c_void_p, C.c_size_t, C.c_void_p, C.c_void_p, C.c_int64], None),
            "oracle_span_key": ([C.c_uint64, C.c_uint64, C.c_uint64], C.c_uint64),
            "oracle_fill_span": ([C.c_uint64, C.c_uint64, C.c_uint64, C.c_void_p, C.c_size_t, C.c_int,
                                  C.c_float], None),
            "oracle_to_bf16": ([C.c_float], C.c_uint16),
            "oracle_to_e4m3": ([C.c_float], C.c_uint8),
            "oracle_digest_records": ([C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t, C.c_void_p,
                                       C.c_void_p, C.c_int], C.c_int),
            "oracle_copy_threads": ([C.c_size_t, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                     C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t, C.c_int], C.c_int),
        }
        for name, (args, res) in sig.items():
            fn = getattr(handle, name)
            fn.argtypes, fn.restype = args, res
        _lib = handle
    return _lib


def _buffer(data):
    """(address, length, keepalive) of bytes-like or numpy data."""
    if isinstance(data, np.ndarray):
        arr = np.ascontiguousarray(data)
        return arr.ctypes.data, arr.nbytes, arr
    raw = bytes(data)
    buf = C.create_string_buffer(raw, len(raw))
    return C.addressof(buf), len(raw), buf


# ---------------------------------------------------------------- CRC32C / SHA-256

def crc32c(data, prior: int = 0) -> int:
    addr, n, keep = _buffer(data)
    return int(lib().oracle_crc32c(addr, n, prior))


def crc32c_bitwise(data, prior: int = 0) -> int:
    addr, n, keep = _buffer(data)
    return int(lib().oracle_crc32c_bitwise(addr, n, prior))


def crc32c_at(address: int, size: int, prior: int = 0) -> int:
    return int(lib().oracle_crc32c(address, size, prior))


def sha256(data) -> bytes:
    addr, n, keep = _buffer(data)
    out = C.create_string_buffer(32)
    lib().oracle_sha256(addr, n, out)
    return out.raw


def sha256_select(allow_extensions: bool):
    """Hash with the portable FIPS 180-4 rounds only (False) or with the CPU's SHA extensions (True)."""
    lib().oracle_sha256_select(1 if allow_extensions else 0)


def digest_records(address: int, record_bytes: int, pitch: int, n: int, *, crc=True, sha=True,
                   threads: int = 1):
    """Per-record (CRC32C array uint32, SHA-256 array [n, 32] uint8) of records in host memory."""
    crcs = np.zeros(n, dtype=np.uint32) if crc else None
    shas = np.zeros((n, 32), dtype=np.uint8) if sha else None
    rc = lib().oracle_digest_records(address, record_bytes, pitch, n,
                                     crcs.ctypes.data if crc else None, shas.ctypes.data if sha else None,
                                     threads)
    if rc:
        raise RuntimeError("oracle digest threads failed to start")
    return crcs, shas


# ---------------------------------------------------------------- geometry

def register_layout(name, shape, stride, element_size, block_size, dtype="torch.bfloat16"):
    """TorchBlockDataPlane.__init__'s per-layer rule (dataplane.py:233-247), restated.

    Returns the layer dict the reference records, or raises ValueError.
    """
    if len(shape) != 4 or shape[2] != block_size or stride[3] != 1:
        raise ValueError(f"unsupported KV layout for {name}")
    dense = 1
    for st, size in sorted((stride[i], shape[i]) for i in (1, 2, 3) if shape[i] > 1):
        if st != dense:
            raise ValueError(f"unsupported KV layout for {name}: block has holes or overlapping axes")
        dense *= size
    if stride[0] < dense:
        raise ValueError(f"unsupported KV layout for {name}: overlapping blocks")
    numel = shape[1] * shape[2] * shape[3]
    return {"name": name, "shape": list(shape[1:]), "dtype": dtype, "stride": list(stride[1:]),
            "bytes": numel * element_size}


def gather(spans, block_ids, block_bytes):
    """Records (numpy uint8 [n, block_bytes]) for host-memory spans.

    ``spans`` is a list of (base_address, pitch_bytes, record_offset, nbytes).
    """
    n = len(block_ids)
    out = np.zeros((n, block_bytes), dtype=np.uint8)
    if n == 0:
        return out
    base = np.array([s[0] for s in spans], dtype=np.uint64)
    pitch = np.array([s[1] for s in spans], dtype=np.int64)
    off = np.array([s[2] for s in spans], dtype=np.int64)
    size = np.array([s[3] for s in spans], dtype=np.int64)
    ids = np.array(block_ids, dtype=np.int64)
    lib().oracle_gather(len(spans), base.ctypes.data, pitch.ctypes.data, off.ctypes.data, size.ctypes.data,
                        ids.ctypes.data, n, out.ctypes.data, block_bytes)
    return out


def scatter(spans, block_ids, source_addresses):
    """Write each packed record at source_addresses[i] into block block_ids[i] of the spans."""
    n = len(block_ids)
    if n == 0:
        return
    base = np.array([s[0] for s in spans], dtype=np.uint64)
    pitch = np.array([s[1] for s in spans], dtype=np.int64)
    off = np.array([s[2] for s in spans], dtype=np.int64)
    size = np.array([s[3] for s in spans], dtype=np.int64)
    ids = np.array(block_ids, dtype=np.int64)
    src = np.array(source_addresses, dtype=np.uint64)
    lib().oracle_scatter(len(spans), base.ctypes.data, pitch.ctypes.data, off.ctypes.data, size.ctypes.data,
                         ids.ctypes.data, src.ctypes.data, n)


def zero_tail(record: np.ndarray, layers, valid: int):
    """_zero_tail (dataplane.py:262-272) on one packed record (numpy uint8, modified in place)."""
    offsets, geometry, offset = [], [], 0
    for layer in layers:
        if len(layer["shape"]) == 4:
            # [2, N, H, C] K/V-split layer (an extension of the reference
            # layout): the same rule applied to its K and V halves.
            _, n, h, c = layer["shape"]
            _, sn, sh, _ = layer["stride"]
            half = layer["bytes"] // 2
            esize = half // h // n // c
            for k in range(2):
                offsets.append(offset + k * half)
                geometry.extend([h, n, c, sh, sn, esize])
        else:
            h, n, c = layer["shape"]
            sh, sn, _ = layer["stride"]
            esize = layer["bytes"] // h // n // c
            offsets.append(offset)
            geometry.extend([h, n, c, sh, sn, esize])
        offset += layer["bytes"]
    offs = np.array(offsets, dtype=np.int64)
    geo = np.array(geometry, dtype=np.int64)
    assert record.flags.c_contiguous and record.dtype == np.uint8
    lib().oracle_zero_tail(record.ctypes.data, len(offsets), offs.ctypes.data, geo.ctypes.data, valid)


# ---------------------------------------------------------------- synthetic input

KIND_BF16, KIND_E4M3, KIND_BYTES = 0, 1, 2


def span_key(seed, span, block):
    return int(lib().oracle_span_key(seed, span, block))


def fill_span(seed, span, block, nbytes, kind=KIND_BF16, inv_scale=1.0) -> np.ndarray:
    out = np.empty(nbytes, dtype=np.uint8)
    lib().oracle_fill_span(seed, span, block, out.ctypes.data, nbytes, kind, inv_scale)
    return out


def to_bf16(x: float) -> int:
    return int(lib().oracle_to_bf16(x))


def to_e4m3(x: float) -> int:
    return int(lib().oracle_to_e4m3(x))


# ---------------------------------------------------------------- host-side logic

EARLY_REPORT_BYTES = 128 << 20      # vllm.py:67


def copy_left(progress):
    """vllm.py:672-679: bytes not yet known complete, or None until every launch is queued.

    ``progress`` holds (event-or-None, bytes-left) pairs; an event is a callable
    returning True when complete.
    """
    if not progress or progress[-1][1]:
        return None
    for event, left in reversed(progress):
        if event is None or event():
            return left
    return None


HEADER = struct.Struct("<8sIQI8s")   # store/common.py:10-11
MAGIC = b"KVSBLOB1"


def blob_header(payload: bytes) -> bytes:
    """blobs.py:97: the 32-byte header written before a blob's payload."""
    return HEADER.pack(MAGIC, 1, len(payload), crc32c(payload), b"\0" * 8)


def content_id(data) -> str:
    """A record's blob id: SHA-256 as lowercase hex (blobs.py:33-36, volatile.py:151)."""
    return sha256(data).hex()


def dedup(records):
    """volatile.py:261-270: unique blob ids in first-seen order, and each record's id."""
    seen, ids = {}, []
    for rec in records:
        key = content_id(rec)
        ids.append(key)
        seen.setdefault(key, len(seen))
    return list(seen), ids


def hashlib_sha256(data) -> bytes:
    """The library routine the reference calls, for cross-checks."""
    return hashlib.sha256(bytes(data)).digest()
