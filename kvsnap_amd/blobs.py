"""Snapshot blob files: the on-disk record format and the disk-staged read path.

Format (reference ``kvsnap/store/common.py:10-11``, ``kvsnap/store/blobs.py:94-111``):
a 32-byte little-endian header ``<8sIQI8s`` = (b"KVSBLOB1", version 1, payload
length, CRC32C of the payload, 8 zero bytes), then the payload.  A blob's file
name is its payload's SHA-256 in lowercase hex plus ``.blob``; files are
written to a temporary name, optionally fdatasync'ed, and renamed.

``save`` is the save side: GPU gather, GPU ids and CRCs, blob writes, and
delta saves of a growing session.  ``read_prepared_into`` is the restore's
disk stage (reference
``kvsnap/store/store.py:686-723``): block ``first_block + i`` is pread into
``address + i * block_bytes`` of a pinned buffer, by ``workers`` threads,
under a shared lock on ``<root>/.blob.lock``.  Every block's CRC32C is checked
against its segment before the caller copies anything to the GPU -- on the
host (the reference's way) or, with ``verify="none"``, left to the caller's
GPU check (see ``TorchBlockDataPlane.load_scatter_verified``).
"""
from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor
from contextlib import contextmanager
import ctypes as C
import errno
import fcntl
import os
from pathlib import Path
import re
import struct
import uuid

import numpy as np

from .native_io import NativeIO, get_io_backend

HEADER = struct.Struct("<8sIQI8s")
_BLOB_ID = re.compile("[0-9a-f]{64}")
MAGIC = b"KVSBLOB1"
VERSION = 1


class CorruptSnapshotError(RuntimeError):
    """A blob is missing, truncated, or fails its checksum; nothing was copied to the GPU."""


def pack_header(length: int, crc32c: int) -> bytes:
    return HEADER.pack(MAGIC, VERSION, length, crc32c, b"\0" * 8)


def parse_header(raw: bytes):
    """(payload length, CRC32C) of a header, or CorruptSnapshotError."""
    if len(raw) != HEADER.size:
        raise CorruptSnapshotError("truncated blob header")
    magic, version, length, checksum, reserved = HEADER.unpack(raw)
    if magic != MAGIC or version != VERSION or reserved != b"\0" * 8:
        raise CorruptSnapshotError("invalid blob header")
    return length, checksum


class BlobDirectory:
    """The blob files under ``<root>/blobs``, written and read through one I/O backend."""

    def __init__(self, root, *, io_backend=None):
        self.root = Path(root)
        self.blob_dir = self.root / "blobs"
        self.blob_dir.mkdir(parents=True, exist_ok=True)
        self._blob_dir_str = str(self.blob_dir)
        self.io = get_io_backend(io_backend)

    def path(self, blob_id: str) -> Path:
        if type(blob_id) is not str or not _BLOB_ID.fullmatch(blob_id):
            raise CorruptSnapshotError("invalid blob identifier")
        return self.blob_dir / (blob_id + ".blob")

    def _path_str(self, blob_id: str) -> str:
        """:meth:`path` as a string (a read plan builds thousands of them; pathlib takes 4 us each)."""
        if type(blob_id) is not str or not _BLOB_ID.fullmatch(blob_id):
            raise CorruptSnapshotError("invalid blob identifier")
        return f"{self._blob_dir_str}/{blob_id}.blob"

    def write_blob(self, blob_id, data, crc32c, *, durable=False):
        """Write one blob unless a file of that name already exists (content-addressed dedup).

        ``data`` is bytes-like, or ``(address, size)`` of memory written in
        place (pinned records).  Returns whether a file was written.
        """
        final = self.path(blob_id)
        size = data[1] if isinstance(data, tuple) else len(data)
        if final.exists():
            fd = os.open(final, os.O_RDONLY)
            try:
                length, checksum = parse_header(os.pread(fd, HEADER.size, 0))
                if length != size or checksum != crc32c:
                    raise CorruptSnapshotError("existing blob differs from its content id")
                if durable:
                    # Written earlier without a sync: a durable snapshot now refers to it, so it is made durable
                    # (the caller syncs the directory entry; reference kvsnap/store/blobs.py:80-92).
                    os.fdatasync(fd)
            finally:
                os.close(fd)
            return False
        temporary = self.blob_dir / f"{blob_id}.{uuid.uuid4().hex}.tmp"
        fd = os.open(temporary, os.O_CREAT | os.O_EXCL | os.O_WRONLY, 0o600)
        try:
            self.io.pwrite_all(fd, pack_header(size, crc32c), 0)
            if isinstance(data, tuple):
                self.io.pwrite_at(fd, data[0], size, HEADER.size)
            else:
                self.io.pwrite_all(fd, data, HEADER.size)
            if durable:
                os.fdatasync(fd)
        finally:
            os.close(fd)
        os.replace(temporary, final)
        return True

    def write_blocks(self, blocks, digests, *, durable=False, workers=8):
        """Write each block under its (sha256 hex, crc32c); returns the segments, one per block.

        A block whose id repeats, in this call or an earlier one, is written
        once (reference dedup, kvsnap/connector/volatile.py:261-270,
        kvsnap/store/store.py:623-627).  ``self.written`` counts the files
        this call created.
        """
        if len(blocks) != len(digests):
            raise ValueError("one digest per block is required")
        unique = {}
        for data, (blob_id, crc) in zip(blocks, digests):
            unique.setdefault(blob_id, (data, crc))
        with ThreadPoolExecutor(max_workers=workers, thread_name_prefix="kvsnap-write") as pool:
            written = list(pool.map(lambda item: self.write_blob(item[0], item[1][0], item[1][1], durable=durable),
                                    unique.items()))
        self.written = sum(written)
        if durable:
            self._sync_directory()
        return [dict(blob_id=blob_id, offset=0, length=data[1] if isinstance(data, tuple) else len(data),
                     first_block=index, nblocks=1, crc32c=crc)
                for index, (data, (blob_id, crc)) in enumerate(zip(blocks, digests))]

    def save(self, plane, block_ids, num_kv_tokens, *, previous=None, durable=False, workers=8, fenced=None,
             chunk_bytes=64 << 20):
        """Save a session's blocks as blob files; returns the snapshot ``{block_ids, num_kv_tokens, segments}``.

        The blocks are gathered on the GPU into pinned staging, hashed there
        (SHA-256 id and CRC32C per block) and written under their ids, with
        repeated ids written once.  With ``previous`` (a snapshot of this
        session saved here, or restored into the same block ids), the
        unchanged prefix (:func:`kvsnap_amd.host_tier.unchanged_prefix`)
        keeps its segments, whose blobs already exist, and only the rest is
        gathered, copied, hashed and written: the reference's blob writer
        rehashes every block (``store.py:616-628``).  The segments equal those
        of a full save.  ``fenced.set()`` is called once the GPU blocks may be
        freed, before the hashes and writes.  ``self.gathered_blocks`` counts
        the blocks this call gathered.
        """
        from .host_tier import unchanged_prefix
        block_size, size = plane.block_size, plane.block_bytes
        block_ids = list(block_ids)
        if len(block_ids) != (num_kv_tokens + block_size - 1) // block_size:
            raise ValueError("block count does not cover computed tokens")
        keep = unchanged_prefix(block_ids, previous, block_size)
        for index in range(keep):
            if not self.path(previous["segments"][index]["blob_id"]).exists():
                keep = index
                break
        segments = [dict(segment, first_block=i) for i, segment in enumerate(previous["segments"][:keep])] \
            if keep else []
        fresh = block_ids[keep:]
        self.gathered_blocks = len(fresh)
        self.written = 0
        identity = plane.layout_identity
        if durable and keep:
            # The kept blobs may have been written without a sync; this durable snapshot refers to them.
            self._make_durable(segment["blob_id"] for segment in segments)
        if not fresh:
            if fenced is not None:
                fenced.set()
            return dict(block_ids=block_ids, num_kv_tokens=num_kv_tokens, segments=segments, kv_layout=identity)
        from .dataplane import CopyFailed
        with plane.staging(len(fresh)) as staged:
            digests = []
            try:
                plane.save_gather(fresh, [(staged, i * size) for i in range(len(fresh))],
                                  num_kv_tokens - keep * block_size, chunk_bytes=chunk_bytes, digests=digests)
            except Exception as exc:
                raise CopyFailed("blob save: device-to-host completion could not be proven") from exc
            if fenced is not None:
                fenced.set()
            new = self.write_blocks([(staged.pointer + i * size, size) for i in range(len(fresh))],
                                    digests[0].result(), durable=durable, workers=workers)
        segments += [dict(segment, first_block=keep + segment["first_block"]) for segment in new]
        return dict(block_ids=block_ids, num_kv_tokens=num_kv_tokens, segments=segments, kv_layout=identity)

    def _make_durable(self, blob_ids):
        """fdatasync the blobs ``blob_ids`` and their directory."""
        for blob_id in set(blob_ids):
            fd = os.open(self.path(blob_id), os.O_RDONLY)
            try:
                os.fdatasync(fd)
            finally:
                os.close(fd)
        self._sync_directory()

    def _sync_directory(self):
        fd = os.open(self.blob_dir, os.O_RDONLY | os.O_DIRECTORY)
        try:
            os.fsync(fd)
        finally:
            os.close(fd)

    def _read_plan(self, segments, address, block_bytes, first_block):
        """(blob path, pinned target, payload offset, length, CRC32C, block index) per segment, after checking
        that the segments map blocks ``first_block, first_block + 1, ...`` one whole KV block each.

        The checks run a column at a time (a plan of 2048 blocks took 2.6 ms
        segment by segment, in the restore's time before its first copy); a
        plan that fails one is walked segment by segment for its first error.
        """
        n = len(segments)
        try:
            ids = [segment["blob_id"] for segment in segments]
            firsts = [segment["first_block"] for segment in segments]
            counts = [segment["nblocks"] for segment in segments]
            offsets = [segment["offset"] for segment in segments]
            lengths = [segment["length"] for segment in segments]
            crcs = [segment["crc32c"] for segment in segments]
        except (KeyError, TypeError):
            return self._read_plan_by_segment(segments, address, block_bytes, first_block)
        if not (n and firsts == list(range(first_block, first_block + n)) and counts.count(1) == n
                and set(map(type, offsets)) == {int} and min(offsets) >= 0
                and set(map(type, lengths)) == {int} and lengths.count(block_bytes) == n
                and set(map(type, ids)) == {str}):
            return self._read_plan_by_segment(segments, address, block_bytes, first_block)
        # n ids of 64 lowercase hex digits each: the joined ids are ASCII, n - 1 newlines at every 65th byte
        # and nothing else but hex digits.
        try:
            joined = "\n".join(ids).encode("ascii")
        except UnicodeEncodeError:
            joined = b""
        if (len(joined) != 65 * n - 1 or joined.count(b"\n") != n - 1 or joined[64::65] != b"\n" * (n - 1)
                or joined.translate(None, b"0123456789abcdef\n")):
            return self._read_plan_by_segment(segments, address, block_bytes, first_block)
        prefix = self._blob_dir_str + "/"
        return list(zip([prefix + blob_id + ".blob" for blob_id in ids],
                        [address + i * block_bytes for i in range(n)], [HEADER.size + offset for offset in offsets],
                        lengths, crcs, range(first_block, first_block + n)))

    def _read_plan_by_segment(self, segments, address, block_bytes, first_block):
        plan = []
        for position, segment in enumerate(segments):
            block = first_block + position
            if segment["first_block"] != block or segment["nblocks"] != 1:
                raise CorruptSnapshotError(f"noncontiguous block mapping: segment {position} is not block {block}")
            offset, length = segment["offset"], segment["length"]
            if type(offset) is not int or type(length) is not int or offset < 0 or length != block_bytes:
                raise CorruptSnapshotError(f"segment {position} is not one KV block of the block size "
                                           f"({block_bytes} bytes)")
            plan.append((self._path_str(segment["blob_id"]), address + position * block_bytes, HEADER.size + offset,
                         length, segment["crc32c"], block))
        return plan

    @contextmanager
    def ring_reader(self, segments, ring, block_bytes, per_chunk, slots, *, first_block=0, workers=8,
                    verify="host"):
        """Native threads reading ``segments`` (blocks ``first_block``, ...) into a ring of pinned chunk slots.

        Chunk k is blocks ``[k * per_chunk, (k + 1) * per_chunk)`` of the
        segments; it lands in slot ``k % slots`` of the ring at ``ring`` (each
        slot ``per_chunk * block_bytes`` bytes).  The readers refill a slot only
        after :meth:`BlobRingReader.release` of the chunk it held.  Under the
        shared ``.blob.lock`` for the reader's lifetime; every header is checked
        and, with ``verify="host"``, every block's CRC32C.  Needs the native
        I/O backend.
        """
        if verify not in ("host", "none"):
            raise ValueError("verify must be host or none")
        if not isinstance(self.io, NativeIO):
            raise RuntimeError("the ring reader needs the native I/O backend")
        plan = self._read_plan(segments, 0, block_bytes, first_block)
        with (self.root / ".blob.lock").open("a+b") as lock:
            fcntl.flock(lock, fcntl.LOCK_SH)
            reader = BlobRingReader(self.io, plan, block_bytes, ring, per_chunk, slots, workers, verify == "host")
            try:
                yield reader
            finally:
                reader.close()

    def read_prepared_into(self, segments, address, block_bytes, *, first_block=0, workers=8, verify="host"):
        """Read a snapshot's blocks from their blob files into packed pinned memory.

        Segment i (block ``first_block + i``) lands at ``address + i *
        block_bytes``, read by ``workers`` threads under a shared lock on
        ``<root>/.blob.lock`` (reference ``store.py:686-723``).  Every blob's
        header is checked and the segment must lie inside its payload; with
        ``verify="host"`` each block's CRC32C is compared in place (a
        mismatch raises ``CorruptSnapshotError`` before anything reaches the
        GPU); ``verify="none"`` leaves the comparison to the caller's GPU check.
        """
        if verify not in ("host", "none"):
            raise ValueError("verify must be host or none")
        if isinstance(self.io, NativeIO):
            # One chunk of every block: ``workers`` native threads, none of them holding the interpreter lock.
            if segments:
                with self.ring_reader(segments, address, block_bytes, len(segments), 1, first_block=first_block,
                                      workers=workers, verify=verify) as reader:
                    reader.wait(0)
            else:
                self._read_plan(segments, address, block_bytes, first_block)
            return
        plan = self._read_plan(segments, address, block_bytes, first_block)
        io = self.io

        def fetch(job):
            path, target, payload_at, length, crc, block = job
            try:
                fd = os.open(path, os.O_RDONLY)
            except OSError as exc:
                raise CorruptSnapshotError(f"unreadable blob {os.path.basename(path)}: {exc}") from exc
            try:
                stored, _ = parse_header(io.pread_all(fd, HEADER.size, 0))
                if payload_at - HEADER.size + length > stored:
                    raise CorruptSnapshotError(f"block {block} runs past the payload of {os.path.basename(path)}")
                io.pread_into(fd, target, length, payload_at)
            except OSError as exc:
                raise CorruptSnapshotError(f"unreadable blob {os.path.basename(path)}: {exc}") from exc
            finally:
                os.close(fd)
            if verify == "host" and io.crc32c_at(target, length) != crc:
                raise CorruptSnapshotError(f"block {block} fails its checksum (CRC32C)")

        with (self.root / ".blob.lock").open("a+b") as lock:
            fcntl.flock(lock, fcntl.LOCK_SH)
            with ThreadPoolExecutor(max_workers=workers, thread_name_prefix="kvsnap-read") as pool:
                for _ in pool.map(fetch, plan):
                    pass


class BlobRingReader:
    """The native blob ring reader (``kvsnap_blob_reader_*`` in ``libkvsnap_io.so``) over one read plan.

    Errors are raised as :class:`CorruptSnapshotError` with the messages of
    the Python read path: an unreadable blob, an invalid header, a block past
    its blob's payload, a CRC32C mismatch.
    """

    def __init__(self, io, plan, block_bytes, ring, per_chunk, slots, workers, verify):
        if type(per_chunk) is not int or type(slots) is not int or per_chunk < 1 or slots < 1:
            raise ValueError("a ring needs at least one slot of at least one block")
        if type(workers) is not int or not 1 <= workers <= 64:
            raise ValueError("1-64 read workers")
        self.lib, self.plan = io.lib, plan
        n = len(plan)
        self.chunks = -(-n // per_chunk)
        # The paths as one buffer of NUL-terminated names and a table of pointers into it (one encode and a
        # vector pass, where a bytes object and a ctypes pointer per path took about 1 ms for 2048 blocks).
        self._names = os.fsencode("\0".join(job[0] for job in plan)) + b"\0" if n else b""
        ends = np.flatnonzero(np.frombuffer(self._names, dtype=np.uint8) == 0)
        if len(ends) != n:
            raise CorruptSnapshotError("a blob path holds a NUL byte")
        base = C.cast(C.c_char_p(self._names), C.c_void_p).value
        self._paths = np.concatenate(([0], ends[:-1] + 1)).astype(np.uint64)[:n] + np.uint64(base or 0)
        self._offsets = np.array([job[2] - HEADER.size for job in plan], dtype=np.uint64)
        self._crcs = np.array([job[4] & 0xFFFFFFFF for job in plan], dtype=np.uint32)
        self.handle = self.lib.kvsnap_blob_reader_start(
            self._paths.ctypes.data, self._offsets.ctypes.data, self._crcs.ctypes.data, n,
            block_bytes, ring, per_chunk, slots, workers, 1 if verify else 0)
        if not self.handle:
            raise RuntimeError("the blob ring reader could not be started")

    def _raise(self, code, failed):
        path, block = os.path.basename(self.plan[failed][0]), self.plan[failed][5]
        if code == errno.EILSEQ:
            raise CorruptSnapshotError(f"block {block} fails its checksum (CRC32C)")
        if code == errno.ERANGE:
            raise CorruptSnapshotError(f"block {block} runs past the payload of {path}")
        if code == errno.EBADMSG:
            raise CorruptSnapshotError(f"invalid blob header ({path})")
        raise CorruptSnapshotError(f"unreadable blob {path}: {os.strerror(code)}")

    def wait(self, k):
        """Return once chunk k is in its slot; raise the first failure at or before chunk k's end."""
        failed = C.c_int64(-1)
        code = self.lib.kvsnap_blob_reader_wait(self.handle, k, C.byref(failed))
        if code == errno.EINVAL and failed.value < 0:
            raise ValueError(f"no chunk {k} in this read")
        if code:
            self._raise(code, failed.value)

    def release(self, k):
        """Chunk k's slot may be refilled (its bytes are copied out)."""
        if self.lib.kvsnap_blob_reader_release(self.handle, k):
            raise ValueError(f"no chunk {k} in this read")

    def close(self):
        """Stop the readers and wait for them: the ring may be freed afterwards."""
        if self.handle:
            handle, self.handle = self.handle, None
            self.lib.kvsnap_blob_reader_finish(handle, None)
