"""Host tier: saved KV blocks held in pinned memory by content id, hashed on the GPU, saved by delta.

The reference's host tier (``kvsnap/connector/volatile.py:208-279``) keeps each
saved block in a pinned allocation of its own, keyed by the block's SHA-256.
A block whose id is already held is dropped (its allocation closed), and the
snapshot's segment points at the held copy.  The reference computes every id
on 8 CPU threads after the D2H (``_digest``, ``volatile.py:141-151``), for
every block of every save (``README.md:795``: "Saves rehash every block").

:class:`HostTier` keeps that adoption rule, its capacity accounting and the
prepared record's shape (segments in block order; ``locations`` by blob id),
with two changes on the data path:

* the ids and CRC32Cs come from the GPU
  (``TorchBlockDataPlane.save_gather(..., digests=[])``), computed from the
  save's device staging while the D2H runs;
* ``save(..., previous=snapshot)`` gathers, copies and hashes only the blocks
  past the unchanged prefix (:func:`unchanged_prefix`): positions that hold
  the same block id as the previous snapshot of the session and were full
  there.  vLLM never rewrites a full block while a request holds it, so such
  a block's bytes, and so its id and CRC, are the previous snapshot's.

Lifetimes are reference counts: every snapshot a save returns holds its
blocks until :meth:`HostTier.release`.  The reference's cross-process IPC,
SQLite reconciliation and preparation intents are control plane and are not
mirrored here.
"""
from __future__ import annotations

from contextlib import contextmanager
import threading
import uuid

from .blobs import CorruptSnapshotError
from .dataplane import CopyFailed, PinnedCapacityError
from .layout import require_layout


def unchanged_prefix(block_ids, previous, block_size):
    """How many leading blocks of ``block_ids`` a save may take from ``previous`` unchanged.

    Block i qualifies when the previous snapshot held the same block id at
    position i and that block was full there (i < its tokens // block_size):
    a partial block gains tokens in the next turn, and a different id is
    different memory.
    """
    if not previous:
        return 0
    old = previous["block_ids"]
    limit = min(len(block_ids), len(old), previous["num_kv_tokens"] // block_size, len(previous["segments"]))
    keep = 0
    while keep < limit and block_ids[keep] == old[keep]:
        keep += 1
    return keep


class HostTier:
    """Pinned KV blocks of host-tier snapshots, one allocation per distinct content id."""

    def __init__(self, plane, capacity_bytes):
        if type(capacity_bytes) is not int or capacity_bytes < 0:
            raise ValueError("host tier capacity must be nonnegative")
        self.plane = plane
        self.capacity_bytes = capacity_bytes
        self._lock = threading.RLock()
        self._entries = {}        # blob id -> dict(allocation, handle, crc32c, refs)
        self._resident = 0
        self.gathered_blocks = 0  # blocks the last save gathered and hashed

    def stats(self):
        with self._lock:
            return dict(resident_bytes=self._resident, blob_count=len(self._entries),
                        capacity_bytes=self.capacity_bytes)

    # ------------------------------------------------------------- adoption

    def adopt(self, allocations, digests, *, reuse=(), first_block=None):
        """Hold ``allocations`` under their ``(sha256 hex, crc32c)`` digests; return the segments.

        ``reuse`` are segments of a snapshot this tier still holds, placed
        first; the new blocks follow them.  Every returned segment takes one
        reference.  The allocations are consumed on every path, as in
        ``VolatileOwner.prepare_allocations``: one whose id is already held is
        closed, and on any error every allocation not held before is closed
        and the tier is left as it was.
        """
        allocations = list(allocations)
        reuse = list(reuse)
        first = len(reuse) if first_block is None else first_block
        adopted, added, retained = set(), [], []
        try:
            if len(digests) != len(allocations):
                raise ValueError("one digest per allocation is required")
            with self._lock:
                segments = []
                for index, segment in enumerate(reuse):
                    entry = self._entries.get(segment["blob_id"])
                    if entry is None or entry["crc32c"] != segment["crc32c"] or \
                            entry["allocation"].size != segment["length"]:
                        raise CorruptSnapshotError("previous snapshot's block is no longer held")
                    segments.append(dict(segment, first_block=index))
                used = self._resident
                for index, (allocation, (blob_id, crc)) in enumerate(zip(allocations, digests)):
                    size = allocation.size
                    if type(size) is not int or size <= 0:
                        raise ValueError("empty host-tier block")
                    entry = self._entries.get(blob_id)
                    if entry is None:
                        if used + size > self.capacity_bytes:
                            raise PinnedCapacityError("pinned capacity exhausted; request durable spill explicitly")
                        self._entries[blob_id] = dict(allocation=allocation, handle=uuid.uuid4().hex, crc32c=crc,
                                                      refs=0)
                        added.append(blob_id)
                        adopted.add(id(allocation))
                        used += size
                    elif entry["crc32c"] != crc or entry["allocation"].size != size:
                        raise CorruptSnapshotError("held block differs from its content id")
                    segments.append(dict(blob_id=blob_id, offset=0, length=size, first_block=first + index,
                                         nblocks=1, crc32c=crc))
                for segment in segments:
                    self._entries[segment["blob_id"]]["refs"] += 1
                    retained.append(segment["blob_id"])
                self._resident = used
                return segments
        except BaseException:
            with self._lock:
                for key in retained:
                    self._entries[key]["refs"] -= 1
                for key in added:
                    self._entries.pop(key)["allocation"].close()
            raise
        finally:
            for allocation in allocations:
                if id(allocation) not in adopted:
                    allocation.close()

    def locations(self, segments):
        with self._lock:
            return {s["blob_id"]: dict(handle=self._entries[s["blob_id"]]["handle"], length=s["length"])
                    for s in segments}

    def release(self, snapshot):
        """Drop one snapshot's references; blocks no snapshot holds are freed."""
        with self._lock:
            for segment in snapshot["segments"]:
                entry = self._entries.get(segment["blob_id"])
                if entry is None or entry["refs"] <= 0:
                    raise ValueError("snapshot released more often than it was saved")
                entry["refs"] -= 1
                if entry["refs"] == 0:
                    del self._entries[segment["blob_id"]]
                    self._resident -= entry["allocation"].size
                    entry["allocation"].close()

    def _held_prefix(self, segments):
        with self._lock:
            keep = 0
            for segment in segments:
                entry = self._entries.get(segment["blob_id"])
                if entry is None or entry["crc32c"] != segment["crc32c"]:
                    break
                keep += 1
            return keep

    # ------------------------------------------------------------- data path

    def save(self, block_ids, num_kv_tokens, *, previous=None, chunk_bytes=64 << 20, fenced=None):
        """Save a session's blocks into the tier; returns the snapshot (held until :meth:`release`).

        With ``previous`` (a snapshot of this session saved or restored into
        the same block ids), the unchanged prefix is taken from it, and only
        the rest is gathered, copied to pinned memory and hashed on the GPU.
        The segments equal those of a full save of the same blocks.
        ``fenced.set()`` is called once the copies to pinned memory are done
        and the GPU blocks may be freed, before the hashes are waited for
        (the reference's save job, ``vllm.py:601-608``).
        """
        plane = self.plane
        block_size, size = plane.block_size, plane.block_bytes
        block_ids = list(block_ids)
        if len(block_ids) != (num_kv_tokens + block_size - 1) // block_size:
            raise ValueError("block count does not cover computed tokens")
        keep = unchanged_prefix(block_ids, previous, block_size)
        if keep:
            keep = self._held_prefix(previous["segments"][:keep])
        reuse = previous["segments"][:keep] if keep else []
        fresh = block_ids[keep:]
        allocations = []
        try:
            for _ in fresh:
                allocations.append(plane.pool.reserve(size))
        except BaseException:
            for allocation in allocations:
                allocation.close()
            raise
        digests = []
        if fresh:
            # A failure here leaves the pinned memory to the pool (the DMA may
            # still be using it), as the reference's save does (vllm.py:602-607).
            try:
                plane.save_gather(fresh, [(allocation, 0) for allocation in allocations],
                                  num_kv_tokens - keep * block_size, chunk_bytes=chunk_bytes, digests=digests)
            except Exception as exc:
                raise CopyFailed("host-tier save: device-to-host completion could not be proven") from exc
        if fenced is not None:
            fenced.set()
        ids = digests[0].result() if fresh else []
        self.gathered_blocks = len(fresh)
        segments = self.adopt(allocations, ids, reuse=reuse)
        return dict(block_ids=block_ids, num_kv_tokens=num_kv_tokens, segments=segments,
                    locations=self.locations(segments), kv_layout=plane.layout_identity)

    def restore(self, block_ids, snapshot, *, verify=False, progress=None, chunk_bytes=None):
        """Scatter a held snapshot into ``block_ids``; returns the snapshot as restored there.

        Every block is checked as held before any copy, and the blocks stay
        held until the copies have completed.  ``verify=True`` checks each
        block's CRC32C on the GPU before it reaches the cache
        (``load_scatter_verified``), where the reference checks in place on
        the host (``volatile.py:302-305``); ``verify="checked"`` checks it in
        the restore's own pass (``load_scatter_checked``: no extra pass, but
        on a mismatch the blocks hold the copied bytes and must be treated as
        not restored).  The returned view has no
        references of its own; pass it as ``previous`` to the session's next
        save.
        """
        segments = snapshot["segments"]
        if len(block_ids) != len(segments):
            raise ValueError("one target block per segment is required")
        if verify not in (False, True, "checked"):
            raise ValueError("verify must be False, True or 'checked'")
        require_layout(snapshot, self.plane.layout_identity)
        with self.borrow(segments, snapshot["locations"]) as sources:
            if verify == "checked":
                self.plane.load_scatter_checked(list(block_ids), sources, [s["crc32c"] for s in segments],
                                                progress=progress, chunk_bytes=chunk_bytes)
            elif verify:
                self.plane.load_scatter_verified(list(block_ids), sources, [s["crc32c"] for s in segments],
                                                 progress=progress, chunk_bytes=chunk_bytes)
            else:
                self.plane.load_scatter(list(block_ids), sources, progress=progress, chunk_bytes=chunk_bytes)
        return dict(snapshot, block_ids=list(block_ids))

    @contextmanager
    def borrow(self, segments, locations):
        """The held pinned blocks of ``segments`` as ``(allocation, 0)`` sources, held until the block exits.

        Every block is checked as held (same handle, length and whole-block
        segment) before any is lent, as ``VolatileOwner.borrow`` checks its
        handles (reference ``volatile.py:281-314``); a block no longer held
        raises :class:`CorruptSnapshotError` and nothing is lent.  The caller
        must not exit the block before its copies out of the sources have
        completed (``load_scatter`` returns after its last one).
        """
        with self._lock:
            sources = []
            for segment in segments:
                entry = self._entries.get(segment["blob_id"])
                location = locations.get(segment["blob_id"], {})
                if entry is None or entry["handle"] != location.get("handle") or \
                        entry["allocation"].size != segment["length"] or segment["offset"] != 0:
                    raise CorruptSnapshotError("host-tier block no longer held")
                sources.append((entry["allocation"], 0))
            for segment in segments:
                self._entries[segment["blob_id"]]["refs"] += 1
        try:
            yield sources
        finally:
            self.release(dict(segments=segments))
