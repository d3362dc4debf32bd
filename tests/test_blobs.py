"""Blob files and the disk-staged read (reference kvsnap/store/blobs.py:78-111, store.py:686-723)."""
import ctypes as C
import hashlib
import os
import struct

import numpy as np
import pytest

import oracle
from kvsnap_amd.blobs import BlobDirectory, CorruptSnapshotError, HEADER, pack_header, parse_header


def records(n, size, seed=0):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, 256, size, dtype=np.uint8).tobytes() for _ in range(n)]


def digests(blocks):
    return [(hashlib.sha256(b).hexdigest(), oracle.crc32c(b)) for b in blocks]


def test_header_is_the_reference_struct_parsed_independently():
    header = pack_header(1000, 0xDEADBEEF)
    assert struct.unpack("<8sIQI8s", header) == (b"KVSBLOB1", 1, 1000, 0xDEADBEEF, bytes(8))
    assert parse_header(header) == (1000, 0xDEADBEEF)
    for bad in (header[:31], b"KVSBLOB2" + header[8:], header[:8] + struct.pack("<I", 2) + header[12:],
                header[:24] + b"\x01" + header[25:]):
        with pytest.raises(CorruptSnapshotError):
            parse_header(bad)


def test_blob_files_match_the_reference_format_and_dedup_by_content(tmp_path):
    store = BlobDirectory(tmp_path, io_backend="native")
    blocks = records(4, 4096)
    blocks.append(blocks[1])                                  # a repeated block is one blob
    segments = store.write_blocks(blocks, digests(blocks))
    assert len(list((tmp_path / "blobs").glob("*.blob"))) == 4
    for block, segment in zip(blocks, segments):
        raw = (tmp_path / "blobs" / (segment["blob_id"] + ".blob")).read_bytes()
        magic, version, length, checksum, reserved = HEADER.unpack(raw[:32])
        assert (magic, version, length, reserved) == (b"KVSBLOB1", 1, 4096, bytes(8))
        assert raw[32:] == block and checksum == oracle.crc32c(block)
        assert hashlib.sha256(raw[32:]).hexdigest() == segment["blob_id"]
    assert [s["first_block"] for s in segments] == list(range(5))
    assert store.write_blob(segments[0]["blob_id"], blocks[0], segments[0]["crc32c"]) is False


def test_read_prepared_into_lands_each_block_in_its_slot_and_checks_crc(tmp_path):
    store = BlobDirectory(tmp_path, io_backend="native")
    size = 65536 + 48
    blocks = records(6, size, seed=3)
    segments = store.write_blocks(blocks, digests(blocks), durable=True)
    target = C.create_string_buffer(size * 6)
    store.read_prepared_into(segments, C.addressof(target), size, workers=3)
    assert target.raw == b"".join(blocks)
    # a restore that skips its first blocks: segments from first_block on are
    # checked against their block index and packed from the buffer's start
    target2 = C.create_string_buffer(size * 4)
    store.read_prepared_into(segments[2:], C.addressof(target2), size, first_block=2)
    assert target2.raw == b"".join(blocks[2:])


def test_a_corrupt_or_missing_blob_is_refused_before_any_copy(tmp_path):
    store = BlobDirectory(tmp_path, io_backend="native")
    blocks = records(3, 8192, seed=4)
    segments = store.write_blocks(blocks, digests(blocks))
    path = tmp_path / "blobs" / (segments[1]["blob_id"] + ".blob")
    raw = bytearray(path.read_bytes())
    raw[-1] ^= 1
    path.write_bytes(bytes(raw))
    target = C.create_string_buffer(8192 * 3)
    with pytest.raises(CorruptSnapshotError, match="checksum"):
        store.read_prepared_into(segments, C.addressof(target), 8192)
    store.read_prepared_into(segments, C.addressof(target), 8192, verify="none")     # left to a GPU check
    os.unlink(path)
    with pytest.raises(CorruptSnapshotError, match="unreadable"):
        store.read_prepared_into(segments, C.addressof(target), 8192)
    bad = dict(segments[0], first_block=5)
    with pytest.raises(CorruptSnapshotError, match="noncontiguous"):
        store.read_prepared_into([bad], C.addressof(target), 8192)
    with pytest.raises(CorruptSnapshotError, match="block size"):
        store.read_prepared_into(segments[:1], C.addressof(target), 4096)
    with pytest.raises(CorruptSnapshotError, match="identifier"):
        store.path("../etc/passwd")


def test_blocks_written_from_memory_in_place_and_dedup_counts(tmp_path):
    store = BlobDirectory(tmp_path, io_backend="native")
    blocks = records(3, 5000, seed=8)
    buf = C.create_string_buffer(b"".join(blocks), 15000)
    parts = [(C.addressof(buf) + i * 5000, 5000) for i in range(3)]
    segments = store.write_blocks(parts, digests(blocks))
    assert store.written == 3 and [s["length"] for s in segments] == [5000] * 3
    for block, segment in zip(blocks, segments):
        assert (tmp_path / "blobs" / (segment["blob_id"] + ".blob")).read_bytes()[32:] == block
    child = blocks[:2] + records(1, 5000, seed=9)
    store.write_blocks(child, digests(child))
    assert store.written == 1 and len(list((tmp_path / "blobs").glob("*.blob"))) == 4


def _chunk(blocks, k, per_chunk):
    return b"".join(blocks[k * per_chunk:(k + 1) * per_chunk])


@pytest.mark.parametrize("per_chunk,slots,workers", [(1, 2, 1), (4, 3, 7), (5, 2, 16), (64, 1, 8)])
def test_the_ring_reader_fills_slots_in_order_and_never_before_their_release(tmp_path, per_chunk, slots, workers):
    """Native readers fill chunk k into slot k % slots only after chunk k - slots was released: a slot still
    holds its chunk's bytes however long the caller keeps it (here: past the time every other read takes)."""
    import time
    store = BlobDirectory(tmp_path, io_backend="native")
    size = 6144
    blocks = records(37, size, seed=11)
    segments = store.write_blocks(blocks, digests(blocks))
    ring = C.create_string_buffer(per_chunk * slots * size)
    chunks = -(-37 // per_chunk)
    with store.ring_reader(segments, C.addressof(ring), size, per_chunk, slots, workers=workers) as reader:
        assert reader.chunks == chunks
        for k in range(chunks):
            reader.wait(k)
            at = (k % slots) * per_chunk * size
            want = _chunk(blocks, k, per_chunk)
            assert ring.raw[at:at + len(want)] == want, k
            time.sleep(0.01)                 # the readers may run ahead into the other slots, never into this one
            assert ring.raw[at:at + len(want)] == want, k
            reader.release(k)
        with pytest.raises(ValueError):
            reader.wait(chunks)


def test_the_ring_reader_reports_each_failure_at_its_chunk_with_the_python_path_s_message(tmp_path):
    """A bad block stops the read: the chunks before it still arrive whole; waiting on its chunk raises the
    message the Python read path raises (checksum, header, payload range, unreadable file)."""
    size = 4096
    for damage, match in [("crc", "block 9 fails its checksum"), ("header", "invalid blob header"),
                          ("short", "unreadable blob"), ("missing", "unreadable blob"),
                          ("range", "block 9 runs past the payload")]:
        folder = tmp_path / damage
        store = BlobDirectory(folder, io_backend="native")
        blocks = records(12, size, seed=12)
        segments = store.write_blocks(blocks, digests(blocks))
        path = folder / "blobs" / (segments[9]["blob_id"] + ".blob")
        raw = bytearray(path.read_bytes())
        if damage == "crc":
            raw[40] ^= 1
        elif damage == "header":
            raw[0:8] = b"KVSBLOB9"
        elif damage == "short":
            raw = raw[:100]
        elif damage == "range":
            segments[9] = dict(segments[9], offset=8)
        if damage == "missing":
            os.unlink(path)
        else:
            path.write_bytes(bytes(raw))
        ring = C.create_string_buffer(4 * 3 * size)
        with store.ring_reader(segments, C.addressof(ring), size, 4, 3, workers=4) as reader:
            for k in range(2):
                reader.wait(k)
                at = (k % 3) * 4 * size
                assert ring.raw[at:at + 4 * size] == _chunk(blocks, k, 4), (damage, k)
                reader.release(k)
            with pytest.raises(CorruptSnapshotError, match=match):
                reader.wait(2)


def test_the_ring_reader_leaves_crc_checks_to_the_caller_when_asked(tmp_path):
    store = BlobDirectory(tmp_path, io_backend="native")
    blocks = records(3, 4096, seed=13)
    segments = store.write_blocks(blocks, digests(blocks))
    path = tmp_path / "blobs" / (segments[1]["blob_id"] + ".blob")
    raw = bytearray(path.read_bytes())
    raw[-1] ^= 1
    path.write_bytes(bytes(raw))
    ring = C.create_string_buffer(3 * 4096)
    with store.ring_reader(segments, C.addressof(ring), 4096, 3, 1, verify="none") as reader:
        reader.wait(0)
    assert ring.raw[4096:8191] == blocks[1][:4095] and ring.raw[8191] == blocks[1][4095] ^ 1
    with pytest.raises(RuntimeError, match="native"):
        with BlobDirectory(tmp_path, io_backend="python").ring_reader(segments, C.addressof(ring), 4096, 3, 1):
            pass


def test_the_read_plan_checks_a_whole_plan_as_the_walk_over_its_segments_does(tmp_path):
    """The read plan's column checks pass exactly the plans that the segment-by-segment walk passes, and a
    plan that fails one gets the walk's error (a newline inside an id, upper-case or non-ASCII hex, a gap, a
    segment of two blocks, a negative offset, a bool offset, a float length, a missing key)."""
    store = BlobDirectory(tmp_path, io_backend="native")
    ids = [hashlib.sha256(bytes([i])).hexdigest() for i in range(5)]
    segments = [dict(blob_id=blob_id, first_block=3 + i, nblocks=1, offset=64 * i, length=4096, crc32c=i)
                for i, blob_id in enumerate(ids)]
    walked = store._read_plan_by_segment(segments, 1 << 20, 4096, 3)
    walk, store._read_plan_by_segment = store._read_plan_by_segment, None      # a valid plan is not walked
    plan = store._read_plan(segments, 1 << 20, 4096, 3)
    store._read_plan_by_segment = walk
    assert plan == walked
    assert plan[4] == (str(store.path(ids[4])), (1 << 20) + 4 * 4096, HEADER.size + 256, 4096, 4, 7)
    assert store._read_plan([], 0, 4096, 0) == []
    bad = [(1, dict(blob_id=ids[1][:30] + "\n" + ids[1][31:]), "identifier"),
           (2, dict(blob_id=ids[2].upper()), "identifier"),
           (4, dict(blob_id=ids[4][:63] + "é"), "identifier"),
           (3, dict(blob_id=ids[3][:63]), "identifier"),
           (0, dict(first_block=9), "noncontiguous"),
           (3, dict(nblocks=2), "noncontiguous"),
           (1, dict(offset=-1), "block size"),
           (2, dict(offset=True), "block size"),
           (2, dict(length=4096.0), "block size")]
    for position, change, match in bad:
        changed = list(segments)
        changed[position] = dict(segments[position], **change)
        with pytest.raises(CorruptSnapshotError, match=match):
            store._read_plan(changed, 1 << 20, 4096, 3)
    changed = list(segments)
    changed[1] = {key: value for key, value in segments[1].items() if key != "crc32c"}
    with pytest.raises(KeyError):
        store._read_plan(changed, 1 << 20, 4096, 3)
