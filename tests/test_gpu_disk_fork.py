"""The disk-staged restore with fork dedup (the fourth workload), at a reduced size, against the oracle.

A parent session is saved as blob files; a forked child whose first blocks
hold byte-identical copies of the parent's (in blocks of its own) plus new
blocks is saved into the same directory.  The blob ids must dedup exactly
the shared content: every snapshot's ids and CRC32Cs equal the oracle's
digests of the oracle's records, the directory holds one file per distinct
record, the child's shared blocks name the parent's blobs and no other.  The
child is then restored from disk through the pipelined reader (pread into a
pinned ring, CRC32C checked on the GPU and on the host), and the cache must
equal the oracle's scatter of the child's records into the targets
(reference kvsnap/store/store.py:616-627, 686-723; results/restore-qwen3-8b.json).
"""
import os
import random

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from kvsnap_amd import synth
from kvsnap_amd.blobs import HEADER, BlobDirectory
from kvsnap_amd.dataplane import TorchBlockDataPlane

pytestmark = pytest.mark.gpu

LAYERS, BLOCKS, BLOCK_SIZE = 36, 640, 16
SESSION, SHARED = 160, 120          # blocks of each session; the child's first SHARED copy the parent's


@pytest.mark.parametrize("verify", ["gpu", "host"])
def test_a_forked_child_dedups_exactly_its_shared_blocks_and_restores_from_disk(hip_library, oracle_lib, tmp_path,
                                                                               verify):
    caches, backing = synth.make_caches(LAYERS, BLOCKS, layout="kv_split")
    plane = TorchBlockDataPlane(caches, BLOCK_SIZE, 2 * SESSION * LAYERS * 65536 + (64 << 20))
    try:
        plane.warm_up()
        keep = synth.fill(plane, 21)
        torch.cuda.synchronize()
        del keep
        size = plane.block_bytes
        rng = random.Random(8)
        order = rng.sample(range(1, BLOCKS), 3 * SESSION + SHARED)
        parent = order[:SESSION]
        copies = order[SESSION:SESSION + SHARED]            # the child's own blocks holding the parent's bytes
        fresh = order[SESSION + SHARED:2 * SESSION]
        target = order[2 * SESSION:3 * SESSION]
        child = copies + fresh
        backing[:, :, torch.tensor(copies, device="cuda")] = backing[:, :, torch.tensor(parent[:SHARED], device="cuda")]
        torch.cuda.synchronize()
        host = backing.view(torch.uint8).cpu().numpy().reshape(-1).copy()
        base = backing.data_ptr()
        spans = [(host.ctypes.data + (s[1] - base), s[2], s[0], s[3]) for s in plane.spans()]

        store = BlobDirectory(tmp_path)
        snapshots = {name: store.save(plane, ids, SESSION * BLOCK_SIZE, durable=True)
                     for name, ids in (("parent", parent), ("child", child))}
        records = {name: oracle_lib.gather(spans, ids, size) for name, ids in (("parent", parent), ("child", child))}
        for name, snapshot in snapshots.items():
            crcs, shas = oracle_lib.digest_records(records[name].ctypes.data, size, size, SESSION, threads=8)
            assert [(s["blob_id"], s["crc32c"]) for s in snapshot["segments"]] == \
                [(bytes(h).hex(), int(c)) for h, c in zip(shas, crcs)], name
        unique, _ = oracle_lib.dedup(list(records["parent"]) + list(records["child"]))
        assert len(unique) == 2 * SESSION - SHARED
        assert sorted(os.listdir(tmp_path / "blobs")) == sorted(key + ".blob" for key in unique)
        parent_ids = [s["blob_id"] for s in snapshots["parent"]["segments"]]
        child_ids = [s["blob_id"] for s in snapshots["child"]["segments"]]
        assert child_ids[:SHARED] == parent_ids[:SHARED]
        assert not set(child_ids[SHARED:]) & set(parent_ids)
        for segment, record in zip(snapshots["child"]["segments"][SHARED:SHARED + 4], records["child"][SHARED:]):
            raw = store.path(segment["blob_id"]).read_bytes()
            assert raw[HEADER.size + segment["offset"]:][:segment["length"]] == record.tobytes()

        # The child from disk into fresh blocks: a 24-block chunk, so the reader and the copies overlap.
        backing[:, :, torch.tensor(target, device="cuda")] = 0
        progress = []
        launches = plane.load_from_disk(target, store, snapshots["child"]["segments"], chunk_bytes=24 * size,
                                        verify=verify, progress=progress)
        torch.cuda.synchronize()
        assert launches >= SESSION // 24 and progress[0] == (None, SESSION * size) and progress[-1][1] == 0
        oracle_lib.scatter(spans, target, [records["child"].ctypes.data + i * size for i in range(SESSION)])
        after = backing.view(torch.uint8).cpu().numpy().reshape(-1)
        changed = np.flatnonzero(after != host)
        assert changed.size == 0, f"{changed.size} bytes differ from the oracle's scatter, first at {changed[0]}"
    finally:
        torch.cuda.synchronize()
        plane.close()


def span_rows(plane, ids):
    """Per span of the plane: host copies (numpy uint8, one row of the span's bytes per block of ``ids``), read by
    torch's own indexing from the caches' raw storage bytes."""
    index = torch.tensor(ids, dtype=torch.int64, device="cuda")
    storage = next(iter(plane.caches.values())).untyped_storage()     # every layer carved from one allocation
    flat = torch.empty(0, dtype=torch.uint8, device="cuda").set_(storage)
    rows = []
    for _, base, pitch, nbytes in plane.spans():
        start = base - storage.data_ptr()
        blocks = (storage.nbytes() - start - nbytes) // pitch + 1
        rows.append(flat.as_strided((blocks, nbytes), (pitch, 1), start)[index].contiguous().cpu().numpy())
    return rows


def oracle_records(oracle_lib, plane, ids):
    rows = span_rows(plane, ids)
    spans = [(row.ctypes.data, nbytes, offset, nbytes) for row, (offset, _, _, nbytes) in zip(rows, plane.spans())]
    return oracle_lib.gather(spans, list(range(len(ids))), plane.block_bytes)


def test_the_fourth_workload_at_full_size(hip_library, oracle_lib, tmp_path):
    """The fourth workload as the benchmark runs it: 16384-block Qwen3-8B caches (36 GiB), a 32k-token parent
    (2048 records, 4,831,838,208 B) and a child whose first 1536 blocks hold the parent's bytes in blocks of its
    own, saved as blob files: the ids and CRC32Cs equal the oracle's digests of the oracle's records (gathered from
    host copies of the blocks), the directory holds exactly 2560 blobs and the child names 1536 of the parent's.
    The child restored from disk (pipelined reader, 128 MiB chunks, every CRC32C checked on the GPU before its
    placement) leaves every target block equal to the oracle's record of its child block."""
    num_blocks, n, shared = 16384, 2048, 1536
    caches, backing = synth.make_caches(LAYERS, num_blocks, layout="kv_split")
    plane = TorchBlockDataPlane(caches, BLOCK_SIZE, n * LAYERS * 65536 + (600 << 20), restore_mode="dma")
    try:
        plane.warm_up()
        keep = synth.fill(plane, 0)
        torch.cuda.synchronize()
        del keep
        size = plane.block_bytes
        order = random.Random(9).sample(range(1, num_blocks), 3 * n + shared)
        parent = order[:n]
        copies = order[n:n + shared]
        fresh = order[n + shared:2 * n]
        target = order[2 * n:3 * n]
        child = copies + fresh
        index_copies, index_parent = torch.tensor(copies, device="cuda"), torch.tensor(parent[:shared], device="cuda")
        for view in caches.values():           # [2, blocks, N, H, D]
            view[:, index_copies] = view[:, index_parent]
        torch.cuda.synchronize()
        store = BlobDirectory(tmp_path)
        snapshots = {}
        for name, ids in (("parent", parent), ("child", child)):
            print(f"full-size disk fork: saving the {name}", flush=True)
            snapshots[name] = store.save(plane, ids, n * BLOCK_SIZE, chunk_bytes=512 << 20)
            for first in range(0, n, 512):
                records = oracle_records(oracle_lib, plane, ids[first:first + 512])
                crcs, shas = oracle_lib.digest_records(records.ctypes.data, size, size, len(records), threads=16)
                assert [(s["blob_id"], s["crc32c"]) for s in snapshots[name]["segments"][first:first + 512]] == \
                    [(bytes(h).hex(), int(c)) for h, c in zip(shas, crcs)], (name, first)
        parent_ids = [s["blob_id"] for s in snapshots["parent"]["segments"]]
        child_ids = [s["blob_id"] for s in snapshots["child"]["segments"]]
        assert len(os.listdir(tmp_path / "blobs")) == len(set(parent_ids) | set(child_ids)) == 2 * n - shared
        assert child_ids[:shared] == parent_ids[:shared] and not set(child_ids[shared:]) & set(parent_ids)

        print("full-size disk fork: restoring the child from disk", flush=True)
        index_target = torch.tensor(target, device="cuda")
        for view in caches.values():
            view[:, index_target] = 0
        progress = []
        launches = plane.load_from_disk(target, store, snapshots["child"]["segments"], verify="gpu",
                                        progress=progress)
        torch.cuda.synchronize()
        assert launches == -(-n // ((128 << 20) // size)) and progress[0] == (None, n * size)
        assert progress[-1][1] == 0
        for first in range(0, n, 512):
            want = oracle_records(oracle_lib, plane, child[first:first + 512])
            got = oracle_records(oracle_lib, plane, target[first:first + 512])
            bad = [first + i for i in range(len(want)) if not np.array_equal(want[i], got[i])]
            assert not bad, bad[:8]
    finally:
        torch.cuda.synchronize()
        plane.close()
