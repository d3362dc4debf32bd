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
