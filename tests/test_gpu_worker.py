"""The worker hooks on the GPU: a session saved through them into the host tier and blob files, loaded
into other blocks, and read by the next forward on the engine stream with no host synchronisation.

The forward is ordered after the copy only by what the worker does: an early-reported load's last
event joins the next forward's waits (reference kvsnap/connector/vllm.py:454-467, 649-670).
"""
import random
import time

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from kvsnap_amd import synth
from kvsnap_amd.blobs import HEADER, BlobDirectory
from kvsnap_amd.dataplane import TorchBlockDataPlane
from kvsnap_amd.host_tier import HostTier
from kvsnap_amd.worker import KvsnapMetadata, KvsnapWorker, Transfer

pytestmark = pytest.mark.gpu

LAYERS, BLOCKS, BLOCK_SIZE = 4, 96, 16


def run_until(worker, condition, seconds=60, finished=()):
    """Step boundaries (bind, report, clear) until ``condition(sending, receiving)`` holds; ``finished`` are
    the requests vLLM reports finished at each step."""
    deadline = time.monotonic() + seconds
    while time.monotonic() < deadline:
        worker.bind_connector_metadata(KvsnapMetadata())
        sending, receiving = worker.get_finished(set(finished))
        worker.clear_connector_metadata()
        if condition(sending, receiving):
            return sending, receiving
        torch.cuda.synchronize()
        time.sleep(1e-4)
    raise AssertionError("the worker never reported")


@pytest.mark.parametrize("durability", ["volatile", "durable"])
@pytest.mark.parametrize("verify", ["gpu", "host"])
def test_a_session_saved_and_loaded_through_the_worker_is_what_the_next_forward_reads(hip_library, oracle_lib,
                                                                                      tmp_path, durability, verify):
    caches, backing = synth.make_caches(LAYERS, BLOCKS, layout="kv_split")
    plane = TorchBlockDataPlane(caches, BLOCK_SIZE, 256 << 20)
    plane.warm_up()
    keep = synth.fill(plane, 3)
    torch.cuda.synchronize()
    del keep
    tier = HostTier(plane, 128 << 20)
    # The 10 MiB session is one launch: a 64 MiB threshold reports it as soon as that launch is queued.
    worker = KvsnapWorker(plane, host_tier=tier, blobs=BlobDirectory(tmp_path), verify=verify,
                          early_report_bytes=64 << 20)
    try:
        rng = random.Random(4)
        source = rng.sample(range(1, BLOCKS), 40)
        target = rng.sample([b for b in range(1, BLOCKS) if b not in source], 40)
        src = torch.tensor(source, device="cuda")
        dst = torch.tensor(target, device="cuda")
        expected = backing[:, :, src].clone()
        tokens = 40 * BLOCK_SIZE - 5           # a partial last block: its tail is zeroed in the snapshot

        # Turn end: the save is handed off after this step's kernels, fenced, then prepared.
        worker.bind_connector_metadata(KvsnapMetadata(saves=[Transfer("r", source, durability=durability,
                                                                      num_kv_tokens=tokens)]))
        worker.wait_for_save()
        run_until(worker, lambda sending, receiving: "r" in sending, finished={"r"})    # the blocks are fenced
        run_until(worker, lambda sending, receiving: not worker._saves)                 # and the save is booked
        meta = worker.build_connector_worker_meta()
        assert meta.errors == {}
        snapshot = meta.prepared["r"]
        assert len(snapshot["segments"]) == 40 and snapshot["kv_layout"] == plane.layout_identity

        # The oracle's records of the cache (the last one's tail past the computed tokens zeroed): the
        # snapshot's segments carry their SHA-256 ids and CRC32Cs, and each blob file (durable) holds one.
        size = plane.block_bytes
        host = backing.view(torch.uint8).cpu().numpy().reshape(-1).copy()
        base = backing.data_ptr()
        host_spans = [(host.ctypes.data + (s[1] - base), s[2], s[0], s[3]) for s in plane.spans()]
        records = oracle_lib.gather(host_spans, source, size)
        oracle_lib.zero_tail(records[-1], plane.layers, tokens % BLOCK_SIZE)
        crcs, shas = oracle_lib.digest_records(records.ctypes.data, size, size, len(source), threads=4)
        assert [(s["blob_id"], s["crc32c"]) for s in snapshot["segments"]] == \
            [(bytes(h).hex(), int(c)) for h, c in zip(shas, crcs)]
        if durability == "durable":
            blobs = BlobDirectory(tmp_path)
            for segment, record in zip(snapshot["segments"], records):
                raw = blobs.path(segment["blob_id"]).read_bytes()
                assert raw[HEADER.size + segment["offset"]:][:segment["length"]] == record.tobytes()
        # What the load must leave: the oracle's scatter of those records into the target blocks.
        oracle_lib.scatter(host_spans, target, [records.ctypes.data + i * size for i in range(len(target))])

        # The next turn: load into other blocks; the forward that reads them runs as soon as the
        # load is reported, ordered after the copy on the GPU by the worker's forward waits.
        backing[:, :, dst] = 0
        worker.bind_connector_metadata(KvsnapMetadata(loads=[Transfer("r", target, snapshot=snapshot,
                                                                      durability=durability)]))
        worker.start_load_kv(None)
        deadline = time.monotonic() + 60
        while "r" not in worker.get_finished(set())[1]:
            assert time.monotonic() < deadline, "the load was never reported"
            time.sleep(50e-6)
        worker.bind_connector_metadata(KvsnapMetadata())      # the forward's waits
        restored = backing[:, :, dst].clone()                  # the forward, on the engine stream
        torch.cuda.synchronize()
        # The snapshot's last block carries zeros past the computed tokens.
        expected[:, :, -1, 16 - 5:] = 0
        assert torch.equal(restored.view(torch.int16), expected.view(torch.int16))
        whole = backing.view(torch.uint8).cpu().numpy().reshape(-1)
        changed = np.flatnonzero(whole != host)
        assert changed.size == 0, f"{changed.size} bytes differ from the oracle's scatter, first at {changed[0]}"
        run_until(worker, lambda sending, receiving: not worker._loads)
        loaded = worker.build_connector_worker_meta()
        assert loaded.loaded == ["r"] and loaded.failed_loads == []
        assert worker.get_block_ids_with_load_errors() == set()

        # Prefix caching: the first three blocks are already in the cache and are not copied.
        backing[:, :, dst] = 0
        backing[:, :, dst[:3]] = 1
        worker.bind_connector_metadata(KvsnapMetadata(loads=[Transfer("p", target, snapshot=snapshot,
                                                                      durability=durability, skip_blocks=3)]))
        worker.start_load_kv(None)
        run_until(worker, lambda sending, receiving: "p" in receiving)
        torch.cuda.synchronize()
        assert bool((backing[:, :, dst[:3]] == 1).all())
        assert torch.equal(backing[:, :, dst[3:]].view(torch.int16), expected[:, :, 3:].view(torch.int16))
        run_until(worker, lambda sending, receiving: not worker._loads)
        assert worker.build_connector_worker_meta().failed_loads == []
    finally:
        worker.shutdown()
        torch.cuda.synchronize()
        plane.close()


@pytest.mark.parametrize("restore_mode", ["kernel", "dma"])
def test_a_worker_that_registers_vllm_s_caches_saves_and_loads_what_the_oracle_says(hip_library, oracle_lib,
                                                                                   restore_mode):
    """register_kv_caches (reference vllm.py:226-240): the worker builds and warms the plane and its host
    tier, publishes the layout every snapshot then records, and a turn saved and loaded through the hooks
    leaves the cache equal to the oracle's scatter of the oracle's records."""
    from kvsnap_amd.layout import describe_layer, layout_identity
    caches, backing = synth.make_caches(LAYERS, BLOCKS, layout="vllm")
    worker = KvsnapWorker(host_tier_bytes=64 << 20, block_size=BLOCK_SIZE, capacity_bytes=160 << 20,
                          plane_options={"restore_mode": restore_mode}, verify="gpu")
    try:
        layout = worker.register_kv_caches(caches)
        plane = worker.dataplane
        assert plane.restore_mode == restore_mode and worker.host_tier is not None
        assert layout == layout_identity([describe_layer(n, caches[n], BLOCK_SIZE) for n in sorted(caches)])
        keep = synth.fill(plane, 6)
        torch.cuda.synchronize()
        del keep
        rng = random.Random(12)
        source = rng.sample(range(1, BLOCKS), 24)
        target = rng.sample([b for b in range(1, BLOCKS) if b not in source], 24)
        tokens = 24 * BLOCK_SIZE - 9
        size = plane.block_bytes
        host = backing.view(torch.uint8).cpu().numpy().reshape(-1).copy()
        base = backing.data_ptr()
        host_spans = [(host.ctypes.data + (s[1] - base), s[2], s[0], s[3]) for s in plane.spans()]
        records = oracle_lib.gather(host_spans, source, size)
        oracle_lib.zero_tail(records[-1], plane.layers, tokens % BLOCK_SIZE)

        worker.bind_connector_metadata(KvsnapMetadata(saves=[Transfer("s", source, num_kv_tokens=tokens)]))
        worker.wait_for_save()
        worker.clear_connector_metadata()
        run_until(worker, lambda sending, receiving: "s" in sending, finished={"s"})
        run_until(worker, lambda sending, receiving: not worker._saves)
        snapshot = worker.build_connector_worker_meta().prepared["s"]
        assert snapshot["kv_layout"] == layout
        crcs, shas = oracle_lib.digest_records(records.ctypes.data, size, size, len(source), threads=4)
        assert [(s["blob_id"], s["crc32c"]) for s in snapshot["segments"]] == \
            [(bytes(h).hex(), int(c)) for h, c in zip(shas, crcs)]

        worker.bind_connector_metadata(KvsnapMetadata(loads=[Transfer("l", target, snapshot=snapshot)]))
        worker.start_load_kv(None)
        worker.clear_connector_metadata()
        run_until(worker, lambda sending, receiving: "l" in receiving)
        run_until(worker, lambda sending, receiving: not worker._loads)
        torch.cuda.synchronize()
        report = worker.build_connector_worker_meta()
        assert report.loaded == ["l"] and report.failed_loads == []
        oracle_lib.scatter(host_spans, target, [records.ctypes.data + i * size for i in range(len(target))])
        after = backing.view(torch.uint8).cpu().numpy().reshape(-1)
        changed = np.flatnonzero(after != host)
        assert changed.size == 0, f"{changed.size} bytes differ from the oracle's scatter, first at {changed[0]}"
    finally:
        worker.shutdown()
        torch.cuda.synchronize()
        if worker.dataplane is not None:
            worker.dataplane.close()


def test_the_vllm_connector_class_saves_and_loads_what_the_oracle_says(hip_library, oracle_lib, tmp_path):
    """KvsnapConnector (KVConnectorBase_V1, worker role), imported through stand-in vLLM modules as vLLM would
    build it from its KV-transfer config: register_kv_caches, then one durable save (blob files under
    store_path) and its load into other blocks through the connector's hooks; the snapshot's ids and CRC32Cs
    equal the oracle's digests, and the cache equals the oracle's scatter of the oracle's records."""
    import importlib
    import sys
    from unittest.mock import patch
    from test_connector import BASE, stand_in_vllm, vllm_config
    with patch.dict(sys.modules, stand_in_vllm()):
        sys.modules.pop("kvsnap_amd.connector", None)
        connector_module = importlib.import_module("kvsnap_amd.connector")
    sys.modules.pop("kvsnap_amd.connector", None)
    role = stand_in_vllm()[BASE].KVConnectorRole
    caches, backing = synth.make_caches(LAYERS, BLOCKS, layout="kv_split")
    connector = connector_module.KvsnapConnector(vllm_config(tmp_path, pinned_pool_bytes=160 << 20,
                                                             host_tier_bytes=64 << 20), role.WORKER, None)
    try:
        connector.register_kv_caches(caches)
        plane = connector.worker.dataplane
        keep = synth.fill(plane, 8)
        torch.cuda.synchronize()
        del keep
        rng = random.Random(14)
        source = rng.sample(range(1, BLOCKS), 20)
        target = rng.sample([b for b in range(1, BLOCKS) if b not in source], 20)
        tokens = 20 * BLOCK_SIZE - 3
        size = plane.block_bytes
        host = backing.view(torch.uint8).cpu().numpy().reshape(-1).copy()
        base = backing.data_ptr()
        host_spans = [(host.ctypes.data + (s[1] - base), s[2], s[0], s[3]) for s in plane.spans()]
        records = oracle_lib.gather(host_spans, source, size)
        oracle_lib.zero_tail(records[-1], plane.layers, tokens % BLOCK_SIZE)

        Metadata = connector_module.KvsnapConnectorMetadata
        connector.bind_connector_metadata(Metadata(saves=[Transfer("s", source, durability="durable",
                                                                   num_kv_tokens=tokens)]))
        connector.wait_for_save()
        connector.clear_connector_metadata()
        run_until(connector, lambda sending, receiving: "s" in sending, finished={"s"})
        run_until(connector, lambda sending, receiving: not connector.worker._saves)
        snapshot = connector.build_connector_worker_meta().prepared["s"]
        crcs, shas = oracle_lib.digest_records(records.ctypes.data, size, size, len(source), threads=4)
        assert [(s["blob_id"], s["crc32c"]) for s in snapshot["segments"]] == \
            [(bytes(h).hex(), int(c)) for h, c in zip(shas, crcs)]
        assert all((tmp_path / "blobs" / (s["blob_id"] + ".blob")).is_file() for s in snapshot["segments"])

        connector.bind_connector_metadata(Metadata(loads=[Transfer("l", target, snapshot=snapshot,
                                                                   durability="durable")]))
        connector.start_load_kv(None)
        connector.clear_connector_metadata()
        run_until(connector, lambda sending, receiving: "l" in receiving)
        run_until(connector, lambda sending, receiving: not connector.worker._loads)
        torch.cuda.synchronize()
        report = connector.build_connector_worker_meta()
        assert report.loaded == ["l"] and report.failed_loads == []
        oracle_lib.scatter(host_spans, target, [records.ctypes.data + i * size for i in range(len(target))])
        after = backing.view(torch.uint8).cpu().numpy().reshape(-1)
        changed = np.flatnonzero(after != host)
        assert changed.size == 0, f"{changed.size} bytes differ from the oracle's scatter, first at {changed[0]}"
    finally:
        torch.cuda.synchronize()
        connector.shutdown()
