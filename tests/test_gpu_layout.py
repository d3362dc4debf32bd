"""A snapshot taken under one KV layout is refused by caches of another layout with the same record size.

A K/V-split Qwen3-shaped cache and a vLLM-layout one make records of the
same size that put different elements at the same offsets; each snapshot
records the layout it was taken under, and a load into caches of another
layout is refused before any copy, as a recompute miss (reference
kvsnap/connector/vllm.py:236, 438-444).  On the GPU: through the worker
(blob files and the host tier) and through the host tier directly, with not
one byte of the refusing cache written, while the same snapshots still load
into caches of their own layout.
"""
import random
import time

import pytest

torch = pytest.importorskip("torch")

from kvsnap_amd import synth
from kvsnap_amd.blobs import BlobDirectory
from kvsnap_amd.dataplane import TorchBlockDataPlane
from kvsnap_amd.host_tier import HostTier
from kvsnap_amd.layout import LayoutMismatch
from kvsnap_amd.worker import KvsnapMetadata, KvsnapWorker, Transfer

pytestmark = pytest.mark.gpu

LAYERS, BLOCKS, BLOCK_SIZE, SESSION = 4, 64, 16, 12


def _reported(worker, request, seconds=60):
    """Step boundaries until ``request`` has been reported received and its load is booked."""
    deadline, seen = time.monotonic() + seconds, False
    while time.monotonic() < deadline:
        worker.bind_connector_metadata(KvsnapMetadata())
        seen |= request in worker.get_finished(set())[1]
        worker.clear_connector_metadata()
        if seen and not worker._loads:
            return
        time.sleep(1e-4)
    raise AssertionError(f"{request} was never reported")


def test_a_k_v_split_snapshot_is_refused_by_vllm_layout_caches_with_no_byte_written(hip_library, tmp_path):
    split_caches, split_backing = synth.make_caches(LAYERS, BLOCKS, layout="kv_split")
    vllm_caches, vllm_backing = synth.make_caches(LAYERS, BLOCKS, layout="vllm")
    split = TorchBlockDataPlane(split_caches, BLOCK_SIZE, 64 << 20)
    vllm = TorchBlockDataPlane(vllm_caches, BLOCK_SIZE, 64 << 20)
    worker = None
    try:
        assert split.block_bytes == vllm.block_bytes and split.layout_identity != vllm.layout_identity
        keep = [synth.fill(split, 1), synth.fill(vllm, 2)]
        torch.cuda.synchronize()
        del keep
        rng = random.Random(5)
        source = rng.sample(range(1, BLOCKS), SESSION)
        target = rng.sample([b for b in range(1, BLOCKS) if b not in source], SESSION)
        tokens = SESSION * BLOCK_SIZE
        on_disk = BlobDirectory(tmp_path).save(split, source, tokens)
        split_tier = HostTier(split, 32 << 20)
        held = split_tier.save(source, tokens)
        assert on_disk["kv_layout"] == held["kv_layout"] == split.layout_identity
        torch.cuda.synchronize()
        before = vllm_backing.clone()

        vllm_tier = HostTier(vllm, 32 << 20)
        worker = KvsnapWorker(vllm, host_tier=vllm_tier, blobs=BlobDirectory(tmp_path))
        for durability, snapshot in (("durable", on_disk), ("volatile", held)):
            request = f"load-{durability}"
            worker.bind_connector_metadata(KvsnapMetadata(loads=[Transfer(request, target, snapshot=snapshot,
                                                                          durability=durability)]))
            worker.start_load_kv(None)
            worker.clear_connector_metadata()
            _reported(worker, request)
            assert worker.get_block_ids_with_load_errors() == set(target), durability
            report = worker.build_connector_worker_meta()
            assert report.failed_loads == [request] and report.loaded == [request], durability
            assert report.invalid_snapshots == [], durability
        with pytest.raises(LayoutMismatch):
            vllm_tier.restore(target, held)
        torch.cuda.synchronize()
        assert torch.equal(vllm_backing.view(torch.int16), before.view(torch.int16))

        # The refusal is the layout's: the same snapshots load into caches of the layout they were taken under.
        split_backing[:, :, target] = 0
        split_tier.restore(target, held)
        torch.cuda.synchronize()
        assert torch.equal(split_backing[:, :, target].view(torch.int16),
                           split_backing[:, :, source].view(torch.int16))
        split_backing[:, :, target] = 0
        split.load_from_disk(target, BlobDirectory(tmp_path), on_disk["segments"])
        torch.cuda.synchronize()
        assert torch.equal(split_backing[:, :, target].view(torch.int16),
                           split_backing[:, :, source].view(torch.int16))
    finally:
        if worker is not None:
            worker.shutdown()
        torch.cuda.synchronize()
        vllm.close()
        split.close()
