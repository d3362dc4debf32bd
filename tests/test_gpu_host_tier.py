"""Host tier on the GPU: delta saves against full saves and the oracle, restores from the tier.

A delta save's snapshot must equal a full save's, segment for segment (the
reference rehashes every block, kvsnap/connector/volatile.py:208-279; with
the same bytes that yields the same ids and CRCs), and its ids must be the
SHA-256 of the records the oracle gathers.
"""
import ctypes as C
import hashlib
import random

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from kvsnap_amd import synth
from kvsnap_amd.blobs import CorruptSnapshotError
from kvsnap_amd.dataplane import TorchBlockDataPlane
from kvsnap_amd.host_tier import HostTier

pytestmark = pytest.mark.gpu

LAYERS, BLOCKS, BLOCK_SIZE = 4, 64, 16


@pytest.fixture
def plane(hip_library):
    caches, backing = synth.make_caches(LAYERS, BLOCKS, layout="kv_split")
    made = TorchBlockDataPlane(caches, BLOCK_SIZE, 256 << 20)
    made.warm_up()
    keep = synth.fill(made, 5)
    torch.cuda.synchronize()
    del keep
    made.backing = backing
    yield made
    torch.cuda.synchronize()
    made.close()


def refill(plane, blocks, seed):
    """New content in ``blocks`` (one synthetic-fill launch per block)."""
    keep = [synth.fill(plane, seed, first_block=b, num_blocks=1) for b in blocks]
    torch.cuda.synchronize()
    del keep


def expected_segments(plane, oracle_lib, block_ids, tokens):
    backing = plane.backing
    torch.cuda.synchronize()
    host = backing.contiguous().view(torch.uint8).cpu().numpy().reshape(-1).copy()
    base = backing.data_ptr()
    spans = [(host.ctypes.data + (s[1] - base), s[2], s[0], s[3]) for s in plane.spans()]
    records = oracle_lib.gather(spans, block_ids, plane.block_bytes)
    if tokens % BLOCK_SIZE:
        oracle_lib.zero_tail(records[-1], plane.layers, tokens % BLOCK_SIZE)
    return [(hashlib.sha256(r.tobytes()).hexdigest(), oracle_lib.crc32c(r.tobytes())) for r in records]


def ids_crcs(snapshot):
    return [(s["blob_id"], s["crc32c"]) for s in snapshot["segments"]]


def test_delta_save_equals_a_full_save_and_gathers_only_changed_blocks(plane, oracle_lib):
    ids = random.Random(11).sample(range(1, BLOCKS), 30)
    delta, full = HostTier(plane, 256 << 20), HostTier(plane, 256 << 20)
    first = delta.save(ids[:20], 19 * BLOCK_SIZE + 6)
    assert delta.gathered_blocks == 20
    assert ids_crcs(first) == expected_segments(plane, oracle_lib, ids[:20], 19 * BLOCK_SIZE + 6)
    # The next turn: the partial block 19 gains tokens and blocks 20..25 are new.
    refill(plane, ids[19:26], 77)
    second = delta.save(ids[:26], 25 * BLOCK_SIZE + 10, previous=first)
    assert delta.gathered_blocks == 7
    reference = full.save(ids[:26], 25 * BLOCK_SIZE + 10)
    assert full.gathered_blocks == 26
    assert second["segments"] == reference["segments"]
    assert ids_crcs(second) == expected_segments(plane, oracle_lib, ids[:26], 25 * BLOCK_SIZE + 10)
    assert [s["first_block"] for s in second["segments"]] == list(range(26))
    # 19 blocks are shared by both snapshots; the tier holds them once.
    assert delta.stats()["blob_count"] == 20 + 7
    delta.release(first)
    assert delta.stats()["blob_count"] == 26
    # A save with nothing new gathers nothing.
    third = delta.save(ids[:25], 25 * BLOCK_SIZE, previous=second)
    assert delta.gathered_blocks == 0 and third["segments"] == second["segments"][:25]
    for tier, snapshots in ((delta, (second, third)), (full, (reference,))):
        for snapshot in snapshots:
            tier.release(snapshot)
        assert tier.stats() == dict(resident_bytes=0, blob_count=0, capacity_bytes=256 << 20)


@pytest.mark.parametrize("verify", [False, True, "checked"])
def test_restore_from_the_tier_then_delta_save_into_the_restored_blocks(plane, oracle_lib, verify):
    rng = random.Random(3)
    ids = rng.sample(range(1, BLOCKS), 40)
    source, target = ids[:12], ids[12:26]
    tier = HostTier(plane, 256 << 20)
    saved = tier.save(source, 12 * BLOCK_SIZE)
    before = plane.backing.view(torch.int16).clone()
    progress = []
    view = tier.restore(target[:12], saved, verify=verify, progress=progress)
    torch.cuda.synchronize()
    after = plane.backing.view(torch.int16)
    # The K/V-split backing is [layers, 2, blocks, N, H, D]: blocks are dimension 2.
    assert max(source + target) < plane.backing.shape[2]
    expected = before.clone()
    expected[:, :, target[:12]] = before[:, :, source]
    assert torch.equal(after, expected)
    assert progress[0][1] == 12 * plane.block_bytes and progress[-1][1] == 0
    # The resumed session writes two new blocks after the restored ones.
    refill(plane, target[12:14], 91)
    resumed = tier.save(target[:14], 13 * BLOCK_SIZE + 1, previous=view)
    assert tier.gathered_blocks == 2
    assert resumed["segments"][:12] == [dict(s) for s in saved["segments"]]
    assert ids_crcs(resumed) == expected_segments(plane, oracle_lib, target[:14], 13 * BLOCK_SIZE + 1)
    tier.release(saved)
    tier.release(resumed)
    assert tier.stats()["blob_count"] == 0


def test_a_released_snapshot_cannot_be_restored_or_reused(plane):
    ids = random.Random(5).sample(range(1, BLOCKS), 8)
    tier = HostTier(plane, 256 << 20)
    snapshot = tier.save(ids[:4], 4 * BLOCK_SIZE)
    tier.release(snapshot)
    with pytest.raises(CorruptSnapshotError):
        tier.restore(ids[4:], snapshot)
    # A delta save from it falls back to gathering every block.
    again = tier.save(ids[:4], 4 * BLOCK_SIZE, previous=snapshot)
    assert tier.gathered_blocks == 4
    assert [s["blob_id"] for s in again["segments"]] == [s["blob_id"] for s in snapshot["segments"]]
    tier.release(again)


def test_a_corrupted_held_block_is_refused_by_the_verified_restore(plane):
    ids = random.Random(6).sample(range(1, BLOCKS), 8)
    tier = HostTier(plane, 256 << 20)
    snapshot = tier.save(ids[:4], 4 * BLOCK_SIZE)
    before = plane.backing.view(torch.int16).clone()
    held = tier._entries[snapshot["segments"][2]["blob_id"]]["allocation"]
    byte = C.c_uint8.from_address(held.pointer + 12345)
    byte.value ^= 0x10
    with pytest.raises(CorruptSnapshotError):
        tier.restore(ids[4:], snapshot, verify=True)
    torch.cuda.synchronize()
    assert torch.equal(plane.backing.view(torch.int16), before), "no KV block is written"
    byte.value ^= 0x10
    tier.restore(ids[4:], snapshot, verify=True)
    tier.release(snapshot)


def test_a_corrupted_held_block_fails_the_checked_restore_after_its_copy(plane):
    ids = random.Random(7).sample(range(1, BLOCKS), 8)
    tier = HostTier(plane, 256 << 20)
    snapshot = tier.save(ids[:4], 4 * BLOCK_SIZE)
    held = tier._entries[snapshot["segments"][1]["blob_id"]]["allocation"]
    byte = C.c_uint8.from_address(held.pointer + 54321)
    byte.value ^= 0x01
    progress = []
    with pytest.raises(CorruptSnapshotError, match=r"1 of 4 .*block 1\)"):
        tier.restore(ids[4:], snapshot, verify="checked", progress=progress)
    assert progress == []
    byte.value ^= 0x01
    tier.restore(ids[4:], snapshot, verify="checked")
    torch.cuda.synchronize()
    src, dst = torch.tensor(ids[:4], device="cuda"), torch.tensor(ids[4:], device="cuda")
    assert torch.equal(plane.backing[:, :, dst].view(torch.int16), plane.backing[:, :, src].view(torch.int16))
    with pytest.raises(ValueError):
        tier.restore(ids[4:], snapshot, verify="staged")
    tier.release(snapshot)


@pytest.mark.parametrize("verify", ["gpu", "host"])
def test_disk_delta_save_equals_a_full_save_and_restores_byte_exact(plane, oracle_lib, tmp_path, verify):
    from kvsnap_amd.blobs import BlobDirectory
    ids = random.Random(21).sample(range(1, BLOCKS), 26)
    delta, full = BlobDirectory(tmp_path / "delta"), BlobDirectory(tmp_path / "full")
    first = delta.save(plane, ids[:20], 19 * BLOCK_SIZE + 6)
    assert delta.gathered_blocks == 20 and delta.written == 20
    refill(plane, ids[19:26], 55)
    second = delta.save(plane, ids[:26], 25 * BLOCK_SIZE + 10, previous=first)
    assert delta.gathered_blocks == 7 and delta.written == 7
    reference = full.save(plane, ids[:26], 25 * BLOCK_SIZE + 10)
    assert full.gathered_blocks == 26 and full.written == 26
    assert second["segments"] == reference["segments"]
    assert ids_crcs(second) == expected_segments(plane, oracle_lib, ids[:26], 25 * BLOCK_SIZE + 10)
    # The delta snapshot restores from disk into other blocks, byte for byte.
    others = [b for b in range(1, BLOCKS) if b not in ids]
    targets = random.Random(22).sample(others, 26)
    before = plane.backing.view(torch.int16).clone()
    assert plane.load_from_disk(targets, delta, second["segments"], chunk_bytes=8 * plane.block_bytes,
                                workers=2, verify=verify) == 4
    torch.cuda.synchronize()
    assert max(ids + targets) < plane.backing.shape[2]
    expected = before.clone()
    expected[:, :, targets] = before[:, :, ids]    # [layers, 2, blocks, N, H, D]
    expected[:, :, targets[-1], 10:] = 0            # the snapshot's last block: slots past token 10 are zero
    assert torch.equal(plane.backing.view(torch.int16), expected)
