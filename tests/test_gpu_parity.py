"""HIP kernels against the CPU oracle on the same seeded inputs, at sizes the oracle finishes in seconds.

Bit-exact throughout: records, restored caches, CRC32C and SHA-256 (the
reference compares bit for bit too, tests/connector/test_copy_kernel_cuda.py:63).
"""
import ctypes as C
import hashlib
import random
import threading

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from kvsnap_amd import synth
from kvsnap_amd.dataplane import (TorchBlockDataPlane, _check, digest_device_records, gather_crc32c_launcher,
                                  kernel_library)

pytestmark = pytest.mark.gpu

LAYERS, BLOCKS, BLOCK_SIZE, HEADS, WIDTH = 6, 96, 16, 8, 256


def vllm_caches(layers, blocks, seed=0):
    """The reference's GPU fixture: random bf16 bits, [blocks, H, N, 2D] views of [blocks, N, H, 2D] storage."""
    generator = torch.Generator(device="cuda").manual_seed(seed)
    backing = torch.randint(-2**15, 2**15, (layers, blocks, BLOCK_SIZE, HEADS, WIDTH), dtype=torch.int16,
                            device="cuda", generator=generator).view(torch.bfloat16)
    return backing, {f"model.layers.{i}.self_attn.attn": backing[i].permute(0, 2, 1, 3) for i in range(layers)}


def host_copy(backing):
    torch.cuda.synchronize()
    return backing.contiguous().view(torch.uint8).cpu().numpy().reshape(-1).copy()


def host_spans(plane, backing, host):
    """The plane's spans re-based onto a host copy of ``backing``."""
    base = backing.data_ptr()
    return [(host.ctypes.data + (s[1] - base), s[2], s[0], s[3]) for s in plane.spans()]


def pinned_bytes(allocation, offset, size):
    return np.frombuffer(C.string_at(allocation.pointer + offset, size), dtype=np.uint8)


@pytest.mark.parametrize("restore_mode", ["kernel", "dma", "dma-in-turn"])
def test_a_saved_snapshot_restores_bit_for_bit_into_shuffled_blocks(planes, monkeypatch, restore_mode):
    """The reference's own GPU case (test_copy_kernel_cuda.py:41-63), on the HIP kernels: the restore kernel
    reading pinned records in place, or the copy engines staging them for the scatter kernel, which places
    each chunk on the plane's aside stream while the next is copied, or in turn on the restore stream."""
    from kvsnap_amd import dataplane as dataplane_module
    monkeypatch.setattr(dataplane_module, "PLACE_ASIDE", restore_mode == "dma")
    backing, caches = vllm_caches(LAYERS, BLOCKS)
    plane = planes(caches, restore_mode="kernel" if restore_mode == "kernel" else "dma")
    if restore_mode == "dma":
        assert plane.stream_report()["aside_stream"] is True
    rng = random.Random(1)
    saved = rng.sample(range(1, BLOCKS), 20)
    restored = rng.sample([b for b in range(1, BLOCKS) if b not in saved], 20)
    size = plane.block_bytes
    before = backing.view(torch.int16).clone()
    for kind in ("staging", "per-block"):
        owned = ([plane.pool.reserve(size * len(saved))] if kind == "staging"
                 else [plane.pool.reserve(size) for _ in saved])
        targets = ([(owned[0], i * size) for i in range(len(saved))] if kind == "staging"
                   else [(allocation, 0) for allocation in owned])
        plane.save_gather(saved, targets, len(saved) * BLOCK_SIZE)
        progress = []
        assert plane.load_scatter(restored, targets, progress=progress, chunk_bytes=3 * size) == 7
        assert all(event.query() for event, _ in progress[1:])
        torch.cuda.synchronize()
        after = backing.view(torch.int16).clone()
        expected = before.clone()
        expected[:, restored] = before[:, saved]
        assert torch.equal(after, expected), kind
        backing.view(torch.int16).copy_(before)
        for allocation in owned:
            allocation.close()


@pytest.mark.parametrize("checked", [False, True])
def test_saves_and_restores_from_two_threads_overlap_byte_exact(planes, oracle_lib, checked):
    """The connector's save thread and loader thread at once (reference vllm.py:202-203), restores on their
    own stream through the copy engines: session k is restored while session k + 1 is saved into the other
    pinned buffer.  Every restore must hold exactly the bytes its save saw; checked restores also pass the
    CRC32Cs their save computed on the GPU."""
    import threading
    caches, backing = synth.make_caches(LAYERS, 96, layout="kv_split")
    plane = planes(caches, capacity=2 * 16 * LAYERS * 65536 + (64 << 20), restore_stream="split",
                   restore_mode="dma")
    rng = random.Random(8)
    source = rng.sample(range(1, 96), 16)
    target = rng.sample([b for b in range(1, 96) if b not in source], 16)
    assert max(source + target) < backing.shape[2]       # [layers, 2, blocks, N, H, D]
    size = plane.block_bytes
    buffers = [plane.pool.reserve(16 * size) for _ in range(2)]
    targets = [[(b, i * size) for i in range(16)] for b in buffers]
    steps = 6
    saved = [threading.Event() for _ in range(steps)]
    restored = [threading.Event() for _ in range(steps)]
    expected, failures, digests = {}, [], []
    src = torch.tensor(source, device="cuda")
    dst = torch.tensor(target, device="cuda")

    def saver():
        try:
            for k in range(steps):
                if k >= 2:
                    restored[k - 2].wait(60)
                keep = [synth.fill(plane, 100 + k, first_block=b, num_blocks=1) for b in source]
                expected[k] = backing[:, :, src].clone()
                plane.save_gather(source, targets[k % 2], 16 * BLOCK_SIZE, digests=digests)
                del keep
                saved[k].set()
        except BaseException as exc:
            failures.append(exc)
            for event in saved:
                event.set()

    def loader():
        try:
            for k in range(steps):
                saved[k].wait(60)
                if failures:
                    return
                if checked:
                    crcs = [crc for _, crc in digests[k].result()]
                    plane.load_scatter_checked(target, targets[k % 2], crcs, chunk_bytes=5 * size)
                else:
                    plane.load_scatter(target, targets[k % 2], chunk_bytes=5 * size)
                torch.cuda.synchronize()
                if not torch.equal(backing[:, :, dst].view(torch.int16), expected[k].view(torch.int16)):
                    failures.append(AssertionError(f"restore {k} differs from save {k}"))
                # Save k's GPU digests against the oracle's over its pinned records (not reused before this).
                crcs, shas = oracle_lib.digest_records(buffers[k % 2].pointer, size, size, 16)
                got = digests[k].result()
                if [c for _, c in got] != crcs.tolist() or [h for h, _ in got] != [bytes(s).hex() for s in shas]:
                    failures.append(AssertionError(f"save {k}'s digests differ from the oracle's"))
                restored[k].set()
        except BaseException as exc:
            failures.append(exc)
            for event in restored:
                event.set()

    threads = [threading.Thread(target=saver), threading.Thread(target=loader)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(120)
    assert not any(t.is_alive() for t in threads)
    assert not failures, failures
    for b in buffers:
        b.close()


def test_the_split_restore_and_hash_streams_are_the_plane_s_own_and_distinct(planes):
    """With ``restore_stream="split"`` the restore stream and every hash stream are streams the plane made
    itself, none of them the pool's copy stream or another of them.  (Whether they landed on hardware queues
    and copy engines of their own is a timing matter: the bench reports it, as ``streams``.)"""
    caches, _ = synth.make_caches(2, 16, layout="kv_split")
    plane = planes(caches, restore_stream="split", restore_mode="dma")
    copy = plane._copy_stream.cuda_stream
    others = [plane._restore_stream().cuda_stream] + [s.cuda_stream for s in plane._hash_streams()]
    assert copy not in others and len(set(others)) == len(others)
    assert set(others) <= set(plane._owned_streams)


def test_a_plane_closed_with_work_in_flight_and_an_exception_alive_exits_cleanly(hip_library, tmp_path):
    """A test process once crashed at exit after a failing test: pinned tensors copied ``non_blocking`` on the
    plane's own streams, kept alive by the failure's traceback, were freed after ``close`` had destroyed
    those streams, and torch's pinned allocator then queried events recorded on them.  The plane no longer
    copies torch pinned tensors on its streams (tables go through its own staging and the library's copies),
    so this child process -- split streams, a save whose hash job is still running, a restore, an exception
    whose traceback outlives ``close``, then more pinned allocations -- must exit 0."""
    import subprocess
    import sys
    script = tmp_path / "close_with_exception.py"
    script.write_text("""
import sys
import torch
from kvsnap_amd import synth
from kvsnap_amd.dataplane import TorchBlockDataPlane
caches, backing = synth.make_caches(4, 64, layout="kv_split")
plane = TorchBlockDataPlane(caches, 16, 64 << 20, restore_stream="split", restore_mode="dma")
plane.warm_up()
keep = synth.fill(plane, 5)
torch.cuda.synchronize()
staged = plane.pool.reserve(8 * plane.block_bytes)
targets = [(staged, i * plane.block_bytes) for i in range(8)]
digests = []
plane.save_gather(list(range(1, 9)), targets, 8 * 16, digests=digests)      # its hash job is in flight
held = None
try:
    pinned = torch.empty(1 << 20, dtype=torch.uint8, pin_memory=True)
    plane.load_scatter(list(range(20, 28)), targets)
    raise RuntimeError("planted failure")
except RuntimeError:
    held = sys.exc_info()              # the traceback keeps this frame, and the pinned tensor, alive
staged.close()
plane.close()
del pinned
held = None
for _ in range(4):                     # the pinned allocator processes its events on these
    extra = torch.empty(1 << 20, dtype=torch.uint8, pin_memory=True)
    extra.to("cuda").sum().item()
torch.cuda.synchronize()
print("clean exit", flush=True)
""")
    env = dict(__import__("os").environ, PYTHONPATH=str(__import__("pathlib").Path(__file__).resolve().parents[1]))
    done = subprocess.run([sys.executable, str(script)], capture_output=True, text=True, timeout=120, env=env)
    assert done.returncode == 0 and "clean exit" in done.stdout, (done.returncode, done.stdout[-2000:],
                                                                  done.stderr[-2000:])


@pytest.mark.parametrize("layout", ["vllm", "kv_split"])
@pytest.mark.parametrize("kind", [synth.KIND_BF16, synth.KIND_E4M3, synth.KIND_BYTES])
def test_synthetic_fill_matches_the_oracle_generator(planes, oracle_lib, layout, kind):
    dtype = torch.float8_e4m3fn if kind == synth.KIND_E4M3 else torch.bfloat16
    caches, backing = synth.make_caches(3, 8, layout=layout, dtype=dtype)
    plane = planes(caches)
    scales = [0.5 + 0.25 * i for i in range(len(plane.spans()))] if kind == synth.KIND_E4M3 else None
    keep = synth.fill(plane, 1234, kind=kind, inv_scales=scales)
    host = host_copy(backing)
    del keep
    for index, (host_addr, pitch, _, nbytes) in enumerate(host_spans(plane, backing, host)):
        for block in range(8):
            start = host_addr - host.ctypes.data + block * pitch
            got = host[start:start + nbytes]
            expected = oracle_lib.fill_span(1234, index, block, nbytes, kind, scales[index] if scales else 1.0)
            assert np.array_equal(got, expected), (index, block)


@pytest.mark.parametrize("layout", ["vllm", "kv_split"])
def test_save_gather_matches_the_oracle_records_and_zeroes_the_tail(planes, oracle_lib, layout):
    caches, backing = synth.make_caches(LAYERS, 24, layout=layout)
    plane = planes(caches)
    keep = synth.fill(plane, 5, kind=synth.KIND_BYTES)
    host = host_copy(backing)
    del keep
    block_ids, tokens = [7, 2, 9, 3, 4], 4 * BLOCK_SIZE + 5
    size = plane.block_bytes
    records = oracle_lib.gather(host_spans(plane, backing, host), block_ids, size)
    oracle_lib.zero_tail(records[-1], plane.layers, 5)
    for kind, copies in (("per-block", 5), ("staging", 3)):
        owned = ([plane.pool.reserve(size * len(block_ids))] if kind == "staging"
                 else [plane.pool.reserve(size) for _ in block_ids])
        targets = ([(owned[0], i * size) for i in range(len(block_ids))] if kind == "staging"
                   else [(allocation, 0) for allocation in owned])
        assert plane.save_gather(block_ids, targets, tokens, chunk_bytes=2 * size) == copies
        for index, (allocation, offset) in enumerate(targets):
            assert np.array_equal(pinned_bytes(allocation, offset, size), records[index]), (kind, index)
        assert np.array_equal(host_copy(backing), host), "the KV cache is only read"
        for allocation in owned:
            allocation.close()


def test_gpu_digests_match_the_oracle_and_hashlib(planes, oracle_lib):
    caches, backing = synth.make_caches(LAYERS, 40, layout="vllm")
    plane = planes(caches)
    keep = synth.fill(plane, 9)
    torch.cuda.synchronize()
    del keep
    block_ids = random.Random(3).sample(range(1, 40), 17)
    tokens = 16 * 16 + 3
    size = plane.block_bytes
    staged = plane.pool.reserve(size * len(block_ids))
    targets = [(staged, i * size) for i in range(len(block_ids))]
    digests = []
    plane.save_gather(block_ids, targets, tokens, digests=digests)
    got = digests[0].result()
    for index, (hexdigest, crc) in enumerate(got):
        record = C.string_at(staged.pointer + index * size, size)
        assert crc == oracle_lib.crc32c(record), index
        assert hexdigest == hashlib.sha256(record).hexdigest() == oracle_lib.sha256(record).hex(), index
    staged.close()


@pytest.mark.parametrize("lead", [True, False], ids=["lead-stream", "one-gather"])
@pytest.mark.parametrize("layout", ["vllm", "kv_split"])
def test_a_hashed_save_gathered_over_two_streams_matches_the_oracle(planes, oracle_lib, monkeypatch, layout, lead):
    """A hashed save longer than one chunk: its first chunk is gathered on the copy stream and the rest,
    with the last record's tail, on the lead stream, whose copies wait for it.  Records, CRC32C and SHA-256
    equal the oracle's with the lead stream and without it."""
    from kvsnap_amd import dataplane as dataplane_module
    monkeypatch.setattr(dataplane_module, "SAVE_LEAD", lead)
    caches, backing = synth.make_caches(LAYERS, 24, layout=layout)
    plane = planes(caches)
    report = plane.stream_report()
    assert report["save_lead"] is lead and (report["aside_stream"] is True or not lead)
    keep = synth.fill(plane, 17, kind=synth.KIND_BYTES)
    host = host_copy(backing)
    del keep
    block_ids, tokens = [7, 2, 9, 3, 4, 11, 20], 6 * BLOCK_SIZE + 3
    size = plane.block_bytes
    records = oracle_lib.gather(host_spans(plane, backing, host), block_ids, size)
    oracle_lib.zero_tail(records[-1], plane.layers, 3)
    # One copy per run of back-to-back targets, and a run is cut where the lead stream's records start.
    for kind, copies in (("per-block", 7), ("staging", 2 if lead else 1)):
        owned = ([plane.pool.reserve(size * len(block_ids))] if kind == "staging"
                 else [plane.pool.reserve(size) for _ in block_ids])
        targets = ([(owned[0], i * size) for i in range(len(block_ids))] if kind == "staging"
                   else [(allocation, 0) for allocation in owned])
        digests = []
        assert plane.save_gather(block_ids, targets, tokens, chunk_bytes=2 * size, digests=digests) == copies
        for index, (allocation, offset) in enumerate(targets):
            assert np.array_equal(pinned_bytes(allocation, offset, size), records[index]), (kind, index)
        for index, ((hexdigest, crc), record) in enumerate(zip(digests[0].result(), records)):
            assert crc == oracle_lib.crc32c(record), (kind, index)
            assert hexdigest == hashlib.sha256(record.tobytes()).hexdigest(), (kind, index)
        for allocation in owned:
            allocation.close()
    assert np.array_equal(host_copy(backing), host), "the KV cache is only read"


@pytest.mark.parametrize("record_bytes", [0, 1, 5, 16, 63, 64, 65, 119, 120, 192, 4095, 4096, 4097, 65520,
                                          65536, 65552, 200000, 2 * 65536 + 48])
def test_crc32c_and_sha256_kernels_on_odd_record_sizes(hip_library, oracle_lib, record_bytes):
    n = 5
    for pitch in {record_bytes, record_bytes + (-record_bytes % 16), record_bytes + 24}:
        pitch = max(pitch, 1)
        data = torch.randint(0, 256, (n * pitch + 16,), dtype=torch.uint8, device="cuda")
        for shift in (0, 8, 3):
            stream = torch.cuda.current_stream()
            crc, sha, workspace = digest_device_records(torch, data.data_ptr() + shift, record_bytes, pitch, n,
                                                        data.device, stream)
            torch.cuda.synchronize()
            host = data.cpu().numpy()
            for r in range(n):
                rec = host[shift + r * pitch: shift + r * pitch + record_bytes].tobytes()
                assert (int(crc[r]) & 0xFFFFFFFF) == oracle_lib.crc32c(rec), (record_bytes, pitch, shift, r)
                assert bytes(sha[r].cpu().numpy()) == hashlib.sha256(rec).digest(), (record_bytes, pitch, shift, r)
            del workspace


@pytest.mark.parametrize("record_bytes,n", [(12000, 8192), (20380, 2048), (70000, 2048), (40968, 1024),
                                             (294912, 512), (589840, 16)])
def test_crc32c_kernel_on_the_stripe_plans_of_many_records(hip_library, oracle_lib, record_bytes, n):
    """Records in the stripe plans the CRC32C launch takes (1 KiB groups, 6 chains per lane): one stripe of
    12 groups with a partial first group (12000 bytes), two stripes of 10 (20380), two of 35 whose first
    group is all padding (70000), unaligned records (40968), a tensor-parallel shard's records (294912:
    eight stripes of 36 groups) -- all combined inside their workgroup -- and 58 stripes of 10 groups,
    three of them padding, combined by a second launch (589840 bytes, 16 records)."""
    lib = kernel_library()
    data = torch.randint(0, 256, (n * record_bytes + 16,), dtype=torch.uint8, device="cuda")
    out = torch.zeros(n, dtype=torch.int32, device="cuda")
    work_bytes = int(lib.kvsnap_crc32c_workspace_bytes(record_bytes, n))
    work = torch.empty(max(work_bytes, 16), dtype=torch.uint8, device="cuda")
    _check(lib, lib.kvsnap_crc32c_records(data.data_ptr(), record_bytes, record_bytes, n, 0, out.data_ptr(),
                                          work.data_ptr(), work_bytes, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    host = data.cpu().numpy()
    want, _ = oracle_lib.digest_records(host.ctypes.data, record_bytes, record_bytes, n, sha=False)
    got = out.cpu().numpy().astype(np.uint32)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, (record_bytes, n, bad[:8])


@pytest.mark.parametrize("record_bytes,n,pitch", [((1 << 31) - 1024, 1, (1 << 31) - 1024),
                                                  ((1 << 31) + 48, 2, (1 << 31) + 64)])
def test_crc32c_kernel_on_records_of_two_gib(hip_library, oracle_lib, record_bytes, n, pitch):
    """The largest record the aligned kernels take (2 GiB - 1 KiB, 32-bit word offsets) and records past 2 GiB,
    which the host sends down the unaligned path (64-bit offsets, 64 stripes of 32 MiB and a combine launch):
    every CRC32C equals the oracle's (csrc/dataplane/io.cpp:39-44)."""
    lib = kernel_library()
    data = torch.randint(0, 256, (n * pitch,), dtype=torch.uint8, device="cuda")
    out = torch.zeros(n, dtype=torch.int32, device="cuda")
    work_bytes = int(lib.kvsnap_crc32c_workspace_bytes(record_bytes, n))
    work = torch.empty(max(work_bytes, 16), dtype=torch.uint8, device="cuda")
    print(f"CRC32C of {n} records of {record_bytes} B, pitch {pitch}", flush=True)
    _check(lib, lib.kvsnap_crc32c_records(data.data_ptr(), record_bytes, pitch, n, 0, out.data_ptr(),
                                          work.data_ptr(), work_bytes, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    host = data.cpu().numpy()
    want = [oracle_lib.crc32c_at(host.ctypes.data + r * pitch, record_bytes) for r in range(n)]
    assert [value & 0xFFFFFFFF for value in out.tolist()] == want
    del data, host, work


@pytest.mark.parametrize("n", [1, 31, 33, 64, 65, 131])
def test_sha256_kernel_covers_every_lane_of_both_round_waves(hip_library, oracle_lib, n):
    """Records are hashed two lanes each, 32 per round wave and 64 per workgroup: partial and full groups."""
    record_bytes, pitch = 1000, 1008
    data = torch.randint(0, 256, (n * pitch,), dtype=torch.uint8, device="cuda")
    crc, sha, workspace = digest_device_records(torch, data.data_ptr(), record_bytes, pitch, n, data.device,
                                                torch.cuda.current_stream())
    torch.cuda.synchronize()
    host = data.cpu().numpy()
    for r in range(n):
        rec = host[r * pitch: r * pitch + record_bytes].tobytes()
        assert bytes(sha[r].cpu().numpy()) == hashlib.sha256(rec).digest(), (n, r)
        assert (int(crc[r]) & 0xFFFFFFFF) == oracle_lib.crc32c(rec), (n, r)
    del workspace


@pytest.mark.parametrize("record_bytes", [0, 55, 56, 119, 120, 1000, 4097, 65552])
@pytest.mark.parametrize("shift", [0, 3])
def test_sha256_over_block_ranges_equals_one_pass(hip_library, oracle_lib, record_bytes, shift):
    """A chain run as several launches (state carried between them) gives the one-launch digest and hashlib's:
    ranges of 1, 3, 4 and 7 compressions, ranges that hold only the padding blocks, aligned and unaligned."""
    lib = kernel_library()
    n, pitch = 70, record_bytes + 16
    nblocks = int(lib.kvsnap_sha256_blocks(record_bytes))
    assert nblocks == record_bytes // 64 + (1 if record_bytes % 64 + 9 <= 64 else 2)
    data = torch.randint(0, 256, (n * pitch + 16,), dtype=torch.uint8, device="cuda")
    base = data.data_ptr() + shift
    stream = torch.cuda.current_stream().cuda_stream
    whole = torch.zeros((n, 32), dtype=torch.uint8, device="cuda")
    _check(lib, lib.kvsnap_sha256_records(base, record_bytes, pitch, n, whole.data_ptr(), stream))
    host = data.cpu().numpy()
    expected = [hashlib.sha256(host[shift + r * pitch: shift + r * pitch + record_bytes].tobytes()).digest()
                for r in range(n)]
    for step in (1, 3, 4, 7):
        state = torch.zeros((n, 8), dtype=torch.int32, device="cuda")
        out = torch.zeros((n, 32), dtype=torch.uint8, device="cuda")
        bounds = list(range(0, nblocks, step)) + [nblocks]
        for first, end in zip(bounds, bounds[1:]):
            _check(lib, lib.kvsnap_sha256_records_range(base, record_bytes, pitch, n, first, end, state.data_ptr(),
                                                        out.data_ptr(), stream))
        torch.cuda.synchronize()
        assert torch.equal(out, whole), (record_bytes, shift, step)
        assert [bytes(out[r].cpu().numpy()) for r in range(n)] == expected, (record_bytes, shift, step)
    # Ranges out of order, past the chain, or missing their state are refused.
    for first, end, state_ptr in ((1, 1, 1), (0, nblocks + 1, 1), (1, nblocks, 0)):
        with pytest.raises(RuntimeError):
            _check(lib, lib.kvsnap_sha256_records_range(base, record_bytes, pitch, n, first, end,
                                                        state_ptr and whole.data_ptr(), whole.data_ptr(), stream))


def test_sha256_ranges_of_several_record_sets_in_one_launch_equal_hashlib(hip_library):
    """kvsnap_sha256_ranges: three record sets of different sizes, counts, pitches and alignment, each
    advanced by its own ranges of compressions (a different step per set, so ranges of unequal length share
    a launch and a set ends while others go on), give every record's SHA-256; bad tables are refused."""
    lib = kernel_library()
    stream = torch.cuda.current_stream().cuda_stream
    sets = [(12000, 12016, 37, 0, 3), (64, 64, 130, 8, 1), (20380, 20384, 5, 0, 7)]  # bytes, pitch, n, shift, step
    data, expected, outs, states, nblocks = [], [], [], [], []
    for record_bytes, pitch, n, shift, _ in sets:
        buf = torch.randint(0, 256, (n * pitch + 16,), dtype=torch.uint8, device="cuda")
        host = buf.cpu().numpy()
        data.append((buf, buf.data_ptr() + shift))
        expected.append([hashlib.sha256(host[shift + r * pitch: shift + r * pitch + record_bytes].tobytes()).digest()
                         for r in range(n)])
        outs.append(torch.zeros((n, 32), dtype=torch.uint8, device="cuda"))
        states.append(torch.zeros((n, 8), dtype=torch.int32, device="cuda"))
        nblocks.append(int(lib.kvsnap_sha256_blocks(record_bytes)))
    done = [0] * len(sets)
    launches = 0
    while any(d < total for d, total in zip(done, nblocks)):
        live = [i for i in range(len(sets)) if done[i] < nblocks[i]]
        k = len(live)
        columns = [(C.c_uint64 * k)() for _ in range(7)]
        counts = (C.c_int64 * k)()
        for j, i in enumerate(live):
            record_bytes, pitch, n, _, step = sets[i]
            end = min(done[i] + step, nblocks[i])
            for column, value in zip(columns, (data[i][1], record_bytes, pitch, done[i], end, states[i].data_ptr(),
                                               outs[i].data_ptr())):
                column[j] = value
            counts[j] = n
            done[i] = end
        records, record_bytes_, pitches, firsts, ends, state_ptrs, out_ptrs = columns
        _check(lib, lib.kvsnap_sha256_ranges(k, records, record_bytes_, pitches, counts, firsts, ends, state_ptrs,
                                              out_ptrs, stream))
        launches += 1
    torch.cuda.synchronize()
    assert launches == max(-(-total // s[4]) for total, s in zip(nblocks, sets))
    for i in range(len(sets)):
        assert [bytes(outs[i][r].cpu().numpy()) for r in range(sets[i][2])] == expected[i], i
    one = [(C.c_uint64 * 1)(v) for v in (data[0][1], 12000, 12016, 0, 1, states[0].data_ptr(), outs[0].data_ptr())]
    n_one = (C.c_int64 * 1)(37)
    with pytest.raises(RuntimeError):        # a range past the chain
        bad = [(C.c_uint64 * 1)(v) for v in (data[0][1], 12000, 12016, 0, nblocks[0] + 1, 0, outs[0].data_ptr())]
        _check(lib, lib.kvsnap_sha256_ranges(1, bad[0], bad[1], bad[2], n_one, bad[3], bad[4], bad[5], bad[6], stream))
    with pytest.raises(RuntimeError):        # more ranges than one launch carries
        _check(lib, lib.kvsnap_sha256_ranges(9, one[0], one[1], one[2], n_one, one[3], one[4], one[5], one[6], stream))


def test_saves_that_share_one_hash_stream_hash_side_by_side_and_equal_the_oracle(oracle_lib, monkeypatch):
    """With one hash stream, three saves issued from three threads share each SHA-256 launch (their chains
    advance together instead of one save after another); every save's ids and CRC32Cs equal the oracle's
    digests of its pinned records."""
    from kvsnap_amd import dataplane as dataplane_module
    monkeypatch.setattr(dataplane_module, "HASH_STREAMS", 1)
    monkeypatch.setattr(dataplane_module, "HASH_SLICE_BLOCKS", 64)
    caches, _ = synth.make_caches(LAYERS, BLOCKS, layout="kv_split")
    plane = TorchBlockDataPlane(caches, 16, 64 << 20)
    try:
        plane.warm_up()
        keep = synth.fill(plane, 17)
        torch.cuda.synchronize()
        del keep
        size = plane.block_bytes
        rng = random.Random(23)
        sessions = [rng.sample(range(1, BLOCKS), count) for count in (9, 20, 14)]
        pinned = [plane.pool.reserve(len(ids) * size) for ids in sessions]
        found = [[] for _ in sessions]
        errors = []

        def save(i):
            try:
                plane.save_gather(sessions[i], [(pinned[i], b * size) for b in range(len(sessions[i]))],
                                  len(sessions[i]) * 16, digests=found[i])
            except BaseException as exc:
                errors.append(exc)

        threads = [threading.Thread(target=save, args=(i,)) for i in range(len(sessions))]
        for t in threads:
            t.start()
        for t in threads:
            t.join(120)
        assert not errors, errors
        assert plane.stream_report()["hash_streams"] == 1
        for i, ids in enumerate(sessions):
            crcs, shas = oracle_lib.digest_records(pinned[i].pointer, size, size, len(ids), threads=4)
            assert found[i][0].result() == [(bytes(h).hex(), int(c)) for h, c in zip(shas, crcs)], i
        for p in pinned:
            p.close()
    finally:
        torch.cuda.synchronize()
        plane.close()


def test_crc32c_kernel_extends_a_prior_value(hip_library, oracle_lib):
    lib = kernel_library()
    data = torch.randint(0, 256, (3 * 70000,), dtype=torch.uint8, device="cuda")
    out = torch.zeros(3, dtype=torch.int32, device="cuda")
    work_bytes = lib.kvsnap_crc32c_workspace_bytes(70000, 3)
    work = torch.empty(work_bytes, dtype=torch.uint8, device="cuda")
    for prior in (0, 1, 0xE3069283, 0xFFFFFFFF):
        _check(lib, lib.kvsnap_crc32c_records(data.data_ptr(), 70000, 70000, 3, prior, out.data_ptr(),
                                              work.data_ptr(), work_bytes, torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        host = data.cpu().numpy()
        for r in range(3):
            assert (int(out[r]) & 0xFFFFFFFF) == oracle_lib.crc32c(host[r * 70000:(r + 1) * 70000].tobytes(), prior)


@pytest.mark.parametrize("strides", [(96, 32, 8, 1), (96, 8, 24, 1), (192, 32, 8, 1), (192, 8, 24, 1)])
def test_tail_zeroing_and_restore_follow_the_actual_strides(planes, strides):
    """The reference's stride permutations (test_scatter_gather.py:291-317) through the HIP kernels."""
    shape = (5, 3, 4, 8)
    storage = torch.arange(5 * strides[0], dtype=torch.int16, device="cuda").view(torch.bfloat16)
    cache = storage.as_strided(shape, strides)
    plane = planes({"layer.0": cache}, block_size=4, capacity=1 << 20)
    before = storage.clone()
    owned = [plane.pool.reserve(plane.block_bytes) for _ in range(2)]
    targets = [(allocation, 0) for allocation in owned]
    plane.save_gather([1, 3], targets, 6)
    # The last block keeps tokens 0-1: the elements of tokens 2-3 (any head, any of the 8 channels) are zero.
    heads, tokens, channels = np.meshgrid(np.arange(3), np.arange(2, 4), np.arange(8), indexing="ij")
    dropped = (heads * strides[1] + tokens * strides[2] + channels).ravel()
    for position, block in enumerate((1, 3)):
        want = before.view(torch.int16)[block * strides[0]:(block + 1) * strides[0]][:96].cpu().numpy().copy()
        if position == 1:
            want[dropped] = 0
        got = np.frombuffer(C.string_at(owned[position].pointer, 192), dtype=np.int16)
        assert np.array_equal(got, want)
    assert torch.equal(storage.view(torch.int16), before.view(torch.int16))
    plane.load_scatter([0, 4], targets)
    torch.cuda.synchronize()
    expected = before.view(torch.int16).clone()
    for block, allocation in zip((0, 4), owned):
        payload = torch.from_numpy(np.frombuffer(C.string_at(allocation.pointer, 192), dtype=np.int16).copy())
        expected[block * strides[0]:block * strides[0] + 96] = payload.cuda()
    assert torch.equal(storage.view(torch.int16), expected)
    for allocation in owned:
        allocation.close()


def test_kv_split_layout_round_trips_through_pinned_records(planes, oracle_lib):
    caches, backing = synth.make_caches(4, 32, layout="kv_split")
    plane = planes(caches)
    keep = synth.fill(plane, 77)
    host = host_copy(backing)
    del keep
    saved, restored = synth.block_tables(32, 10)
    size = plane.block_bytes
    staged = plane.pool.reserve(size * 10)
    targets = [(staged, i * size) for i in range(10)]
    plane.save_gather(saved, targets, 10 * BLOCK_SIZE)
    records = oracle_lib.gather(host_spans(plane, backing, host), saved, size)
    assert np.array_equal(pinned_bytes(staged, 0, 10 * size), records.reshape(-1))
    assert plane.load_scatter(restored, targets) == 1
    after = host_copy(backing)
    expected = host.copy()
    oracle_lib.scatter(host_spans(plane, backing, expected), restored,
                       [staged.pointer + i * size for i in range(10)])
    assert np.array_equal(after, expected)
    staged.close()


def test_restore_from_device_memory_uses_the_same_kernel(planes):
    """Sources may be device addresses (a staged H2D copy) as well as pinned host addresses."""
    backing, caches = vllm_caches(3, 16, seed=4)
    plane = planes(caches)
    size = plane.block_bytes
    records = torch.randint(-2**15, 2**15, (4, size // 2), dtype=torch.int16, device="cuda")
    tables = plane._load_tables()
    from kvsnap_amd.dataplane import copy_host_blocks
    sources = torch.tensor([records[i].data_ptr() for i in range(4)], dtype=torch.int64, device="cuda")
    blocks = torch.tensor([3, 9, 1, 14], dtype=torch.int64, device="cuda")
    copy_host_blocks(sources, blocks, *tables)
    torch.cuda.synchronize()
    for i, block in enumerate([3, 9, 1, 14]):
        for layer, name in enumerate(sorted(caches)):
            span = caches[name][block].permute(1, 0, 2).contiguous().view(torch.int16).reshape(-1)
            assert torch.equal(span, records[i][layer * 32768:(layer + 1) * 32768])


@pytest.mark.parametrize("layout", ["vllm", "kv_split"])
def test_direct_save_writes_pinned_records_in_place(hip_library, oracle_lib, layout):
    caches, backing = synth.make_caches(LAYERS, 24, layout=layout)
    plane = TorchBlockDataPlane(caches, BLOCK_SIZE, 64 << 20, save_mode="direct")
    try:
        plane.warm_up()
        keep = synth.fill(plane, 13, kind=synth.KIND_BYTES)
        host = host_copy(backing)
        del keep
        block_ids, tokens = [7, 2, 9, 3, 4], 4 * BLOCK_SIZE + 5
        size = plane.block_bytes
        records = oracle_lib.gather(host_spans(plane, backing, host), block_ids, size)
        oracle_lib.zero_tail(records[-1], plane.layers, 5)
        for kind in ("per-block", "staging"):
            owned = ([plane.pool.reserve(size * len(block_ids))] if kind == "staging"
                     else [plane.pool.reserve(size) for _ in block_ids])
            targets = ([(owned[0], i * size) for i in range(len(block_ids))] if kind == "staging"
                       else [(allocation, 0) for allocation in owned])
            digests = []
            assert plane.save_gather(block_ids, targets, tokens, chunk_bytes=2 * size, digests=digests) == 3
            for index, (allocation, offset) in enumerate(targets):
                assert np.array_equal(pinned_bytes(allocation, offset, size), records[index]), (kind, index)
            for (hexdigest, crc), record in zip(digests[0].result(), records):
                assert crc == oracle_lib.crc32c(record) and hexdigest == hashlib.sha256(record.tobytes()).hexdigest()
            for allocation in owned:
                allocation.close()
        assert np.array_equal(host_copy(backing), host)
    finally:
        torch.cuda.synchronize()
        plane.close()


def test_verified_restore_checks_every_block_before_writing_any(planes, oracle_lib):
    from kvsnap_amd.blobs import CorruptSnapshotError
    caches, backing = synth.make_caches(LAYERS, 40, layout="kv_split")
    plane = planes(caches)
    keep = synth.fill(plane, 21)
    torch.cuda.synchronize()
    del keep
    saved, restored = synth.block_tables(40, 12)
    size = plane.block_bytes
    staged = plane.pool.reserve(12 * size)
    sources = [(staged, i * size) for i in range(12)]
    digests = []
    plane.save_gather(saved, sources, 12 * BLOCK_SIZE, digests=digests)
    crcs = [crc for _, crc in digests[0].result()]
    before = host_copy(backing)
    # one flipped bit in the tenth staged block: nothing may reach the cache
    C.memmove(staged.pointer + 9 * size + 777, bytes([C.string_at(staged.pointer + 9 * size + 777, 1)[0] ^ 4]), 1)
    with pytest.raises(CorruptSnapshotError, match="block 9"):
        plane.load_scatter_verified(restored, sources, crcs)
    assert np.array_equal(host_copy(backing), before)
    C.memmove(staged.pointer + 9 * size + 777, bytes([C.string_at(staged.pointer + 9 * size + 777, 1)[0] ^ 4]), 1)
    progress = []
    assert plane.load_scatter_verified(restored, sources, crcs, progress=progress, chunk_bytes=5 * size) == 3
    assert [left for _, left in progress] == [12 * size, 7 * size, 2 * size, 0]
    expected = before.copy()
    oracle_lib.scatter(host_spans(plane, backing, expected), restored, [staged.pointer + i * size for i in range(12)])
    assert np.array_equal(host_copy(backing), expected)
    staged.close()


def test_synthetic_decode_reads_every_block_of_every_sequence(planes):
    caches, backing = synth.make_caches(4, 64, layout="kv_split", dtype=torch.float8_e4m3fn)
    plane = planes(caches)
    keep = synth.fill(plane, 5, kind=synth.KIND_BYTES)
    torch.cuda.synchronize()
    del keep
    lib = kernel_library()
    spans = plane.spans()
    bases = torch.tensor([s[1] for s in spans], dtype=torch.int64, device="cuda")
    pitches = torch.tensor([s[2] for s in spans], dtype=torch.int64, device="cuda")
    words = torch.tensor([s[3] // 8 for s in spans], dtype=torch.int64, device="cuda")
    table = torch.tensor([random.Random(q).sample(range(64), 9) for q in range(3)], dtype=torch.int64, device="cuda")
    out = torch.zeros(3 * len(spans), dtype=torch.int32, device="cuda")
    _check(lib, lib.kvsnap_synth_decode(bases.data_ptr(), pitches.data_ptr(), words.data_ptr(), len(spans),
                                        table.data_ptr(), 3, 9, out.data_ptr(), 0,
                                        torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    host = host_copy(backing)
    base = backing.data_ptr()
    for q in range(3):
        for s, (_, b0, pitch, nbytes) in enumerate(spans):
            total = 0
            for block in table[q].tolist():
                start = b0 - base + block * pitch
                w = host[start:start + nbytes].view(np.uint32).reshape(-1, 4).astype(np.uint64)
                total += int((w[:, 0].astype(np.uint32) ^ w[:, 1].astype(np.uint32) ^ w[:, 2].astype(np.uint32)
                              ^ w[:, 3].astype(np.uint32)).astype(np.uint64).sum())
            assert (int(out[q * len(spans) + s]) & 0xFFFFFFFF) == total & 0xFFFFFFFF


def test_qwen3_1_7b_round_trip_at_the_cpu_reference_shape(planes, oracle_lib):
    """28 layers, 4096-block cache, a 2048-token (128-block) session: gather, CRC32C, scatter, compare."""
    caches, backing = synth.make_caches(28, 4096, layout="vllm")
    plane = planes(caches, capacity=256 << 20)
    keep = synth.fill(plane, 0)
    torch.cuda.synchronize()
    del keep
    assert plane.block_bytes == 1835008
    saved, restored = synth.block_tables(4096, 128)
    size = plane.block_bytes
    staged = plane.pool.reserve(128 * size)
    targets = [(staged, i * size) for i in range(128)]
    digests = []
    plane.save_gather(saved, targets, 2048, digests=digests)
    # records against the oracle's generator (no device copy involved) and its CRC
    for index in (0, 57, 127):
        record = pinned_bytes(staged, index * size, size)
        for s, (offset, _, _, nbytes) in enumerate(plane.spans()):
            assert np.array_equal(record[offset:offset + nbytes],
                                  oracle_lib.fill_span(0, s, saved[index], nbytes, synth.KIND_BF16)), (index, s)
    crcs, _ = oracle_lib.digest_records(staged.pointer, size, size, 128, sha=False, threads=8)
    assert [crc for _, crc in digests[0].result()] == crcs.tolist()
    plane.load_scatter(restored, targets)
    torch.cuda.synchronize()
    src = torch.tensor(saved, device="cuda")
    dst = torch.tensor(restored, device="cuda")
    for view in caches.values():
        assert torch.equal(view[src].view(torch.int16), view[dst].view(torch.int16))
    staged.close()


def test_qwen3_8b_8k_session_at_full_size(planes, oracle_lib):
    """The headline workload's shape: 36 K/V-split layers in a 16384-block cache (36 GiB), an 8192-token
    session of 512 records (1,207,959,552 bytes).  Save with GPU digests: all 512 pinned records equal the
    oracle's gather over a host copy of the session's blocks (taken by torch's own indexing), and every CRC32C
    and SHA-256 equals the oracle's.  Restore into a fresh table, then again with every block's CRC32C
    checked in the copy (the checked restore at its default chunking: batched copies, two device slots,
    placements on the aside stream): each time the target blocks equal the oracle's scatter, i.e. the
    source blocks, and the checked restore's CRC32Cs pass."""
    caches, backing = synth.make_caches(36, 16384, layout="kv_split")
    size = 36 * 65536
    plane = planes(caches, capacity=512 * size + (64 << 20))
    keep = synth.fill(plane, 0)
    torch.cuda.synchronize()
    del keep
    assert plane.block_bytes == size == 2359296
    saved, restored = synth.block_tables(16384, 512)
    assert max(saved + restored) < 16384
    staged = plane.pool.reserve(512 * size)
    targets = [(staged, i * size) for i in range(512)]
    digests = []
    plane.save_gather(saved, targets, 8192, digests=digests)
    got = digests[0].result()
    crcs, shas = oracle_lib.digest_records(staged.pointer, size, size, 512, threads=16)
    assert [crc for _, crc in got] == crcs.tolist()
    assert [sha for sha, _ in got] == [bytes(s).hex() for s in shas]
    # The oracle's gather over host copies of the session's blocks, layer by layer ([2, 512, N, H, D] each,
    # K half then V half, in the plane's sorted layer order): block j of the copy is block saved[j].
    src, dst = torch.tensor(saved, device="cuda"), torch.tensor(restored, device="cuda")
    copies, host_spans_ = [], []
    for name, view in plane.caches.items():
        host = view[:, src].contiguous().view(torch.uint8).cpu().numpy().reshape(-1)
        half = host.size // 2
        copies.append(host)
        host_spans_ += [(host.ctypes.data, half // 512, None, half // 512),
                        (host.ctypes.data + half, half // 512, None, half // 512)]
    spans = [(base, pitch, offset, nbytes) for (base, pitch, _, nbytes), (offset, *_rest)
             in zip(host_spans_, plane.spans())]
    assert [s[3] for s in spans] == [s[3] for s in plane.spans()]
    expected = oracle_lib.gather(spans, list(range(512)), size)
    pinned = np.ctypeslib.as_array((C.c_uint8 * (512 * size)).from_address(staged.pointer)).reshape(512, size)
    mismatched = [i for i in range(512) if not np.array_equal(pinned[i], expected[i])]
    assert not mismatched, mismatched[:8]
    del expected, copies
    assert plane.load_scatter(restored, targets) == 19
    torch.cuda.synchronize()
    for view in caches.values():               # [2, blocks, N, H, D]
        assert torch.equal(view[:, src].view(torch.int16), view[:, dst].view(torch.int16))
        view[:, dst] = 0
    assert plane.load_scatter_checked(restored, targets, [crc for _, crc in got]) == 19
    torch.cuda.synchronize()
    for view in caches.values():
        assert torch.equal(view[:, src].view(torch.int16), view[:, dst].view(torch.int16))
    staged.close()


@pytest.mark.parametrize("layers,layout,dtype,block_size,heads,head_dim,source_shift", [
    (4, "vllm", "bf16", 16, 8, 128, 0),        # 64 KiB spans, 16-byte accesses
    (4, "kv_split", "bf16", 16, 8, 128, 8),    # 32 KiB spans from sources 8 bytes off 16: 8-byte accesses
    (4, "kv_split", "fp8", 16, 8, 128, 0),     # 16 KiB spans
    (4, "kv_split", "bf16", 16, 1, 40, 0),     # 1280-byte spans: 80 slots, a short last row of 16
    (4, "vllm", "bf16", 3, 1, 4, 0),           # 48-byte spans: 3 slots
    (4, "kv_split", "bf16", 3, 1, 4, 8),       # 24-byte spans: 1 slot and an 8-byte word; blocks 8 bytes off 16
    (36, "kv_split", "bf16", 16, 1, 128, 0),   # a TP = 8 shard of Qwen3-8B: 72 spans of 4 KiB per record
])
def test_the_checked_restore_kernel_gives_every_record_s_crc32c_and_the_restore_s_bytes(
        planes, oracle_lib, layers, layout, dtype, block_size, heads, head_dim, source_shift):
    """kvsnap_restore_blocks_checked + kvsnap_restore_checked_crc32c through the C-ABI: the KV cache after the
    copy equals the oracle's scatter of the same records, and every record's CRC32C equals the oracle's
    (kvsnap_crc32c_extend, csrc/dataplane/io.cpp:39-44), over spans of every length class the kernel handles."""
    torch_dtype = torch.bfloat16 if dtype == "bf16" else torch.float8_e4m3fn
    caches, backing = synth.make_caches(layers, 64, block_size=block_size, heads=heads, head_dim=head_dim,
                                        dtype=torch_dtype, layout=layout)
    raw = backing.view(torch.uint8)
    generator = torch.Generator(device="cuda").manual_seed(5)
    raw.copy_(torch.randint(0, 256, raw.shape, dtype=torch.uint8, device="cuda", generator=generator))
    plane = planes(caches, block_size=block_size)
    size, n = plane.block_bytes, 29
    staging = plane.pool.reserve(n * size + 16)
    records = np.random.default_rng(6).integers(0, 256, n * size, dtype=np.uint8)
    C.memmove(staging.pointer + source_shift, records.ctypes.data, n * size)
    addresses = [staging.pointer + source_shift + i * size for i in range(n)]
    targets = random.Random(7).sample(range(64), n)
    expected = host_copy(backing)
    oracle_lib.scatter(host_spans(plane, backing, expected), targets, addresses)
    crcs = [oracle_lib.crc32c_at(address, size) for address in addresses]

    tables = plane._load_tables()
    n_spans = tables[0].numel()
    lib = kernel_library()
    table = torch.tensor(addresses + targets, dtype=torch.int64, device="cuda")
    partial = torch.full((n * n_spans,), -1, dtype=torch.int32, device="cuda")
    out = torch.zeros(n, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    for first, last in ((0, 17), (17, n)):      # two launches, each writing its blocks' partials
        _check(lib, lib.kvsnap_restore_blocks_checked(
            table.data_ptr() + 8 * first, table.data_ptr() + 8 * (n + first), last - first,
            *(t.data_ptr() for t in tables), n_spans, 64, partial.data_ptr() + 4 * first * n_spans, stream))
    _check(lib, lib.kvsnap_restore_checked_crc32c(partial.data_ptr(), n, tables[0].data_ptr(), tables[3].data_ptr(),
                                                  n_spans, size, out.data_ptr(), stream))
    torch.cuda.synchronize()
    assert [value & 0xFFFFFFFF for value in out.tolist()] == crcs
    assert np.array_equal(host_copy(backing), expected)
    staging.close()


@pytest.mark.parametrize("layers,layout,dtype,block_size,heads,head_dim,shift,to_host,with_stage,programs", [
    (4, "vllm", "bf16", 16, 8, 128, 0, True, True, 4),        # 64 KiB spans into pinned memory, and a device copy
    (4, "kv_split", "bf16", 16, 8, 128, 8, True, False, 4),   # 32 KiB spans, destinations 8 bytes off 16
    (4, "kv_split", "fp8", 16, 8, 128, 0, False, True, 0),    # 16 KiB spans, device to device, full grid
    (4, "kv_split", "bf16", 16, 1, 40, 0, False, False, 0),   # 1280-byte spans: a short last row
    (4, "vllm", "bf16", 3, 1, 4, 0, True, True, 2),           # 48-byte spans
    (4, "kv_split", "bf16", 3, 1, 4, 8, False, True, 0),      # 24-byte spans: an 8-byte word; 8-byte alignment
    (36, "kv_split", "bf16", 16, 1, 128, 0, False, True, 0),  # a TP = 8 shard of Qwen3-8B: 72 spans of 4 KiB
])
def test_the_checked_gather_kernel_gives_the_oracle_s_records_and_crc32cs(
        planes, oracle_lib, layers, layout, dtype, block_size, heads, head_dim, shift, to_host, with_stage, programs):
    """kvsnap_gather_blocks_checked + kvsnap_restore_checked_crc32c through the C-ABI: every record written (into
    pinned memory over the link, or device memory; and its device copy when asked) equals the oracle's gather of
    the same blocks, and every record's CRC32C equals the oracle's (csrc/dataplane/io.cpp:39-44), over spans of
    every length class the kernel handles; the cache is only read."""
    torch_dtype = torch.bfloat16 if dtype == "bf16" else torch.float8_e4m3fn
    caches, backing = synth.make_caches(layers, 64, block_size=block_size, heads=heads, head_dim=head_dim,
                                        dtype=torch_dtype, layout=layout)
    raw = backing.view(torch.uint8)
    generator = torch.Generator(device="cuda").manual_seed(15)
    raw.copy_(torch.randint(0, 256, raw.shape, dtype=torch.uint8, device="cuda", generator=generator))
    plane = planes(caches, block_size=block_size)
    size, n = plane.block_bytes, 29
    blocks = random.Random(17).sample(range(64), n)
    before = host_copy(backing)
    expected = oracle_lib.gather(host_spans(plane, backing, before), blocks, size)
    if to_host:
        staging = plane.pool.reserve(n * size + 16)
        base, host = staging.pointer + shift, None
    else:
        host = torch.zeros(n * size + 16, dtype=torch.uint8, device="cuda")
        base, staging = host.data_ptr() + shift, None
    stage = torch.zeros(n * size, dtype=torch.uint8, device="cuda") if with_stage else None
    tables = plane._load_tables()
    n_spans = tables[0].numel()
    lib = kernel_library()
    table = torch.tensor([base + i * size for i in range(n)] + blocks, dtype=torch.int64, device="cuda")
    partial = torch.full((n * n_spans,), -1, dtype=torch.int32, device="cuda")
    out = torch.zeros(n, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    for first, last in ((0, 17), (17, n)):      # two launches, each writing its blocks' partials
        _check(lib, lib.kvsnap_gather_blocks_checked(
            table.data_ptr() + 8 * first, table.data_ptr() + 8 * (n + first), last - first,
            *(t.data_ptr() for t in tables), n_spans, stage.data_ptr() + first * size if with_stage else None, size,
            programs, partial.data_ptr() + 4 * first * n_spans, stream))
    _check(lib, lib.kvsnap_restore_checked_crc32c(partial.data_ptr(), n, tables[0].data_ptr(), tables[3].data_ptr(),
                                                  n_spans, size, out.data_ptr(), stream))
    torch.cuda.synchronize()
    if to_host:
        written = np.ctypeslib.as_array((C.c_uint8 * (n * size)).from_address(base)).reshape(n, size).copy()
        staging.close()
    else:
        written = host.cpu().numpy()[shift:shift + n * size].reshape(n, size)
    assert np.array_equal(written, expected)
    if with_stage:
        assert np.array_equal(stage.cpu().numpy().reshape(n, size), expected)
    assert [value & 0xFFFFFFFF for value in out.tolist()] == [oracle_lib.crc32c(r.tobytes()) for r in expected]
    assert np.array_equal(host_copy(backing), before)


@pytest.mark.parametrize("layers,layout,heads,head_dim,blocks_total,n,gap", [
    (4, "vllm", 8, 128, 64, 29, 0),         # 64 KiB spans: 256-group records
    (4, "kv_split", 8, 128, 64, 29, 1024),  # 32 KiB spans, records 1 KiB apart past their ends
    (36, "kv_split", 1, 128, 64, 29, 0),    # a TP = 8 shard of Qwen3-8B: 72 spans of 4 KiB, 288 groups
    (36, "vllm", 1, 128, 64, 3, 0),         # 3 records: most of the grid's waves have none
    (17, "vllm", 1, 16, 5200, 5000, 0),     # 17-group records: a padded first stripe, short batches, two rounds
])
def test_the_gather_with_crc32c_gives_the_oracle_s_records_and_crc32cs(planes, oracle_lib, layers, layout, heads,
                                                                       head_dim, blocks_total, n, gap):
    """kvsnap_gather_crc32c through the C-ABI over the plane's groups' table: every device record equals the
    oracle's gather of its block and every CRC32C the oracle's (csrc/dataplane/io.cpp:39-44), for stripe plans
    with and without front padding, partial batches, idle waves and more records than one round; the cache is
    only read and nothing past a record is written."""
    caches, backing = synth.make_caches(layers, blocks_total, block_size=16, heads=heads, head_dim=head_dim,
                                        layout=layout)
    raw = backing.view(torch.uint8)
    generator = torch.Generator(device="cuda").manual_seed(25)
    raw.copy_(torch.randint(0, 256, raw.shape, dtype=torch.uint8, device="cuda", generator=generator))
    plane = planes(caches, block_size=16)
    size = plane.block_bytes
    pitch = size + gap
    blocks = random.Random(27).sample(range(blocks_total), n)
    before = host_copy(backing)
    expected = oracle_lib.gather(host_spans(plane, backing, before), blocks, size)
    groups = plane.group_tables()
    assert groups is not None and groups[0].numel() == size // 1024
    out = torch.full((n * pitch,), 0xA5, dtype=torch.uint8, device="cuda")
    crcs = torch.zeros(n, dtype=torch.int32, device="cuda")
    ids = torch.tensor(blocks, dtype=torch.int64, device="cuda")
    print(f"gather with CRC32C: {layers} layers {layout}, {size} B records, n={n}, pitch={pitch}", flush=True)
    gather_crc32c_launcher(ids, *groups, size, out.data_ptr(), pitch, crcs)()
    torch.cuda.synchronize()
    written = out.cpu().numpy().reshape(n, pitch)
    assert np.array_equal(written[:, :size], expected)
    assert (written[:, size:] == 0xA5).all()
    assert [value & 0xFFFFFFFF for value in crcs.tolist()] == [oracle_lib.crc32c(r.tobytes()) for r in expected]
    assert np.array_equal(host_copy(backing), before)


@pytest.mark.parametrize("groups,n,blocks_total,seed", [
    (1, 5, 9, 41),          # one-group records: every stripe a single partial batch
    (7, 300, 320, 42),      # odd group count, many records a workgroup
    (300, 40, 48, 43),      # long records, several stripes each
    (17, 5000, 5100, 44),   # more records than one round of the grid
])
def test_the_gather_with_crc32c_follows_any_groups_table(oracle_lib, groups, n, blocks_total, seed):
    """kvsnap_gather_crc32c through the C-ABI over a random groups' table, not a plane's: each 1 KiB group of a
    record comes from one of two regions of different block pitch, at a random KiB of the block's row, in any
    order and some twice.  Every record equals the oracle's gather of its block by the same table, every
    CRC32C the oracle's (csrc/dataplane/io.cpp:39-44), and nothing past a record is written."""
    rng = random.Random(seed)
    pitches = (9 * 1024, 3 * 1024 + 1024)                   # bytes per block in each region
    starts = (0, blocks_total * pitches[0])
    total = starts[1] + blocks_total * pitches[1]
    cache = torch.randint(0, 256, (total,), dtype=torch.uint8, device="cuda",
                          generator=torch.Generator(device="cuda").manual_seed(seed))
    picks = []
    for _ in range(groups):
        region = rng.randrange(2)
        picks.append((region, rng.randrange(pitches[region] // 1024)))
    bases = [cache.data_ptr() + starts[r] + 1024 * k for r, k in picks]
    group_pitches = [pitches[r] for r, _ in picks]
    blocks = [rng.randrange(blocks_total) for _ in range(n)]
    host = cache.cpu().numpy()
    expected = np.stack([np.concatenate([host[starts[r] + b * pitches[r] + 1024 * k:][:1024] for r, k in picks])
                         for b in blocks])
    size, gap = groups * 1024, 48
    pitch = size + gap
    out = torch.full((n * pitch,), 0x5A, dtype=torch.uint8, device="cuda")
    crcs = torch.zeros(n, dtype=torch.int32, device="cuda")
    device_tables = [torch.tensor(v, dtype=torch.int64, device="cuda") for v in (blocks, bases, group_pitches)]
    print(f"gather with CRC32C, random table: {groups} groups, n={n}, seed={seed}", flush=True)
    gather_crc32c_launcher(*device_tables, size, out.data_ptr(), pitch, crcs)()
    torch.cuda.synchronize()
    written = out.cpu().numpy().reshape(n, pitch)
    assert np.array_equal(written[:, :size], expected)
    assert (written[:, size:] == 0x5A).all()
    assert [value & 0xFFFFFFFF for value in crcs.tolist()] == [oracle_lib.crc32c(r.tobytes()) for r in expected]
    assert np.array_equal(cache.cpu().numpy(), host)


@pytest.mark.parametrize("tokens", [12 * BLOCK_SIZE, 12 * BLOCK_SIZE - 7])
def test_a_hashed_direct_save_is_one_checked_gather_and_its_digests_are_the_oracle_s(planes, oracle_lib, tokens):
    """save_mode="direct" with digests: the checked gather writes the pinned records and their device copy and
    folds their CRC32Cs in one pass over the cache; the SHA-256 reads the device copy.  Records (last tail zeroed),
    CRC32Cs and SHA-256s equal the oracle's."""
    caches, backing = synth.make_caches(LAYERS, 40, layout="kv_split")
    plane = planes(caches, save_mode="direct", restore_programs=4)
    keep = synth.fill(plane, 29)
    torch.cuda.synchronize()
    del keep
    saved, _ = synth.block_tables(40, 12)
    size = plane.block_bytes
    before = host_copy(backing)
    expected = oracle_lib.gather(host_spans(plane, backing, before), saved, size)
    staged = plane.pool.reserve(12 * size)
    digests = []
    assert plane.save_gather(saved, [(staged, i * size) for i in range(12)], tokens, digests=digests) == 1
    got = digests[0].result()
    if tokens % BLOCK_SIZE:
        oracle_lib.zero_tail(expected[11], plane.layers, tokens % BLOCK_SIZE)
    pinned = np.ctypeslib.as_array((C.c_uint8 * (12 * size)).from_address(staged.pointer)).reshape(12, size).copy()
    assert np.array_equal(pinned, expected)
    crcs, shas = oracle_lib.digest_records(staged.pointer, size, size, 12, threads=8)
    assert got == [(bytes(h).hex(), int(c)) for h, c in zip(shas, crcs)]
    staged.close()


@pytest.mark.parametrize("restore_mode", ["kernel", "dma"])
def test_a_checked_restore_loads_clean_blocks_and_reports_a_corrupt_one_only_after_the_copy(planes, oracle_lib,
                                                                                           restore_mode):
    from kvsnap_amd.blobs import CorruptSnapshotError
    caches, backing = synth.make_caches(LAYERS, 40, layout="kv_split")
    plane = planes(caches, restore_mode=restore_mode)
    keep = synth.fill(plane, 23)
    torch.cuda.synchronize()
    del keep
    saved, restored = synth.block_tables(40, 12)
    size = plane.block_bytes
    staged = plane.pool.reserve(12 * size)
    sources = [(staged, i * size) for i in range(12)]
    digests = []
    plane.save_gather(saved, sources, 12 * BLOCK_SIZE, digests=digests)
    crcs = [crc for _, crc in digests[0].result()]
    before = host_copy(backing)
    expected = before.copy()
    oracle_lib.scatter(host_spans(plane, backing, expected), restored, [staged.pointer + i * size for i in range(12)])
    # One flipped bit in the tenth block: the copy completes, the load is refused and nothing is reported.
    flip = staged.pointer + 9 * size + 4321
    C.memmove(flip, bytes([C.string_at(flip, 1)[0] ^ 16]), 1)
    progress = []
    with pytest.raises(CorruptSnapshotError, match=r"1 of 12 .*block 9\)"):
        plane.load_scatter_checked(restored, sources, crcs, progress=progress)
    assert progress == []
    torch.cuda.synchronize()
    corrupt = expected.copy()
    oracle_lib.scatter(host_spans(plane, backing, corrupt), restored, [staged.pointer + i * size for i in range(12)])
    assert np.array_equal(host_copy(backing), corrupt)
    C.memmove(flip, bytes([C.string_at(flip, 1)[0] ^ 16]), 1)
    assert plane.load_scatter_checked(restored, sources, crcs, progress=progress, chunk_bytes=5 * size) == 3
    assert [left for _, left in progress] == [12 * size, 0] and progress[1][0].query()
    assert np.array_equal(host_copy(backing), expected)
    staged.close()


@pytest.mark.parametrize("heads", [1, 2, 4])
@pytest.mark.parametrize("layout", ["kv_split", "vllm"])
@pytest.mark.parametrize("restore_mode", ["kernel", "dma"])
def test_a_tensor_parallel_shard_round_trips_with_short_spans(planes, oracle_lib, layout, restore_mode, heads):
    """One tensor-parallel rank's shard of Qwen3-8B (TP = 8, 4 and 2: 1, 2 and 4 KV heads, 4-16 KiB K/V spans,
    8-32 KiB vLLM spans), where the copy launches put several spans in one workgroup and a hashed save takes
    the gather with CRC32C: the gathered records equal the oracle's fill, their digests the oracle's, and the
    restore is the identity, through the restore kernel and the copy engines."""
    caches, backing = synth.make_caches(36, 600, heads=heads, layout=layout)
    plane = planes(caches, capacity=128 * 36 * 8192 * heads + (64 << 20), restore_mode=restore_mode)
    assert plane.min_span_bytes == (4096 if layout == "kv_split" else 8192) * heads
    assert plane.group_tables() is not None
    keep = synth.fill(plane, 3)
    torch.cuda.synchronize()
    del keep
    size = plane.block_bytes
    assert size == 36 * 8192 * heads
    saved, restored = synth.block_tables(600, 128, seed_source=5, seed_target=6)
    assert max(saved + restored) < 600
    staged = plane.pool.reserve(128 * size)
    targets = [(staged, i * size) for i in range(128)]
    digests = []
    plane.save_gather(saved, targets, 128 * 16 - 5, digests=digests)
    got = digests[0].result()
    crcs, shas = oracle_lib.digest_records(staged.pointer, size, size, 128, threads=16)
    assert [crc for _, crc in got] == crcs.tolist()
    assert [sha for sha, _ in got] == [bytes(h).hex() for h in shas]
    for index in (0, 77):
        record = pinned_bytes(staged, index * size, size)
        for s, (offset, _, _, nbytes) in enumerate(plane.spans()):
            assert np.array_equal(record[offset:offset + nbytes],
                                  oracle_lib.fill_span(3, s, saved[index], nbytes, synth.KIND_BF16)), (index, s)
    plane.load_scatter(restored, targets, chunk_bytes=40 * size)
    torch.cuda.synchronize()
    src, dst = torch.tensor(saved[:-1], device="cuda"), torch.tensor(restored[:-1], device="cuda")
    for view in caches.values():
        if layout == "kv_split":               # [2, blocks, N, H, D]
            assert torch.equal(view[:, src].view(torch.int16), view[:, dst].view(torch.int16))
        else:                                   # [blocks, H, N, 2D]
            assert torch.equal(view[src].view(torch.int16), view[dst].view(torch.int16))
    staged.close()


def early_report_scenario(planes):
    """The connector's protocol (reference vllm.py:454-466, 663-679): a loader thread runs the restore while the
    engine polls its progress; at most 128 MiB left, the load is reported and the next forward waits on the last
    launch's event (wait_on_engine_stream).  Checks that work on the engine stream after that wait sees every
    restored byte; returns the slowest progress poll in seconds."""
    import threading
    import time
    from kvsnap_amd.ordering import EARLY_REPORT_BYTES, early_report
    caches, backing = synth.make_caches(36, 1100, layout="kv_split")
    size = 36 * 65536
    plane = planes(caches, capacity=512 * size + (64 << 20))
    keep = synth.fill(plane, 17)
    torch.cuda.synchronize()
    del keep
    saved, restored = synth.block_tables(1100, 512)
    assert max(saved + restored) < 1100
    staged = plane.pool.reserve(512 * size)
    sources = [(staged, i * size) for i in range(512)]
    plane.save_gather(saved, sources, 512 * BLOCK_SIZE)
    dst = torch.tensor(restored, device="cuda")
    src = torch.tensor(saved, device="cuda")
    for view in caches.values():                # [2, blocks, N, H, D]
        view[:, dst] = 0
    torch.cuda.synchronize()
    progress, failure = [], []

    def loader():
        try:
            plane.load_scatter(restored, sources, progress=progress)
        except BaseException as exc:
            failure.append(exc)

    thread = threading.Thread(target=loader)
    thread.start()
    report, deadline, slowest = None, time.monotonic() + 30, 0.0
    while report is None and time.monotonic() < deadline and not failure:
        start = time.monotonic()
        report = early_report(list(progress))
        slowest = max(slowest, time.monotonic() - start)
        time.sleep(0.0002)
    assert report is not None and not failure
    left, last = report
    assert left <= EARLY_REPORT_BYTES
    plane.wait_on_engine_stream(last)
    # The next "forward": reads of the restored blocks, queued on the engine stream.
    seen = [view[:, dst].clone() for view in caches.values()]
    torch.cuda.current_stream().synchronize()
    thread.join()
    for view, got in zip(caches.values(), seen):
        assert torch.equal(got.view(torch.int16), view[:, src].view(torch.int16))
    staged.close()
    return slowest


def test_an_early_reported_restore_is_complete_for_the_engine_stream(planes):
    """The early-report protocol's ordering, with no wall-clock bound (the poll's latency is checked by
    tests/test_zy_timing.py, collected after every parity test)."""
    early_report_scenario(planes)


@pytest.mark.parametrize("seed", range(6))
def test_copy_kernels_on_random_span_tables_including_8_byte_alignment(hip_library, oracle_lib, seed):
    """Random geometries: odd word counts, pitches that are odd multiples of 8 bytes, bases offset by 8,
    so the kernels' 8-byte path runs beside the 16-byte one; gather, restore, scatter and gather-to-records.
    The span-length hint only shapes the launches: unknown, right, far too short and far too long all give
    the oracle's bytes.  With a known hint and a grid sized to the work, the gather and scatter go one wave
    per KiB of a span: the spans here differ in length, so some pieces lie past a span's end and some last
    pieces loop over the rest of a longer span."""
    rng = np.random.default_rng(100 + seed)
    blocks = int(rng.integers(4, 40))
    n_spans = int(rng.integers(1, 9))
    words = [int(rng.integers(1, 3000 if s % 2 else 700)) for s in range(n_spans)]
    hint = [0, 8 * min(words), 16, 1 << 20, 8 * min(words), 4096][seed]
    pitches = [w + int(rng.integers(0, 5)) for w in words]                     # 8-byte words
    shifts = [int(rng.integers(0, 2)) for _ in range(n_spans)]                 # 0 or 1 word of misalignment
    offsets = np.cumsum([0] + words[:-1]).tolist()
    record_words = sum(words)
    stores = [torch.randint(-2**62, 2**62, (blocks * p + 2,), dtype=torch.int64, device="cuda") for p in pitches]
    lib = kernel_library()
    stream = torch.cuda.current_stream().cuda_stream

    def dev(values):
        return torch.tensor(values, dtype=torch.int64, device="cuda")

    offs = dev([o * 8 for o in offsets])
    bases = dev([s.data_ptr() + 8 * sh for s, sh in zip(stores, shifts)])
    pitch_b = dev([p * 8 for p in pitches])
    words_t = dev(words)
    count = int(rng.integers(1, blocks + 1))
    ids = rng.choice(blocks, count, replace=False).tolist()
    host_before = [s.cpu().numpy().copy() for s in stores]
    spans = [(h.ctypes.data + 8 * sh, p * 8, o * 8, w * 8)
             for h, sh, p, o, w in zip(host_before, shifts, pitches, offsets, words)]
    expected = oracle_lib.gather(spans, ids, record_words * 8)
    # gather into a device buffer at an 8-byte (not 16) offset
    out = torch.zeros(count * record_words + 1, dtype=torch.int64, device="cuda")
    _check(lib, lib.kvsnap_gather_blocks(dev(ids).data_ptr(), count, offs.data_ptr(), bases.data_ptr(),
                                         pitch_b.data_ptr(), words_t.data_ptr(), n_spans, hint, out.data_ptr() + 8,
                                         record_words * 8, 0, stream))
    torch.cuda.synchronize()
    got = out.cpu().numpy()[1:].view(np.uint8).reshape(count, -1)
    assert np.array_equal(got, expected)
    # gather-to-records: per-record destinations
    dests = torch.zeros(count * (record_words + 1), dtype=torch.int64, device="cuda")
    dest_ptrs = dev([dests.data_ptr() + 8 * i * (record_words + 1) for i in range(count)])
    _check(lib, lib.kvsnap_gather_to_records(dest_ptrs.data_ptr(), dev(ids).data_ptr(), count, offs.data_ptr(),
                                             bases.data_ptr(), pitch_b.data_ptr(), words_t.data_ptr(), n_spans,
                                             hint, 7, stream))
    torch.cuda.synchronize()
    rows = dests.cpu().numpy().reshape(count, record_words + 1)[:, :record_words]
    assert np.array_equal(rows.view(np.uint8).reshape(count, -1), expected)
    # restore the gathered records into other blocks
    targets = rng.choice(blocks, count, replace=False).tolist()
    sources = dev([out.data_ptr() + 8 + i * record_words * 8 for i in range(count)])
    _check(lib, lib.kvsnap_restore_blocks(sources.data_ptr(), dev(targets).data_ptr(), count, offs.data_ptr(),
                                          bases.data_ptr(), pitch_b.data_ptr(), words_t.data_ptr(), n_spans, hint,
                                          5, stream))
    torch.cuda.synchronize()
    after = [s.cpu().numpy() for s in stores]
    oracle_lib.scatter(spans, targets, [expected[i].ctypes.data for i in range(count)])
    for a, h in zip(after, host_before):
        assert np.array_equal(a, h)
    # scatter the same device records (record pitch, 8-byte offset) into a third and a fourth set of blocks,
    # on a fixed grid and on one sized to the work (one wave per KiB of a span where the hint is known)
    for programs in (3, 0):
        third = rng.choice(blocks, count, replace=False).tolist()
        _check(lib, lib.kvsnap_scatter_blocks(out.data_ptr() + 8, record_words * 8, dev(third).data_ptr(), count,
                                              offs.data_ptr(), bases.data_ptr(), pitch_b.data_ptr(),
                                              words_t.data_ptr(), n_spans, hint, programs, stream))
        torch.cuda.synchronize()
        after = [s.cpu().numpy() for s in stores]
        oracle_lib.scatter(spans, third, [expected[i].ctypes.data for i in range(count)])
        for a, h in zip(after, host_before):
            assert np.array_equal(a, h), programs


def test_gather_and_scatter_of_more_blocks_than_one_launch_takes(hip_library, oracle_lib):
    """70,000 blocks of two 1 KiB spans: the pieces launches carry at most 65,535 blocks each, so the gather and
    the scatter each take two; records and scattered blocks equal the oracle's."""
    blocks, n, words = 70_010, 70_000, [128, 128]
    rng = np.random.default_rng(5)
    stores = [torch.randint(-2**62, 2**62, (blocks * w,), dtype=torch.int64, device="cuda") for w in words]
    lib = kernel_library()
    stream = torch.cuda.current_stream().cuda_stream

    def dev(values):
        return torch.tensor(values, dtype=torch.int64, device="cuda")

    offs, bases, pitches, words_t = dev([0, 1024]), dev([s.data_ptr() for s in stores]), dev([1024, 1024]), dev(words)
    ids = rng.choice(blocks, n, replace=False).tolist()
    host = [s.cpu().numpy() for s in stores]
    spans = [(h.ctypes.data, 1024, o, 1024) for h, o in zip(host, (0, 1024))]
    expected = oracle_lib.gather(spans, ids, 2048)
    out = torch.zeros(n * 256, dtype=torch.int64, device="cuda")
    _check(lib, lib.kvsnap_gather_blocks(dev(ids).data_ptr(), n, offs.data_ptr(), bases.data_ptr(),
                                         pitches.data_ptr(), words_t.data_ptr(), 2, 1024, out.data_ptr(), 2048, 0,
                                         stream))
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint8).reshape(n, -1), expected)
    # the records back into the blocks in reverse order
    targets = ids[::-1]
    _check(lib, lib.kvsnap_scatter_blocks(out.data_ptr(), 2048, dev(targets).data_ptr(), n, offs.data_ptr(),
                                          bases.data_ptr(), pitches.data_ptr(), words_t.data_ptr(), 2, 1024, 0,
                                          stream))
    torch.cuda.synchronize()
    oracle_lib.scatter(spans, targets, [expected[i].ctypes.data for i in range(n)])
    for store, h in zip(stores, host):
        assert np.array_equal(store.cpu().numpy(), h)


@pytest.mark.parametrize("verify", ["gpu", "host"])
def test_pipelined_disk_restore_is_byte_exact_and_refuses_corrupt_blobs(planes, oracle_lib, tmp_path, verify):
    from kvsnap_amd.blobs import BlobDirectory, CorruptSnapshotError
    caches, backing = synth.make_caches(LAYERS, 48, layout="kv_split")
    plane = planes(caches, capacity=128 << 20)
    keep = synth.fill(plane, 31)
    torch.cuda.synchronize()
    del keep
    saved, restored = synth.block_tables(48, 20)
    size = plane.block_bytes
    staged = plane.pool.reserve(20 * size)
    digests = []
    plane.save_gather(saved, [(staged, i * size) for i in range(20)], 20 * BLOCK_SIZE, digests=digests)
    store = BlobDirectory(tmp_path)
    segments = store.write_blocks([(staged.pointer + i * size, size) for i in range(20)], digests[0].result())
    expected = host_copy(backing)
    oracle_lib.scatter(host_spans(plane, backing, expected), restored, [staged.pointer + i * size for i in range(20)])
    progress = []
    launches = plane.load_from_disk(restored, store, segments, chunk_bytes=6 * size, workers=3, verify=verify,
                                    progress=progress)
    assert launches == 4 and progress[0] == (None, 20 * size) and progress[-1][1] == 0
    assert [left for _, left in progress[1:]] == [14 * size, 8 * size, 2 * size, 0]
    assert np.array_equal(host_copy(backing), expected)
    # again through a pool that holds two 3-block chunks: the staging ring, not the snapshot, sizes it
    small = planes(caches, capacity=6 * size + (1 << 20))
    targets = torch.tensor(restored, device="cuda")
    for view in caches.values():              # [2, blocks, N, H, D]; ids < 48
        view[:, targets] = 0
    assert small.load_from_disk(restored, store, segments, chunk_bytes=3 * size, workers=2, verify=verify,
                                ring=2) == 7
    assert np.array_equal(host_copy(backing), expected)
    # a flipped payload bit in the third chunk's blob
    path = store.path(segments[13]["blob_id"])
    raw = bytearray(path.read_bytes())
    raw[-100] ^= 8
    path.write_bytes(bytes(raw))
    with pytest.raises(CorruptSnapshotError):
        plane.load_from_disk(restored, store, segments, chunk_bytes=6 * size, workers=3, verify=verify)
    staged.close()


def test_the_sha_round_probe_times_the_round_sequence(hip_library):
    """kvsnap_sha_round_probe: the round sequence on one wave takes at least its 9 VALU at 4 cycles each a slot
    (and not wildly more), the engine clock it reports is a plausible MI355X clock, and the slots were run (the
    checksum depends on the seed)."""
    out = torch.zeros(3, dtype=torch.int64, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    lib = kernel_library()
    sums = []
    for seed in (1, 2):
        _check(lib, lib.kvsnap_sha_round_probe(seed, 1 << 16, out.data_ptr(), stream))
        cycles, ticks, checksum = out.tolist()
        sums.append(checksum)
    slot = cycles / (1 << 16)
    ghz = cycles / (ticks * 10.0)
    assert 36 <= slot < 60, slot
    assert 0.8 < ghz < 2.6, ghz
    assert sums[0] != sums[1]


@pytest.mark.parametrize("nbytes", [16, 4096 + 16, (1 << 20) + 48, 512 * 294912 + 16])
def test_the_read_probe_reads_every_word_once(hip_library, nbytes):
    """kvsnap_read_probe: the XOR of its sink is the XOR of the buffer's 32-bit words, for a buffer smaller
    than one wave's loads, a ragged one, and a TP = 8 shard's records with one word more (its tail path)."""
    generator = torch.Generator(device="cuda").manual_seed(nbytes)
    buffer = torch.randint(-2**31, 2**31, (nbytes // 4,), dtype=torch.int32, device="cuda", generator=generator)
    sink = torch.zeros(4096, dtype=torch.int32, device="cuda")
    lib = kernel_library()
    _check(lib, lib.kvsnap_read_probe(buffer.data_ptr(), nbytes, sink.data_ptr(),
                                      torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    want = np.bitwise_xor.reduce(buffer.cpu().numpy().view(np.uint32))
    assert np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32)) == want


@pytest.mark.parametrize("nbytes", [16, 4096 + 16, (1 << 20) + 48, 512 * 294912 + 16])
def test_the_copy_probe_copies_every_word_and_nothing_past(hip_library, nbytes):
    """kvsnap_copy_probe: the destination equals the source, and the 64 bytes after it are untouched."""
    generator = torch.Generator(device="cuda").manual_seed(nbytes + 1)
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda", generator=generator)
    dst = torch.full((nbytes + 64,), 0xA5, dtype=torch.uint8, device="cuda")
    lib = kernel_library()
    _check(lib, lib.kvsnap_copy_probe(src.data_ptr(), dst.data_ptr(), nbytes, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert torch.equal(dst[:nbytes], src)
    assert bool((dst[nbytes:] == 0xA5).all())
