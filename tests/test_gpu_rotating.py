"""Rotating fp8 sessions saved and restored beside a decode, against the oracle (the fifth workload).

Qwen3-1.7B's KV shape with an fp8-e4m3 cache: 28 layers of [2, blocks, 16,
8, 128], per-layer scales, 917,504-byte records.  Four sessions of 1k, 2k, 4k
and 8k tokens (64/128/256/512 blocks) are saved (the gather kernel writing
pinned records directly, SHA-256 and CRC32C computed on the GPU) and restored
into other blocks (the copy engines staging each chunk, the scatter kernel
placing it) round-robin from a side thread, while the compute stream runs a
16-sequence synthetic decode that reads random paged blocks of every layer --
the reference's rotating-sessions-under-load measurement
(results/resume-phases.json:351,396).

Every session's pinned records must equal the oracle's gather of the cache,
every digest the oracle's, and the cache afterwards the oracle's scatter of
those records into the restore targets, with every other block untouched.
"""
import random
import threading

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from kvsnap_amd import synth
from kvsnap_amd.dataplane import TorchBlockDataPlane, _check, kernel_library

pytestmark = pytest.mark.gpu

LAYERS, BLOCKS, BLOCK_SIZE = 28, 2048, 16
SESSION_TOKENS = (1024, 2048, 4096, 8192)


def test_rotating_fp8_sessions_beside_a_decode_equal_the_oracle(hip_library, oracle_lib):
    caches, backing = synth.make_caches(LAYERS, BLOCKS, layout="kv_split", dtype=torch.float8_e4m3fn)
    size = LAYERS * 2 * BLOCK_SIZE * 8 * 128
    assert size == 917504
    blocks_needed = sum(t // BLOCK_SIZE for t in SESSION_TOKENS)
    plane = TorchBlockDataPlane(caches, BLOCK_SIZE, blocks_needed * size + (64 << 20), save_mode="direct",
                                restore_programs=4, restore_mode="dma")
    try:
        plane.warm_up()
        assert plane.block_bytes == size
        scales = random.Random(4)
        inverse = [scales.uniform(0.5, 2.0) for _ in range(LAYERS)]
        keep = synth.fill(plane, 9, kind=synth.KIND_E4M3, inv_scales=[inverse[s // 2] for s in range(2 * LAYERS)])
        torch.cuda.synchronize()
        del keep
        before = backing.view(torch.uint8).cpu().numpy().reshape(-1).copy()

        free = list(range(1, BLOCKS))
        random.Random(11).shuffle(free)
        sessions = []
        for tokens in SESSION_TOKENS:
            count = tokens // BLOCK_SIZE
            source, target = free[:count], free[count:2 * count]
            del free[:2 * count]
            pinned = plane.pool.reserve(count * size)
            sessions.append((tokens, source, target, pinned, [(pinned, i * size) for i in range(count)]))

        # The decode: 16 sequences of 256 random blocks, every layer's K and V, on the compute stream.
        lib = kernel_library()
        spans = plane.spans()
        bases, pitches, words = (torch.tensor(column, dtype=torch.int64, device="cuda") for column in
                                 ([s[1] for s in spans], [s[2] for s in spans], [s[3] // 8 for s in spans]))
        seqs, per_seq = 16, 256
        table = torch.tensor([random.Random(100 + q).sample(range(1, BLOCKS), per_seq) for q in range(seqs)],
                             dtype=torch.int64, device="cuda")
        sums = torch.zeros(seqs * len(spans), dtype=torch.int32, device="cuda")
        compute = torch.cuda.current_stream()

        digests, failures, rounds = {}, [], 2

        def rotate():
            try:
                for _ in range(rounds):
                    for tokens, source, target, pinned, targets in sessions:
                        found = []
                        plane.save_gather(source, targets, tokens, digests=found)
                        plane.load_scatter(target, targets)
                        digests[tokens] = found[0]
            except BaseException as exc:
                failures.append(exc)

        side = threading.Thread(target=rotate)
        side.start()
        steps = 0
        while side.is_alive() or steps < 8:
            _check(lib, lib.kvsnap_synth_decode(bases.data_ptr(), pitches.data_ptr(), words.data_ptr(), len(spans),
                                                table.data_ptr(), seqs, per_seq, sums.data_ptr(), 0,
                                                compute.cuda_stream))
            compute.synchronize()
            steps += 1
        side.join(120)
        assert not side.is_alive() and not failures, failures
        torch.cuda.synchronize()

        # The oracle, over the host copy of the cache taken before the first save.
        base = backing.data_ptr()
        host_spans = [(before.ctypes.data + (s[1] - base), s[2], s[0], s[3]) for s in spans]
        expected_cache = before.copy()
        expected_spans = [(expected_cache.ctypes.data + (s[1] - base), s[2], s[0], s[3]) for s in spans]
        for tokens, source, target, pinned, _ in sessions:
            records = oracle_lib.gather(host_spans, source, size)
            landed = np.frombuffer(pinned.read(), dtype=np.uint8).reshape(len(source), size)
            assert np.array_equal(landed, records), tokens
            crcs, shas = oracle_lib.digest_records(records.ctypes.data, size, size, len(source), threads=8)
            assert digests[tokens].result() == [(bytes(s).hex(), int(c)) for s, c in zip(shas, crcs)], tokens
            oracle_lib.scatter(expected_spans, target, [records.ctypes.data + i * size for i in range(len(target))])
        after = backing.view(torch.uint8).cpu().numpy().reshape(-1)
        assert np.array_equal(after, expected_cache)
        assert steps >= 8
        for *_, pinned, _ in sessions:
            pinned.close()
    finally:
        torch.cuda.synchronize()
        plane.close()
