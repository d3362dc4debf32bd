#!/usr/bin/env python
"""KV snapshot save + restore on one MI355X.

Default workload (one step): save an 8192-token Qwen3-8B session -- 512
blocks out of a 16384-block paged cache (36 layers x {K,V}, 8 KV heads,
head_dim 128, block_size 16, bf16 ~N(0,1) from seed 0, block ids seeded) --
with the GPU gather, DMA into pinned host memory and per-block CRC32C +
SHA-256 on the GPU, then restore it from the pinned records into a fresh
seeded block table with the restore kernel.  1,207,959,552 bytes each way.

    python bench.py [--steps K] [--warmup W] [--layout kv_split|vllm]

prints one JSON line: ``value`` = (save bytes + restore bytes) / time per
step, with the cache resident in HBM.  In the timed steps a save's digests are
collected ``--hash-depth`` (2) steps later, so the hashes of consecutive saves
run side by side on their own streams; every digest is complete before the
timer stops.  Also reported: one-at-a-time save/restore latency and GB/s, the
measured pinned<->device DMA peaks and the fractions of them reached,
early-readiness latency, per-kernel HIP-event durations, the rooflines, and
the CPU path timed on this host's cores.

Other workloads (one JSON line each, for the record; not the headline):
    --workload disk-fork      32768-token session saved as blob files with a
                              forked child sharing its first 1536 blocks, then
                              the child restored from disk (pread into pinned
                              staging, CRC32C-verified on the host or the GPU)
    --workload rotating-fp8   Qwen3-1.7B fp8-e4m3 sessions of 1k/2k/4k/8k tokens
                              saved and restored round-robin beside a synthetic
                              16-sequence decode on the compute stream
    --workload turns          an 8192-token Qwen3-8B session growing by 512
                              tokens a turn, each turn end saved into the host
                              tier in full (every block gathered and hashed, as
                              the reference rehashes every block) and by delta
                              (only the blocks past the unchanged prefix), and
                              by delta as blob files
    --workload cpu-roundtrip  the reference's CPU-runnable case (Qwen3-1.7B shape,
                              4096-block cache, 2048-token session): gather,
                              CRC32C, scatter, compare -- on the host cores
                              (the reference's path, restated by the oracle)
                              and on the GPU on the same bytes, the GPU
                              restore checked against the CPU's CRC32Cs
    --workload duplex         the default workload's saves and restores from two
                              threads: session k restored (copy engines, then
                              the scatter kernel) while session k + 1 is saved
    --workload kernels        each kernel alone plus a plain copy of known size
                              (the driver for rocprofv3 counter runs);
                              --kv-heads 4/2/1 gives one tensor-parallel rank's
                              shard at TP = 2/4/8 (4-16 KiB spans)
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import random
import statistics
import sys
import tempfile
import threading
import time

HBM_PEAK_GBPS = 8000.0
LATENCY_SAMPLES = 20
# MI355X's host link, PCIe 5.0 x16: 32 GT/s x 16 lanes, 128b/130b encoding, per direction.
PCIE5_X16_GBPS = round(32 * 16 * 128 / 130 / 8, 2)
# SHA-256 runs one dependency chain per record (two lanes of a round wave).
# The round wave issues 596 VALU per 64-byte block (counted in the gfx950 ISA
# of sha256_kernel: 192 alignbit, 192 bitop3, 74 DPP adds, 64 add3, 64 xad,
# 10 others); a wave64 VALU takes 4 cycles of its SIMD at the 2.4 GHz peak
# engine clock.  All chains run side by side (one round wave per 32 records).
# The round's own 9-VALU sequence is also timed live on one wave
# (kvsnap_sha_round_probe: shader cycles and the 100 MHz constant clock), which
# gives the rate a slot runs at and the engine clock meanwhile; the bound at
# that rate is reported beside the nominal one.
SHA_VALU_PER_BLOCK = 596
SHA_CYCLES_PER_VALU = 4
ENGINE_CLOCK_GHZ = 2.4
SHA_PROBE_SLOTS = 1 << 18
# A floor that does not come from the kernel: FIPS 180-4's round in gfx950
# instructions.  A round is six 32-bit additions (T1 = h + Sigma1 + Ch + (W+K),
# e = d + T1, T2 = Sigma0 + Maj, a = T1 + T2; W+K comes summed from the message
# schedule), two Sigma functions of three rotations XORed, and Ch and Maj.  With
# v_add3_u32 (two additions), v_alignbit_b32 (a rotation) and v_bitop3_b32 (any
# three-input boolean function) that is 3 + 2 * (3 + 1) + 2 = 13 instructions.
# One lane per record issues all 13 in turn; split over two lanes of one wave
# (which run one instruction stream), at best half of them each, rounded up,
# plus one instruction that hands a value to the partner lane: 8.  The chain of
# a record is then 64 rounds of 8 wave64 instructions a block, plus the 8
# additions of the feed-forward (4 a lane).
SHA_FIPS_ROUND_INSTRUCTIONS = 13
SHA_FIPS_TWO_LANE_ROUND = (SHA_FIPS_ROUND_INSTRUCTIONS + 1) // 2 + 1
SHA_FIPS_FEED_FORWARD = 4


def sha_round_rate(torch):
    """The SHA-256 round sequence timed on one wave (median of 5): shader cycles a slot and the engine clock in
    GHz (cycles over the 100 MHz constant clock's ticks)."""
    from kvsnap_amd.dataplane import _check, kernel_library
    lib = kernel_library()
    out = torch.zeros(3, dtype=torch.int64, device="cuda")
    stream = torch.cuda.current_stream()
    samples = []
    for seed in range(6):
        _check(lib, lib.kvsnap_sha_round_probe(seed, SHA_PROBE_SLOTS, out.data_ptr(), stream.cuda_stream))
        cycles, ticks, _ = out.tolist()
        if seed:                       # the first launch warms the clock up
            samples.append((cycles / SHA_PROBE_SLOTS, cycles / (ticks * 10.0)))
    samples.sort()
    return samples[len(samples) // 2]


def sha_issue_bound(record_bytes, records, ms, round_rate):
    """Fraction of the per-chain VALU issue bound the SHA-256 kernel reached; ``round_rate`` is
    sha_round_rate's (cycles a slot, engine GHz)."""
    blocks = record_bytes // 64 + (1 if record_bytes % 64 + 9 <= 64 else 2)
    bound_ms = blocks * SHA_VALU_PER_BLOCK * SHA_CYCLES_PER_VALU / (ENGINE_CLOCK_GHZ * 1e6)
    total = record_bytes * records
    slot_cycles, clock_ghz = round_rate
    sequence_ms = blocks * 64 * slot_cycles / (ENGINE_CLOCK_GHZ * 1e6)
    fips_ms = blocks * (64 * SHA_FIPS_TWO_LANE_ROUND + SHA_FIPS_FEED_FORWARD) * SHA_CYCLES_PER_VALU / (
        ENGINE_CLOCK_GHZ * 1e6)
    one_lane_ms = blocks * (64 * SHA_FIPS_ROUND_INSTRUCTIONS + 2 * SHA_FIPS_FEED_FORWARD) * SHA_CYCLES_PER_VALU / (
        ENGINE_CLOCK_GHZ * 1e6)
    return {"bound": "valu-issue (one chain per record)", "valu_per_block": SHA_VALU_PER_BLOCK,
            "fips_floor": {"instructions_per_round": SHA_FIPS_ROUND_INSTRUCTIONS,
                           "two_lane_instructions_per_round": SHA_FIPS_TWO_LANE_ROUND,
                           "two_lane_floor_ms": round(fips_ms, 3), "frac": round(fips_ms / ms, 4),
                           "one_lane_floor_ms": round(one_lane_ms, 3),
                           "source": "FIPS 180-4 round operations in gfx950 instructions (add3, alignbit, bitop3)"},
            "cycles_per_valu": SHA_CYCLES_PER_VALU, "clock_ghz": ENGINE_CLOCK_GHZ, "bound_ms": round(bound_ms, 3),
            "achieved": round(total / (ms * 1e6), 2), "peak": round(total / (bound_ms * 1e6), 2), "unit": "GB/s",
            "frac": round(bound_ms / ms, 4), "round_cycles_measured": round(slot_cycles, 2),
            "round_probe_clock_ghz": round(clock_ghz, 3),
            "round_probe": "kvsnap_sha_round_probe: the round sequence alone on one wave, s_memtime / s_memrealtime",
            "round_sequence_bound_ms": round(sequence_ms, 3), "frac_of_round_sequence_rate": round(sequence_ms / ms, 4)}


def log(*args):
    print(*args, file=sys.stderr, flush=True)


def median_ms(torch, stream, fn, reps=5, batch=1):
    """Median over ``reps`` of the time per call of ``fn``.  With ``batch`` > 1 a call is queued first and the
    events bracket ``batch`` more, so the GPU never waits for the host to launch (short kernels)."""
    times = []
    for _ in range(reps):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        if batch > 1:
            fn()
        start.record(stream)
        for _ in range(batch):
            fn()
        end.record(stream)
        end.synchronize()
        times.append(start.elapsed_time(end) / batch)
    return statistics.median(times)


def percentile(values, q):
    ordered = sorted(values)
    return ordered[min(len(ordered) - 1, int(round(q / 100 * (len(ordered) - 1))))]


def link_peaks(torch, staged, stream, nbytes):
    """Measured contiguous pinned <-> device DMA rates (GB/s) for one nbytes copy."""
    buffer = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    h2d_ms = median_ms(torch, stream, lambda: staged.copy(buffer.data_ptr(), nbytes, 0, to_host=False))
    d2h_ms = median_ms(torch, stream, lambda: staged.copy(buffer.data_ptr(), nbytes, 0, to_host=True))
    return nbytes / h2d_ms / 1e6, nbytes / d2h_ms / 1e6


def host_threads():
    """(os.cpu_count(), CPUs this process may run on, threads the baseline uses).  One GPU's share of a
    host is taken as 16 CPUs whatever the machine has, so the widest leg runs on at most 16 threads."""
    count = os.cpu_count() or 1
    allowed = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else count
    return count, allowed, max(1, min(16, allowed))


def _timed(fn, seconds):
    """Best of repeated calls of ``fn`` (at least two, for about ``seconds``), in seconds per call."""
    best, spent, calls = float("inf"), 0.0, 0
    while calls < 2 or spent < seconds:
        t0 = time.perf_counter()
        fn()
        took = time.perf_counter() - t0
        best, spent, calls = min(best, took), spent + took, calls + 1
    return best


def cpu_baseline(layers, span, records=512, seconds_per_leg=0.6):
    """The reference's CPU path for the default snapshot, on this host's cores, leg by leg.

    The snapshot: ``records`` records of ``layers`` x ``span`` bytes, gathered
    from seeded random blocks of a host cache of ``2 * records`` blocks (the
    default workload's 512 records of 2,359,296 B: 1.21 GB).  Legs, each in GB/s
    of record bytes and ms for the snapshot:

    * gather / scatter: per-(layer, block) memcpy between the cache and
      packed records (the oracle's restatement of ``dataplane.py:388-437``);
    * crc32c: the SSE4.2 CRC32C of every record (``io.cpp:16-47``);
    * sha256: SHA-256 of every record with the SHA extensions (hashlib's role
      at ``store.py:621-622``, ``volatile.py:229-232``);
    * pread: the records read back from a page-cached file into host memory
      by reader threads, each taking one record at a time and checking its
      CRC32C (``read_prepared_into``, ``store.py:686-723``), through this
      repository's ``io.cpp`` pool (the reference's I/O C-ABI).

    Each leg runs on 1 thread, on 8 (the reference's hash and read pools) and
    on the host's share ``N`` (``host_threads``).  ``value``: save + restore
    bytes over gather + CRC32C + SHA-256 + scatter at ``N`` threads.
    """
    import concurrent.futures
    import numpy as np
    import oracle
    from kvsnap_amd.native_io import IO_LIBRARY, NativeIO
    oracle.build()
    oracle.sha256_select(True)
    lib = oracle.lib()
    count, allowed, widest = host_threads()
    record = layers * span
    host_blocks = 2 * records
    rng = np.random.default_rng(0)
    cache = np.empty(layers * host_blocks * span, dtype=np.uint8)
    chunk = rng.integers(0, 256, size=64 << 20, dtype=np.uint8)
    for at in range(0, cache.size, chunk.size):
        cache[at:at + chunk.size] = chunk[:cache.size - at]
    base = cache.ctypes.data
    span_base = np.array([base + l * host_blocks * span for l in range(layers)], dtype=np.uint64)
    span_pitch = np.full(layers, span, dtype=np.int64)
    span_off = np.arange(layers, dtype=np.int64) * span
    span_len = np.full(layers, span, dtype=np.int64)
    order = random.Random(1).sample(range(host_blocks), host_blocks)
    ids = np.array(order[:records], dtype=np.int64)
    dst = np.array(order[records:], dtype=np.int64)
    packed = np.zeros(records * record, dtype=np.uint8)
    sources = np.arange(records, dtype=np.uint64) * record + packed.ctypes.data
    crcs = np.zeros(records, dtype=np.uint32)
    shas = np.zeros((records, 32), dtype=np.uint8)
    copy_args = (layers, span_base.ctypes.data, span_pitch.ctypes.data, span_off.ctypes.data, span_len.ctypes.data)

    def gather(threads):
        lib.oracle_copy_threads(*copy_args, ids.ctypes.data, None, records, packed.ctypes.data, record, threads)

    def scatter(threads):
        lib.oracle_copy_threads(*copy_args, dst.ctypes.data, sources.ctypes.data, records, None, record, threads)

    def crc(threads):
        lib.oracle_digest_records(packed.ctypes.data, record, record, records, crcs.ctypes.data, None, threads)

    def sha(threads):
        lib.oracle_digest_records(packed.ctypes.data, record, record, records, None, shas.ctypes.data, threads)

    gather(widest)
    crc(widest)
    expected = crcs.copy()
    legs = {"gather": gather, "scatter": scatter, "crc32c": crc, "sha256": sha}
    thread_counts = sorted({1, 8, widest})
    result = {name: {} for name in list(legs) + ["pread"]}
    with tempfile.TemporaryDirectory(prefix="kvsnap-cpu-") as folder:
        path = os.path.join(folder, "records")
        with open(path, "wb") as f:
            f.write(memoryview(packed))
        fd = os.open(path, os.O_RDONLY)
        try:
            def pread(threads):
                # The reference's read path (store.py:686-723): reader threads each pread one record through a
                # native I/O pool of as many workers (this repository's io.cpp, the same C-ABI) and check its
                # CRC32C (the oracle's SSE4.2 restatement of io.cpp:16-47).
                io = NativeIO(IO_LIBRARY, workers=threads, queue_bytes=64 << 20)

                def one(i):
                    at = packed.ctypes.data + i * record
                    io.pread_into(fd, at, record, i * record)
                    if oracle.crc32c_at(at, record) != expected[i]:
                        raise RuntimeError("a record read back fails its CRC32C")
                try:
                    with concurrent.futures.ThreadPoolExecutor(threads) as readers:
                        list(readers.map(one, range(records)))
                finally:
                    io.close()

            legs["pread"] = pread
            for threads in thread_counts:
                for name, fn in legs.items():
                    seconds = _timed(lambda: fn(threads), seconds_per_leg)
                    result[name][threads] = seconds
        finally:
            os.close(fd)
    total = records * record
    save_restore = {t: 2 * total / sum(result[n][t] for n in ("gather", "crc32c", "sha256", "scatter")) / 1e9
                    for t in thread_counts}
    return {"value": round(save_restore[widest], 3), "unit": "GB/s", "cores": widest, "kind": "port",
            "nproc": count, "affinity_cpus": allowed, "threads": thread_counts,
            "legs_gbps": {name: {str(t): round(total / s / 1e9, 3) for t, s in times.items()}
                          for name, times in result.items()},
            "legs_ms": {name: {str(t): round(s * 1e3, 2) for t, s in times.items()} for name, times in result.items()},
            "save_restore_gbps": {str(t): round(v, 3) for t, v in save_restore.items()},
            "pread_kind": "this repository's io.cpp pool (threads workers) + the oracle's CRC32C",
            "sample": (f"the {records}-record snapshot ({records} x {record} B = {total} B) gathered from and "
                       f"scattered into a {host_blocks}-block host cache; best of repeated runs per leg; pread from "
                       f"a page-cached file"),
            "threads_note": "widest leg = min(16, CPUs this process may use): one GPU's share of the host's CPUs"}


def measured_traffic(kernel):
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3 counter summary
    (FETCH_SIZE and WRITE_SIZE, each scaled by a plain copy of known size), or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "qwen3-8b-8k-kernels.traffic.json")
    try:
        with open(path) as f:
            return round(json.load(f)["kernels"][kernel]["traffic_bytes"])
    except (OSError, KeyError, ValueError):
        return None


def span_rows(torch, plane, ids):
    """Per span of the plane: a host copy (numpy uint8, ``len(ids)`` rows of the span's bytes) of blocks ``ids``,
    read by torch from the raw storage bytes, whatever the caches' layout."""
    index = torch.tensor(ids, dtype=torch.int64, device="cuda")
    out = []
    for _, base, pitch, nbytes in plane.spans():
        tensor = next(t for t in plane.caches.values()
                      if t.untyped_storage().data_ptr() <= base < t.untyped_storage().data_ptr() + t.untyped_storage().nbytes())
        storage = tensor.untyped_storage()
        flat = torch.empty(0, dtype=torch.uint8, device="cuda").set_(storage)
        blocks = (storage.nbytes() - (base - storage.data_ptr()) - nbytes) // pitch + 1
        view = flat.as_strided((blocks, nbytes), (pitch, 1), base - storage.data_ptr())
        out.append(view[index].contiguous().cpu().numpy())
    return out


def same_blocks(torch, caches, a, b):
    ia, ib = torch.tensor(a, device="cuda"), torch.tensor(b, device="cuda")
    return all(torch.equal(t[:, ia].view(torch.int16), t[:, ib].view(torch.int16)) if t.ndim == 5
               else torch.equal(t[ia].view(torch.int16), t[ib].view(torch.int16)) for t in caches.values())


# ---------------------------------------------------------------- default workload

def run_save_restore(args):
    import torch
    from kvsnap_amd import synth
    from kvsnap_amd.dataplane import (KernelTimer, TorchBlockDataPlane, _check, gather_blocks, kernel_library,
                                      scatter_blocks)
    from kvsnap_amd.ordering import early_launch_index

    layers, num_blocks, block_size, tokens = 36, 16384, 16, 8192
    session = tokens // block_size
    caches, backing = synth.make_caches(layers, num_blocks, block_size=block_size, layout=args.layout)
    # Nothing else runs on the GPU here, so the restore kernel reads the pinned records in place (about 1 %
    # faster than the copy engines, the library's default for serving beside a decode; --restore-mode dma
    # measures that default).
    plane = TorchBlockDataPlane(caches, block_size, session * layers * 65536 + (64 << 20),
                                restore_mode=args.restore_mode or "kernel")
    plane.warm_up()
    keep = synth.fill(plane, 0)
    torch.cuda.synchronize()
    del keep
    size = plane.block_bytes
    total = session * size
    source, target = synth.block_tables(num_blocks, session)
    staged = plane.pool.reserve(total)
    targets = [(staged, i * size) for i in range(session)]
    log(f"setup: {layers} layers x {num_blocks} blocks ({args.layout}), record {size} B, session {total} B")
    h2d_peak, d2h_peak = link_peaks(torch, staged, plane._copy_stream, total)
    log(f"DMA peaks: H2D {h2d_peak:.1f} GB/s, D2H {d2h_peak:.1f} GB/s")

    # Latency, one operation at a time (not the timed region): save until the
    # D2H fence, save until its CRC32C and SHA-256 are ready, restore, and the
    # checked restore (every block's CRC32C folded in as it is copied, then
    # compared with the save's), none of them carrying timing events (events
    # around each of a restore's 19 launches add 0.24 ms to it).  Then a
    # restore with every launch timed, for the early-readiness point and for
    # where a slow restore spent its time: the host's wall clock against the
    # GPU's span from its first launch's start to its last launch's end, and
    # the longest launch.  Last, a save with no digests asked for, as the
    # reference's connector calls it (its staging copied in 512 MiB rounds
    # instead of the hashed save's one).  Medians, maxima and nearest-rank p99
    # over ``LATENCY_SAMPLES`` samples after one discarded, every sample
    # reported.
    latency = {"save": [], "hashed": [], "save_plain": [], "restore": [], "early": [], "checked": [],
               "timed_restore": [], "timed_restore_gpu_span": [], "timed_restore_longest_launch": []}
    lat_timer = KernelTimer()
    for i in range(LATENCY_SAMPLES + 1):
        digests, progress = [], []
        t0 = time.perf_counter()
        plane.save_gather(source, targets, tokens, digests=digests)
        t1 = time.perf_counter()
        saved_crcs = [crc for _, crc in digests[0].result()]
        t2 = time.perf_counter()
        plane.load_scatter(target, targets)
        t3 = time.perf_counter()
        plane.load_scatter_checked(target, targets, saved_crcs)
        t4 = time.perf_counter()
        lat_timer.reset()
        plane.timer = lat_timer if i else None
        plane.load_scatter(target, targets, progress=progress)
        t5 = time.perf_counter()
        plane.load_scatter_checked(target, targets, saved_crcs)
        plane.timer = None
        t6 = time.perf_counter()
        plane.save_gather(source, targets, tokens)          # the connector's save: no digests asked for
        t7 = time.perf_counter()
        if i:
            latency["save_plain"].append((t7 - t6) * 1e3)
            latency["checked"].append((t4 - t3) * 1e3)
            latency["save"].append((t1 - t0) * 1e3)
            latency["hashed"].append((t2 - t0) * 1e3)
            latency["restore"].append((t3 - t2) * 1e3)
            latency["timed_restore"].append((t5 - t4) * 1e3)
            # Per launch: the restore kernel's spans, or with copy-engine restores the placements' (the copies
            # are timed per copy, up to four launches' blocks at a time); the span opens at the first copy.
            pairs = lat_timer.pairs["restore" if plane.restore_mode == "kernel" else "place"]
            start = lat_timer.pairs["restore"][0][0]
            latency["early"].append(start.elapsed_time(pairs[early_launch_index(progress)][1]))
            latency["timed_restore_gpu_span"].append(start.elapsed_time(pairs[-1][1]))
            latency["timed_restore_longest_launch"].append(max(a.elapsed_time(b) for a, b in pairs))
    lat = {k: statistics.median(v) for k, v in latency.items()}
    checked_launch_ms = lat_timer.summary()["restore_checked"]["avg_ms"]

    # Throughput: each step saves the session (gather, D2H, GPU CRC32C +
    # SHA-256) and restores it into the target blocks.  A save's digests are
    # collected ``hash_depth`` steps later, as a connector's commit thread
    # would; the timed region ends only when every digest is complete.
    from collections import deque
    pending, collected = deque(), []

    def step():
        digests = []
        plane.save_gather(source, targets, tokens, digests=digests)
        plane.load_scatter(target, targets)
        pending.append(digests[0])
        while len(pending) > args.hash_depth:
            collected[:] = [pending.popleft().result()]

    def drain():
        while pending:
            collected[:] = [pending.popleft().result()]
        return collected[0]

    for _ in range(args.warmup):
        step()
    drain()
    # In the timed steps only the roofline's kernel, the gather (one launch a step), carries timing events:
    # a pair around each of a step's ~50 launches added about 0.15 ms of stream time per step.
    timer = KernelTimer(names={"gather"})
    plane.timer = timer
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(args.steps):
        step()
    digests = drain()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    plane.timer = None
    ms_per_step = elapsed * 1e3 / args.steps
    # The other kernels' in-step times: a few more steps, every launch timed, after the timed region.
    instrumented_steps = 3
    plane.timer = in_step = KernelTimer()
    for _ in range(instrumented_steps):
        step()
    drain()
    plane.timer = None
    kernels = dict(in_step.summary(), gather=timer.summary()["gather"])
    launches = len(plane._launch_bounds(session, 64 << 20))     # a restore's launches at the default chunking

    # Parity of the last step, outside the timed region.
    import oracle
    exact = same_blocks(torch, caches, source, target)
    crcs, shas = oracle.digest_records(staged.pointer, size, size, session, threads=min(16, os.cpu_count() or 1))
    digests_exact = all(crc == int(c) and sha == bytes(s).hex() for (sha, crc), c, s in zip(digests, crcs, shas))
    log(f"parity: restore byte-exact={exact}, CRC32C+SHA-256 bit-exact={digests_exact}")

    gather, restore, crc, sha = kernels["gather"], kernels["restore"], kernels["crc32c"], kernels["sha256"]
    # Read + write of every record, over the save's gather launches: the first chunk's on the copy stream
    # and the rest's on the lead stream (one launch where the plane has no lead stream).
    gather_per_save = gather["launches"] // args.steps
    gather_achieved = 2 * total * args.steps / (gather["total_ms"] * 1e6)
    restore_link = (total * instrumented_steps / restore["launches"]) / (restore["avg_ms"] * 1e6)
    # After the timed region, on the session's records gathered into device memory: the scatter (the
    # verified restore's last step) into the restore targets, which already hold the same bytes, and the
    # CRC32C kernel alone (in the steps it shares the GPU with earlier saves' SHA-256 kernels).
    records = torch.empty(total, dtype=torch.uint8, device="cuda")
    tables = plane._load_tables()
    src_ids = torch.tensor(source, dtype=torch.int64, device="cuda")
    dst_ids = torch.tensor(target, dtype=torch.int64, device="cuda")
    gather_blocks(src_ids, *tables, records.data_ptr(), size, min_span_bytes=plane.min_span_bytes)
    stream = torch.cuda.current_stream()
    scatter_ms = median_ms(torch, stream, lambda: scatter_blocks(records.data_ptr(), size, dst_ids, *tables,
                                                                 min_span_bytes=plane.min_span_bytes),
                           reps=5, batch=4)
    lib = kernel_library()
    crc_out = torch.empty(session, dtype=torch.int32, device="cuda")
    work_bytes = int(lib.kvsnap_crc32c_workspace_bytes(size, session))
    work = torch.empty(work_bytes, dtype=torch.uint8, device="cuda")
    crc_alone_ms = median_ms(torch, stream, lambda: _check(lib, lib.kvsnap_crc32c_records(
        records.data_ptr(), size, size, session, 0, crc_out.data_ptr(), work.data_ptr(), work_bytes,
        stream.cuda_stream)), reps=5, batch=4)
    # SHA-256 alone, one launch over the whole chain (in the steps a save's hash is fed as block-range
    # launches beside the copies and the earlier saves' hashes, so its in-step span counts their overlap).
    sha_out = torch.empty((session, 32), dtype=torch.uint8, device="cuda")
    sha_alone_ms = median_ms(torch, stream, lambda: _check(lib, lib.kvsnap_sha256_records(
        records.data_ptr(), size, size, session, sha_out.data_ptr(), stream.cuda_stream)), reps=3)
    # What the same bytes take with nothing but the copy or the read: a contiguous copy with the gather and
    # scatter kernels' shape (kvsnap_copy_probe) and a plain read with the CRC32C kernel's (kvsnap_read_probe).
    copied = torch.empty(total, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(4096, dtype=torch.int32, device="cuda")
    copy_probe_ms = median_ms(torch, stream, lambda: _check(lib, lib.kvsnap_copy_probe(
        records.data_ptr(), copied.data_ptr(), total, stream.cuda_stream)), reps=5, batch=4)
    read_probe_ms = median_ms(torch, stream, lambda: _check(lib, lib.kvsnap_read_probe(
        records.data_ptr(), total, sink.data_ptr(), stream.cuda_stream)), reps=5, batch=4)
    del records, work, sha_out, copied
    scatter_achieved = 2 * total / (scatter_ms * 1e6)
    crc_achieved = total / (crc_alone_ms * 1e6)
    copy_probe = 2 * total / (copy_probe_ms * 1e6)
    read_probe = total / (read_probe_ms * 1e6)
    cpu = None if args.no_cpu_baseline else cpu_baseline(layers, 65536, session, args.cpu_seconds)
    out = {
        "metric": "8k Qwen3-8B KV restore/save GB/s and ms; % of host-link and HBM roofline",
        "value": round(2 * total / (ms_per_step * 1e6), 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic (seeded bf16 ~N(0,1) KV, seeded block tables)",
        "config": {"workload": "qwen3-8b-8k-token-snapshot-save-then-restore", "layers": layers, "kv_heads": 8,
                   "head_dim": 128, "block_size": block_size, "cache_blocks": num_blocks, "session_blocks": session,
                   "snapshot_bytes": total, "kv_dtype": "bf16", "layout": args.layout,
                   "restore_mode": plane.restore_mode, "parallelism": "none (one GPU)"},
        "hash_depth": args.hash_depth,
        "save_ms": round(lat["save"], 3),
        "save_gbps": round(total / lat["save"] / 1e6, 2),
        "save_hashed_ms": round(lat["hashed"], 3),
        # The same digests on this box's host cores instead (SHA-NI and SSE4.2 over the pinned records once the
        # D2H has landed, the reference's way): the save, then the CPU baseline's SHA-256 and CRC32C legs.
        "hashes_ready_host_ms": None if cpu is None else {
            threads: round(lat["save"] + cpu["legs_ms"]["sha256"][threads] + cpu["legs_ms"]["crc32c"][threads], 3)
            for threads in cpu["legs_ms"]["sha256"]},
        "save_plain_ms": round(lat["save_plain"], 3),
        "restore_ms": round(lat["restore"], 3),
        "restore_gbps": round(total / lat["restore"] / 1e6, 2),
        "restore_launches": launches,
        "restore_early_ready_ms": round(lat["early"], 3),
        "restore_checked_ms": round(lat["checked"], 3),
        "restore_checked_gbps": round(total / lat["checked"] / 1e6, 2),
        "restore_checked_frac_of_h2d": round(total / lat["checked"] / 1e6 / h2d_peak, 4),
        "restore_checked_launch_ms": round(checked_launch_ms, 4),
        "latency_samples_ms": {k: [round(v, 2) for v in vs] for k, vs in latency.items()},
        "latency_max_ms": {k: round(max(vs), 3) for k, vs in latency.items()},
        "latency_p99_ms": {k: round(percentile(vs, 99), 3) for k, vs in latency.items()},
        "latency_median_ms": {k: round(v, 3) for k, v in lat.items()},
        "streams": plane.stream_report(),
        "h2d_peak_gbps": round(h2d_peak, 2),
        "d2h_peak_gbps": round(d2h_peak, 2),
        "restore_frac_of_h2d": round(total / lat["restore"] / 1e6 / h2d_peak, 4),
        "save_frac_of_d2h": round(total / lat["save"] / 1e6 / d2h_peak, 4),
        "pcie5_x16_gbps": PCIE5_X16_GBPS,
        "restore_frac_of_pcie5_x16": round(total / lat["restore"] / 1e6 / PCIE5_X16_GBPS, 4),
        "save_frac_of_pcie5_x16": round(total / lat["save"] / 1e6 / PCIE5_X16_GBPS, 4),
        "kernels_ms": {name: round(k["total_ms"] / args.steps if name == "gather" else k["avg_ms"], 4)
                       for name, k in kernels.items()},
        "kernels_ms_source": "gather: HIP events in the timed steps, summed over a save's launches; the others: "
                             "3 steps after them with every launch timed, per launch",
        "roofline": {"kernel": "gather_pieces_kernel", "bound": "hbm", "achieved": round(gather_achieved, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(gather_achieved / HBM_PEAK_GBPS, 4),
                     "launches_per_save": gather_per_save,
                     "traffic": measured_traffic("gather_pieces_kernel"), "algorithmic_bytes": 2 * total,
                     "traffic_source": "profiles/qwen3-8b-8k-kernels.traffic.md (rocprofv3 FETCH_SIZE, WRITE_SIZE)",
                     "copy_probe_gbps": round(copy_probe, 1),
                     "frac_of_copy_probe": round(gather_achieved / copy_probe, 4),
                     "copy_probe": "kvsnap_copy_probe: the same bytes copied contiguously, a 64-lane workgroup a KiB"},
        "link_roofline": {"kernel": "restore_kernel", "bound": "host-link", "achieved": round(restore_link, 2),
                          "peak": round(h2d_peak, 2), "unit": "GB/s", "frac": round(restore_link / h2d_peak, 4)},
        "scatter_roofline": {"kernel": "scatter_pieces_kernel (device records to cache)", "bound": "hbm",
                             "achieved": round(scatter_achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                             "frac": round(scatter_achieved / HBM_PEAK_GBPS, 4), "ms": round(scatter_ms, 4),
                             "frac_of_copy_probe": round(scatter_achieved / copy_probe, 4)},
        "crc_roofline": {"kernel": "crc_records_kernel", "bound": "hbm", "achieved": round(crc_achieved, 1),
                         "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(crc_achieved / HBM_PEAK_GBPS, 4),
                         "ms": round(crc_alone_ms, 4), "in_step_ms": round(crc["avg_ms"], 4),
                         "read_probe_gbps": round(read_probe, 1),
                         "frac_of_read_probe": round(crc_achieved / read_probe, 4),
                         "read_probe": "kvsnap_read_probe: the same bytes read with this kernel's workgroup shape"},
        "sha256": {"kernel": "sha256_kernel", "ms": round(sha_alone_ms, 3),
                   "gbps": round(total / (sha_alone_ms * 1e6), 2), "records": session,
                   "in_step_ms": round(sha["avg_ms"], 3),
                   "issue_roofline": sha_issue_bound(size, session, sha_alone_ms, sha_round_rate(torch)),
                   "cpu_ms_by_threads": cpu["legs_ms"]["sha256"] if cpu else None},
        "parity": {"restore_byte_exact": exact, "digests_bit_exact": digests_exact},
        "cpu_baseline": cpu,
    }
    staged.close()
    plane.close()
    del plane, staged, targets, tables
    torch.cuda.empty_cache()
    if not args.no_disk_fork:
        # The fourth workload at full size on the same caches.
        out["disk_fork"] = disk_fork(args, caches)
    del caches, backing
    torch.cuda.empty_cache()
    if not args.no_rotating:
        # The fifth workload beside this one, in the same line.
        rotating = run_rotating(args, hashed=True)
        out["rotating_fp8"] = {key: rotating[key] for key in (
            "metric", "value", "unit", "copy_alone_gbps", "rounds", "record_bytes", "sessions_tokens",
            "decode_step_ms", "p99_compute_stall_ms", "save_mode", "restore_mode", "restore_programs",
            "byte_exact", "saves_hashed", "digests_exact", "streams")}
    if not args.no_duplex:
        # The same session's saves and restores overlapped from two threads, as a connector's save threads
        # and loader thread issue them (every save still hashed): the link's two directions at once.  It ran
        # in a process of its own before this one touched the GPU, as a connector's plane would: a process's
        # first planes find restore streams on the fast copy engines (89-91 GB/s), its third plane did not
        # (70-82 GB/s when this line measured it in-process).
        duplex = getattr(args, "duplex_result", None)
        process = "its own, run before this one touched the GPU"
        if duplex is None:
            duplex, process = run_duplex(args), "this one (a later plane)"
        out["duplex"] = {key: duplex[key] for key in (
            "metric", "value", "unit", "steps", "ms_per_step", "duplex_link_gbps", "restore_mode", "save_mode",
            "restore_stream_check", "parity", "streams")}
        out["duplex"]["process"] = process
        if duplex is args.duplex_result:
            # The same workload again in this process, whose earlier planes (the 8k plane, the disk-fork plane
            # and the rotating fp8 plane) created their streams first: what a process's later plane finds.
            later = run_duplex(args)
            out["duplex"]["in_this_process"] = {key: later[key] for key in (
                "value", "ms_per_step", "duplex_link_gbps", "restore_stream_check", "parity")}
            out["duplex"]["in_this_process"]["plane"] = "the fourth plane of the bench process"
    out["hw_queues"] = os.environ.get("GPU_MAX_HW_QUEUES")
    return out


# ---------------------------------------------------------------- disk-staged restore with fork dedup

def run_disk_fork(args):
    from kvsnap_amd import synth
    caches, _ = synth.make_caches(36, 16384, block_size=16, layout=args.layout)
    return disk_fork(args, caches)


def disk_fork(args, caches):
    """The fourth workload on 16384-block Qwen3-8B caches (filled here with seed 0): a 32k-token parent session
    (2048 records, 4,831,838,208 B) and a forked child whose first 1536 blocks hold the parent's bytes in blocks
    of its own, each saved as blob files (GPU gather, D2H, GPU CRC32C + SHA-256 ids, content-addressed writes:
    2560 blobs), then the child restored from disk into fresh blocks by the pipelined reader with every block's
    CRC32C checked before its placement (reference store.py:616-628, 686-723; results/restore-qwen3-8b.json).
    Checks: the ids and CRC32Cs equal the oracle's digests of the pinned records; a sample of restored blocks
    equals the oracle's scatter of the blob files' payloads; every restored block equals its source block."""
    import numpy as np
    import torch
    import oracle
    from kvsnap_amd.blobs import BlobDirectory
    from kvsnap_amd.dataplane import KernelTimer, TorchBlockDataPlane
    from kvsnap_amd.native_io import IO_LIBRARY, NativeIO

    layers, block_size, tokens, shared = 36, 16, 32768, 1536
    num_blocks = next(iter(caches.values())).shape[1 if args.layout == "kv_split" else 0]
    n = tokens // block_size
    size = layers * 65536
    ring, chunk = 4, 128 << 20
    plane = TorchBlockDataPlane(caches, block_size, n * size + ring * chunk + (64 << 20), restore_mode="dma")
    plane.warm_up()
    # Seed-0 contents in every block (an earlier workload's restores copied blocks onto others, and a parent
    # holding two equal blocks would dedup within itself).
    from kvsnap_amd import synth
    keep = synth.fill(plane, 0)
    torch.cuda.synchronize()
    del keep
    parent = random.Random(1).sample(range(1, num_blocks), n)
    taken = set(parent)
    fresh = random.Random(3).sample([b for b in range(1, num_blocks) if b not in taken], n - shared)
    child = parent[:shared] + fresh
    taken |= set(fresh)
    target = random.Random(2).sample([b for b in range(1, num_blocks) if b not in taken], n)
    root = tempfile.mkdtemp(prefix="kvsnap-blobs-", dir=args.disk_dir)
    store = BlobDirectory(root)
    io = store.io = NativeIO(IO_LIBRARY, workers=8, queue_bytes=64 << 20)
    phases, written, segments, digests_exact = {}, {}, {}, True
    threads = host_threads()[2]
    staged = plane.pool.reserve(n * size)
    for name, ids in (("parent", parent), ("child", child)):
        targets = [(staged, i * size) for i in range(n)]
        digests = []
        t0 = time.perf_counter()
        plane.save_gather(ids, targets, tokens, digests=digests)
        t1 = time.perf_counter()
        dig = digests[0].result()
        t2 = time.perf_counter()
        segments[name] = store.write_blocks([(staged.pointer + i * size, size) for i in range(n)], dig)
        t3 = time.perf_counter()
        written[name] = store.written
        crcs, shas = oracle.digest_records(staged.pointer, size, size, n, threads=threads)
        digests_exact &= dig == [(bytes(h).hex(), int(c)) for h, c in zip(shas, crcs)]
        phases[name] = {"gather_d2h_ms": round((t1 - t0) * 1e3, 2), "hashes_ready_ms": round((t2 - t0) * 1e3, 2),
                        "blob_write_ms": round((t3 - t2) * 1e3, 2)}
    staged.close()
    shared_ids = sum(1 for a, b in zip(segments["parent"], segments["child"]) if a["blob_id"] == b["blob_id"])
    blobs = len(os.listdir(os.path.join(root, "blobs")))
    log(f"disk-fork: {blobs} blobs, child shares {shared_ids} with parent, wrote {written}")
    crcs = [s["crc32c"] for s in segments["child"]]
    target_index = torch.tensor(target, device="cuda")

    def scrub():
        for t in caches.values():
            if t.ndim == 5:
                t[:, target_index] = 0
            else:
                t[target_index] = 0
        torch.cuda.synchronize()

    # The two stages apart, then pipelined: the reader alone into a ring that is released at once (no copy),
    # and the copies, checks and placements alone from records already in pinned memory.
    ring_alloc = plane.pool.reserve(ring * chunk)
    per_chunk = chunk // size
    t0 = time.perf_counter()
    with store.ring_reader(segments["child"], ring_alloc.pointer, size, per_chunk, ring, workers=8,
                           verify="none") as reader:
        for k in range(reader.chunks):
            reader.wait(k)
            reader.release(k)
    read_alone_ms = (time.perf_counter() - t0) * 1e3
    ring_alloc.close()
    restores = {}
    for label, workers in (("workers_8", 8), ("workers_16", 16)):
        samples = []
        for rep in range(3):
            scrub()
            timer = KernelTimer()
            plane.timer = timer
            t0 = time.perf_counter()
            plane.load_from_disk(target, store, segments["child"], workers=workers, verify="gpu", chunk_bytes=chunk,
                                 ring=ring)
            samples.append((time.perf_counter() - t0) * 1e3)
            plane.timer = None
        exact = same_blocks(torch, caches, child, target)
        # The per-chunk timeline of the last repetition: each chunk's copy start and end, and its placement's
        # end, in ms after the first copy started (GPU clock).
        pairs = timer.pairs
        zero = pairs["disk_copy"][0][0]
        timeline = [[round(zero.elapsed_time(a), 3), round(zero.elapsed_time(b), 3),
                     round(zero.elapsed_time(p[1]), 3)] for (a, b), p in zip(pairs["disk_copy"], pairs["place"])]
        copy_busy = sum(a.elapsed_time(b) for a, b in pairs["disk_copy"])
        best = min(samples)
        restores[label] = {"read_workers": workers, "ms": round(best, 2), "gbps": round(n * size / best / 1e6, 2),
                           "samples_ms": [round(v, 2) for v in samples], "byte_exact": exact,
                           "copy_engine_busy_ms": round(copy_busy, 2), "chunks": len(timeline),
                           "timeline_ms": timeline}
    # Copies, checks and placements alone (the records already pinned, as the reader leaves them).
    pinned = plane.pool.reserve(n * size)
    store.read_prepared_into(segments["child"], pinned.pointer, size, workers=16, verify="none")
    scrub()
    t0 = time.perf_counter()
    plane.load_scatter_verified(target, [(pinned, i * size) for i in range(n)], crcs)
    copy_alone_ms = (time.perf_counter() - t0) * 1e3
    # A sample of the restored blocks against the oracle's scatter of the blob files' payloads: each span of
    # the sampled target blocks is copied to the host by torch (raw storage bytes, any layout), and the oracle
    # gathers records from those host copies.
    sample = sorted(random.Random(5).sample(range(n), 64))
    rows = span_rows(torch, plane, [target[i] for i in sample])
    spans_host = [(row.ctypes.data, nbytes, offset, nbytes) for row, (offset, _, _, nbytes) in zip(rows, plane.spans())]
    got = oracle.gather(spans_host, list(range(len(sample))), size)
    expected = np.zeros((len(sample), size), dtype=np.uint8)
    for j, i in enumerate(sample):
        with open(store.path(segments["child"][i]["blob_id"]), "rb") as f:
            expected[j] = np.frombuffer(f.read()[32:], dtype=np.uint8)
    sample_exact = bool(np.array_equal(got, expected))
    pinned.close()
    io.close()
    import shutil
    shutil.rmtree(root, ignore_errors=True)
    plane.close()
    best = restores["workers_8"]
    return {"metric": "disk-staged restore with fork dedup, 32k-token Qwen3-8B", "workload": "disk-fork",
            "value": best["gbps"], "unit": "GB/s (blob files to KV blocks: pread by 8 native threads, one "
                                           "copy-engine transfer per 128 MiB chunk, every CRC32C checked on the GPU "
                                           "before placement, pipelined)",
            "restore_ms": best["ms"], "snapshot_bytes": n * size, "blocks": n,
            "blobs_on_disk": blobs, "child_blocks_shared_with_parent": shared_ids, "blobs_written": written,
            "crc32c_checked": n, "ids_and_crcs_match_oracle": digests_exact,
            "restored_equals_source_blocks": all(r["byte_exact"] for r in restores.values()),
            "sample_matches_oracle_scatter_of_blob_payloads": sample_exact, "sample_blocks": len(sample),
            "read_alone_ms": round(read_alone_ms, 2), "read_alone_gbps": round(n * size / read_alone_ms / 1e6, 2),
            "copy_check_place_alone_ms": round(copy_alone_ms, 2),
            "copy_check_place_alone_gbps": round(n * size / copy_alone_ms / 1e6, 2),
            "saves": phases, "restores": restores, "ring": {"slots": ring, "chunk_bytes": chunk},
            "page_cache": "warm (the blob files were just written)", "layout": args.layout,
            "reference": "114.5 ms read + CRC32C of 1.2 GB warm, then the H2D (results/restore-qwen3-8b.json:3358, 3611)"}


# ---------------------------------------------------------------- rotating fp8 sessions under decode load

def run_rotating(args, hashed=None):
    """Qwen3-1.7B fp8-e4m3 sessions of 1k/2k/4k/8k tokens saved and restored round-robin from a side thread
    beside a synthetic 16-sequence decode on the compute stream (reference results/resume-phases.json:351,
    396).  ``hashed`` (default: ``--digests``) has every save compute its CRC32C and SHA-256 on the GPU;
    the last round's are then checked against the oracle's digests of the records."""
    import torch
    hashed = args.digests if hashed is None else hashed
    from kvsnap_amd import synth
    from kvsnap_amd.dataplane import TorchBlockDataPlane, _check, kernel_library

    layers, num_blocks, block_size = 28, 16384, 16
    caches, backing = synth.make_caches(layers, num_blocks, block_size=block_size, layout="kv_split",
                                        dtype=torch.float8_e4m3fn)
    sessions_tokens = [1024, 2048, 4096, 8192]
    size = layers * 32768
    # Copies beside decode: direct saves on 4-workgroup grids and restores through the copy engines moved
    # 41 GB/s with a 0.17 ms p99 decode stall.  The restore kernel reading pinned memory in place holds CUs
    # through the link's latency and stalled the decode 0.85 ms at p99; staged saves (full-grid gathers)
    # moved only 14 GB/s beside it.
    plane = TorchBlockDataPlane(caches, block_size, sum(t // block_size for t in sessions_tokens) * size + (64 << 20),
                                save_mode=args.save_mode or "direct", restore_programs=args.programs or 4,
                                restore_mode=args.restore_mode or "dma",
                                gather_programs=args.gather_programs)
    plane.warm_up()
    scales_rng = random.Random(4)
    layer_inv = [scales_rng.uniform(0.5, 2.0) for _ in range(layers)]
    keep = synth.fill(plane, 0, kind=synth.KIND_E4M3, inv_scales=[layer_inv[s // 2] for s in range(2 * layers)])
    torch.cuda.synchronize()
    del keep
    rng = random.Random(1)
    free = list(range(1, num_blocks))
    rng.shuffle(free)
    sessions = []
    for t in sessions_tokens:
        count = t // block_size
        src, dst = free[:count], free[count:2 * count]
        del free[:2 * count]
        staged = plane.pool.reserve(count * size)
        sessions.append((t, src, dst, staged, [(staged, i * size) for i in range(count)]))
    # decode stand-in: 16 sequences x 4096 tokens (256 blocks) of random paged blocks, every layer's K and V
    lib = kernel_library()
    spans = plane.spans()
    bases = torch.tensor([s[1] for s in spans], dtype=torch.int64, device="cuda")
    pitches = torch.tensor([s[2] for s in spans], dtype=torch.int64, device="cuda")
    words = torch.tensor([s[3] // 8 for s in spans], dtype=torch.int64, device="cuda")
    seqs, per_seq = 16, 256
    table = torch.tensor([random.Random(100 + q).sample(range(1, num_blocks), per_seq) for q in range(seqs)],
                         dtype=torch.int64, device="cuda")
    out = torch.zeros(seqs * len(spans), dtype=torch.int32, device="cuda")
    compute = torch.cuda.current_stream()

    def decode_step():
        _check(lib, lib.kvsnap_synth_decode(bases.data_ptr(), pitches.data_ptr(), words.data_ptr(), len(spans),
                                            table.data_ptr(), seqs, per_seq, out.data_ptr(), 0, compute.cuda_stream))

    def run_steps(count=None, until=None, depth=32):
        pairs = []
        i = 0
        while (count is not None and i < count) or (until is not None and until()):
            if len(pairs) >= depth:
                pairs[-depth][1].synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(compute)
            decode_step()
            b.record(compute)
            pairs.append((a, b))
            i += 1
        torch.cuda.synchronize()
        return [a.elapsed_time(b) for a, b in pairs]

    run_steps(50)
    baseline = run_steps(400)
    base_med, base_p99 = statistics.median(baseline), percentile(baseline, 99)
    moved = [0]

    digests = []

    def rotate(rounds):
        for _ in range(rounds):
            for tokens, src, dst, staged, targets in sessions:
                plane.save_gather(src, targets, tokens, digests=digests if hashed else None)
                plane.load_scatter(dst, targets)
                moved[0] += 2 * len(src) * size
        for d in digests:
            d.result()

    t0 = time.perf_counter()
    rotate(1)                                           # copies alone
    alone_gbps = moved[0] / (time.perf_counter() - t0) / 1e9
    moved[0] = 0
    worker = threading.Thread(target=rotate, args=(args.rounds,))
    t0 = time.perf_counter()
    worker.start()
    loaded = run_steps(until=worker.is_alive)
    worker.join()
    elapsed = time.perf_counter() - t0
    exact = all(same_blocks(torch, caches, src, dst) for _, src, dst, _, _ in sessions)
    digests_exact = None
    if hashed:
        import oracle
        digests_exact = True
        for (tokens, src, _, staged, _), found in zip(sessions, digests[-len(sessions):]):
            crcs, shas = oracle.digest_records(staged.pointer, size, size, len(src), threads=host_threads()[2])
            digests_exact &= found.result() == [(bytes(h).hex(), int(c)) for h, c in zip(shas, crcs)]
    stalls = [max(0.0, t - base_med) for t in loaded]
    streams = plane.stream_report()
    for *_, staged, _ in sessions:
        staged.close()
    plane.close()
    step_bytes = seqs * per_seq * len(spans) * (size // len(spans))
    return {"metric": "rotating fp8 sessions under decode load, Qwen3-1.7B", "workload": "rotating-fp8",
            "value": round(moved[0] / elapsed / 1e9, 3), "unit": "GB/s (copy, beside decode)",
            "copy_alone_gbps": round(alone_gbps, 3), "rounds": args.rounds,
            "record_bytes": size, "sessions_tokens": sessions_tokens,
            "decode_step_ms": {"baseline_median": round(base_med, 4), "baseline_p99": round(base_p99, 4),
                               "loaded_median": round(statistics.median(loaded), 4),
                               "loaded_p99": round(percentile(loaded, 99), 4), "steps": len(loaded)},
            "decode_hbm_gbps_baseline": round(step_bytes / base_med / 1e6, 1),
            "p99_compute_stall_ms": round(percentile(stalls, 99), 4),
            "save_mode": plane.save_mode, "restore_programs": plane.restore_programs,
            "restore_mode": plane.restore_mode, "gather_programs": plane.gather_programs, "byte_exact": exact,
            "saves_hashed": bool(hashed), "digests_exact": digests_exact, "streams": streams,
            "note": "beside this decode (median / p99 stall): direct saves on 4 workgroups with copy-engine "
                    "restores 41 GB/s (+10 % / 0.17 ms), on 2-3 workgroups 30-36 GB/s (+9 % / 0.11 ms), on 6 "
                    "39 GB/s (0.71 ms); with the in-place restore kernel on 4 workgroups 29 GB/s (+21 % / 0.85 ms); "
                    "staged saves 14 GB/s"}


# ---------------------------------------------------------------- save and restore overlapped on the link

def run_duplex_process(args):
    """run_duplex in a child process (this same script, --workload duplex); its JSON line back.  Called before
    this process touches the GPU."""
    import subprocess
    command = [sys.executable, "-u", os.path.abspath(__file__), "--workload", "duplex", "--layout", args.layout]
    if args.restore_mode:
        command += ["--restore-mode", args.restore_mode]
    if args.save_mode:
        command += ["--save-mode", args.save_mode]
    if args.no_digests:
        command.append("--no-digests")
    done = subprocess.run(command, capture_output=True, text=True, timeout=600)
    lines = [line for line in done.stdout.splitlines() if line.startswith("{")]
    if done.returncode != 0 or not lines:
        raise RuntimeError(f"duplex child process failed ({done.returncode}): {done.stderr[-2000:]}")
    return json.loads(lines[-1])


def run_duplex(args):
    """The default workload's saves and restores from two host threads, as the connector's save threads and
    loader thread issue them: session k is restored while session k + 1 is saved.  Restores run on their own
    stream (restore_stream="split") through the copy engines (restore_mode="dma"), so a restore's
    host-to-device copies and a save's device-to-host copies use the two directions of the link at once.
    Two pinned staging buffers alternate between the sessions."""
    import torch
    from kvsnap_amd import synth
    from kvsnap_amd.dataplane import TorchBlockDataPlane

    layers, num_blocks, block_size, tokens = 36, 16384, 16, 8192
    session = tokens // block_size
    caches, backing = synth.make_caches(layers, num_blocks, block_size=block_size, layout=args.layout)
    plane = TorchBlockDataPlane(caches, block_size, 2 * session * layers * 65536 + (64 << 20),
                                restore_stream="split", restore_mode=args.restore_mode or "dma",
                                save_mode=args.save_mode)
    plane.warm_up()
    keep = synth.fill(plane, 0)
    torch.cuda.synchronize()
    del keep
    size = plane.block_bytes
    total = session * size
    source, target = synth.block_tables(num_blocks, session)
    buffers = [plane.pool.reserve(total) for _ in range(2)]
    targets = [[(b, i * size) for i in range(session)] for b in buffers]

    def run(steps):
        saved = [threading.Event() for _ in range(steps)]
        restored = [threading.Event() for _ in range(steps)]
        digests, errors = [], []

        def saver():
            try:
                for k in range(steps):
                    if k >= 2:
                        restored[k - 2].wait()          # its buffer is free again
                    plane.save_gather(source, targets[k % 2], tokens, digests=None if args.no_digests else digests)
                    saved[k].set()
            except BaseException as exc:
                errors.append(exc)
                for e in saved:
                    e.set()

        def loader():
            try:
                for k in range(steps):
                    saved[k].wait()
                    if errors:
                        return
                    plane.load_scatter(target, targets[k % 2])
                    restored[k].set()
            except BaseException as exc:
                errors.append(exc)
                for e in restored:
                    e.set()

        threads = [threading.Thread(target=saver), threading.Thread(target=loader)]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for t in threads:
            t.start()
        for t in threads:
            t.join()
        values = [d.result() for d in digests]
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        if errors:
            raise errors[0]
        return elapsed, values

    run(args.warmup)
    elapsed, values = run(args.steps)
    ms_per_step = elapsed * 1e3 / args.steps
    import oracle
    exact = same_blocks(torch, caches, source, target)
    last = buffers[(args.steps - 1) % 2]
    crcs, shas = oracle.digest_records(last.pointer, size, size, session, threads=min(16, os.cpu_count() or 1))
    digests_exact = None if args.no_digests else all(v == values[-1] for v in values) and all(
        crc == int(c) and sha == bytes(h).hex() for (sha, crc), c, h in zip(values[-1], crcs, shas))
    # After the timed runs (its streams would otherwise take hardware queues first): the link both ways
    # at once, one pinned->device and one device->pinned copy of the session's size.
    up_src = torch.empty(total, dtype=torch.uint8, pin_memory=True)
    down_dst = torch.empty(total, dtype=torch.uint8, pin_memory=True)
    dev_a = torch.empty(total, dtype=torch.uint8, device="cuda")
    dev_b = torch.empty(total, dtype=torch.uint8, device="cuda")
    s_up, s_down = torch.cuda.Stream(), torch.cuda.Stream()
    duplex = []
    for _ in range(3):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        with torch.cuda.stream(s_up):
            dev_a.copy_(up_src, non_blocking=True)
        with torch.cuda.stream(s_down):
            down_dst.copy_(dev_b, non_blocking=True)
        torch.cuda.synchronize()
        duplex.append(2 * total / (time.perf_counter() - t0) / 1e9)
    del up_src, down_dst, dev_a, dev_b
    log(f"both directions at once: {max(duplex):.1f} GB/s aggregate")

    streams = plane.stream_report()
    for b in buffers:
        b.close()
    plane.close()
    return {"metric": "8k Qwen3-8B KV restore/save GB/s, saves and restores overlapped", "workload": "duplex",
            "value": round(2 * total / (ms_per_step * 1e6), 3), "unit": "GB/s", "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms_per_step, 3), "snapshot_bytes": total,
            "duplex_link_gbps": round(max(duplex), 2), "layout": args.layout, "restore_mode": plane.restore_mode,
            "save_mode": plane.save_mode, "restore_stream_check": plane.restore_stream_check, "streams": streams,
            "parity": {"restore_byte_exact": exact, "digests_bit_exact": digests_exact},
            "note": "session k restored while session k + 1 is saved (two host threads, two pinned buffers); "
                    "each step still saves 1.208 GB with CRC32C + SHA-256 and restores 1.208 GB"}


# ---------------------------------------------------------------- kernels alone (profiling driver)

def run_kernels(args):
    """Each kernel of the default workload alone, HIP-event timed on its stream, plus a plain
    device-to-device copy of the same byte count (the reference point for rocprof's traffic counters),
    a plain read of the records (what the CRC32C kernel could take at this size) and a contiguous copy of
    them with the gather and scatter kernels' shape (what those could take)."""
    import torch
    from kvsnap_amd import synth
    from kvsnap_amd.dataplane import (_check, copy_host_blocks, digest_device_records, gather_blocks,
                                      gather_crc32c_launcher, kernel_library, scatter_blocks, TorchBlockDataPlane)

    layers, num_blocks, block_size, tokens = 36, 16384, 16, 8192
    session = tokens // block_size
    caches, backing = synth.make_caches(layers, num_blocks, block_size=block_size, heads=args.kv_heads,
                                        layout=args.layout)
    plane = TorchBlockDataPlane(caches, block_size, session * layers * 8192 * args.kv_heads + (64 << 20))
    plane.warm_up()
    keep = synth.fill(plane, 0)
    torch.cuda.synchronize()
    del keep
    size = plane.block_bytes
    total = session * size
    source, target = synth.block_tables(num_blocks, session)
    tables = plane._load_tables()
    stream = torch.cuda.current_stream()
    # With --rotate N the HBM kernels cycle over N sets of blocks and buffers, so that no launch finds the bytes
    # of the launch before it in the last-level cache (a TP = 8 shard's 151 MB would otherwise stay there).
    rot = max(1, args.rotate)
    used = set(source) | set(target)
    spare = [b for b in range(num_blocks) if b not in used]
    extra = random.Random(11).sample(spare, 2 * (rot - 1) * session) if rot > 1 else []
    sources = [source] + [extra[2 * k * session:(2 * k + 1) * session] for k in range(rot - 1)]
    targets_ = [target] + [extra[(2 * k + 1) * session:(2 * k + 2) * session] for k in range(rot - 1)]
    id_sets = [torch.tensor(x, dtype=torch.int64, device="cuda") for x in sources]
    dst_sets = [torch.tensor(x, dtype=torch.int64, device="cuda") for x in targets_]
    stages = [torch.empty(total, dtype=torch.uint8, device="cuda") for _ in range(rot)]
    others = [torch.empty(total, dtype=torch.uint8, device="cuda") for _ in range(rot)]
    ids, stage, dst = id_sets[0], stages[0], dst_sets[0]
    staged = plane.pool.reserve(total)
    pinned = torch.tensor([staged.pointer + i * size for i in range(session)], dtype=torch.int64, device="cuda")
    lib = kernel_library()
    crc = torch.empty(session, dtype=torch.int32, device="cuda")
    work_bytes = int(lib.kvsnap_crc32c_workspace_bytes(size, session))
    work = torch.empty(work_bytes, dtype=torch.uint8, device="cuda")
    sha = torch.empty((session, 32), dtype=torch.uint8, device="cuda")
    hint = plane.min_span_bytes
    records_at = [torch.tensor([st.data_ptr() + i * size for i in range(session)], dtype=torch.int64, device="cuda")
                  for st in stages]
    partial = torch.empty(session * tables[0].numel(), dtype=torch.int32, device="cuda")
    sink = torch.zeros(4096, dtype=torch.int32, device="cuda")

    def cycling(launch):
        """launch(k) on set 0, 1, ..., rot - 1, 0, ... in turn, and launch itself for set k."""
        turn = [0]

        def next_set():
            k, turn[0] = turn[0], (turn[0] + 1) % rot
            return launch(k)
        next_set.on = launch
        return next_set

    def gather_checked(k):
        _check(lib, lib.kvsnap_gather_blocks_checked(
            records_at[k].data_ptr(), id_sets[k].data_ptr(), session, *(t.data_ptr() for t in tables),
            tables[0].numel(), None, 0, 0, partial.data_ptr(), stream.cuda_stream))
        _check(lib, lib.kvsnap_restore_checked_crc32c(partial.data_ptr(), session, tables[0].data_ptr(),
                                                      tables[3].data_ptr(), tables[0].numel(), size, crc.data_ptr(),
                                                      stream.cuda_stream))

    runs = {
        "plain_copy": (cycling(lambda k: others[k].copy_(stages[k])), 2 * total, args.reps),
        # The same bytes read and nothing else done with them (kvsnap_read_probe, the CRC32C kernels' 1024-lane
        # workgroups, one a CU): what a read of this size can take, the CRC32C kernel's own ceiling.
        "plain_read": (cycling(lambda k: _check(lib, lib.kvsnap_read_probe(
            stages[k].data_ptr(), total, sink.data_ptr(), stream.cuda_stream))), total, args.reps),
        # The records copied contiguously with the gather and scatter kernels' shape (kvsnap_copy_probe: one
        # 64-lane workgroup a KiB, nothing scattered): their own ceiling at this size.
        "streaming_copy": (cycling(lambda k: _check(lib, lib.kvsnap_copy_probe(
            stages[k].data_ptr(), others[k].data_ptr(), total, stream.cuda_stream))), 2 * total, args.reps),
        "gather_pieces_kernel": (cycling(lambda k: gather_blocks(id_sets[k], *tables, stages[k].data_ptr(), size,
                                                                 min_span_bytes=hint)), 2 * total, args.reps),
        # 512 records take the one-launch plan (crc_records_kernel: stripes combined in the workgroup).
        "crc_records_kernel": (cycling(lambda k: _check(lib, lib.kvsnap_crc32c_records(
            stages[k].data_ptr(), size, size, session, 0, crc.data_ptr(), work.data_ptr(), work_bytes,
            stream.cuda_stream))), total, args.reps),
        "restore_kernel": (lambda: copy_host_blocks(pinned, dst, *tables, min_span_bytes=hint), 2 * total,
                           args.reps),
        # The copy-engine restore's scatter: records in device staging, one wave per KiB of a span.
        "scatter_pieces_kernel": (cycling(lambda k: scatter_blocks(stages[k].data_ptr(), size, dst_sets[k], *tables,
                                                                   min_span_bytes=hint)), 2 * total, args.reps),
        "sha256_kernel": (lambda: _check(lib, lib.kvsnap_sha256_records(
            stage.data_ptr(), size, size, session, sha.data_ptr(), stream.cuda_stream)), total, 1),
        # The gather with every record's CRC32C folded in, into device records on a full grid, and its finish
        # (the save's record bytes and CRC32Cs from one read of the cache): read + write, like the gather.
        "gather_checked_kernel": (cycling(gather_checked), 2 * total, args.reps),
        # Its finish alone (every record's CRC32C from its spans' partials): a few microseconds, not HBM-bound.
        "restore_checked_finish_kernel": (lambda: _check(lib, lib.kvsnap_restore_checked_crc32c(
            partial.data_ptr(), session, tables[0].data_ptr(), tables[3].data_ptr(), tables[0].numel(), size,
            crc.data_ptr(), stream.cuda_stream)), 4 * session * tables[0].numel(), args.reps),
    }
    # The gather with CRC32C into device records (whole-KiB spans): the CRC32C kernel's stripes and tables with
    # its loads from the cache and its words written to the records, one launch; read + write, like the gather.
    groups = plane.group_tables()
    if groups is not None:
        fused = [torch.empty(total, dtype=torch.uint8, device="cuda") for _ in range(rot)]
        fused_crc = torch.empty(session, dtype=torch.int32, device="cuda")
        launches = [gather_crc32c_launcher(id_sets[k], *groups, size, fused[k].data_ptr(), size, fused_crc)
                    for k in range(rot)]
        runs["gather_crc_kernel"] = (cycling(lambda k: launches[k]()), 2 * total, args.reps)
    out = {}
    for name, (fn, algorithmic, reps) in runs.items():
        for _ in range(rot):
            fn()
        ms = median_ms(torch, stream, fn, reps=reps, batch=1 if name == "sha256_kernel" else 4 * rot)
        out[name] = {"ms": round(ms, 4), "algorithmic_bytes": algorithmic,
                     "gbps": round(algorithmic / ms / 1e6, 1)}
    out["crc_records_kernel"]["of_plain_read"] = round(out["plain_read"]["ms"] / out["crc_records_kernel"]["ms"], 3)
    for name in ("gather_pieces_kernel", "scatter_pieces_kernel"):
        out[name]["of_streaming_copy"] = round(out["streaming_copy"]["ms"] / out[name]["ms"], 3)
    out["sha256_kernel"]["issue_roofline"] = sha_issue_bound(size, session, out["sha256_kernel"]["ms"],
                                                          sha_round_rate(torch))
    # The checked gather's CRC32Cs against the CRC kernel's over the same records (set 0's).
    runs["gather_pieces_kernel"][0].on(0)
    runs["crc_records_kernel"][0].on(0)
    want = crc.clone()
    gather_checked(0)
    torch.cuda.synchronize()
    out["gather_checked_kernel"]["crc32c_equal_crc_kernel"] = bool(torch.equal(want, crc))
    if groups is not None:     # its records against the gather kernel's, its CRC32Cs against the CRC kernel's
        launches[0]()
        torch.cuda.synchronize()
        out["gather_crc_kernel"]["records_equal_gather"] = bool(torch.equal(fused[0], stage))
        out["gather_crc_kernel"]["crc32c_equal_crc_kernel"] = bool(torch.equal(want, fused_crc))
    staged.close()
    plane.close()
    return {"workload": "kernels", "snapshot_bytes": total, "layout": args.layout, "kv_heads": args.kv_heads,
            "rotate": rot,
            "span_bytes": sorted({s[3] for s in plane.spans()}), "kernels": out,
            "note": "restore_kernel reads pinned host records (link) and writes HBM; bytes counted both ways"}


# ---------------------------------------------------------------- the reference's CPU round trip

def run_cpu_roundtrip(args):
    import numpy as np
    import torch
    import oracle
    from kvsnap_amd import synth
    from kvsnap_amd.dataplane import TorchBlockDataPlane

    layers, num_blocks, block_size, tokens = 28, 4096, 16, 2048
    session = tokens // block_size
    caches, backing = synth.make_caches(layers, num_blocks, block_size=block_size, layout=args.layout)
    plane = TorchBlockDataPlane(caches, block_size, session * layers * 65536 + (64 << 20))
    plane.warm_up()
    keep = synth.fill(plane, 0)
    torch.cuda.synchronize()
    del keep
    size = plane.block_bytes
    total = session * size
    source, target = synth.block_tables(num_blocks, session)

    # CPU leg: a host cache of the same geometry; the source blocks hold the bytes the GPU cache holds (the
    # oracle's generator is the GPU's, bit for bit).
    oracle.build()
    lib = oracle.lib()
    host = np.zeros(backing.numel() * backing.element_size(), dtype=np.uint8)
    base = backing.data_ptr()
    spans = plane.spans()
    for s, (_, span_base, pitch, nbytes) in enumerate(spans):
        start = span_base - base
        for b in source:
            host[start + b * pitch:start + b * pitch + nbytes] = oracle.fill_span(0, s, b, nbytes)
    span_base = np.array([host.ctypes.data + (sp[1] - base) for sp in spans], dtype=np.uint64)
    span_pitch = np.array([sp[2] for sp in spans], dtype=np.int64)
    span_off = np.array([sp[0] for sp in spans], dtype=np.int64)
    span_len = np.array([sp[3] for sp in spans], dtype=np.int64)
    src_ids, dst_ids = np.array(source, dtype=np.int64), np.array(target, dtype=np.int64)
    records = np.zeros(total, dtype=np.uint8)
    crcs = np.zeros(session, dtype=np.uint32)
    addresses = np.array([records.ctypes.data + i * size for i in range(session)], dtype=np.uint64)

    def cpu_round_trip(threads):
        lib.oracle_copy_threads(len(spans), span_base.ctypes.data, span_pitch.ctypes.data, span_off.ctypes.data,
                                span_len.ctypes.data, src_ids.ctypes.data, None, session, records.ctypes.data,
                                size, threads)
        lib.oracle_digest_records(records.ctypes.data, size, size, session, crcs.ctypes.data, None, threads)
        lib.oracle_copy_threads(len(spans), span_base.ctypes.data, span_pitch.ctypes.data, span_off.ctypes.data,
                                span_len.ctypes.data, dst_ids.ctypes.data, addresses.ctypes.data, session, None,
                                size, threads)

    cpu_round_trip(1)                                   # first touch of the target pages, untimed
    threads_max = max(1, min(16, os.cpu_count() or 1))
    cpu = {}
    for threads in sorted({1, threads_max}):
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            cpu_round_trip(threads)
            times.append(time.perf_counter() - t0)
        cpu[threads] = min(times)
    cpu_exact = np.array_equal(oracle.gather([(int(span_base[i]), int(span_pitch[i]), int(span_off[i]),
                                               int(span_len[i])) for i in range(len(spans))], target, size),
                               records.reshape(session, size))

    # GPU leg: save into pinned records, then a verified restore that must match the CPU's CRC32Cs.
    staged = plane.pool.reserve(total)
    targets = [(staged, i * size) for i in range(session)]
    expected = [int(c) for c in crcs]
    gpu = []
    for _ in range(4):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        plane.save_gather(source, targets, tokens)
        plane.load_scatter_verified(target, targets, expected)
        torch.cuda.synchronize()
        gpu.append(time.perf_counter() - t0)
    gpu_ms = statistics.median(gpu[1:]) * 1e3
    records_equal = np.array_equal(np.frombuffer(ctypes.string_at(staged.pointer, total), dtype=np.uint8), records)
    exact = same_blocks(torch, caches, source, target)
    staged.close()
    plane.close()
    return {"metric": "CPU reference round trip at the Qwen3-1.7B shape (gather, CRC32C, scatter, compare)",
            "workload": "cpu-roundtrip", "value": round(2 * total / (gpu_ms * 1e6), 2),
            "unit": "GB/s (GPU: save + CRC-verified restore, save and restore bytes)", "record_bytes": size,
            "session_blocks": session, "gpu_ms": round(gpu_ms, 2),
            "cpu_baseline": {"value": round(2 * total / cpu[threads_max] / 1e9, 3), "unit": "GB/s",
                             "cores": threads_max, "kind": "port",
                             "single_thread_gbps": round(2 * total / cpu[1] / 1e9, 3),
                             "ms": {str(t): round(v * 1e3, 2) for t, v in cpu.items()},
                             "sample": f"the whole case: {session} blocks x {size} B gathered, CRC32C'd and "
                                       "scattered into a fresh table, best of 3"},
            # load_scatter_verified raises before any KV write unless every GPU CRC32C equals the CPU's.
            "parity": {"cpu_round_trip_exact": bool(cpu_exact), "gpu_records_equal_cpu_records": bool(records_equal),
                       "gpu_crc32c_equal_cpu": True, "gpu_restore_exact": exact},
            "layout": args.layout}


# ---------------------------------------------------------------- turn-2 time to first forward through the worker hooks

def run_ttft(args):
    """Turn 2 of a session restored through the worker hooks while an engine steps (the data plane's part
    of the reference's bench/restore_ttft.py).

    An 8k-token Qwen3-8B session is saved at turn end through ``KvsnapWorker`` into the host tier and as
    blob files.  Then, each repetition, the engine steps a 16-sequence synthetic decode of 8k-token
    contexts (19 GB of KV reads a step, synchronised every step as sampling does); the request arrives,
    its load starts after that step's forward, and it runs in the first forward after the worker reports
    it.  Time to first forward: from the arrival to the end of that forward, which reads every restored
    block and must fold them to the checksums the saved blocks gave.  With early report the request is
    reported once at most 128 MiB of its copy is left and the forward waits on the GPU for the rest; the
    reference's TTFT also holds the gateway, lease and model prefill, which are not here.
    """
    import torch
    from kvsnap_amd import synth
    from kvsnap_amd.blobs import BlobDirectory
    from kvsnap_amd.dataplane import TorchBlockDataPlane, _check, kernel_library
    from kvsnap_amd.host_tier import HostTier
    from kvsnap_amd.ordering import EARLY_REPORT_BYTES
    from kvsnap_amd.worker import KvsnapMetadata, KvsnapWorker, Transfer

    layers, num_blocks, block_size, tokens, seqs = 36, 16384, 16, 8192, 16
    session = tokens // block_size
    caches, backing = synth.make_caches(layers, num_blocks, block_size=block_size, layout=args.layout)
    record = layers * 65536
    plane = TorchBlockDataPlane(caches, block_size, 2 * session * record + (1 << 30))
    plane.warm_up()
    keep = synth.fill(plane, 0)
    torch.cuda.synchronize()
    del keep
    size, total = plane.block_bytes, session * plane.block_bytes
    source, target = synth.block_tables(num_blocks, session)
    taken = set(source) | set(target)
    background = random.Random(3).sample([b for b in range(1, num_blocks) if b not in taken], seqs * session)
    tables = plane._load_tables()
    n_spans = tables[0].numel()
    lib = kernel_library()
    stream = torch.cuda.current_stream()

    def forward(table, n_seqs, out):
        _check(lib, lib.kvsnap_synth_decode(tables[1].data_ptr(), tables[2].data_ptr(), tables[3].data_ptr(), n_spans,
                                            table.data_ptr(), n_seqs, session, out.data_ptr(), 0, stream.cuda_stream))

    batch = torch.tensor(background, dtype=torch.int64, device="cuda")
    batch_out = torch.empty(seqs * n_spans, dtype=torch.int32, device="cuda")
    src_table = torch.tensor(source, dtype=torch.int64, device="cuda")
    dst_table = torch.tensor(target, dtype=torch.int64, device="cuda")
    expected = torch.empty(n_spans, dtype=torch.int32, device="cuda")
    got = torch.empty(n_spans, dtype=torch.int32, device="cuda")
    forward(src_table, 1, expected)
    step_ms = []
    for _ in range(5):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        forward(batch, seqs, batch_out)
        end.record()
        end.synchronize()
        step_ms.append(start.elapsed_time(end))

    root = args.disk_dir or tempfile.mkdtemp(prefix="kvsnap-ttft-")
    tier = HostTier(plane, 2 * total)
    worker = KvsnapWorker(plane, host_tier=tier, blobs=BlobDirectory(root))

    def until(condition, seconds=60, finished=()):
        deadline = time.perf_counter() + seconds
        while not condition():
            if time.perf_counter() > deadline:
                raise RuntimeError("the worker did not report in time")
            worker.bind_connector_metadata(KvsnapMetadata())
            worker.get_finished(set(finished))
            worker.clear_connector_metadata()
            time.sleep(1e-4)

    # Turn end: both saves handed off after the step's kernels, fenced, hashed on the GPU, kept.
    worker.bind_connector_metadata(KvsnapMetadata(saves=[
        Transfer("host", source, durability="volatile", num_kv_tokens=tokens),
        Transfer("disk", source, durability="durable", num_kv_tokens=tokens)]))
    worker.wait_for_save()
    saved = {}
    until(lambda: not worker._saves, finished={"host", "disk"})    # fenced, reported, and booked
    meta = worker.build_connector_worker_meta()
    if meta.errors:
        raise RuntimeError(f"turn-end saves failed: {meta.errors}")
    saved.update(meta.prepared)

    # (snapshot, durability, check, early report, how the plane's restores cross the link)
    arms = [("host", "volatile", "none", True, "kernel"), ("host", "volatile", "none", False, "kernel"),
            ("host", "volatile", "none", True, "dma"), ("host", "volatile", "gpu", True, "kernel"),
            ("host", "volatile", "gpu", True, "dma"), ("disk", "durable", "gpu", True, "kernel")]
    results, exact = {}, True
    for name, durability, verify, early, mode in arms:
        worker.verify = verify
        worker.early_report_bytes = EARLY_REPORT_BYTES if early else -1
        plane.restore_mode = mode
        times, steps, step_times = [], [], []
        for rep in range(args.reps + 1):               # the first repetition warms the arm up
            if args.layout == "kv_split":              # [layers, 2, blocks, ...]
                backing[:, :, dst_table] = 0
            else:                                      # [layers, blocks, ...]
                backing[:, dst_table] = 0
            torch.cuda.synchronize()
            arrival = time.perf_counter()
            runnable, step, marks = False, 0, [arrival]
            while True:
                loads = [Transfer("r", target, snapshot=saved[name], durability=durability)] if step == 0 else []
                worker.bind_connector_metadata(KvsnapMetadata(loads=loads))
                forward(batch, seqs, batch_out)
                if runnable:
                    forward(dst_table, 1, got)
                    torch.cuda.current_stream().synchronize()
                    elapsed = (time.perf_counter() - arrival) * 1e3
                    break
                if loads:
                    worker.start_load_kv(None)         # async loads start after the forward
                torch.cuda.current_stream().synchronize()
                marks.append(time.perf_counter())
                runnable = "r" in worker.get_finished(set())[1]
                step += 1
            until(lambda: not worker._loads)
            loaded = worker.build_connector_worker_meta()
            exact = exact and loaded.failed_loads == [] and torch.equal(got, expected)
            if rep:
                times.append(elapsed)
                steps.append(step)
                step_times.extend((b - a) * 1e3 for a, b in zip(marks, marks[1:]))
        results[f"{name}-verify-{verify}-{'early' if early else 'at-completion'}-{mode}"] = {
            "median_ms": round(statistics.median(times), 2), "min_ms": round(min(times), 2),
            "max_ms": round(max(times), 2), "steps_before_forward": statistics.median(steps),
            "engine_step_ms_while_loading": round(statistics.median(step_times), 2)}
        log(list(results)[-1], results[list(results)[-1]])
    worker.shutdown()
    tier_stats = tier.stats()
    plane.close()
    if not args.disk_dir:
        import shutil
        shutil.rmtree(root, ignore_errors=True)
    best = results["host-verify-none-early-kernel"]
    return {"metric": "turn-2 time to first forward of an 8k-token Qwen3-8B session restored through the worker "
                      "hooks beside a 16-sequence decode (data-plane part of TTFT)",
            "workload": "ttft", "value": best["median_ms"], "unit": "ms", "higher_is_better": False,
            "arms": results, "engine_step_ms": round(statistics.median(step_ms), 3), "snapshot_bytes": total,
            "reps": args.reps, "host_tier": tier_stats, "forward_reads_restored_bytes_exact": exact,
            "note": "arrival -> end of the first forward that reads the restored blocks; early = reported once "
                    "<= 128 MiB is left, the forward waiting on the GPU for the rest; kernel = the restore kernel "
                    "reads pinned memory in place (CUs beside the decode), dma = the copy engines stage each chunk "
                    "and the scatter kernel places it; verify gpu = every block's CRC32C checked on the GPU: host-tier "
                    "blocks by the checked restore kernel as it copies them from pinned memory (kernel) or places "
                    "each staged chunk (dma), the load reported once the check has passed; "
                    "disk blocks in device staging before any KV write"}


# ---------------------------------------------------------------- multi-turn host-tier saves

def run_turns(args):
    import torch
    from kvsnap_amd import synth
    from kvsnap_amd.dataplane import TorchBlockDataPlane
    from kvsnap_amd.blobs import BlobDirectory
    from kvsnap_amd.host_tier import HostTier

    layers, num_blocks, block_size = 36, 16384, 16
    start_tokens, turn_tokens, turns = 8192, 512, args.turns
    final = (start_tokens + turns * turn_tokens) // block_size
    caches, backing = synth.make_caches(layers, num_blocks, block_size=block_size, layout=args.layout)
    size = layers * 65536
    # Both tiers hold one snapshot, and a save reserves its fresh blocks before adopting them.
    plane = TorchBlockDataPlane(caches, block_size, 4 * final * size + (64 << 20))
    plane.warm_up()
    keep = synth.fill(plane, 0)
    torch.cuda.synchronize()
    del keep
    ids = random.Random(1).sample(range(1, num_blocks), final)
    full, delta = HostTier(plane, 2 * final * size), HostTier(plane, 2 * final * size)
    root = tempfile.mkdtemp(prefix="kvsnap-turns-", dir=args.disk_dir)
    disk = BlobDirectory(root)
    prev_full = prev_delta = prev_disk = None
    rows = []
    for turn in range(turns + 1):
        tokens = start_tokens + turn * turn_tokens
        count = tokens // block_size
        if turn:
            # The turn's new tokens: fresh content in its new blocks.
            first = (tokens - turn_tokens) // block_size
            keep = [synth.fill(plane, 1000 + turn, first_block=b, num_blocks=1) for b in ids[first:count]]
            torch.cuda.synchronize()
            del keep
        fence_full, fence_delta = Stamp(), Stamp()
        t0 = time.perf_counter()
        snap_full = full.save(ids[:count], tokens, fenced=fence_full)
        t1 = time.perf_counter()
        snap_delta = delta.save(ids[:count], tokens, previous=prev_delta, fenced=fence_delta)
        t2 = time.perf_counter()
        fence_disk = Stamp()
        t3 = time.perf_counter()
        snap_disk = disk.save(plane, ids[:count], tokens, previous=prev_disk, fenced=fence_disk)
        t4 = time.perf_counter()
        if not snap_full["segments"] == snap_delta["segments"] == snap_disk["segments"]:
            raise RuntimeError(f"turn {turn}: the delta saves' segments differ from the full save's")
        rows.append(dict(turn=turn, tokens=tokens, blocks=count,
                         full_fenced_ms=round((fence_full.at - t0) * 1e3, 2), full_ms=round((t1 - t0) * 1e3, 2),
                         full_gathered=full.gathered_blocks,
                         delta_fenced_ms=round((fence_delta.at - t1) * 1e3, 2), delta_ms=round((t2 - t1) * 1e3, 2),
                         delta_gathered=delta.gathered_blocks,
                         disk_fenced_ms=round((fence_disk.at - t3) * 1e3, 2), disk_ms=round((t4 - t3) * 1e3, 2),
                         disk_written=disk.written))
        log(f"turn {turn}: {tokens} tokens; full: fenced {rows[-1]['full_fenced_ms']} ms, adopted "
            f"{rows[-1]['full_ms']} ms; delta ({delta.gathered_blocks} blocks): fenced "
            f"{rows[-1]['delta_fenced_ms']} ms, adopted {rows[-1]['delta_ms']} ms")
        for tier, previous in ((full, prev_full), (delta, prev_delta)):
            if previous is not None:
                tier.release(previous)
        prev_full, prev_delta, prev_disk = snap_full, snap_delta, snap_disk
    cpu = None if args.no_cpu_baseline else turn_cpu_baseline(full, prev_full, size)
    later = rows[1:]
    median = lambda key: statistics.median(r[key] for r in later)
    for tier, previous in ((full, prev_full), (delta, prev_delta)):
        tier.release(previous)
    plane.close()
    import shutil
    shutil.rmtree(root, ignore_errors=True)
    return {"metric": "turn-end host-tier save of a growing Qwen3-8B session: ms until the GPU blocks are free "
                      "(D2H fenced), delta save",
            "workload": "turns", "value": median("delta_fenced_ms"), "unit": "ms", "higher_is_better": False,
            "full_fenced_ms": median("full_fenced_ms"), "delta_adopted_ms": median("delta_ms"),
            "full_adopted_ms": median("full_ms"), "disk_delta_fenced_ms": median("disk_fenced_ms"),
            "disk_delta_written_ms": median("disk_ms"),
            "fence_speedup": round(median("full_fenced_ms") / median("delta_fenced_ms"), 2),
            "note": "adopted = digests computed on the GPU and the blocks held by content id; a record's "
                    "SHA-256 is one sequential chain, so both saves' adoption waits about one record's hash",
            "record_bytes": size, "start_tokens": start_tokens, "tokens_per_turn": turn_tokens, "turns": rows,
            "segments_equal": True, "layout": args.layout, "cpu_baseline": cpu}


class Stamp:
    """A ``fenced`` event that records when it was set."""
    at = None

    def set(self):
        self.at = time.perf_counter()


def turn_cpu_baseline(tier, snapshot, size):
    """The reference's turn-end rehash (volatile.py:226-229): SHA-256 + CRC32C of every block, 8 threads.

    Timed by the oracle on this host's cores over the last turn's held
    blocks, in place in pinned memory.
    """
    from concurrent.futures import ThreadPoolExecutor
    import oracle
    oracle.build()
    oracle.sha256_select(True)
    pointers = [tier._entries[s["blob_id"]]["allocation"].pointer for s in snapshot["segments"]]
    with ThreadPoolExecutor(max_workers=8) as pool:
        t0 = time.perf_counter()
        list(pool.map(lambda p: oracle.digest_records(p, size, size, 1, threads=1), pointers))
        elapsed = time.perf_counter() - t0
    return {"value": round(elapsed * 1e3, 2), "unit": "ms", "cores": 8, "kind": "port",
            "gbps": round(len(pointers) * size / elapsed / 1e9, 2),
            "sample": f"the last turn's {len(pointers)} held blocks x {size} B, SHA-256 + CRC32C each"}


def main():
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    # 40 steps: the timed region ends when the last save's SHA-256 is done, about 14 ms after its restore,
    # a tail that 10 steps would spread as 1.4 ms over each.
    parser.add_argument("--steps", type=int, default=40)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--layout", choices=("kv_split", "vllm"), default="kv_split")
    parser.add_argument("--workload", choices=("save-restore", "disk-fork", "rotating-fp8", "turns", "cpu-roundtrip",
                                               "kernels", "duplex", "ttft"), default="save-restore")
    parser.add_argument("--reps", type=int, default=5, help="kernels, ttft: timed repetitions per kernel / arm")
    parser.add_argument("--rotate", type=int, default=1,
                        help="kernels: HBM kernels cycle over this many block sets and buffers (no cache reuse)")
    parser.add_argument("--kv-heads", type=int, default=8, choices=(1, 2, 4, 8),
                        help="kernels: KV heads in the cache, 8 / TP for one tensor-parallel rank's shard")
    parser.add_argument("--hash-depth", type=int, default=2,
                        help="save-restore: steps a save's digests may trail before they are collected")
    parser.add_argument("--rounds", type=int, default=4, help="rotating-fp8: rounds over the four sessions")
    parser.add_argument("--turns", type=int, default=6, help="turns: turns after the first save")
    parser.add_argument("--save-mode", choices=("staged", "direct"), default=None,
                        help="rotating-fp8, duplex: save mode of the plane (rotating-fp8 default direct, duplex staged)")
    parser.add_argument("--programs", type=int, default=None,
                        help="rotating-fp8: restore / direct-save workgroups (default 4)")
    parser.add_argument("--gather-programs", type=int, default=None,
                        help="rotating-fp8: workgroups of the plane's gather and scatter grids (default 0: one per job)")
    parser.add_argument("--digests", action="store_true",
                        help="rotating-fp8: every save also computes its CRC32C and SHA-256 on the GPU")
    parser.add_argument("--no-digests", action="store_true",
                        help="duplex: saves without GPU CRC32C / SHA-256 (the link alone)")
    parser.add_argument("--restore-mode", choices=("kernel", "dma"), default=None,
                        help="save-restore, duplex, rotating-fp8: how restores cross the link")
    parser.add_argument("--disk-dir", default=None, help="disk-fork, turns, ttft: where the blob files go")
    parser.add_argument("--cpu-seconds", type=float, default=0.6,
                        help="save-restore: seconds per leg and thread count of the CPU baseline")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-rotating", action="store_true",
                        help="save-restore: leave out the rotating fp8 sessions beside a decode")
    parser.add_argument("--no-disk-fork", action="store_true",
                        help="save-restore: leave out the disk-staged restore with fork dedup (2048 blocks)")
    parser.add_argument("--no-duplex", action="store_true",
                        help="save-restore: leave out the saves and restores overlapped from two threads")
    args = parser.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: every GPU saves and restores its own KV shard over its own host link, "
              "so there is no multi-GPU step to time here (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    # The default workload's duplex field runs first, in a child process, while this one has not touched the GPU.
    args.duplex_result = (run_duplex_process(args)
                          if args.workload == "save-restore" and not args.no_duplex else None)
    import torch
    torch.cuda.set_device(0)
    runner = {"save-restore": run_save_restore, "disk-fork": run_disk_fork, "rotating-fp8": run_rotating,
              "turns": run_turns, "cpu-roundtrip": run_cpu_roundtrip, "kernels": run_kernels, "duplex": run_duplex,
              "ttft": run_ttft}
    print(json.dumps(runner[args.workload](args)), flush=True)


if __name__ == "__main__":
    main()
