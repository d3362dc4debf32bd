#!/usr/bin/env python
"""KV snapshot save + restore on one MI355X: an 8192-token Qwen3-8B session.

Workload (one step): save a 512-block session out of a 16384-block paged
cache (36 layers x {K,V}, 8 KV heads, head_dim 128, block_size 16, bf16
~N(0,1) from seed 0, block ids seeded) -- GPU gather, DMA into pinned host
memory, per-block CRC32C and SHA-256 on the GPU -- then restore it from the
pinned records into a fresh seeded block table with the restore kernel.
1,207,959,552 bytes each way.

    python bench.py [--steps K] [--warmup W] [--layout kv_split|vllm]

Prints one JSON line.  ``value`` is the step's snapshot throughput (save
bytes + restore bytes) / (time per step), with the cache resident in HBM.
Also reported: save and restore latency and GB/s, the measured contiguous
pinned<->device DMA peaks and the fractions of them reached, per-kernel HIP
event durations, the rooflines, and the CPU path on the host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

LAYERS, NUM_BLOCKS, BLOCK_SIZE, HEADS, HEAD_DIM = 36, 16384, 16, 8, 128
TOKENS = 8192
SESSION_BLOCKS = TOKENS // BLOCK_SIZE
HBM_PEAK_GBPS = 8000.0
EARLY_REPORT_BYTES = 128 << 20


def log(*args):
    print(*args, file=sys.stderr, flush=True)


def median_ms(torch, stream, fn, reps=5):
    times = []
    for _ in range(reps):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        fn()
        end.record(stream)
        end.synchronize()
        times.append(start.elapsed_time(end))
    return statistics.median(times)


def cpu_baseline(seconds_budget=20.0):
    """The reference's CPU path restated by the oracle, on this host's cores.

    Per sample block: gather its 36 spans into a packed record (memcpy),
    CRC32C (SSE4.2) and SHA-256 (SHA extensions) of the record, and scatter it
    back into other blocks (memcpy) -- on 1 thread and on min(16, nproc)
    threads.  Sample: 64 blocks of a 256-block host cache, repeated until
    about ``seconds_budget`` seconds have passed.
    """
    import numpy as np
    import oracle
    oracle.build()
    oracle.sha256_select(True)
    lib = oracle.lib()
    span = HEADS * 2 * HEAD_DIM * BLOCK_SIZE * 2       # 65536 bytes per (layer, block)
    host_blocks, sample = 256, 64
    record = LAYERS * span
    cache = np.frombuffer(np.random.default_rng(0).bytes(LAYERS * host_blocks * span), dtype=np.uint8).copy()
    base = cache.ctypes.data
    span_base = np.array([base + l * host_blocks * span for l in range(LAYERS)], dtype=np.uint64)
    span_pitch = np.full(LAYERS, span, dtype=np.int64)
    span_off = np.array([l * span for l in range(LAYERS)], dtype=np.int64)
    span_len = np.full(LAYERS, span, dtype=np.int64)
    import random
    ids = np.array(random.Random(1).sample(range(1, host_blocks), sample), dtype=np.int64)
    dst = np.array(random.Random(2).sample([b for b in range(1, host_blocks) if b not in set(ids.tolist())], sample),
                   dtype=np.int64)
    records = np.zeros(sample * record, dtype=np.uint8)
    crcs = np.zeros(sample, dtype=np.uint32)
    shas = np.zeros((sample, 32), dtype=np.uint8)
    sources = np.array([records.ctypes.data + i * record for i in range(sample)], dtype=np.uint64)
    threads_max = max(1, min(16, os.cpu_count() or 1))
    result = {}
    for threads in sorted({1, threads_max}):
        reps, elapsed = 0, 0.0
        deadline = seconds_budget / 2
        while elapsed < deadline or reps == 0:
            t0 = time.perf_counter()
            lib.oracle_copy_threads(LAYERS, span_base.ctypes.data, span_pitch.ctypes.data, span_off.ctypes.data,
                                    span_len.ctypes.data, ids.ctypes.data, None, sample, records.ctypes.data, record,
                                    threads)
            lib.oracle_digest_records(records.ctypes.data, record, record, sample, crcs.ctypes.data,
                                      shas.ctypes.data, threads)
            lib.oracle_copy_threads(LAYERS, span_base.ctypes.data, span_pitch.ctypes.data, span_off.ctypes.data,
                                    span_len.ctypes.data, dst.ctypes.data, sources.ctypes.data, sample, None, record,
                                    threads)
            elapsed += time.perf_counter() - t0
            reps += 1
        result[threads] = 2 * sample * record * reps / elapsed / 1e9
    return {"value": result[threads_max], "unit": "GB/s", "cores": threads_max, "kind": "port",
            "single_thread_gbps": result[1],
            "sample": (f"{sample} Qwen3-8B blocks ({sample * record} B) of a {host_blocks}-block host cache: "
                       "gather + CRC32C + SHA-256 + scatter, repeated ~{:.0f} s".format(seconds_budget))}


def main():
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=10)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--layout", choices=("kv_split", "vllm"), default="kv_split")
    parser.add_argument("--cpu-seconds", type=float, default=20.0)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    args = parser.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: every GPU saves and restores its own KV shard over its own host link, "
              "so there is no multi-GPU step to time here (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    import torch
    from kvsnap_amd import synth
    from kvsnap_amd.dataplane import KernelTimer, TorchBlockDataPlane

    torch.cuda.set_device(0)
    caches, backing = synth.make_caches(LAYERS, NUM_BLOCKS, block_size=BLOCK_SIZE, heads=HEADS, head_dim=HEAD_DIM,
                                        layout=args.layout)
    plane = TorchBlockDataPlane(caches, BLOCK_SIZE, SESSION_BLOCKS * LAYERS * 65536 + (64 << 20))
    plane.warm_up()
    keep = synth.fill(plane, 0)
    torch.cuda.synchronize()
    del keep
    size = plane.block_bytes
    total = SESSION_BLOCKS * size
    source, target = synth.block_tables(NUM_BLOCKS, SESSION_BLOCKS)
    staged = plane.pool.reserve(total)
    targets = [(staged, i * size) for i in range(SESSION_BLOCKS)]
    stream = plane._copy_stream
    log(f"setup: {LAYERS} layers x {NUM_BLOCKS} blocks ({args.layout}), record {size} B, session {total} B")

    # Measured link peaks: one contiguous pinned <-> device DMA of the whole session.
    device_buffer = torch.empty(total, dtype=torch.uint8, device="cuda")
    h2d_ms = median_ms(torch, stream, lambda: staged.copy(device_buffer.data_ptr(), total, 0, to_host=False))
    d2h_ms = median_ms(torch, stream, lambda: staged.copy(device_buffer.data_ptr(), total, 0, to_host=True))
    del device_buffer
    h2d_peak, d2h_peak = total / h2d_ms / 1e6, total / d2h_ms / 1e6
    log(f"DMA peaks: H2D {h2d_peak:.1f} GB/s, D2H {d2h_peak:.1f} GB/s")

    save_ms, hashed_ms, restore_ms, early_ms = [], [], [], []

    def step(record):
        digests, progress = [], []
        t0 = time.perf_counter()
        plane.save_gather(source, targets, TOKENS, digests=digests)
        t1 = time.perf_counter()
        plane.load_scatter(target, targets, progress=progress)
        t2 = time.perf_counter()
        result = digests[0].result()
        t3 = time.perf_counter()
        if record:
            save_ms.append((t1 - t0) * 1e3)
            restore_ms.append((t2 - t1) * 1e3)
            hashed_ms.append((t3 - t0) * 1e3)
        return result, progress

    for _ in range(args.warmup):
        step(False)
    timer = KernelTimer()
    plane.timer = timer
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(args.steps):
        digests, progress = step(True)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    plane.timer = None
    kernels = timer.summary()
    ms_per_step = elapsed * 1e3 / args.steps

    # Early readiness: launch count and how much was still in flight when the
    # last launch was queued (the connector reports a load once <= 128 MiB remain).
    launches = len(progress) - 1

    # Parity of the last step (outside the timed region): restored blocks equal
    # the saved ones, and the GPU digests equal the oracle's on the pinned records.
    src_ids = torch.tensor(source, device="cuda")
    dst_ids = torch.tensor(target, device="cuda")
    exact = all(torch.equal(t[:, src_ids].view(torch.int16), t[:, dst_ids].view(torch.int16))
                if t.ndim == 5 else torch.equal(t[src_ids].view(torch.int16), t[dst_ids].view(torch.int16))
                for t in caches.values())
    import numpy as np
    import oracle
    crcs, shas = oracle.digest_records(staged.pointer, size, size, SESSION_BLOCKS, threads=min(16, os.cpu_count()))
    digests_exact = all(crc == int(c) and sha == bytes(s).hex()
                        for (sha, crc), c, s in zip(digests, crcs, shas))
    log(f"parity: restore byte-exact={exact}, CRC32C+SHA-256 bit-exact={digests_exact}")

    gather = kernels["gather"]
    restore = kernels["restore"]
    crc = kernels["crc32c"]
    sha = kernels["sha256"]
    gather_achieved = 2 * total / (gather["avg_ms"] * 1e6)        # read + write per launch (one launch per save)
    restore_per_launch = total / restore["launches"] * args.steps   # bytes per launch (pinned read = HBM write)
    restore_link = restore_per_launch / (restore["avg_ms"] * 1e6)
    crc_achieved = total / (crc["avg_ms"] * 1e6)
    cpu = None if args.no_cpu_baseline else cpu_baseline(args.cpu_seconds)
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
        "config": {"workload": "qwen3-8b-8k-token-snapshot-save-then-restore", "layers": LAYERS,
                   "kv_heads": HEADS, "head_dim": HEAD_DIM, "block_size": BLOCK_SIZE, "cache_blocks": NUM_BLOCKS,
                   "session_blocks": SESSION_BLOCKS, "snapshot_bytes": total, "kv_dtype": "bf16",
                   "layout": args.layout, "parallelism": "none (one GPU)"},
        "save_ms": round(statistics.median(save_ms), 3),
        "save_gbps": round(total / statistics.median(save_ms) / 1e6, 2),
        "save_hashed_ms": round(statistics.median(hashed_ms), 3),
        "restore_ms": round(statistics.median(restore_ms), 3),
        "restore_gbps": round(total / statistics.median(restore_ms) / 1e6, 2),
        "restore_launches": launches,
        "h2d_peak_gbps": round(h2d_peak, 2),
        "d2h_peak_gbps": round(d2h_peak, 2),
        "restore_frac_of_h2d": round(total / statistics.median(restore_ms) / 1e6 / h2d_peak, 4),
        "save_frac_of_d2h": round(total / statistics.median(save_ms) / 1e6 / d2h_peak, 4),
        "kernels_ms": {name: round(k["avg_ms"], 4) for name, k in kernels.items()},
        "roofline": {"kernel": "gather_kernel", "bound": "hbm", "achieved": round(gather_achieved, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(gather_achieved / HBM_PEAK_GBPS, 4),
                     "traffic": None},
        "link_roofline": {"kernel": "restore_kernel", "bound": "host-link", "achieved": round(restore_link, 2),
                          "peak": round(h2d_peak, 2), "unit": "GB/s", "frac": round(restore_link / h2d_peak, 4)},
        "crc_roofline": {"kernel": "crc_stripes_kernel", "bound": "hbm", "achieved": round(crc_achieved, 1),
                         "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(crc_achieved / HBM_PEAK_GBPS, 4)},
        "sha256": {"ms": round(sha["avg_ms"], 3), "gbps": round(total / (sha["avg_ms"] * 1e6), 2),
                   "records": SESSION_BLOCKS},
        "parity": {"restore_byte_exact": exact, "digests_bit_exact": digests_exact},
        "cpu_baseline": cpu,
    }
    staged.close()
    plane.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
