"""The hash lane's scheduling on the CPU: saves that hash at the same time share each SHA-256 launch.

A fake kernel library stands in for the HIP one: it records every launch,
fills a record set's digests (hashlib over host memory) and CRC32Cs (the
oracle) when a range ends its chain, and can fail a chosen launch.  The GPU
tests check the chaining state between ranges against hashlib; these check
that the lane merges jobs into shared launches, advances each job by its
own ranges, carries at most eight jobs a launch, reports a failed launch (or
a kernel library that fails to load) to every job in it and keeps serving
later ones, and finishes every job before ``close`` returns.
"""
import ctypes as C
from contextlib import nullcontext
import hashlib
import threading
import time
from types import SimpleNamespace
from unittest.mock import patch

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import oracle
from kvsnap_amd import dataplane
from kvsnap_amd.dataplane import SHA_MAX_RANGES, HashJob, HashLane


class FakeTorch:
    """torch with the CUDA calls a hash lane makes answered on the CPU."""

    class Event:
        def __init__(self, enable_timing=False):
            pass

        def record(self, stream=None):
            pass

        def synchronize(self):
            pass

        def query(self):
            return True

    def __init__(self):
        self.cuda = SimpleNamespace(Event=self.Event, stream=lambda stream: nullcontext())

    def __getattr__(self, name):
        return getattr(torch, name)

    def empty(self, *args, device=None, **kwargs):
        return torch.empty(*args, **kwargs)


class FakeLibrary:
    """The entry points a hash lane calls, on host memory."""

    def __init__(self, fail_launch=None, hold_first_crc=None, launch_seconds=0.0):
        self.launches, self.crcs = [], []
        self.fail_launch, self.hold_first_crc, self.launch_seconds = fail_launch, hold_first_crc, launch_seconds
        self.error = b""

    @staticmethod
    def kvsnap_crc32c_workspace_bytes(record_bytes, n):
        return 64

    @staticmethod
    def kvsnap_sha256_blocks(record_bytes):
        return record_bytes // 64 + (1 if record_bytes % 64 + 9 <= 64 else 2)

    def kvsnap_cuda_error(self):
        return self.error

    def kvsnap_crc32c_records(self, records, record_bytes, pitch, n, prior, out, work, work_bytes, stream):
        if self.hold_first_crc is not None and not self.crcs:
            assert self.hold_first_crc.wait(10)
        self.crcs.append(records)
        values = (C.c_uint32 * n).from_address(out)
        for i in range(n):
            values[i] = oracle.crc32c_at(records + i * pitch, record_bytes)
        return 0

    def kvsnap_sha256_ranges(self, count, records, record_bytes, pitches, counts, firsts, ends, states, outs,
                             stream):
        index = len(self.launches)
        self.launches.append([(records[i], firsts[i], ends[i]) for i in range(count)])
        time.sleep(self.launch_seconds)
        if index == self.fail_launch:
            self.error = b"SHA-256 launch failed"
            return -1
        for i in range(count):
            if ends[i] == self.kvsnap_sha256_blocks(record_bytes[i]):
                digests = (C.c_uint8 * (32 * counts[i])).from_address(outs[i])
                for r in range(counts[i]):
                    data = C.string_at(records[i] + r * pitches[i], record_bytes[i])
                    digests[32 * r:32 * r + 32] = list(hashlib.sha256(data).digest())
        return 0


def record_sets(count, n=3, record_bytes=1000, seed=0):
    rng = np.random.default_rng(seed)
    return [np.frombuffer(rng.bytes(n * record_bytes), dtype=np.uint8).copy() for _ in range(count)]


def submit(lane, sets, record_bytes=1000, n=3, slice_blocks=4):
    return [HashJob(lane.torch, s.ctypes.data, record_bytes, record_bytes, n, "cuda", lane, slice_blocks)
            for s in sets]


def check_digests(job, records, record_bytes=1000, n=3):
    job.synchronize()
    for r in range(n):
        data = records[r * record_bytes:(r + 1) * record_bytes].tobytes()
        assert bytes(job.sha[r].numpy()) == hashlib.sha256(data).digest()
        assert int(job.crc[r]) & 0xFFFFFFFF == oracle.crc32c(data)


def test_jobs_that_arrive_together_share_every_launch_and_get_their_own_digests():
    held = threading.Event()
    fake = FakeLibrary(hold_first_crc=held)
    with patch.object(dataplane, "kernel_library", lambda library=None: fake):
        lane = HashLane(FakeTorch(), SimpleNamespace(cuda_stream=7, synchronize=lambda: None))
        blocker = record_sets(1, seed=9)
        first = submit(lane, blocker)       # the lane takes it and holds at its CRC32C ...
        deadline = time.monotonic() + 10
        while lane._incoming and time.monotonic() < deadline:
            time.sleep(1e-4)
        sets = record_sets(4)
        jobs = submit(lane, sets)           # ... while four more arrive together
        held.set()
        check_digests(first[0], blocker[0])
        for job, records in zip(jobs, sets):
            check_digests(job, records)
        lane.close()
    nblocks = FakeLibrary.kvsnap_sha256_blocks(1000)
    carried = [[i for i, launch in enumerate(fake.launches) if records.ctypes.data in {a for a, _, _ in launch}]
               for records in sets]
    assert carried[0] and all(c == carried[0] for c in carried)      # the four in the same launches
    assert len(carried[0]) == -(-nblocks // 4)                       # one launch per range, shared
    assert fake.launches[0] == [(blocker[0].ctypes.data, 0, 4)]      # the blocker started alone


def test_a_job_that_arrives_later_joins_the_launches_already_running():
    held = threading.Event()
    fake = FakeLibrary(hold_first_crc=held, launch_seconds=0.005)
    with patch.object(dataplane, "kernel_library", lambda library=None: fake):
        lane = HashLane(FakeTorch(), SimpleNamespace(cuda_stream=7, synchronize=lambda: None))
        early = record_sets(1, seed=1)
        first = submit(lane, early, slice_blocks=2)[0]
        held.set()
        while not fake.launches:            # the first job's chain has started alone
            pass
        late = record_sets(1, seed=2)
        second = submit(lane, late, slice_blocks=2)[0]
        check_digests(first, early[0])
        check_digests(second, late[0])
        lane.close()
    shared = [launch for launch in fake.launches if len(launch) == 2]
    assert shared and fake.launches[0] == [(early[0].ctypes.data, 0, 2)]


def test_a_launch_carries_at_most_eight_jobs_and_every_job_finishes():
    held = threading.Event()
    fake = FakeLibrary(hold_first_crc=held)
    with patch.object(dataplane, "kernel_library", lambda library=None: fake):
        lane = HashLane(FakeTorch(), SimpleNamespace(cuda_stream=7, synchronize=lambda: None))
        sets = record_sets(SHA_MAX_RANGES + 3, seed=3)
        jobs = submit(lane, sets)
        held.set()
        for job, records in zip(jobs, sets):
            check_digests(job, records)
        lane.close()
    assert max(len(launch) for launch in fake.launches) == SHA_MAX_RANGES
    nblocks = FakeLibrary.kvsnap_sha256_blocks(1000)
    for records in sets:                    # each job's ranges cover its chain once, in order
        ranges = [(first, end) for launch in fake.launches for address, first, end in launch
                  if address == records.ctypes.data]
        assert ranges == [(a, min(a + 4, nblocks)) for a in range(0, nblocks, 4)]


def test_a_failed_launch_fails_its_jobs_and_the_lane_serves_the_next():
    held = threading.Event()
    fake = FakeLibrary(fail_launch=2, hold_first_crc=held)
    with patch.object(dataplane, "kernel_library", lambda library=None: fake):
        lane = HashLane(FakeTorch(), SimpleNamespace(cuda_stream=7, synchronize=lambda: None))
        sets = record_sets(2, seed=4)
        jobs = submit(lane, sets)
        held.set()
        for job in jobs:
            with pytest.raises(RuntimeError, match="SHA-256 launch failed"):
                job.synchronize()
            assert job.finished(timeout=0) and job.keepalive is None
        after = record_sets(1, seed=5)
        check_digests(submit(lane, after)[0], after[0])
        lane.close()


def test_close_finishes_every_job_and_refuses_new_ones():
    fake = FakeLibrary()
    with patch.object(dataplane, "kernel_library", lambda library=None: fake):
        lane = HashLane(FakeTorch(), SimpleNamespace(cuda_stream=7, synchronize=lambda: None))
        sets = record_sets(4, seed=6)
        jobs = submit(lane, sets)
        lane.close()
        assert all(job.finished(timeout=0) for job in jobs)
        for job, records in zip(jobs, sets):
            check_digests(job, records)
        with pytest.raises(RuntimeError, match="closed"):
            submit(lane, record_sets(1, seed=7))


def test_a_library_that_fails_to_load_fails_the_jobs_and_the_lane_serves_the_next():
    fake, calls = FakeLibrary(), []

    def library(library=None):          # the lane thread's first load fails
        if threading.current_thread().name == "kvsnap-hash":
            calls.append(1)
            if len(calls) == 1:
                raise RuntimeError("HIP dataplane library not built")
        return fake

    with patch.object(dataplane, "kernel_library", library):
        lane = HashLane(FakeTorch(), SimpleNamespace(cuda_stream=7, synchronize=lambda: None))
        first = submit(lane, record_sets(1, seed=8))[0]
        with pytest.raises(RuntimeError, match="not built"):
            first.synchronize()
        later = record_sets(1, seed=9)
        check_digests(submit(lane, later)[0], later[0])
        lane.close()
