"""The pinned pool's control flow on the CPU: our pool.cpp built against a fault-injecting HIP stand-in.

Mirrors the reference's tests/unit/test_independent_native.py and
tests/connector/test_native_lifetime.py, and runs the same scenarios against
the reference's own pool (csrc/dataplane/cuda_pool.cpp built with its own
tests/native/fake_cuda.cpp into oracle/_ref) where that library was built, so
both pools are held to the same return codes.
"""
import ctypes as C
import gc
import os
import shutil
import subprocess
import threading
import weakref
from pathlib import Path
from unittest.mock import patch

import pytest

from kvsnap_amd.dataplane import CudaPool, PinnedCapacityError
from kvsnap_amd.pool import POOL_SIGNATURES, declare

ROOT = Path(__file__).resolve().parents[1]
REF_POOL = ROOT / "oracle" / "_ref" / "libkvsnap_pool_fakecuda_ref.so"

# The pool's own entry points as the binding types them, plus the stand-in runtime's fault hooks.
SIGNATURES = dict(POOL_SIGNATURES, kvsnap_test_pending="int <-", kvsnap_test_fail_next_record="void <-",
                  kvsnap_test_fail_next_stream_sync="void <-")


def _typed(path):
    lib = C.CDLL(str(path))
    for name, signature in SIGNATURES.items():
        declare(lib, name, signature)
    return lib


@pytest.fixture(scope="module")
def fake_pool_path(tmp_path_factory):
    if not shutil.which("g++"):
        pytest.skip("g++ unavailable")
    out = tmp_path_factory.mktemp("pool") / "libpool_fakehip.so"
    # -Bsymbolic binds the pool to the stand-in even if a real HIP runtime is loaded.
    subprocess.run(["g++", "-std=c++17", "-shared", "-fPIC", "-pthread", "-Wl,-Bsymbolic", "-Wall", "-Wextra",
                    "-Werror", "-I", str(ROOT / "tests" / "native"), str(ROOT / "kvsnap_amd" / "csrc" / "pool.cpp"),
                    str(ROOT / "tests" / "native" / "fake_hip.cpp"), "-o", str(out)],
                   check=True, capture_output=True, text=True, timeout=120)
    return out


@pytest.fixture(scope="module")
def lib(fake_pool_path):
    handle = _typed(fake_pool_path)
    for name, signature in {"kvsnap_test_fail_next_host_alloc": "void <-", "kvsnap_test_map_elsewhere": "void <- int",
                            "kvsnap_test_live_events": "int <-", "kvsnap_test_last_copy_stream": "size <-",
                            "kvsnap_test_last_host_flags": "u32 <-",
                            "kvsnap_pool_copy_stream": "int <- ptr size*"}.items():
        declare(handle, name, signature)
    return handle


def pools():
    """Our pool, and the reference's where its fake-CUDA build exists."""
    yield "ours"
    if REF_POOL.is_file():
        yield "reference"


def _reserve(lib, pool, size):
    ident, ptr = C.c_uint64(), C.c_void_p()
    rc = lib.kvsnap_pool_reserve(pool, size, C.byref(ident), C.byref(ptr))
    return rc, ident.value, ptr.value


def scenario_record_failure(lib):
    pool = lib.kvsnap_pool_create(16, 0)
    try:
        rc, ident, _ = _reserve(lib, pool, 16)
        destination = C.create_string_buffer(16)
        lib.kvsnap_test_fail_next_record()
        copy_rc = lib.kvsnap_pool_copy(pool, ident, 0, destination, 16, 0, 0)
        released = lib.kvsnap_pool_release(pool, ident)
        return (rc, copy_rc, released, lib.kvsnap_test_pending() if released == 0 else None)
    finally:
        lib.kvsnap_pool_destroy(pool)


def scenario_strided(lib):
    pool = lib.kvsnap_pool_create(24, 0)
    try:
        rc, ident, ptr = _reserve(lib, pool, 24)
        C.memmove(ptr, bytes(range(24)), 24)
        device = C.create_string_buffer(b"\xee" * 18, 18)
        ok = lib.kvsnap_pool_copy_2d(pool, ident, 4, 8, device, 6, 4, 3, 0, 0)
        waited = lib.kvsnap_pool_wait(pool, ident)
        raw = device.raw
        too_long = lib.kvsnap_pool_copy_2d(pool, ident, 4, 8, device, 6, 5, 3, 0, 0)
        narrow = lib.kvsnap_pool_copy_2d(pool, ident, 0, 2, device, 6, 4, 3, 0, 0)
        released = lib.kvsnap_pool_release(pool, ident)
        return (rc, ok, waited, raw, too_long, narrow, released)
    finally:
        lib.kvsnap_pool_destroy(pool)


def scenario_capacity_and_drain(lib):
    pool = lib.kvsnap_pool_create(16, 0)
    try:
        rc, ident, _ = _reserve(lib, pool, 16)
        over, _, _ = _reserve(lib, pool, 1)
        destination = C.create_string_buffer(16)
        outside = lib.kvsnap_pool_copy(pool, ident, 0, destination, 17, 0, 0)
        inside = lib.kvsnap_pool_copy(pool, ident, 0, destination, 16, 0, 0)
        ready = lib.kvsnap_pool_ready(pool, ident)
        released = lib.kvsnap_pool_release(pool, ident)
        pending = lib.kvsnap_test_pending()
        again, _, _ = _reserve(lib, pool, 16)
        return (rc, over, outside, inside, ready, released, pending, again)
    finally:
        lib.kvsnap_pool_destroy(pool)


def scenario_failed_drain(lib):
    pool = lib.kvsnap_pool_create(16, 0)
    try:
        rc, ident, _ = _reserve(lib, pool, 16)
        destination = C.create_string_buffer(16)
        lib.kvsnap_test_fail_next_record()
        failed_copy = lib.kvsnap_pool_copy(pool, ident, 0, destination, 16, 0, 0)
        lib.kvsnap_test_fail_next_stream_sync()
        failed_release = lib.kvsnap_pool_release(pool, ident)
        still_pending = lib.kvsnap_test_pending() > 0
        blocked, _, _ = _reserve(lib, pool, 1)
        released = lib.kvsnap_pool_release(pool, ident)
        pending = lib.kvsnap_test_pending()
        return (rc, failed_copy, failed_release, still_pending, blocked, released, pending)
    finally:
        lib.kvsnap_pool_destroy(pool)


SCENARIOS = [scenario_record_failure, scenario_strided, scenario_capacity_and_drain, scenario_failed_drain]


@pytest.mark.parametrize("scenario", SCENARIOS, ids=lambda f: f.__name__)
def test_pool_matches_the_reference_pool_on_every_scenario(lib, scenario):
    ours = scenario(lib)
    if not REF_POOL.is_file():
        pytest.skip("reference pool not built (no /root/reference when oracle/_ref was made)")
    reference = scenario(_typed(REF_POOL))
    assert ours == reference


def test_record_failure_never_releases_inflight_pinned_bytes(lib):
    rc, copy_rc, released, pending = scenario_record_failure(lib)
    assert (rc, copy_rc) == (0, -1)
    if released == 0:
        assert pending == 0, "allocation released while a copy is still queued"


def test_strided_copy_moves_one_layer_of_consecutive_blocks_and_checks_bounds(lib):
    rc, ok, waited, raw, too_long, narrow, released = scenario_strided(lib)
    assert (rc, ok, waited, released) == (0, 0, 0, 0)
    assert raw == bytes([4, 5, 6, 7, 0xee, 0xee, 12, 13, 14, 15, 0xee, 0xee, 20, 21, 22, 23, 0xee, 0xee])
    assert (too_long, narrow) == (-1, -1)


def test_normal_async_copy_drains_before_release_and_checks_capacity(lib):
    assert scenario_capacity_and_drain(lib) == (0, -1, -1, 0, 0, 0, 0, 0)


def test_failed_stream_drain_keeps_allocation_unavailable_for_reuse(lib):
    assert scenario_failed_drain(lib) == (0, -1, -1, True, -1, 0, 0)


def test_first_fit_reuses_a_released_hole(lib):
    pool = lib.kvsnap_pool_create(48, 0)
    try:
        got = [_reserve(lib, pool, 16) for _ in range(3)]
        assert [g[0] for g in got] == [0, 0, 0]
        assert lib.kvsnap_pool_release(pool, got[1][1]) == 0
        rc, ident, ptr = _reserve(lib, pool, 16)
        assert rc == 0 and ptr == got[1][2] and ident not in {g[1] for g in got}
        rc, _, _ = _reserve(lib, pool, 1)
        assert rc == -1 and b"pinned capacity exhausted" in lib.kvsnap_cuda_error()
    finally:
        lib.kvsnap_pool_destroy(pool)


def test_reserve_rejects_zero_and_oversized_and_unknown_ids_fail(lib):
    pool = lib.kvsnap_pool_create(64, 0)
    try:
        assert _reserve(lib, pool, 0)[0] == -1
        assert _reserve(lib, pool, 65)[0] == -1
        assert b"pinned capacity exhausted" in lib.kvsnap_cuda_error()
        assert lib.kvsnap_pool_wait(pool, 12345) == -1
        assert b"unknown pinned allocation" in lib.kvsnap_cuda_error()
        assert lib.kvsnap_pool_ready(pool, 12345) == -1
        assert lib.kvsnap_pool_release(pool, 12345) == -1
    finally:
        lib.kvsnap_pool_destroy(pool)


def test_create_refuses_an_arena_mapped_at_another_device_address(lib):
    lib.kvsnap_test_map_elsewhere(1)
    try:
        assert not lib.kvsnap_pool_create(64, 0)
        assert b"not mapped at its host address" in lib.kvsnap_cuda_error()
    finally:
        lib.kvsnap_test_map_elsewhere(0)
    lib.kvsnap_test_fail_next_host_alloc()
    assert not lib.kvsnap_pool_create(64, 0)
    assert not lib.kvsnap_pool_create(0, 0)
    assert b"capacity must be positive" in lib.kvsnap_cuda_error()


@pytest.mark.parametrize("value,flag", [("1", 0x40000000), ("0", 0x80000000), (None, 0)])
def test_arena_coherence_follows_the_environment(lib, value, flag):
    env = {} if value is None else {"KVSNAP_PINNED_COHERENT": value}
    with patch.dict(os.environ, env, clear=False):
        if value is None:
            os.environ.pop("KVSNAP_PINNED_COHERENT", None)
        pool = lib.kvsnap_pool_create(64, 0)
        try:
            flags = lib.kvsnap_test_last_host_flags()
            assert flags & 0x3 == 0x3                      # portable | mapped
            assert flags & 0xC0000000 == flag
        finally:
            lib.kvsnap_pool_destroy(pool)


def test_copies_run_on_the_pool_stream_and_events_are_freed(lib, fake_pool_path):
    before = lib.kvsnap_test_live_events()
    pool = CudaPool(32, library=fake_pool_path)
    source = C.create_string_buffer(b"0123456789abcdef", 16)
    with pool.borrow_copy_stream() as stream:
        allocation = pool.reserve(16)
        allocation.copy(C.addressof(source), 16, to_host=True)
        assert lib.kvsnap_test_last_copy_stream() == stream
        assert allocation.read() == b"0123456789abcdef"
        allocation.close()
    pool.close()
    assert lib.kvsnap_test_live_events() == before
    with pytest.raises(RuntimeError, match="pool closed"):
        with pool.borrow_copy_stream():
            pass


def test_failed_checked_close_preserves_the_pool_until_a_retry_drains(lib, fake_pool_path):
    pool = CudaPool(16, library=fake_pool_path)
    source = C.create_string_buffer(b"0123456789abcdef", 16)
    allocation = pool.reserve(16)
    allocation.copy(C.addressof(source), 16, to_host=True)
    assert lib.kvsnap_test_pending() == 1
    handle = pool.handle
    lib.kvsnap_test_fail_next_stream_sync()
    with pytest.raises(RuntimeError):
        pool.close()
    assert pool.handle == handle
    assert not allocation.ready()
    with pytest.raises(PinnedCapacityError):
        pool.reserve(1)
    pool.close()
    assert pool.handle is None and lib.kvsnap_test_pending() == 0


def test_pinned_allocation_reads_writes_zeroes_and_bounds(lib, fake_pool_path):
    pool = CudaPool(64, library=fake_pool_path)
    try:
        allocation = pool.reserve(16)
        allocation.write(b"A" * 16)
        allocation.zero(4, 8)
        assert allocation.read() == b"AAAA" + bytes(8) + b"AAAA"
        assert allocation.read_range(2, 4) == b"AA\0\0"
        for bad in ((-1, 2), (15, 2), (0, 17)):
            with pytest.raises(ValueError):
                allocation.read_range(*bad)
        with pytest.raises(ValueError):
            allocation.zero(10, 8)
        with pytest.raises(ValueError):
            allocation.write(b"short")
        with pytest.raises(ValueError):
            allocation.copy(-1, 4, to_host=True)
        allocation.close()
        with pytest.raises(RuntimeError, match="closed"):
            allocation.read()
    finally:
        pool.close()


# ---------------------------------------------------------------- Python lifetime, against a scripted library


class Entry:
    """One entry point of the scripted library: callable, and typeable as ctypes functions are."""

    def __init__(self, body):
        self.body, self.argtypes, self.restype = body, None, None

    def __call__(self, *args):
        return self.body(*args)


class ScriptedPool:
    """The pool C-ABI answered in Python, to drive the binding's lifetime rules without a runtime.

    One pool (handle 101) and one allocation (id 7 at address 128).  A copy
    stops at a gate until the test opens it, and records whether the pool or
    the allocation went away while it was inside.
    """

    HANDLE = 101

    def __init__(self):
        self.inside, self.gate = threading.Event(), threading.Event()
        self.gone = {"pool": False, "allocation": False}
        self.close_result, self.violations = 0, []
        self.set(kvsnap_pool_abi_version=lambda: 2, kvsnap_cuda_error=lambda: b"scripted failure",
                 kvsnap_pool_create=lambda capacity, device: self.HANDLE, kvsnap_pool_destroy=lambda pool: None,
                 kvsnap_pool_close_checked=self._close, kvsnap_pool_reserve=self._reserve,
                 kvsnap_pool_copy=self._copy, kvsnap_pool_copy_2d=self._copy,
                 kvsnap_pool_wait=lambda pool, ident: 0, kvsnap_pool_ready=lambda pool, ident: 1,
                 kvsnap_pool_release=self._release)

    def set(self, **bodies):
        for name, body in bodies.items():
            setattr(self, name, Entry(body))

    def _close(self, pool):
        if self.close_result == 0:
            self.gone["pool"] = True
        return self.close_result

    def _reserve(self, pool, size, ident, pointer):
        C.cast(ident, C.POINTER(C.c_uint64)).contents.value = 7
        C.cast(pointer, C.POINTER(C.c_void_p)).contents.value = 128
        return 0

    def _release(self, pool, ident):
        self.gone["allocation"] = True
        return 0

    def _copy(self, *args):
        self.inside.set()
        if not self.gate.wait(5):
            self.violations.append("the gate was never opened")
        if any(self.gone.values()):
            self.violations.append(f"ended inside a copy: {self.gone}")
        return 0


def binding_over(library):
    """A CudaPool whose library is ``library`` (ctypes loading intercepted)."""
    with patch.object(C, "CDLL", return_value=library):
        return CudaPool(4096)


@pytest.mark.parametrize("shape,closing", [("flat", "pool"), ("strided", "allocation")])
def test_closing_waits_for_a_copy_in_flight(shape, closing):
    library = ScriptedPool()
    pool = binding_over(library)
    allocation = pool.reserve(128)
    finished = threading.Event()
    failures = []

    def in_thread(work, done=None):
        def run():
            try:
                work()
            except BaseException as exc:
                failures.append(exc)
            finally:
                if done is not None:
                    done.set()
        thread = threading.Thread(target=run)
        thread.start()
        return thread

    copy = (lambda: allocation.copy(256, 128, to_host=True)) if shape == "flat" else \
        (lambda: allocation.copy_2d(256, 64, 0, 64, 64, 2, to_host=True))
    copier = in_thread(copy)
    assert library.inside.wait(2)
    closer = in_thread(pool.close if closing == "pool" else allocation.close, finished)
    held = not finished.wait(0.05)
    library.gate.set()
    copier.join(3)
    closer.join(3)
    pool.close()
    assert held, "close returned while a copy was still inside the library"
    assert failures == [] and library.violations == []


def test_owners_stay_alive_until_a_wait_or_release_succeeds():
    library = ScriptedPool()
    pool = binding_over(library)
    allocation = pool.reserve(128)
    owner = type("Owner", (), {})()
    allocation._tensor_references = [owner]
    watch_allocation, watch_owner = weakref.ref(allocation), weakref.ref(owner)
    library.set(kvsnap_pool_wait=lambda pool, ident: -1, kvsnap_pool_release=lambda pool, ident: -1)
    with pytest.raises(RuntimeError, match="scripted failure"):
        allocation.wait()
    with pytest.raises(RuntimeError, match="scripted failure"):
        allocation.close()
    del allocation, owner
    gc.collect()
    assert watch_allocation() is not None and watch_owner() is not None    # the pool keeps both
    library.set(kvsnap_pool_release=lambda pool, ident: 0)
    watch_allocation().close()
    gc.collect()
    assert watch_owner() is None and watch_allocation() is None
    pool.close()


def test_a_failed_pool_close_can_be_retried_with_everything_in_place():
    library = ScriptedPool()
    pool = binding_over(library)
    allocation = pool.reserve(128)
    owner = object()
    allocation._tensor_references = [owner]
    library.close_result = -1
    with pytest.raises(RuntimeError):
        pool.close()
    assert (pool.handle, library.gone["pool"], allocation._tensor_references) == (ScriptedPool.HANDLE, False, [owner])
    library.close_result = 0
    pool.close()
    assert pool.handle is None and allocation.closed and allocation._tensor_references == []


def test_another_abi_version_is_refused_before_any_pool_exists():
    library = ScriptedPool()
    created = []
    library.set(kvsnap_pool_abi_version=lambda: 1,
                kvsnap_pool_create=lambda capacity, device: created.append(capacity) or ScriptedPool.HANDLE)
    with pytest.raises(RuntimeError, match="unsupported.*ABI"):
        binding_over(library)
    assert created == []


def test_a_forked_child_may_not_touch_the_pool():
    pool = binding_over(ScriptedPool())
    owner_pid = pool._pid
    pool._pid = owner_pid + 1          # as seen from a child: the pool belongs to another process
    for call in (lambda: pool.reserve(1), pool.close):
        with pytest.raises(RuntimeError, match="fork"):
            call()
    pool._pid = owner_pid
    pool.close()


def test_only_the_capacity_message_becomes_pinned_capacity_error():
    library = ScriptedPool()
    message = [b"pinned capacity exhausted: 64 bytes free"]
    library.set(kvsnap_pool_reserve=lambda *args: -1, kvsnap_cuda_error=lambda: message[0])
    pool = binding_over(library)
    with pytest.raises(PinnedCapacityError):
        pool.reserve(1)
    message[0] = b"some other failure"
    with pytest.raises(RuntimeError, match="some other failure") as raised:
        pool.reserve(1)
    assert not isinstance(raised.value, PinnedCapacityError)
    pool.close()
