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

ROOT = Path(__file__).resolve().parents[1]
REF_POOL = ROOT / "oracle" / "_ref" / "libkvsnap_pool_fakecuda_ref.so"

API = {
    "kvsnap_pool_create": ([C.c_size_t, C.c_int], C.c_void_p),
    "kvsnap_pool_destroy": ([C.c_void_p], None),
    "kvsnap_pool_close_checked": ([C.c_void_p], C.c_int),
    "kvsnap_pool_reserve": ([C.c_void_p, C.c_size_t, C.POINTER(C.c_uint64), C.POINTER(C.c_void_p)], C.c_int),
    "kvsnap_pool_copy": ([C.c_void_p, C.c_uint64, C.c_size_t, C.c_void_p, C.c_size_t, C.c_int, C.c_size_t], C.c_int),
    "kvsnap_pool_copy_2d": ([C.c_void_p, C.c_uint64, C.c_size_t, C.c_size_t, C.c_void_p, C.c_size_t, C.c_size_t,
                             C.c_size_t, C.c_int, C.c_size_t], C.c_int),
    "kvsnap_pool_release": ([C.c_void_p, C.c_uint64], C.c_int),
    "kvsnap_pool_wait": ([C.c_void_p, C.c_uint64], C.c_int),
    "kvsnap_pool_ready": ([C.c_void_p, C.c_uint64], C.c_int),
    "kvsnap_cuda_error": ([], C.c_char_p),
    "kvsnap_test_pending": ([], C.c_int),
    "kvsnap_test_fail_next_record": ([], None),
    "kvsnap_test_fail_next_stream_sync": ([], None),
}


def _typed(path):
    lib = C.CDLL(str(path))
    for name, (args, result) in API.items():
        fn = getattr(lib, name)
        fn.argtypes, fn.restype = args, result
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
    for name, (args, result) in {"kvsnap_test_fail_next_host_alloc": ([], None),
                                 "kvsnap_test_map_elsewhere": ([C.c_int], None),
                                 "kvsnap_test_live_events": ([], C.c_int),
                                 "kvsnap_test_last_copy_stream": ([], C.c_size_t),
                                 "kvsnap_test_last_host_flags": ([], C.c_uint),
                                 "kvsnap_pool_copy_stream": ([C.c_void_p, C.POINTER(C.c_size_t)], C.c_int),
                                 "kvsnap_pool_abi_version": ([], C.c_int)}.items():
        fn = getattr(handle, name)
        fn.argtypes, fn.restype = args, result
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


# ---------------------------------------------------------------- Python lifetime with a blocking ABI


class Function:
    def __init__(self, implementation):
        self.implementation = implementation

    def __call__(self, *args):
        return self.implementation(*args)


class BlockingABI:
    """A stand-in ABI whose copy blocks until released, to race close against it."""

    def __init__(self):
        self.entered, self.proceed = threading.Event(), threading.Event()
        self.destroyed = self.released = self.fail_close = False
        self.kvsnap_pool_abi_version = Function(lambda: 2)
        self.kvsnap_cuda_error = Function(lambda: b"stand-in error")
        self.kvsnap_pool_create = Function(lambda capacity, device: 101)
        self.kvsnap_pool_destroy = Function(lambda pool: setattr(self, "destroyed", True))
        self.kvsnap_pool_close_checked = Function(self.close_checked)
        self.kvsnap_pool_reserve = Function(self.reserve)
        self.kvsnap_pool_copy = Function(self.copy)
        self.kvsnap_pool_copy_2d = Function(self.copy)
        self.kvsnap_pool_wait = Function(lambda pool, allocation: 0)
        self.kvsnap_pool_ready = Function(lambda pool, allocation: 1)
        self.kvsnap_pool_release = Function(self.release)

    def close_checked(self, pool):
        if self.fail_close:
            return -1
        self.destroyed = True
        return 0

    def reserve(self, pool, size, ident, pointer):
        C.cast(ident, C.POINTER(C.c_uint64))[0] = 7
        C.cast(pointer, C.POINTER(C.c_void_p))[0] = 128
        return 0

    def release(self, pool, allocation):
        self.released = True
        return 0

    def copy(self, *args):
        self.entered.set()
        if not self.proceed.wait(3):
            raise RuntimeError("copy gate timed out")
        if self.destroyed or self.released:
            raise AssertionError("native lifetime ended during an active copy")
        return 0


def _pool_with(abi):
    with patch("kvsnap_amd.dataplane.C.CDLL", return_value=abi):
        return CudaPool(4096)


@pytest.mark.parametrize("strided,close_pool", [(False, True), (True, False)])
def test_close_waits_for_an_inflight_copy(strided, close_pool):
    abi = BlockingABI()
    pool = _pool_with(abi)
    allocation = pool.reserve(128)
    errors, closed = [], threading.Event()

    def copy():
        try:
            if strided:
                allocation.copy_2d(256, 64, 0, 64, 64, 2, to_host=True)
            else:
                allocation.copy(256, 128, to_host=True)
        except BaseException as exc:
            errors.append(exc)

    def close():
        try:
            (pool.close if close_pool else allocation.close)()
        except BaseException as exc:
            errors.append(exc)
        finally:
            closed.set()

    copier, closer = threading.Thread(target=copy), threading.Thread(target=close)
    copier.start()
    assert abi.entered.wait(2)
    closer.start()
    try:
        assert not closed.wait(0.05), "close returned while a copy still borrowed the pool"
    finally:
        abi.proceed.set()
        copier.join(2)
        closer.join(2)
        pool.close()
    assert errors == []


def test_failed_wait_and_release_keep_owners_alive():
    abi = BlockingABI()
    pool = _pool_with(abi)
    allocation = pool.reserve(128)
    tensor = type("Storage", (), {})()
    allocation._tensor_references = [tensor]
    allocation_ref, tensor_ref = weakref.ref(allocation), weakref.ref(tensor)
    abi.kvsnap_pool_wait = Function(lambda pool, allocation: -1)
    abi.kvsnap_pool_release = Function(lambda pool, allocation: -1)
    with pytest.raises(RuntimeError):
        allocation.wait()
    with pytest.raises(RuntimeError):
        allocation.close()
    del allocation, tensor
    gc.collect()
    try:
        assert allocation_ref() is not None and tensor_ref() is not None
        abi.kvsnap_pool_release = Function(abi.release)
        allocation_ref().close()
        gc.collect()
        assert tensor_ref() is None and allocation_ref() is None
    finally:
        pool.close()


def test_failed_pool_close_keeps_handle_and_references_for_retry():
    abi = BlockingABI()
    pool = _pool_with(abi)
    allocation = pool.reserve(128)
    marker = object()
    allocation._tensor_references = [marker]
    abi.fail_close = True
    with pytest.raises(RuntimeError):
        pool.close()
    assert pool.handle == 101 and not abi.destroyed and allocation._tensor_references == [marker]
    abi.fail_close = False
    pool.close()
    assert pool.handle is None


def test_incompatible_abi_is_rejected_before_a_pool_is_created():
    abi = BlockingABI()
    abi.kvsnap_pool_abi_version = Function(lambda: 1)
    created = []
    abi.kvsnap_pool_create = Function(lambda *a: created.append(a) or 101)
    with pytest.raises(RuntimeError, match="unsupported.*ABI"):
        _pool_with(abi)
    assert created == []


def test_pools_refuse_use_after_fork():
    abi = BlockingABI()
    pool = _pool_with(abi)
    pool._pid = -1
    with pytest.raises(RuntimeError, match="fork"):
        pool.reserve(1)
    with pytest.raises(RuntimeError, match="fork"):
        pool.close()
    pool._pid = os.getpid()
    pool.close()


def test_capacity_message_maps_to_pinned_capacity_error():
    abi = BlockingABI()
    abi.kvsnap_pool_reserve = Function(lambda *a: -1)
    abi.kvsnap_cuda_error = Function(lambda: b"pinned capacity exhausted")
    pool = _pool_with(abi)
    with pytest.raises(PinnedCapacityError):
        pool.reserve(1)
    abi.kvsnap_cuda_error = Function(lambda: b"other failure")
    with pytest.raises(RuntimeError, match="other failure"):
        pool.reserve(1)
    pool.close()
