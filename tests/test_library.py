"""The C-ABI libraries load without a GPU and export every symbol include/*.h declares."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HIP_LIBRARY = ROOT / "kvsnap_amd" / "_native" / "libkvsnap_hip.so"
IO_LIBRARY = ROOT / "kvsnap_amd" / "_native" / "libkvsnap_io.so"
LIBRARIES = {"kvsnap_pool.h": HIP_LIBRARY, "kvsnap_kernels.h": HIP_LIBRARY, "kvsnap_io.h": IO_LIBRARY}


def declared(header):
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / header).read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(kvsnap_\w+)\s*\(", text)))


@pytest.fixture(scope="module", autouse=True)
def built():
    if not (HIP_LIBRARY.is_file() and IO_LIBRARY.is_file()):
        from kvsnap_amd import build
        build.build_all()


def test_every_header_declares_something():
    for header in LIBRARIES:
        assert len(declared(header)) >= 3, header


@pytest.mark.parametrize("header", sorted(LIBRARIES))
def test_library_exports_every_declared_symbol(header):
    path = LIBRARIES[header]
    exported = set(subprocess.run(["nm", "-D", "--defined-only", str(path)], check=True, capture_output=True,
                                  text=True).stdout.split())
    missing = [name for name in declared(header) if name not in exported]
    assert not missing, f"{path.name} lacks {missing}"
    lib = C.CDLL(str(path))          # loads without touching a GPU
    for name in declared(header):
        assert getattr(lib, name)


def test_abi_versions_without_a_gpu():
    hip = C.CDLL(str(HIP_LIBRARY))
    assert hip.kvsnap_pool_abi_version() == 2
    assert hip.kvsnap_kernels_abi_version() == 2
    io = C.CDLL(str(IO_LIBRARY))
    assert io.kvsnap_io_abi_version() == 1


def test_library_resolution_needs_no_gpu(monkeypatch):
    from kvsnap_amd.dataplane import resolve_cuda_library
    monkeypatch.delenv("KVSNAP_CUDA_LIBRARY", raising=False)
    monkeypatch.delenv("KVSNAP_HIP_LIBRARY", raising=False)
    assert resolve_cuda_library() == HIP_LIBRARY
    monkeypatch.setenv("KVSNAP_CUDA_LIBRARY", "/tmp/other.so")
    assert str(resolve_cuda_library()) == "/tmp/other.so"
    assert str(resolve_cuda_library("/x/y.so")) == "/x/y.so"


def test_missing_hip_library_fails_loudly(monkeypatch, tmp_path):
    from kvsnap_amd import dataplane
    monkeypatch.setenv("KVSNAP_CUDA_LIBRARY", str(tmp_path / "absent.so"))
    with pytest.raises(RuntimeError, match="not built"):
        dataplane.kernel_library()


def test_the_gather_with_crc32c_takes_whole_kib_records_under_2_gib_only():
    """kvsnap_gather_crc32c_fits (host logic only): whole KiB, more than none, under 2 GiB."""
    hip = C.CDLL(str(HIP_LIBRARY))
    hip.kvsnap_gather_crc32c_fits.argtypes = [C.c_uint64]
    assert [hip.kvsnap_gather_crc32c_fits(n) for n in (1024, 2359296, 294912, (1 << 31) - 1024)] == [1, 1, 1, 1]
    assert [hip.kvsnap_gather_crc32c_fits(n) for n in (0, 16, 1280, 2359296 + 16, 1 << 31, 1 << 40)] == [0] * 6


def test_the_sha_round_probe_refuses_a_bad_count_before_any_gpu_call():
    """kvsnap_sha_round_probe checks its arguments on the host first (no GPU here)."""
    hip = C.CDLL(str(HIP_LIBRARY))
    hip.kvsnap_sha_round_probe.argtypes = [C.c_uint32, C.c_int, C.c_void_p, C.c_size_t]
    hip.kvsnap_cuda_error.restype = C.c_char_p
    for reps in (0, 15, 17, (1 << 24) + 16):
        assert hip.kvsnap_sha_round_probe(0, reps, 8, 0) == -1
        assert b"multiple of 16" in hip.kvsnap_cuda_error()


def test_the_read_probe_refuses_a_bad_buffer_before_any_gpu_call():
    """kvsnap_read_probe checks its arguments on the host first (no GPU here)."""
    hip = C.CDLL(str(HIP_LIBRARY))
    hip.kvsnap_read_probe.argtypes = [C.c_void_p, C.c_uint64, C.c_void_p, C.c_size_t]
    hip.kvsnap_cuda_error.restype = C.c_char_p
    for src, nbytes, sink in ((0, 16, 16), (8, 16, 16), (16, 0, 16), (16, 24, 16), (16, 16, 0), (16, 16, 2)):
        assert hip.kvsnap_read_probe(src, nbytes, sink, 0) == -1
        assert b"read probe" in hip.kvsnap_cuda_error()


def test_the_copy_probe_refuses_a_bad_buffer_before_any_gpu_call():
    """kvsnap_copy_probe checks its arguments on the host first (no GPU here)."""
    hip = C.CDLL(str(HIP_LIBRARY))
    hip.kvsnap_copy_probe.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.c_size_t]
    hip.kvsnap_cuda_error.restype = C.c_char_p
    for src, dst, nbytes in ((0, 16, 16), (16, 0, 16), (8, 16, 16), (16, 24, 16), (16, 16, 0), (16, 32, 40),
                             (16, 32, (1 << 40) + 16)):
        assert hip.kvsnap_copy_probe(src, dst, nbytes, 0) == -1
        assert b"copy probe" in hip.kvsnap_cuda_error()
