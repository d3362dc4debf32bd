"""kvsnap_crc32c_records_noalloc: CRC32C of a batch of records with no allocation at all.

It runs the same kernels as kvsnap_crc32c_records, with the stripes' partial
CRCs in the library's static per-device workspace instead of a caller's
buffer.  Two calls in a row (the second on fewer, shorter records, so stale
partials of the first would show) must give what the workspace entry point
gives, and the oracle's CRC32C; a batch past the static workspace is refused
before anything is launched.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from kvsnap_amd.dataplane import _check, kernel_library

pytestmark = pytest.mark.gpu


def _with_workspace(lib, data, record_bytes, pitch, n, prior, stream):
    out = torch.zeros(n, dtype=torch.int32, device="cuda")
    work_bytes = int(lib.kvsnap_crc32c_workspace_bytes(record_bytes, n))
    work = torch.empty(max(work_bytes, 16), dtype=torch.uint8, device="cuda")
    _check(lib, lib.kvsnap_crc32c_records(data.data_ptr(), record_bytes, pitch, n, prior, out.data_ptr(),
                                          work.data_ptr(), work_bytes, stream))
    torch.cuda.synchronize()
    return out.cpu().numpy().astype(np.uint32)


def test_crc32c_without_allocation_equals_the_workspace_entry_point(hip_library, oracle_lib):
    lib = kernel_library()
    _check(lib, lib.kvsnap_kernels_init(torch.cuda.current_device()))
    stream = torch.cuda.current_stream().cuda_stream
    # Many records combine inside their workgroup and leave the static workspace alone; fewer spread
    # their stripes over the chip and keep them there (the second of those calls on a smaller batch).
    for record_bytes, pitch, n, prior in [(589824, 589824, 512, 0), (589840, 589840, 64, 1),
                                          (70000, 70016, 3, 0xE3069283)]:
        print(f"noalloc crc32c: {n} records of {record_bytes} bytes", flush=True)
        data = torch.randint(0, 256, (n * pitch,), dtype=torch.uint8, device="cuda")
        want = _with_workspace(lib, data, record_bytes, pitch, n, prior, stream)
        out = torch.full((n,), -1, dtype=torch.int32, device="cuda")
        _check(lib, lib.kvsnap_crc32c_records_noalloc(data.data_ptr(), record_bytes, pitch, n, prior,
                                                      out.data_ptr(), stream))
        torch.cuda.synchronize()
        got = out.cpu().numpy().astype(np.uint32)
        assert np.array_equal(got, want), (record_bytes, n)
        host = data.cpu().numpy()
        oracle_crcs = [oracle_lib.crc32c(host[r * pitch:r * pitch + record_bytes].tobytes(), prior) for r in range(n)]
        assert got.tolist() == oracle_crcs, (record_bytes, n)


def test_crc32c_without_allocation_refuses_a_batch_past_its_workspace(hip_library):
    lib = kernel_library()
    _check(lib, lib.kvsnap_kernels_init(torch.cuda.current_device()))
    # Buffers sized for the refused batch, so a regressed guard would still read and write in bounds.
    records = torch.zeros(65537 * 16, dtype=torch.uint8, device="cuda")
    out = torch.zeros(65537, dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="at most 65536 records"):
        _check(lib, lib.kvsnap_crc32c_records_noalloc(records.data_ptr(), 16, 16, 65537, 0, out.data_ptr(),
                                                      torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert not out.any()


FRESH_PROCESS = r"""
import sys
import torch
from kvsnap_amd.dataplane import _check, kernel_library
lib = kernel_library()
records = torch.randint(0, 256, (4 * 1024,), dtype=torch.uint8, device="cuda")
out = torch.full((4,), -1, dtype=torch.int32, device="cuda")
stream = torch.cuda.current_stream().cuda_stream
try:
    _check(lib, lib.kvsnap_crc32c_records_noalloc(records.data_ptr(), 1024, 1024, 4, 0, out.data_ptr(), stream))
except RuntimeError as exc:
    print("refused:", exc, flush=True)
else:
    sys.exit("a call before kvsnap_kernels_init was not refused")
torch.cuda.synchronize()
assert (out == -1).all()
_check(lib, lib.kvsnap_kernels_init(torch.cuda.current_device()))
_check(lib, lib.kvsnap_crc32c_records_noalloc(records.data_ptr(), 1024, 1024, 4, 0, out.data_ptr(), stream))
want = torch.zeros(4, dtype=torch.int32, device="cuda")
work_bytes = int(lib.kvsnap_crc32c_workspace_bytes(1024, 4))
work = torch.empty(max(work_bytes, 16), dtype=torch.uint8, device="cuda")
_check(lib, lib.kvsnap_crc32c_records(records.data_ptr(), 1024, 1024, 4, 0, want.data_ptr(), work.data_ptr(),
                                      work_bytes, stream))
torch.cuda.synchronize()
assert torch.equal(out, want), (out, want)
print("ok", flush=True)
"""


def test_crc32c_without_allocation_needs_the_explicit_init_and_makes_no_synchronous_call(hip_library):
    """In a fresh process no entry point has set the device up: the no-allocation call is refused (nothing
    queued, no table upload of its own), and after kvsnap_kernels_init it gives the workspace entry point's
    CRC32Cs."""
    import os
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    env = dict(os.environ, PYTHONPATH=str(root) + os.pathsep + os.environ.get("PYTHONPATH", ""))
    done = subprocess.run([sys.executable, "-c", FRESH_PROCESS], capture_output=True, text=True, timeout=300,
                          cwd=root, env=env)
    assert done.returncode == 0, done.stdout + done.stderr
    assert "refused: CRC32C without allocation: call kvsnap_kernels_init" in done.stdout
    assert done.stdout.rstrip().endswith("ok")
