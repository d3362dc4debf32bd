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
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="at most 65536 records"):
        _check(lib, lib.kvsnap_crc32c_records_noalloc(out.data_ptr(), 16, 16, 65537, 0, out.data_ptr(),
                                                      torch.cuda.current_stream().cuda_stream))
