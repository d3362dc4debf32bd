"""The plane's per-kernel timer: it times the launches a save and a restore make, and only the named ones."""
import pytest

torch = pytest.importorskip("torch")

from kvsnap_amd.dataplane import KernelTimer
from test_gpu_parity import BLOCK_SIZE, BLOCKS, LAYERS, vllm_caches

pytestmark = pytest.mark.gpu


def test_a_kernel_timer_times_the_plane_s_launches_and_only_the_named_ones(planes):
    backing, caches = vllm_caches(LAYERS, BLOCKS)
    plane = planes(caches, restore_mode="kernel")
    size, n = plane.block_bytes, 8
    staging = plane.pool.reserve(size * n)
    targets = [(staging, i * size) for i in range(n)]

    def step(timer):
        plane.timer = timer
        plane.save_gather(list(range(1, 1 + n)), targets, n * BLOCK_SIZE)
        plane.load_scatter(list(range(40, 40 + n)), targets)
        torch.cuda.synchronize()
        return timer.summary()

    try:
        everything = step(KernelTimer())
        assert "restore" in everything and len(everything) >= 2, everything
        for name, record in everything.items():
            assert record["launches"] >= 1 and record["total_ms"] > 0, (name, record)
            assert record["avg_ms"] == pytest.approx(record["total_ms"] / record["launches"])
        saved = next(name for name in everything if name != "restore")
        for wanted in ({"restore"}, {saved}):
            timer = KernelTimer(wanted)
            summary = step(timer)
            assert set(summary) == wanted, summary
            assert summary[next(iter(wanted))]["launches"] == everything[next(iter(wanted))]["launches"]
            timer.reset()
            assert timer.summary() == {}
        torch.cuda.synchronize()
        restored = backing[:, 40:40 + n].view(torch.int16)
        assert torch.equal(restored, backing[:, 1:1 + n].view(torch.int16))
    finally:
        plane.timer = None
        staging.close()
