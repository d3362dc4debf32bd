import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def _gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def hip_library():
    """The built HIP library; on a machine with a GPU its absence is a failure, not a skip."""
    from kvsnap_amd.dataplane import kernel_library, resolve_cuda_library
    path = resolve_cuda_library()
    assert path.is_file(), f"HIP library not built at {path}"
    return kernel_library()


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    oracle.build()
    return oracle


@pytest.fixture
def planes(hip_library):
    """A maker of warmed-up data planes (block size 16 unless asked), each closed when the test ends."""
    import torch
    from kvsnap_amd.dataplane import TorchBlockDataPlane
    made = []

    def make(caches, block_size=16, capacity=64 << 20, **kwargs):
        plane = TorchBlockDataPlane(caches, block_size, capacity, **kwargs)
        plane.warm_up()
        made.append(plane)
        return plane

    yield make
    torch.cuda.synchronize()
    for plane in made:
        plane.close()
