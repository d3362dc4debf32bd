"""Wall-clock checks, collected after every parity test so that a slow poll on a loaded machine cannot stop
the parity suite under ``pytest -x``."""
import pytest

pytest.importorskip("torch")

from test_gpu_parity import early_report_scenario

pytestmark = pytest.mark.gpu


def test_progress_polls_never_wait_for_the_copy_they_describe(planes):
    """While a loader thread waits on its restore, the engine's progress polls answer at once: a query of the
    event that thread synchronized on used to be held until the whole 21 ms restore was over (HIP), so no load
    was ever reported early.  Every poll must take under 5 ms."""
    slowest = early_report_scenario(planes)
    assert slowest < 0.005, slowest
