"""Restore ordering: when a load may be reported before its copy has finished.

The connector reports an asynchronous load to the engine once every launch is
queued and at most ``EARLY_REPORT_BYTES`` of its copy are not yet known to be
complete; the next forward then waits on the GPU, through
``TorchBlockDataPlane.wait_on_engine_stream``, for the event after which that
much is left (reference ``kvsnap/connector/vllm.py:67, 649-679``).  The
``progress`` list is the one ``load_scatter`` fills: ``(None, total bytes)``
and then, per launch, ``(its completion event, bytes left once it completes)``.
"""
from __future__ import annotations

EARLY_REPORT_BYTES = 128 << 20


def copy_left(progress):
    """Bytes of a load not yet known complete, or None until every launch is queued."""
    if not progress or progress[-1][1]:
        return None
    for event, left in reversed(progress):
        if event is None or event.query():
            return left
    return None


def early_report(progress, limit=EARLY_REPORT_BYTES):
    """(bytes left, event the next forward must wait on) once the load may be reported, else None."""
    left = copy_left(progress)
    if left is None or left > limit:
        return None
    return left, progress[-1][0]


def early_launch_index(progress, limit=EARLY_REPORT_BYTES):
    """Index of the first launch whose completion leaves at most ``limit`` bytes, or None."""
    for index, (event, left) in enumerate(progress[1:]):
        if left <= limit:
            return index
    return None
