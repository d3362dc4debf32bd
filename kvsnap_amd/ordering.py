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
    """Bytes of a load not yet known complete, or None while launches are still being queued.

    The launches run in order on one stream, so their events complete in
    order: the answer is the ``left`` of the last entry known complete,
    found by bisection over the events (the first entry, ``(None, total)``,
    counts as complete).
    """
    if not progress or progress[-1][1] != 0:
        return None                   # the last launch, which leaves nothing, is not queued yet
    known, unknown = 0, len(progress)  # entries before ``unknown`` may be complete; ``known`` is
    while unknown - known > 1:
        middle = (known + unknown) // 2
        event = progress[middle][0]
        if event is None or event.query():
            known = middle
        else:
            unknown = middle
    return progress[known][1]


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
