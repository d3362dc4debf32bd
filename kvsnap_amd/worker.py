"""The connector's worker side over this data plane: loads, saves and what each step reports.

A ROCm vLLM's ``KVConnectorBase_V1`` connector delegates its worker hooks to
:class:`KvsnapWorker`, which keeps the reference connector's hook names,
threads and rules (``kvsnap/connector/vllm.py:226-240, 454-691``):

* ``register_kv_caches`` builds the data plane over vLLM's caches, warms it
  up and publishes the layout identity (``kv_layout``) every snapshot made
  here records.
* ``bind_connector_metadata`` / ``clear_connector_metadata``: the step's
  loads and saves.  The next forward waits, on the GPU, for the copies of
  loads that were reported early; with asynchronous loads the point "work
  queued before this forward" is recorded for this step's loads.
* ``start_load_kv(forward_context)``: each load waits for that point (or,
  synchronous, for everything queued so far) and runs on the one loader
  thread, filling a ``progress`` list as its launches are queued.  Before any
  copy, a snapshot taken under another KV layout, a block no longer held, or
  a corrupt block makes the load fail: vLLM recomputes its blocks.  A copy
  failure is :class:`DMAUnknown`, which stops the engine.  With
  ``verify="gpu"`` every block's CRC32C is checked on the GPU (a volatile
  block's as the restore kernel copies it, a durable block's before it
  reaches the cache); a mismatch found by the copy also fails the load.
* ``wait_for_save``: saves run on two threads after this step's kernels;
  ``fenced`` is set once the device-to-host copy has landed and the GPU
  blocks may be freed, before the digests and the host-tier adoption or blob
  writes finish.
* ``get_finished``: saves whose blocks are fenced, of requests vLLM has
  finished, are reported sending.  A load is reported receiving when it is
  done, or early once every launch is queued and at most
  ``early_report_bytes`` (128 MiB) of its copy is not known complete; its
  event then joins the next forward's waits.  A load that fails after an
  early report stops the engine.

Scheduler metadata are plain :class:`KvsnapMetadata` / :class:`Transfer`
records here.  The manifests, SQLite store, leases, gateway, telemetry,
tensor-parallel shards and cross-process host-tier reads of the reference
are control plane and are not mirrored.
"""
from __future__ import annotations

from concurrent.futures import Future, ThreadPoolExecutor
from dataclasses import dataclass, field
import threading

from .blobs import CorruptSnapshotError
from .dataplane import CopyFailed, StagingUnavailable
from .layout import LayoutMismatch, require_layout
from .native_io import get_io_backend
from .ordering import EARLY_REPORT_BYTES, early_report


class DMAUnknown(RuntimeError):
    """A copy's completion could not be proven; the engine must stop (reference ``vllm.py`` ``DMAUnknown``)."""


class LoadRefused(RuntimeError):
    """A load cannot run (the scheduler's error, another KV layout, a missing tier); nothing was copied."""


@dataclass
class Transfer:
    """One request's load or save, as the scheduler hands it to the worker.

    ``snapshot`` is a host-tier snapshot (``durability="volatile"``) or a blob
    snapshot (``"durable"``) for a load; for a save, ``previous`` may name the
    session's last snapshot, so only the blocks past its unchanged prefix are
    gathered and hashed.  ``skip_blocks`` leading blocks of a load are already
    in the cache (prefix caching) and are not copied.
    """
    request_id: str
    block_ids: list
    snapshot: dict | None = None
    durability: str = "volatile"
    num_kv_tokens: int = 0
    skip_blocks: int = 0
    previous: dict | None = None
    error: str | None = None


@dataclass
class KvsnapMetadata:
    """What one engine step asks of the worker (the reference's ``KvsnapMetadata``)."""
    loads: list = field(default_factory=list)
    saves: list = field(default_factory=list)


@dataclass
class KvsnapWorkerMetadata:
    """What the worker reports back to the scheduler after a step (the reference's worker metadata)."""
    prepared: dict = field(default_factory=dict)           # request id -> saved snapshot
    errors: dict = field(default_factory=dict)             # request id -> why its save failed
    failed_loads: list = field(default_factory=list)       # requests whose blocks must be recomputed
    invalid_snapshots: list = field(default_factory=list)  # request ids whose snapshot was corrupt
    loaded: list = field(default_factory=list)             # requests whose load is over


def _in_chain(exc, kind):
    """Whether ``exc``, or an exception it was raised from or while handling, is a ``kind``."""
    visited = set()
    while exc is not None and id(exc) not in visited:
        if isinstance(exc, kind):
            return True
        visited.add(id(exc))
        exc = exc.__cause__ if exc.__cause__ is not None else exc.__context__
    return False


def _run_now(fn, *args):
    """``fn(*args)`` run on this thread, its outcome wrapped as a finished future."""
    outcome = Future()
    try:
        value = fn(*args)
    except BaseException as exc:
        outcome.set_exception(exc)
    else:
        outcome.set_result(value)
    return outcome


class _SaveJob:
    """A save in flight: its future, the fence that frees its GPU blocks, and what has been reported."""

    __slots__ = ("future", "fenced", "vllm_finished", "sent", "booked")

    def __init__(self, future, fenced):
        self.future, self.fenced = future, fenced
        self.vllm_finished = self.sent = self.booked = False


class _LoadJob:
    """A load in flight: its future, its transfer, the progress its launches fill, and an early report."""

    __slots__ = ("future", "transfer", "progress", "reported")

    def __init__(self, future, transfer, progress):
        self.future, self.transfer, self.progress, self.reported = future, transfer, progress, False


class KvsnapWorker:
    """Worker-side connector hooks over a :class:`kvsnap_amd.dataplane.TorchBlockDataPlane`.

    Pass a registered ``dataplane``, or leave it out and call
    :meth:`register_kv_caches` (with ``block_size`` and ``capacity_bytes``
    given here) as vLLM does.  With ``host_tier_bytes`` a host tier is made
    over the plane at registration.
    """

    def __init__(self, dataplane=None, *, host_tier=None, blobs=None, async_load=True, save_threads=2,
                 verify="gpu", early_report_bytes=EARLY_REPORT_BYTES, block_size=16, capacity_bytes=24 << 30,
                 host_tier_bytes=None, plane_options=None):
        if verify not in ("gpu", "host", "none"):
            raise ValueError("verify must be gpu, host or none")
        self.host_tier, self.blobs = host_tier, blobs
        self.async_load, self.verify, self.early_report_bytes = async_load, verify, early_report_bytes
        self.block_size, self.capacity_bytes = block_size, capacity_bytes
        self.host_tier_bytes, self.plane_options = host_tier_bytes, dict(plane_options or {})
        self.dataplane, self.kv_layout = None, None
        if dataplane is not None:
            self._adopt_plane(dataplane)
        self.loader = ThreadPoolExecutor(max_workers=1, thread_name_prefix="kvsnap-load")
        self.executor = ThreadPoolExecutor(max_workers=save_threads, thread_name_prefix="kvsnap-save")
        self._metadata = KvsnapMetadata()
        self._loads = {}             # request id -> _LoadJob
        self._saves = {}             # request id -> _SaveJob
        self.forward_waits = []      # events the next forward waits on
        self.load_errors = set()
        self.worker_meta = KvsnapWorkerMetadata()
        self._queued_before_forward = None

    # ---- registration --------------------------------------------------------

    def _adopt_plane(self, plane):
        self.dataplane = plane
        self.kv_layout = plane.layout_identity

    def register_kv_caches(self, kv_caches):
        """Register vLLM's KV caches: build the plane, warm it up, publish the layout (``vllm.py:226-240``)."""
        from .dataplane import TorchBlockDataPlane
        if self.dataplane is not None:
            raise RuntimeError("KV caches are already registered")
        plane = TorchBlockDataPlane(kv_caches, self.block_size, self.capacity_bytes, **self.plane_options)
        plane.warm_up()              # kernels loaded, tables built and streams picked now, not on the first load
        self._adopt_plane(plane)
        if self.host_tier is None and self.host_tier_bytes:
            from .host_tier import HostTier
            self.host_tier = HostTier(plane, self.host_tier_bytes)
        return self.kv_layout

    # ---- step boundary -------------------------------------------------------

    def bind_connector_metadata(self, connector_metadata):
        """Take this step's metadata, before its forward (reference ``vllm.py:454-467``)."""
        self._metadata = connector_metadata
        waits, self.forward_waits = self.forward_waits, []
        for event in waits:                          # loads reported early may run in this forward
            self.dataplane.wait_on_engine_stream(event)
        # With every load asynchronous vLLM calls start_load_kv after the forward, and a load's blocks belong
        # to a request this forward does not run: the load waits only for the work queued before it.
        has_loads = bool(getattr(connector_metadata, "loads", None))
        self._queued_before_forward = self.dataplane.producer_event() if self.async_load and has_loads else None

    def clear_connector_metadata(self):
        """Drop this step's metadata once the step is over (``KVConnectorBase_V1``)."""
        self._metadata = KvsnapMetadata()

    # ---- loads ---------------------------------------------------------------

    def start_load_kv(self, forward_context=None, **kwargs):
        """Start this step's loads (reference ``vllm.py:469-481``)."""
        transfers = list(self._metadata.loads)
        if not transfers:
            return
        after = self._queued_before_forward or self.dataplane.producer_event()
        self._queued_before_forward = None
        for transfer in transfers:
            if not self.async_load:
                self._book_load(transfer, _run_now(self._load, transfer, after))
                continue
            progress = []
            future = self.loader.submit(self._load, transfer, after, progress)
            self._loads[transfer.request_id] = _LoadJob(future, transfer, progress)

    def _refuse_early(self, transfer):
        """Every reason to refuse a load that needs no copy to find: raised before anything moves."""
        if transfer.error:
            raise LoadRefused(transfer.error)
        if transfer.snapshot is None:
            raise LoadRefused("the load names no snapshot")
        try:
            require_layout(transfer.snapshot, self.kv_layout)
        except LayoutMismatch as exc:
            raise LoadRefused(str(exc)) from exc
        wanted = len(transfer.block_ids) - transfer.skip_blocks
        have = len(transfer.snapshot["segments"]) - transfer.skip_blocks
        if have != wanted:
            raise LoadRefused(f"the snapshot has {have} blocks for {wanted} targets")
        tier = self.host_tier if transfer.durability == "volatile" else self.blobs
        if tier is None:
            raise LoadRefused(f"no {'host tier' if transfer.durability == 'volatile' else 'blob directory'} "
                              f"for a {transfer.durability} snapshot")

    def _load(self, transfer, after, progress=None):
        """Copy one snapshot into its blocks; returns the launch count."""
        self._refuse_early(transfer)
        skip = transfer.skip_blocks
        targets, segments = list(transfer.block_ids[skip:]), transfer.snapshot["segments"][skip:]
        plane, crcs = self.dataplane, [segment["crc32c"] for segment in segments]
        if transfer.durability != "volatile":
            after.synchronize()
            try:
                return plane.load_from_disk(targets, self.blobs, segments, first_block=skip, progress=progress,
                                            verify="host" if self.verify == "host" else "gpu")
            except CorruptSnapshotError:
                raise      # found before that chunk's copy, after the earlier ones completed: a recompute miss
            except StagingUnavailable as exc:
                raise LoadRefused(f"no device staging for the load: {exc}") from exc     # before any copy
            except Exception as exc:
                raise DMAUnknown("kvsnap H2D completion could not be proven") from exc
        with self.host_tier.borrow(segments, transfer.snapshot["locations"]) as sources:
            if self.verify == "host":       # the reference's verify_host_checksums (volatile.py:302-305)
                io = get_io_backend()
                for (allocation, offset), segment in zip(sources, segments):
                    if io.crc32c_at(allocation.pointer + offset, segment["length"]) != segment["crc32c"]:
                        raise CorruptSnapshotError("host-tier block checksum mismatch")
            after.synchronize()
            try:
                if self.verify == "gpu":
                    return plane.load_scatter_checked(targets, sources, crcs, progress=progress)
                return plane.load_scatter(targets, sources, progress=progress)
            except CorruptSnapshotError:
                raise      # a block failed the checked copy's CRC32C: none of them counts as loaded
            except StagingUnavailable as exc:
                raise LoadRefused(f"no device staging for the load: {exc}") from exc     # before any copy
            except Exception as exc:
                raise DMAUnknown("kvsnap H2D completion could not be proven") from exc

    def _book_load(self, transfer, outcome):
        """Record a load that is over (reference ``vllm.py:536-549``); DMAUnknown propagates."""
        error = outcome.exception()
        if isinstance(error, DMAUnknown):
            raise error
        if error is not None:
            # The request's blocks hold nothing it may use: vLLM recomputes them.
            self.load_errors.update(transfer.block_ids[transfer.skip_blocks:])
            self.worker_meta.failed_loads.append(transfer.request_id)
            if isinstance(error, CorruptSnapshotError):
                self.worker_meta.invalid_snapshots.append(transfer.request_id)
        self.worker_meta.loaded.append(transfer.request_id)

    def wait_for_layer_load(self, layer_name):
        """Loads are over before vLLM schedules their request, so no layer waits."""

    def save_kv_layer(self, layer_name, kv_layer, attn_metadata, **kwargs):
        """Saves take the finished request's blocks at the step boundary, not layer by layer."""

    # ---- saves ---------------------------------------------------------------

    def wait_for_save(self):
        """Hand this step's saves to the save threads (reference ``vllm.py:561-570``)."""
        transfers = list(self._metadata.saves)
        if not transfers:
            return
        after = self.dataplane.producer_event()      # this step's kernels wrote the last KV
        for transfer in transfers:
            fenced = threading.Event()
            future = self.executor.submit(self._save, transfer, after, fenced)
            self._saves[transfer.request_id] = _SaveJob(future, fenced)

    def _save(self, transfer, after, fenced):
        """Land one turn in pinned memory, then hash and keep it; ``fenced`` frees the GPU blocks."""
        try:
            after.synchronize()
            if transfer.durability == "volatile":
                if self.host_tier is None:
                    raise ValueError("no host tier for a volatile save")
                return self.host_tier.save(transfer.block_ids, transfer.num_kv_tokens,
                                           previous=transfer.previous, fenced=fenced)
            if self.blobs is None:
                raise ValueError("no blob directory for a durable save")
            return self.blobs.save(self.dataplane, transfer.block_ids, transfer.num_kv_tokens,
                                   previous=transfer.previous, fenced=fenced)
        except BaseException as exc:
            if _in_chain(exc, CopyFailed):
                # The copy may still use the GPU blocks and the pinned memory: fenced stays unset.  (Releasing
                # a staging buffer whose copy is unproven raises again on the way out, so the copy failure
                # can be the context of the exception that arrives here.)
                raise DMAUnknown("kvsnap D2H completion could not be proven") from exc
            fenced.set()    # failed before the copy started, or after it landed: the blocks may go
            raise

    # ---- step report ---------------------------------------------------------

    def _sending(self, finished_req_ids):
        """Saves to report sending: fenced, of requests vLLM has finished.  Finished saves are booked."""
        for request_id in finished_req_ids:
            job = self._saves.get(request_id)
            if job is not None:
                job.vllm_finished = True
        sending = set()
        for request_id, job in list(self._saves.items()):
            over = job.future.done()          # read before the fence: a finished job has set it or raised
            if not job.sent and job.vllm_finished and job.fenced.is_set():
                job.sent = True
                sending.add(request_id)
            if over and not job.booked:
                job.booked = True
                error = job.future.exception()
                if isinstance(error, DMAUnknown):
                    raise error
                if error is None:
                    self.worker_meta.prepared[request_id] = job.future.result()
                else:
                    self.worker_meta.errors[request_id] = f"{type(error).__name__}: {error}"
            if job.booked and (job.sent or not job.fenced.is_set()):
                del self._saves[request_id]
        return sending

    def _receiving(self):
        """Loads to report receiving: the finished ones, and those whose copy is far enough along."""
        receiving = set()
        for request_id, job in list(self._loads.items()):
            if job.future.done():
                del self._loads[request_id]
                error = job.future.exception()
                if job.reported and error is not None and not isinstance(error, DMAUnknown):
                    # vLLM may already have run the request on these blocks.
                    raise DMAUnknown("a load failed after it was reported") from error
                self._book_load(job.transfer, job.future)
                if not job.reported:
                    receiving.add(request_id)
            elif not job.reported:
                report = early_report(job.progress, self.early_report_bytes)
                if report is not None:
                    job.reported = True
                    receiving.add(request_id)
                    self.forward_waits.append(report[1])
        return receiving

    def get_finished(self, finished_req_ids):
        """(sending, receiving) request ids for this step (reference ``vllm.py:610-670``)."""
        return self._sending(finished_req_ids), self._receiving()

    def build_connector_worker_meta(self):
        """This step's report to the scheduler; the next step starts a new one."""
        report, self.worker_meta = self.worker_meta, KvsnapWorkerMetadata()
        return report

    def get_block_ids_with_load_errors(self):
        """Blocks whose loads failed since the last call: vLLM recomputes them."""
        blocks, self.load_errors = self.load_errors, set()
        return blocks

    def shutdown(self):
        for pool in (self.loader, self.executor):
            pool.shutdown(wait=True)


__all__ = ["DMAUnknown", "KvsnapMetadata", "KvsnapWorker", "KvsnapWorkerMetadata", "LoadRefused", "Transfer"]
