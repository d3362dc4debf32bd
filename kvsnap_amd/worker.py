"""The connector's worker side over this data plane: loads, saves and what each step reports.

Mirrors the data-plane half of the reference's vLLM connector worker
(``kvsnap/connector/vllm.py:454-687``), with the same method names, threads
and rules, so that a ROCm vLLM's ``KVConnectorBase_V1`` worker can delegate to
it:

* ``bind_connector_metadata`` (``vllm.py:454-467``): the next forward waits, on
  the GPU, for the copies of loads reported early; with asynchronous loads the
  point "work queued before this forward" is recorded for them.
* ``start_load_kv`` (``vllm.py:469-481``): each load waits for that point (or,
  synchronous, for everything queued so far) and then runs on the one loader
  thread, filling a ``progress`` list as its launches are queued.
* ``_load`` (``vllm.py:483-513``): a volatile snapshot's blocks are read in
  place from the host tier (:meth:`kvsnap_amd.host_tier.HostTier.borrow`); a
  durable one's from blob files, pipelined through pinned staging and
  CRC-checked (:meth:`TorchBlockDataPlane.load_from_disk`); with
  ``verify="gpu"`` (default) every block's CRC32C is checked on the GPU (a
  volatile block's as the restore kernel copies it,
  :meth:`TorchBlockDataPlane.load_scatter_checked`; a durable block's before
  it reaches the cache), with ``"host"`` on the host cores.  A failure before
  any copy (the scheduler's error, a block no longer held, a corrupt block),
  or a CRC32C mismatch found by the checked copy, is a failed load whose
  blocks are recomputed; a copy failure is :class:`DMAUnknown`, which stops
  the engine.  A checked load is reported once its check has passed.
* ``wait_for_save`` / ``_save`` (``vllm.py:561-608``): saves run on two threads
  after this step's kernels; ``fenced`` is set once the D2H has landed and
  the GPU blocks may be freed, before the digests and the host-tier adoption
  or blob writes finish.
* ``get_finished`` (``vllm.py:610-670``): finished saves whose blocks are
  fenced are reported sending; a load is reported receiving when it is done,
  or early, once every launch is queued and at most ``early_report_bytes``
  (128 MiB) of its copy is not known complete, its last event then joining
  the next forward's waits.  A load that fails after an early report stops
  the engine.

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
from .dataplane import CopyFailed
from .native_io import get_io_backend
from .ordering import EARLY_REPORT_BYTES, copy_left


class DMAUnknown(RuntimeError):
    """A copy's completion could not be proven; the engine must stop (reference ``vllm.py`` ``DMAUnknown``)."""


class LoadRefused(RuntimeError):
    """The scheduler side could not prepare a load (the transfer's ``error``); nothing was copied."""


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


def _caused_by(exc, kind):
    """Whether ``exc`` or any exception it was raised from or while handling is a ``kind``."""
    seen = set()
    while exc is not None and id(exc) not in seen:
        if isinstance(exc, kind):
            return True
        seen.add(id(exc))
        exc = exc.__cause__ or exc.__context__
    return False


def _completed(fn, *args):
    """Run ``fn`` now; its outcome as a finished future (the synchronous path)."""
    future = Future()
    try:
        future.set_result(fn(*args))
    except BaseException as exc:
        future.set_exception(exc)
    return future


class KvsnapWorker:
    """Worker-side connector hooks over a :class:`kvsnap_amd.dataplane.TorchBlockDataPlane`."""

    def __init__(self, dataplane, *, host_tier=None, blobs=None, async_load=True, save_threads=2,
                 verify="gpu", early_report_bytes=EARLY_REPORT_BYTES):
        if verify not in ("gpu", "host", "none"):
            raise ValueError("verify must be gpu, host or none")
        self.dataplane, self.host_tier, self.blobs = dataplane, host_tier, blobs
        self.async_load, self.verify, self.early_report_bytes = async_load, verify, early_report_bytes
        self.loader = ThreadPoolExecutor(max_workers=1, thread_name_prefix="kvsnap-load")
        self.executor = ThreadPoolExecutor(max_workers=save_threads, thread_name_prefix="kvsnap-save")
        self._metadata = KvsnapMetadata()
        self.load_jobs = {}          # request id -> (future, transfer, progress)
        self.save_jobs = {}          # request id -> (future, fenced)
        self.forward_waits = []      # events the next forward waits on
        self.reported_early = set()
        self.finished = set()        # saves whose GPU blocks are fenced
        self.known_finished = set()  # requests vLLM has finished that have a save
        self.load_errors = set()
        self.worker_meta = KvsnapWorkerMetadata()
        self._queued_before_forward = None

    # ---- step boundary -----------------------------------------------------

    def bind_connector_metadata(self, connector_metadata):
        """Take this step's metadata, before its forward (reference ``vllm.py:454-467``)."""
        self._metadata = connector_metadata
        for event in self.forward_waits:            # loads reported early may run in this forward
            self.dataplane.wait_on_engine_stream(event)
        self.forward_waits = []
        # vLLM calls start_load_kv after the forward when every load is asynchronous; an async load's
        # blocks belong to a request this forward does not run, so it waits only for the work queued
        # before the forward (whatever last used its freshly allocated blocks).
        self._queued_before_forward = (self.dataplane.producer_event()
                                       if self.async_load and connector_metadata.loads else None)

    # ---- loads -------------------------------------------------------------

    def start_load_kv(self, forward_context=None, **kwargs):
        """Start this step's loads (reference ``vllm.py:469-481``)."""
        loads = self._metadata.loads
        if not loads:
            return
        ready = self._queued_before_forward or self.dataplane.producer_event()
        self._queued_before_forward = None
        for transfer in loads:
            if self.async_load:
                progress = []
                future = self.loader.submit(self._load, transfer, ready, progress)
                self.load_jobs[transfer.request_id] = (future, transfer, progress)
            else:
                self._finish_load(transfer, _completed(self._load, transfer, ready))

    def _load(self, transfer, ready, progress=None):
        """Copy one snapshot into its blocks; returns the launch count."""
        if transfer.error:
            raise LoadRefused(transfer.error)
        first = transfer.skip_blocks
        targets = list(transfer.block_ids[first:])
        segments = transfer.snapshot["segments"][first:]
        if len(segments) != len(targets):
            raise LoadRefused(f"snapshot has {len(segments)} blocks for {len(targets)} targets")
        plane = self.dataplane
        if transfer.durability == "volatile":
            if self.host_tier is None:
                raise LoadRefused("no host tier for a volatile snapshot")
            with self.host_tier.borrow(segments, transfer.snapshot["locations"]) as sources:
                if self.verify == "host":       # the reference's verify_host_checksums (volatile.py:302-305)
                    io = get_io_backend()
                    for (allocation, offset), segment in zip(sources, segments):
                        if io.crc32c_at(allocation.pointer + offset, segment["length"]) != segment["crc32c"]:
                            raise CorruptSnapshotError("host-tier block checksum mismatch")
                ready.synchronize()
                try:
                    if self.verify == "gpu":
                        return plane.load_scatter_checked(targets, sources, [s["crc32c"] for s in segments],
                                                          progress=progress)
                    return plane.load_scatter(targets, sources, progress=progress)
                except CorruptSnapshotError:
                    raise               # a block failed its CRC32C; none of them is reported loaded
                except Exception as exc:
                    raise DMAUnknown("kvsnap H2D completion could not be proven") from exc
        if self.blobs is None:
            raise LoadRefused("no blob directory for a durable snapshot")
        ready.synchronize()
        try:
            return plane.load_from_disk(targets, self.blobs, segments, first_block=first, progress=progress,
                                        verify="host" if self.verify == "host" else "gpu")
        except CorruptSnapshotError:
            raise                       # raised after every earlier copy completed; the blocks are recomputed
        except Exception as exc:
            raise DMAUnknown("kvsnap H2D completion could not be proven") from exc

    def _finish_load(self, transfer, future):
        """Book a load that is over (reference ``vllm.py:536-549``)."""
        try:
            future.result()
        except DMAUnknown:
            raise
        except Exception as exc:
            # Nothing the request runs on reached the GPU: vLLM recomputes these blocks.
            self.load_errors.update(transfer.block_ids[transfer.skip_blocks:])
            self.worker_meta.failed_loads.append(transfer.request_id)
            if isinstance(exc, CorruptSnapshotError):
                self.worker_meta.invalid_snapshots.append(transfer.request_id)
        self.worker_meta.loaded.append(transfer.request_id)

    def wait_for_layer_load(self, layer_name):
        """Loads are over before vLLM schedules their request, so no layer waits."""

    def save_kv_layer(self, layer_name, kv_layer, attn_metadata, **kwargs):
        """Saves take the finished request's blocks at the step boundary, not layer by layer."""

    # ---- saves -------------------------------------------------------------

    def wait_for_save(self):
        """Hand this step's saves to the save threads (reference ``vllm.py:561-570``)."""
        saves = self._metadata.saves
        if not saves:
            return
        ready = self.dataplane.producer_event()      # this step's kernels wrote the last KV
        for transfer in saves:
            fenced = threading.Event()
            self.save_jobs[transfer.request_id] = (self.executor.submit(self._save, transfer, ready, fenced),
                                                   fenced)

    def _save(self, transfer, ready, fenced):
        """Land one turn in pinned memory, then hash and keep it; ``fenced`` frees the GPU blocks."""
        try:
            ready.synchronize()
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
            if _caused_by(exc, CopyFailed):
                # The DMA may still use the GPU blocks and the pinned memory: fenced stays unset.  (A
                # staging buffer released while its copy is unproven raises again on the way out, so
                # the copy failure can be the context of the exception that arrives here.)
                raise DMAUnknown("kvsnap D2H completion could not be proven") from exc
            fenced.set()    # failed before the copy started (or after it landed): the blocks may go
            raise

    # ---- step report -------------------------------------------------------

    def get_finished(self, finished_req_ids):
        """(sending, receiving) request ids for this step (reference ``vllm.py:610-670``)."""
        self.known_finished.update(r for r in finished_req_ids if r in self.save_jobs or r in self.finished)
        for request_id, (future, fenced) in list(self.save_jobs.items()):
            done = future.done()      # read first: a finished job has always set fenced or raised
            if fenced.is_set():
                self.finished.add(request_id)
            if not done:
                continue
            del self.save_jobs[request_id]
            try:
                self.worker_meta.prepared[request_id] = future.result()
            except DMAUnknown:
                raise
            except Exception as exc:
                self.worker_meta.errors[request_id] = f"{type(exc).__name__}: {exc}"
        sending = self.finished & self.known_finished
        self.finished -= sending
        self.known_finished -= sending
        receiving = set()
        for request_id, (future, transfer, progress) in list(self.load_jobs.items()):
            if future.done():
                del self.load_jobs[request_id]
                if request_id in self.reported_early:
                    self.reported_early.discard(request_id)
                    error = future.exception()
                    if error is not None and not isinstance(error, DMAUnknown):
                        # vLLM may already have run the request on these blocks.
                        raise DMAUnknown("a load failed after it was reported") from error
                    self._finish_load(transfer, future)
                    continue
                self._finish_load(transfer, future)
                receiving.add(request_id)
            elif request_id not in self.reported_early:
                left = copy_left(progress)
                if left is not None and left <= self.early_report_bytes:
                    receiving.add(request_id)
                    self.reported_early.add(request_id)
                    self.forward_waits.append(progress[-1][0])
        return sending, receiving

    def build_connector_worker_meta(self):
        result, self.worker_meta = self.worker_meta, KvsnapWorkerMetadata()
        return result

    def get_block_ids_with_load_errors(self):
        result, self.load_errors = self.load_errors, set()
        return result

    def shutdown(self):
        self.loader.shutdown(wait=True)
        self.executor.shutdown(wait=True)


__all__ = ["DMAUnknown", "KvsnapMetadata", "KvsnapWorker", "KvsnapWorkerMetadata", "LoadRefused", "Transfer"]
