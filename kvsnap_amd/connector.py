"""The vLLM connector class for this data plane: ``KVConnectorBase_V1``, worker role.

vLLM builds it from its KV-transfer config (``kv_connector = "KvsnapConnector"``,
``kv_connector_module_path = "kvsnap_amd.connector"``), as it builds the
reference's ``KvsnapConnector`` (reference ``kvsnap/connector/vllm.py:134-143``).
On the worker every hook is :class:`kvsnap_amd.worker.KvsnapWorker`'s, with
the reference's names and arguments (``vllm.py:436-699``): registration,
``bind_connector_metadata`` / ``clear_connector_metadata``, ``start_load_kv``,
``wait_for_layer_load``, ``save_kv_layer``, ``wait_for_save``,
``get_finished``, ``build_connector_worker_meta``,
``get_block_ids_with_load_errors`` and ``shutdown``.

The scheduler role (snapshot store, manifests, leases, prefix matching) is
control plane and is not implemented here: constructing the connector for
it raises, and its hooks raise ``NotImplementedError``.  The scheduler hands
the worker :class:`KvsnapConnectorMetadata` (the step's load and save
:class:`~kvsnap_amd.worker.Transfer` lists) and reads back
:class:`KvsnapConnectorWorkerMetadata`.

``kv_connector_extra_config`` keys (the reference's where they mean the same):

================================  ==============================================================
``store_path``                    root of the blob directory (durable snapshots), if any
``pinned_pool_bytes``             the pinned pool's capacity (default 24 GiB)
``host_tier_bytes``               host-tier share of the pool (default three quarters of it)
``async_load``                    loads on the loader thread (default true)
``verify``                        "gpu" (default), "host" or "none": where block CRC32Cs are checked;
                                  ``verify_host_checksums: true`` (the reference's key) means "host"
``device_staging_bytes``          device memory the plane reserves at registration for restores
``restore_mode``                  "dma" (copy engines, default) or "kernel" (in-place restore kernel)
================================  ==============================================================
"""
from __future__ import annotations

from dataclasses import dataclass

from vllm.distributed.kv_transfer.kv_connector.v1.base import (
    KVConnectorBase_V1, KVConnectorMetadata, KVConnectorRole, KVConnectorWorkerMetadata,
)

from .worker import KvsnapMetadata, KvsnapWorker, KvsnapWorkerMetadata


@dataclass
class KvsnapConnectorMetadata(KvsnapMetadata, KVConnectorMetadata):
    """One step's loads and saves (lists of :class:`kvsnap_amd.worker.Transfer`), as vLLM passes them."""


@dataclass
class KvsnapConnectorWorkerMetadata(KvsnapWorkerMetadata, KVConnectorWorkerMetadata):
    """One step's report from a worker: prepared snapshots, save errors, failed and finished loads."""


def _setting(extra, key, default, kind):
    value = extra.get(key, default)
    if kind is bool:
        if isinstance(value, str):
            value = value.strip().lower() in ("1", "true", "yes", "on")
        return bool(value)
    return kind(value)


class KvsnapConnector(KVConnectorBase_V1):
    """vLLM's KV connector over :class:`KvsnapWorker` (the worker role)."""

    def __init__(self, vllm_config, role, kv_cache_config=None):
        if role != KVConnectorRole.WORKER:
            raise NotImplementedError("kvsnap_amd provides the connector's worker role only: the scheduler side "
                                      "(snapshot store, manifests, leases) is not part of it")
        parallel = vllm_config.parallel_config
        if getattr(parallel, "pipeline_parallel_size", 1) != 1 or getattr(parallel, "data_parallel_size", 1) != 1:
            raise ValueError("kvsnap supports tensor parallelism only: pipeline and data parallel sizes must be 1")
        if kv_cache_config is not None and len(kv_cache_config.kv_cache_groups) != 1:
            raise ValueError("kvsnap requires one full-attention KV group")
        if getattr(vllm_config, "speculative_config", None):
            raise ValueError("speculative decoding is unsupported")
        if getattr(vllm_config.scheduler_config, "async_scheduling", False):
            raise ValueError("kvsnap requires synchronous scheduling: request_finished must see settled tokens")
        super().__init__(vllm_config, role, kv_cache_config)
        extra = dict(vllm_config.kv_transfer_config.kv_connector_extra_config or {})
        capacity = _setting(extra, "pinned_pool_bytes", 24 << 30, int)
        verify = "host" if _setting(extra, "verify_host_checksums", False, bool) else extra.get("verify", "gpu")
        options = {}
        if "device_staging_bytes" in extra:
            options["device_staging_bytes"] = _setting(extra, "device_staging_bytes", 0, int)
        if "restore_mode" in extra:
            options["restore_mode"] = str(extra["restore_mode"])
        blobs = None
        if extra.get("store_path"):
            from .blobs import BlobDirectory
            blobs = BlobDirectory(extra["store_path"])
        self.worker = KvsnapWorker(blobs=blobs, async_load=_setting(extra, "async_load", True, bool),
                                   verify=verify, block_size=vllm_config.cache_config.block_size,
                                   capacity_bytes=capacity,
                                   host_tier_bytes=_setting(extra, "host_tier_bytes", capacity * 3 // 4, int),
                                   plane_options=options)

    # ---- worker hooks (reference vllm.py:436-699) ------------------------------

    def register_kv_caches(self, kv_caches):
        """Build, warm up and register the data plane over vLLM's caches; returns the layout identity."""
        return self.worker.register_kv_caches(kv_caches)

    def bind_connector_metadata(self, connector_metadata):
        super().bind_connector_metadata(connector_metadata)
        self.worker.bind_connector_metadata(connector_metadata)

    def clear_connector_metadata(self):
        parent = getattr(super(), "clear_connector_metadata", None)
        if parent is not None:
            parent()
        self.worker.clear_connector_metadata()

    def start_load_kv(self, forward_context, **kwargs):
        self.worker.start_load_kv(forward_context, **kwargs)

    def wait_for_layer_load(self, layer_name):
        self.worker.wait_for_layer_load(layer_name)

    def save_kv_layer(self, layer_name, kv_layer, attn_metadata, **kwargs):
        self.worker.save_kv_layer(layer_name, kv_layer, attn_metadata, **kwargs)

    def wait_for_save(self):
        self.worker.wait_for_save()

    def get_finished(self, finished_req_ids):
        return self.worker.get_finished(finished_req_ids)

    def build_connector_worker_meta(self):
        report = self.worker.build_connector_worker_meta()
        return KvsnapConnectorWorkerMetadata(**vars(report))

    def get_block_ids_with_load_errors(self):
        return self.worker.get_block_ids_with_load_errors()

    def shutdown(self):
        """Finish the loads and saves in flight, then close the data plane."""
        self.worker.shutdown()
        if self.worker.dataplane is not None:
            self.worker.dataplane.close()

    # ---- scheduler hooks: not implemented here ---------------------------------

    def _scheduler_only(self, *args, **kwargs):
        raise NotImplementedError("the connector's scheduler side is not implemented in kvsnap_amd")

    get_num_new_matched_tokens = _scheduler_only
    update_state_after_alloc = _scheduler_only
    build_connector_meta = _scheduler_only
    request_finished = _scheduler_only


__all__ = ["KvsnapConnector", "KvsnapConnectorMetadata", "KvsnapConnectorWorkerMetadata"]
