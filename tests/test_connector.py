"""The vLLM connector class (worker role) on the CPU, imported through stand-in vLLM modules.

vLLM is not installed here; as the reference's connector tests do
(tests/connector/test_failure_policy.py:22-44), the modules the connector
imports are stood in for: ``vllm`` and its ``...kv_connector.v1.base`` with a
``KVConnectorBase_V1`` that keeps the bound metadata, the two metadata base
classes and the role enum.  The data plane and the host tier are stand-ins
too (as in tests/test_worker.py): this checks the class vLLM would build, its
configuration and its delegation of one save and one load through the hooks.
"""
from contextlib import nullcontext
import importlib
import sys
from types import ModuleType, SimpleNamespace
from unittest.mock import MagicMock, patch

import pytest

BASE = "vllm.distributed.kv_transfer.kv_connector.v1.base"


def stand_in_vllm():
    base = ModuleType(BASE)

    class KVConnectorBase_V1:
        def __init__(self, vllm_config, role, kv_cache_config=None):
            self._vllm_config, self._role, self._connector_metadata = vllm_config, role, None

        def bind_connector_metadata(self, connector_metadata):
            self._connector_metadata = connector_metadata

        def clear_connector_metadata(self):
            self._connector_metadata = None

        def _get_connector_metadata(self):
            return self._connector_metadata

    base.KVConnectorBase_V1 = KVConnectorBase_V1
    base.KVConnectorMetadata = type("KVConnectorMetadata", (), {})
    base.KVConnectorWorkerMetadata = type("KVConnectorWorkerMetadata", (), {})
    base.KVConnectorRole = SimpleNamespace(SCHEDULER="scheduler", WORKER="worker")
    modules = {"vllm": ModuleType("vllm")}
    for name in ("vllm.distributed", "vllm.distributed.kv_transfer", "vllm.distributed.kv_transfer.kv_connector",
                 "vllm.distributed.kv_transfer.kv_connector.v1"):
        modules[name] = ModuleType(name)
    modules[BASE] = base
    return modules


@pytest.fixture
def connector_module():
    with patch.dict(sys.modules, stand_in_vllm()):
        sys.modules.pop("kvsnap_amd.connector", None)
        module = importlib.import_module("kvsnap_amd.connector")
        yield module
    sys.modules.pop("kvsnap_amd.connector", None)


def vllm_config(tmp_path=None, **extra):
    extra.setdefault("pinned_pool_bytes", 64 << 20)
    if tmp_path is not None:
        extra["store_path"] = str(tmp_path)
    return SimpleNamespace(
        parallel_config=SimpleNamespace(tensor_parallel_size=1, pipeline_parallel_size=1, data_parallel_size=1),
        scheduler_config=SimpleNamespace(async_scheduling=False), speculative_config=None,
        cache_config=SimpleNamespace(block_size=16),
        kv_transfer_config=SimpleNamespace(kv_connector_extra_config=extra))


class RunAtOnce:
    def submit(self, fn, *args):
        from kvsnap_amd.worker import _run_now
        return _run_now(fn, *args)

    def shutdown(self, wait=True):
        pass


def test_the_connector_is_a_kv_connector_base_v1_and_refuses_what_it_does_not_support(connector_module, tmp_path):
    module = connector_module
    role = sys.modules[BASE].KVConnectorRole
    assert issubclass(module.KvsnapConnector, sys.modules[BASE].KVConnectorBase_V1)
    assert issubclass(module.KvsnapConnectorMetadata, sys.modules[BASE].KVConnectorMetadata)
    assert issubclass(module.KvsnapConnectorWorkerMetadata, sys.modules[BASE].KVConnectorWorkerMetadata)
    with pytest.raises(NotImplementedError, match="worker role only"):
        module.KvsnapConnector(vllm_config(), role.SCHEDULER, None)
    config = vllm_config()
    config.parallel_config.pipeline_parallel_size = 2
    with pytest.raises(ValueError, match="tensor parallelism only"):
        module.KvsnapConnector(config, role.WORKER, None)
    config = vllm_config()
    config.scheduler_config.async_scheduling = True
    with pytest.raises(ValueError, match="synchronous scheduling"):
        module.KvsnapConnector(config, role.WORKER, None)
    with pytest.raises(ValueError, match="one full-attention KV group"):
        module.KvsnapConnector(vllm_config(), role.WORKER, SimpleNamespace(kv_cache_groups=[1, 2]))
    connector = module.KvsnapConnector(vllm_config(tmp_path, verify_host_checksums="true", async_load="false",
                                                   host_tier_bytes=32 << 20, device_staging_bytes=0),
                                       role.WORKER, SimpleNamespace(kv_cache_groups=[1]))
    worker = connector.worker
    assert (worker.verify, worker.async_load, worker.block_size, worker.capacity_bytes, worker.host_tier_bytes) == \
        ("host", False, 16, 64 << 20, 32 << 20)
    assert worker.plane_options == {"device_staging_bytes": 0} and worker.blobs.root == tmp_path
    with pytest.raises(NotImplementedError):
        connector.get_num_new_matched_tokens(None, 0)


def test_one_save_and_one_load_through_the_connector_hooks(connector_module):
    """register_kv_caches builds and warms the plane; a step's save goes through wait_for_save and is reported
    sending once vLLM finishes the request, its snapshot in the worker metadata; the next step's load goes
    through start_load_kv and is reported receiving, its blocks restored by the plane from the host tier."""
    from kvsnap_amd.worker import Transfer
    module = connector_module
    role = sys.modules[BASE].KVConnectorRole
    plane = MagicMock(block_bytes=4, layout_identity="layout")
    with patch("kvsnap_amd.dataplane.TorchBlockDataPlane", return_value=plane) as made, \
         patch("kvsnap_amd.host_tier.HostTier") as tier_class:
        connector = module.KvsnapConnector(vllm_config(pinned_pool_bytes=1 << 20), role.WORKER, None)
        for pool in (connector.worker.loader, connector.worker.executor):
            pool.shutdown()
        connector.worker.loader = connector.worker.executor = RunAtOnce()
        caches = {"model.layers.0.self_attn.attn": object()}
        assert connector.register_kv_caches(caches) == "layout"
    made.assert_called_once_with(caches, 16, 1 << 20)
    plane.warm_up.assert_called_once_with()
    tier = tier_class.return_value
    tier_class.assert_called_once_with(plane, (1 << 20) * 3 // 4)

    snapshot = {"segments": [{"blob_id": "a" * 64, "offset": 0, "length": 4, "crc32c": 7}],
                "locations": {"a" * 64: {}}, "kv_layout": "layout"}

    def saved(block_ids, num_kv_tokens, *, previous=None, fenced=None):
        fenced.set()                  # the D2H landed: the GPU blocks may go
        return snapshot
    tier.save.side_effect = saved
    save = Transfer("r1", [5], durability="volatile", num_kv_tokens=16)
    connector.bind_connector_metadata(module.KvsnapConnectorMetadata(saves=[save]))
    connector.start_load_kv(SimpleNamespace())
    connector.wait_for_save()
    assert connector.get_finished({"r1"}) == ({"r1"}, set())
    report = connector.build_connector_worker_meta()
    assert isinstance(report, module.KvsnapConnectorWorkerMetadata) and report.prepared == {"r1": snapshot}
    tier.save.assert_called_once()
    assert tier.save.call_args.args[:2] == ([5], 16)
    connector.clear_connector_metadata()
    assert connector._get_connector_metadata() is None

    tier.borrow.side_effect = lambda segments, locations: nullcontext([("pinned", 0)])
    load = Transfer("r2", [9], snapshot=snapshot, durability="volatile")
    connector.bind_connector_metadata(module.KvsnapConnectorMetadata(loads=[load]))
    connector.start_load_kv(SimpleNamespace())
    assert connector.get_finished(set()) == (set(), {"r2"})
    plane.load_scatter_checked.assert_called_once()
    assert plane.load_scatter_checked.call_args.args == ([9], [("pinned", 0)], [7])
    assert connector.get_block_ids_with_load_errors() == set()
    assert connector.build_connector_worker_meta().loaded == ["r2"]
    connector.shutdown()
    plane.close.assert_called_once_with()
