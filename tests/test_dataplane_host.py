"""TorchBlockDataPlane's host logic on real CPU tensors, with the GPU launches replaced by memmoves.

The geometry is the reference's Qwen3-8B fixture (tests/connector/
test_scatter_gather.py:1-13): 36 layers ``model.layers.N.self_attn.attn``,
each a [blocks, 8 heads, 16 tokens, 256] bf16 view of [blocks, 16, 8, 256]
storage, 64 KiB per (layer, block), 2.25 MiB records.  Only the HIP launches
and the pool's stream are stood in for; registration, chunking, coalescing
of adjacent targets, progress reporting, bounds checks and tail regions are
the data plane's own code.  Expected bytes come from torch's strided
indexing, independently of the data plane's span arithmetic.
"""
import ctypes as C
import sys
from contextlib import contextmanager, nullcontext
from types import SimpleNamespace
from unittest.mock import Mock, patch

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import oracle
from kvsnap_amd import dataplane
from kvsnap_amd.dataplane import TorchBlockDataPlane

LAYERS, HEADS, BLOCK_SIZE, WIDTH = 36, 8, 16, 256


class HostAllocation:
    """A pinned allocation stand-in: host memory, copies are memmoves."""

    def __init__(self, size):
        self.size, self.waits, self.closed = size, 0, False
        self.buffer = C.create_string_buffer(max(size, 1))
        self.pointer = C.addressof(self.buffer)

    def _open(self):
        if self.closed:
            raise RuntimeError("pinned allocation closed")

    def copy(self, device_ptr, size, offset=0, *, to_host, producer_stream=0):
        if min(size, offset) < 0 or offset + size > self.size:
            raise ValueError("copy outside the allocation")
        host = self.pointer + offset
        C.memmove(host if to_host else device_ptr, device_ptr if to_host else host, size)

    def wait(self):
        self.waits += 1

    def zero(self, offset, size):
        C.memset(self.pointer + offset, 0, size)

    def bytes(self, offset, size):
        return C.string_at(self.pointer + offset, size)


class HostPool:
    @contextmanager
    def borrow_copy_stream(self):
        yield 1

    @contextmanager
    def operation(self):
        yield

    def close(self):
        pass


def emulated_restore(sources, blocks, offsets, bases, pitches, words, *, programs=None, min_span_bytes=0):
    spans = list(zip(*(t.tolist() for t in (offsets, bases, pitches, words))))
    for source, block in zip(sources.tolist(), blocks.tolist()):
        for offset, base, pitch, count in spans:
            C.memmove(base + block * pitch, source + offset, count * 8)


def emulated_gather(blocks, offsets, bases, pitches, words, records, record_pitch, *, programs=None,
                    min_span_bytes=0):
    spans = list(zip(*(t.tolist() for t in (offsets, bases, pitches, words))))
    for i, block in enumerate(blocks.tolist()):
        for offset, base, pitch, count in spans:
            C.memmove(records + i * record_pitch + offset, base + block * pitch, count * 8)


def emulated_zero(lib, record_ptr, regions):
    count = regions.numel() // 2
    values = regions.tolist()
    for start, length in zip(values[:count], values[count:]):
        C.memset(record_ptr + start, 0, length)


class Pinnable:
    def __init__(self, tensor):
        self.tensor = tensor

    def pin_memory(self):
        return self.tensor

    def __getattr__(self, name):
        return getattr(self.tensor, name)


class Event:
    def record(self, stream=None):
        pass

    def synchronize(self):
        pass

    def query(self):
        return True


class CpuTorch:
    """torch with its few CUDA calls made CPU no-ops."""
    cuda = SimpleNamespace(stream=lambda stream: nullcontext(), Event=Event,
                           ExternalStream=lambda handle, device=None: Mock(),
                           Stream=lambda device=None: Mock(), current_stream=lambda device=None: Mock())

    def __getattr__(self, name):
        return getattr(torch, name)

    def tensor(self, *args, **kwargs):
        return Pinnable(torch.tensor(*args, **kwargs))


class CudaLabelled:
    device = SimpleNamespace(type="cuda", index=0)

    def __init__(self, tensor):
        self.tensor = tensor

    def __getattr__(self, name):
        return getattr(self.tensor, name)

    def __getitem__(self, index):
        return self.tensor[index]


def emulated_gather_launcher(*args, **kwargs):
    return lambda: emulated_gather(*args, **kwargs)


@pytest.fixture(autouse=True)
def emulated_launches():
    with patch.object(dataplane, "copy_host_blocks", emulated_restore), \
         patch.object(dataplane, "gather_blocks", emulated_gather), \
         patch.object(dataplane, "gather_launcher", emulated_gather_launcher), \
         patch.object(dataplane, "kernel_library", lambda library=None: None), \
         patch.object(TorchBlockDataPlane, "_zero_regions", staticmethod(emulated_zero)):
        yield


def register(caches, block_size=BLOCK_SIZE):
    with patch.dict(sys.modules, {"torch": CpuTorch()}), patch.object(dataplane, "CudaPool", return_value=HostPool()):
        plane = TorchBlockDataPlane({name: CudaLabelled(t) for name, t in caches.items()}, block_size, 1 << 30)
    plane.caches = dict(sorted(caches.items()))
    plane.torch = CpuTorch()
    return plane


def qwen3_8b_caches(blocks, seed=0):
    generator = torch.Generator().manual_seed(seed)
    backing = torch.randint(-2**15, 2**15, (LAYERS, blocks, BLOCK_SIZE, HEADS, WIDTH), dtype=torch.int16,
                            generator=generator).view(torch.bfloat16)
    return {f"model.layers.{i}.self_attn.attn": backing[i].permute(0, 2, 1, 3) for i in range(LAYERS)}


def raw(tensor):
    tensor = tensor.contiguous()
    return C.string_at(tensor.data_ptr(), tensor.numel() * tensor.element_size())


def block_span(view, block):
    """A layer's bytes for one block in storage order (tokens, heads, width)."""
    return raw(view[block].permute(1, 0, 2))


def bits(view):
    return view.permute(0, 2, 1, 3).view(torch.int16)


def snapshot(caches):
    return {name: bits(view).clone() for name, view in caches.items()}


def targets_for(kind, count, size):
    if kind == "per-block":
        return [(HostAllocation(size), 0) for _ in range(count)]
    staged = HostAllocation(size * count)
    return [(staged, i * size) for i in range(count)]


@pytest.fixture
def qwen():
    caches = qwen3_8b_caches(12)
    return caches, register(caches), sorted(caches)


def test_registration_matches_the_layout_vllm_reports(qwen):
    caches, plane, names = qwen
    layer = plane.layers[0]
    assert (layer["shape"], layer["stride"], layer["bytes"]) == ([8, 16, 256], [256, 2048, 1], 65536)
    assert plane.block_bytes == 36 * 65536
    assert [l["name"] for l in plane.layers] == names
    assert names[:3] == ["model.layers.0.self_attn.attn", "model.layers.1.self_attn.attn",
                         "model.layers.10.self_attn.attn"]
    for layer in plane.layers:   # identical to the oracle's restatement of the rule
        view = caches[layer["name"]]
        expected = oracle.register_layout(layer["name"], list(view.shape), list(view.stride()), 2, BLOCK_SIZE)
        assert {k: layer[k] for k in expected} == expected


@pytest.mark.parametrize("kind,copies", [("per-block", 5), ("staging", 3)])
def test_save_gather_packs_layers_in_name_order_and_zeroes_the_tail(qwen, kind, copies):
    caches, plane, names = qwen
    block_ids, tokens = [7, 2, 9, 3, 4], 4 * BLOCK_SIZE + 5
    size = plane.block_bytes
    before = snapshot(caches)
    targets = targets_for(kind, len(block_ids), size)
    assert plane.save_gather(block_ids, targets, tokens, chunk_bytes=2 * size) == copies
    for index, block in enumerate(block_ids):
        allocation, offset = targets[index]
        for position, name in enumerate(names):
            expected = bytearray(block_span(caches[name], block))
            if index == len(block_ids) - 1:
                expected[5 * HEADS * WIDTH * 2:] = bytes((BLOCK_SIZE - 5) * HEADS * WIDTH * 2)
            assert allocation.bytes(offset + position * 65536, 65536) == bytes(expected), (block, name)
    assert all(allocation.waits for allocation, _ in targets)
    for name in names:
        assert torch.equal(bits(caches[name]), before[name])


@pytest.mark.parametrize("kind", ["per-block", "staging"])
def test_load_scatter_writes_only_the_target_blocks(qwen, kind):
    caches, plane, names = qwen
    block_ids = [10, 0, 5, 6, 1]
    size = plane.block_bytes
    sources = targets_for(kind, len(block_ids), size)
    payload = torch.randint(-2**15, 2**15, (len(block_ids), size // 2), dtype=torch.int16,
                            generator=torch.Generator().manual_seed(len(kind)))
    for (allocation, offset), row in zip(sources, payload):
        C.memmove(allocation.pointer + offset, row.data_ptr(), size)
    before = snapshot(caches)
    assert plane.load_scatter(block_ids, sources) == 1
    for index, name in enumerate(names):
        after = bits(caches[name])
        for block in range(12):
            if block in block_ids:
                row = raw(payload[block_ids.index(block)])
                assert block_span(caches[name], block) == row[index * 65536:(index + 1) * 65536]
            else:
                assert torch.equal(after[block], before[name][block])


def test_load_scatter_launches_per_chunk_and_reports_what_is_left(qwen):
    caches, plane, names = qwen
    block_ids, size = [3, 8, 1, 0, 6], plane.block_bytes
    sources = targets_for("staging", len(block_ids), size)
    before = snapshot(caches)
    for (allocation, offset), block in zip(sources, block_ids):
        for position, name in enumerate(names):
            C.memmove(allocation.pointer + offset + position * 65536, raw(bits(caches[name])[(block + 2) % 12]), 65536)
    progress = []
    assert plane.load_scatter(block_ids, sources, progress=progress, chunk_bytes=2 * size) == 3
    assert [left for _, left in progress] == [5 * size, 3 * size, size, 0]
    assert progress[0][0] is None
    for name in names:
        for block in block_ids:
            assert torch.equal(bits(caches[name])[block], before[name][(block + 2) % 12])


def test_load_scatter_checks_every_source_before_the_launch(qwen):
    caches, plane, names = qwen
    size = plane.block_bytes
    before = snapshot(caches)
    closed = HostAllocation(size)
    closed.closed = True
    cases = {"outside": [(HostAllocation(size), 0), (HostAllocation(size - 8), 0)],
             "closed": [(HostAllocation(size), 0), (closed, 0)],
             "negative": [(HostAllocation(2 * size), -8), (HostAllocation(size), 0)]}
    for reason, sources in cases.items():
        with patch.object(dataplane, "copy_host_blocks") as launch:
            with pytest.raises((ValueError, RuntimeError)):
                plane.load_scatter([1, 2], sources)
            launch.assert_not_called()
    for name in names:
        assert torch.equal(bits(caches[name]), before[name])


def test_a_failed_launch_drains_the_copy_stream_before_sources_can_be_released(qwen):
    caches, plane, names = qwen
    plane._load_tables()
    plane._copy_stream = Mock()
    sources = targets_for("staging", 2, plane.block_bytes)
    with patch.object(dataplane, "copy_host_blocks", side_effect=RuntimeError("launch failed")):
        with pytest.raises(RuntimeError, match="launch failed"):
            plane.load_scatter([1, 2], sources)
    plane._copy_stream.synchronize.assert_called_once_with()


def test_a_saved_snapshot_restores_into_other_blocks(qwen):
    caches, plane, names = qwen
    saved, tokens, restored = [3, 4, 5, 8, 11], 5 * BLOCK_SIZE, [0, 1, 2, 6, 7]
    size = plane.block_bytes
    targets = targets_for("staging", len(saved), size)
    expected = {name: [block_span(caches[name], b) for b in saved] for name in names}
    assert plane.save_gather(saved, targets, tokens) == 1
    assert plane.load_scatter(restored, targets) == 1
    for name in names:
        assert [block_span(caches[name], b) for b in restored] == expected[name]


def test_ids_and_counts_are_validated(qwen):
    caches, plane, names = qwen
    size = plane.block_bytes
    for ids in ([12], [-1], [1.0], ["1"]):
        with pytest.raises(ValueError):
            plane.load_scatter(ids, targets_for("staging", 1, size))
    with pytest.raises(ValueError):
        plane.load_scatter([1, 2], targets_for("staging", 1, size))
    with pytest.raises(ValueError):
        plane.save_gather([1, 2], targets_for("staging", 2, size), 33)      # 33 tokens need 3 blocks
    assert plane.save_gather([], [], 0) == 0
    assert plane.load_scatter([], []) == 0


@pytest.mark.parametrize("strides", [(96, 32, 8, 1), (96, 8, 24, 1), (192, 32, 8, 1), (192, 8, 24, 1)])
def test_tail_zeroing_and_restore_follow_the_actual_strides(strides):
    shape = (5, 3, 4, 8)
    storage = torch.arange(5 * strides[0], dtype=torch.int16).view(torch.bfloat16)
    cache = storage.as_strided(shape, strides)
    plane = register({"layer.0": cache}, block_size=4)
    before = storage.clone()
    targets = targets_for("per-block", 2, plane.block_bytes)
    plane.save_gather([1, 3], targets, 6)
    for index, block in enumerate((1, 3)):
        span = before[block * strides[0]:block * strides[0] + 96].view(torch.int16).clone()
        if index == 1:
            for head in range(3):
                for token in (2, 3):
                    start = head * strides[1] + token * strides[2]
                    span[start:start + 8] = 0
        assert targets[index][0].bytes(0, 192) == raw(span)
    assert torch.equal(storage.view(torch.int16), before.view(torch.int16))
    plane.load_scatter([0, 4], targets)
    expected = before.view(torch.int16).clone()
    for block, (allocation, _) in zip((0, 4), targets):
        payload = torch.frombuffer(bytearray(allocation.bytes(0, 192)), dtype=torch.int16)
        expected[block * strides[0]:block * strides[0] + 96] = payload
    assert torch.equal(storage.view(torch.int16), expected)


def test_kv_split_layers_pack_k_then_v_and_zero_both_tails():
    generator = torch.Generator().manual_seed(3)
    backing = torch.randint(-2**15, 2**15, (3, 2, 6, 4, 2, 8), dtype=torch.int16, generator=generator).view(
        torch.bfloat16)                                   # [layers, K/V, blocks, N=4, H=2, C=8]
    caches = {f"layer.{i}": backing[i] for i in range(3)}
    plane = register(caches, block_size=4)
    assert plane.layers[0]["shape"] == [2, 4, 2, 8] and plane.layers[0]["bytes"] == 256
    assert plane.block_bytes == 3 * 256
    targets = targets_for("staging", 2, plane.block_bytes)
    plane.save_gather([4, 1], targets, 7)                  # last block keeps 3 of 4 tokens
    for index, block in enumerate((4, 1)):
        record = targets[0][0].bytes(index * plane.block_bytes, plane.block_bytes)
        for layer in range(3):
            for kv in range(2):
                span = bytearray(raw(backing[layer, kv, block]))
                if index == 1:
                    span[3 * 2 * 8 * 2:] = bytes(128 - 3 * 2 * 8 * 2)
                start = layer * 256 + kv * 128
                assert record[start:start + 128] == bytes(span), (block, layer, kv)
    before = backing.view(torch.int16).clone()
    plane.load_scatter([0, 5], targets)
    after = backing.view(torch.int16)
    record0 = torch.frombuffer(bytearray(targets[0][0].bytes(0, plane.block_bytes)), dtype=torch.int16)
    assert torch.equal(after[:, :, 0].reshape(-1), record0)
    assert torch.equal(after[:, :, 1:5], before[:, :, 1:5])


def test_tail_regions_equal_the_oracle_rule_on_random_records(qwen):
    caches, plane, names = qwen
    rng = np.random.default_rng(0)
    for valid in (1, 5, 15):
        record = rng.integers(0, 256, plane.block_bytes, dtype=np.uint8)
        expected = record.copy()
        oracle.zero_tail(expected, plane.layers, valid)
        got = record.copy()
        for start, length in plane._tail_regions(valid):
            got[start:start + length] = 0
        assert np.array_equal(got, expected)
        assert len(plane._tail_regions(valid)) == LAYERS    # token-major storage: one merged range per layer


def test_digests_are_returned_in_block_order():
    caches = qwen3_8b_caches(6, seed=2)
    plane = register(caches)
    size = plane.block_bytes

    class EmulatedHashJob:
        """The oracle in place of the GPU hash job, with its interface."""

        def __init__(self, torch_module, records_ptr, record_bytes, record_pitch, n, device, stream, slice_blocks, *,
                     timer=None, keepalive=None, executor=None):
            crcs, shas = oracle.digest_records(records_ptr, record_bytes, record_pitch, n)
            self.crc, self.sha = torch.from_numpy(crcs.astype(np.int64)), torch.from_numpy(shas)

        def query(self):
            return True

        def finished(self, timeout=None):
            return True

        def synchronize(self):
            pass

    targets = targets_for("staging", 3, size)
    digests = []
    with patch.object(dataplane, "HashJob", EmulatedHashJob), \
         patch.object(TorchBlockDataPlane, "_hash_streams", lambda self: [Mock()]):
        plane.save_gather([5, 2, 4], targets, 3 * BLOCK_SIZE - 2, digests=digests)
    result = digests[0].result()
    for i, (hexdigest, crc) in enumerate(result):
        record = targets[0][0].bytes(i * size, size)
        assert crc == oracle.crc32c(record) and hexdigest == oracle.sha256(record).hex()


class Descriptor:
    """A tensor descriptor with real shape/stride arithmetic and no storage (test_kv_layout.py)."""

    def __init__(self, shape, strides):
        self.shape, self._strides = tuple(shape), tuple(strides)
        self.device = SimpleNamespace(type="cuda", index=0)
        self.ndim, self.dtype = len(shape), "torch.bfloat16"

    def stride(self, axis=None):
        return self._strides if axis is None else self._strides[axis]

    def element_size(self):
        return 2

    def numel(self):
        n = 1
        for s in self.shape:
            n *= s
        return n

    def __getitem__(self, index):
        return Descriptor(self.shape[1:], self._strides[1:])


@pytest.mark.parametrize("shape,strides,block_size,block_bytes", [
    ((5, 3, 4, 8), (96, 8, 24, 1), 4, 192),              # LBNHC storage, BHNC view
    ((5, 3, 4, 8), (192, 32, 8, 1), 4, 192),             # block-outer interleaved layers
    ((5, 3, 4, 8), (96, 8, 8, 1), 4, None),              # overlapping inner axes
    ((5, 3, 4, 8), (48, 32, 8, 1), 4, None),             # overlapping blocks
    ((5, 3, 5, 8), (120, 40, 8, 1), 4, None),            # tokens != block size
    ((5, 3, 4, 8), (96, 32, 8, 2), 4, None),             # non-contiguous C
    ((2, 5, 4, 3, 8), (480, 96, 24, 8, 1), 4, 384),      # [2, B, N, H, C] K/V split
    ((2, 5, 4, 3, 8), (96, 192, 24, 8, 1), 4, 384),      # [B, 2, N, H, C] storage seen as [2, B, ...]
    ((2, 5, 4, 3, 8), (96, 96, 24, 8, 1), 4, None),      # K and V overlap
    ((3, 5, 4, 3, 8), (480, 96, 24, 8, 1), 4, None),     # not K/V
    ((5, 3, 8), (24, 8, 1), 4, None),                    # wrong rank
])
def test_registration_accepts_dense_blocks_and_rejects_the_rest(shape, strides, block_size, block_bytes):
    with patch.dict(sys.modules, {"torch": SimpleNamespace()}), patch.object(dataplane, "CudaPool", return_value=Mock()):
        if block_bytes is None:
            with pytest.raises(ValueError):
                TorchBlockDataPlane({"layer.0": Descriptor(shape, strides)}, block_size, 4096)
        else:
            plane = TorchBlockDataPlane({"layer.0": Descriptor(shape, strides)}, block_size, 4096)
            assert plane.block_bytes == block_bytes


def test_registration_requires_one_cuda_device():
    with patch.dict(sys.modules, {"torch": SimpleNamespace()}), patch.object(dataplane, "CudaPool", return_value=Mock()):
        with pytest.raises(ValueError):
            TorchBlockDataPlane({}, 4, 4096)
        cpu = Descriptor((5, 3, 4, 8), (96, 8, 24, 1))
        cpu.device = SimpleNamespace(type="cpu", index=None)
        with pytest.raises(ValueError, match="one CUDA device"):
            TorchBlockDataPlane({"layer.0": cpu}, 4, 4096)


def test_early_report_follows_the_reference_rule():
    """vllm.py:649-679 as pinned by test_failure_policy.py:180-206."""
    from kvsnap_amd.ordering import EARLY_REPORT_BYTES, copy_left, early_launch_index, early_report
    mib = 1 << 20
    done, pending = Mock(query=Mock(return_value=True)), Mock(query=Mock(return_value=False))
    progress = [(None, 300 * mib), (done, 200 * mib), (done, 100 * mib), (pending, 0)]
    assert copy_left(progress) == 100 * mib
    assert early_report(progress) == (100 * mib, pending)
    assert early_report([(None, 300 * mib), (done, 200 * mib), (pending, 100 * mib), (pending, 0)]) is None
    assert copy_left([(None, 300 * mib), (done, 100 * mib), (pending, 50 * mib)]) is None     # still queuing
    assert EARLY_REPORT_BYTES == 128 * mib
    assert early_launch_index(progress) == 1
    # the oracle's restatement of the same rule agrees on the same scenario
    assert oracle.copy_left([(None if e is None else e.query, l) for e, l in progress]) == copy_left(progress)


def test_restore_progress_reaches_the_early_report_threshold_at_the_expected_launch(qwen):
    """An 8k-token Qwen3-8B restore: 19 launches of 28 blocks; reportable after the 17th."""
    from kvsnap_amd.ordering import early_launch_index
    size = 36 * 65536
    per_launch = (64 << 20) // size
    progress = [(None, 512 * size)] + [(Mock(), (512 - min(512, (k + 1) * per_launch)) * size)
                                       for k in range(-(-512 // per_launch))]
    assert len(progress) - 1 == 19
    assert early_launch_index(progress) == 16


def test_restore_runs_group_consecutive_records():
    """The DMA restore copies each run of adjacent pinned records with one copy."""
    from kvsnap_amd.dataplane import _runs
    assert _runs([0, 10, 20, 40, 50, 70], 10) == [(0, 3), (3, 2), (5, 1)]
    assert _runs([100, 110, 200], 10, 5) == [(5, 2), (7, 1)]
    assert _runs([30, 20, 10], 10) == [(0, 1), (1, 1), (2, 1)]
    assert _runs([], 10) == []


def test_restore_mode_is_checked():
    caches = {"layer.0": CudaLabelled(torch.zeros(4, 2, BLOCK_SIZE, 8))}
    with patch.dict(sys.modules, {"torch": CpuTorch()}), patch.object(dataplane, "CudaPool", return_value=HostPool()):
        with pytest.raises(ValueError, match="restore_mode"):
            TorchBlockDataPlane(caches, BLOCK_SIZE, 1 << 30, restore_mode="fast")
