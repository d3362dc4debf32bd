"""TorchBlockDataPlane's host logic on CPU tensors, with the HIP library replaced by a CPU one.

The geometry is the reference's Qwen3-8B fixture (tests/connector/
test_scatter_gather.py:1-13): 36 layers ``model.layers.N.self_attn.attn``,
each a [blocks, 8 heads, 16 tokens, 256] bf16 view of [blocks, 16, 8, 256]
storage, 64 KiB per (layer, block), 2.25 MiB records.

What is stood in for, and how:

* ``HostKernels`` implements the kernel C-ABI entry points the plane calls
  (restore, gather, zero, and the copies between "device" and pinned memory)
  on host memory with ``ctypes.memmove``, so the plane's own launch code and
  table uploads run unchanged.
* ``CpuCuda`` is a torch proxy whose CUDA calls (streams, events, device
  allocations) are CPU no-ops or CPU tensors.
* ``Arena`` is the pinned pool: one host buffer carved into allocations, each
  copy a memmove, with counts of waits and copies.

Registration, chunking, copy coalescing, progress, bounds checks and tail
regions are the plane's own code.  Expected bytes come from torch's strided
indexing of the caches, independently of the plane's span arithmetic.
"""
import ctypes as C
import sys
from contextlib import contextmanager, nullcontext
from types import SimpleNamespace
from unittest.mock import MagicMock, patch

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import oracle
from kvsnap_amd import dataplane
from kvsnap_amd.blobs import CorruptSnapshotError
from kvsnap_amd.dataplane import TorchBlockDataPlane

LAYERS, HEADS, TOKENS, WIDTH = 36, 8, 16, 256
SPAN = HEADS * TOKENS * WIDTH * 2

CUDA = SimpleNamespace(type="cuda", index=0)


# ---------------------------------------------------------------- stand-ins


class HostKernels:
    """The kernel library's entry points, executed on host memory (every pointer is a host address)."""

    def __init__(self):
        self.launches = []

    @staticmethod
    def _int64(address, count):
        return list((C.c_int64 * count).from_address(address)) if count else []

    def _spans(self, offsets, bases, pitches, words, n_spans):
        return list(zip(*(self._int64(t, n_spans) for t in (offsets, bases, pitches, words))))

    def kvsnap_restore_blocks(self, sources, blocks, n, offsets, bases, pitches, words, n_spans, hint, programs,
                              stream):
        self.launches.append(("restore", n))
        for source, block in zip(self._int64(sources, n), self._int64(blocks, n)):
            for offset, base, pitch, count in self._spans(offsets, bases, pitches, words, n_spans):
                C.memmove(base + block * pitch, source + offset, 8 * count)
        return 0

    def kvsnap_gather_blocks(self, blocks, n, offsets, bases, pitches, words, n_spans, hint, records, record_pitch,
                             programs, stream):
        self.launches.append(("gather", n))
        for i, block in enumerate(self._int64(blocks, n)):
            for offset, base, pitch, count in self._spans(offsets, bases, pitches, words, n_spans):
                C.memmove(records + i * record_pitch + offset, base + block * pitch, 8 * count)
        return 0

    def kvsnap_scatter_blocks(self, records, record_pitch, blocks, n, offsets, bases, pitches, words, n_spans, hint,
                              programs, stream):
        self.launches.append(("scatter", n))
        for i, block in enumerate(self._int64(blocks, n)):
            for offset, base, pitch, count in self._spans(offsets, bases, pitches, words, n_spans):
                C.memmove(base + block * pitch, records + i * record_pitch + offset, 8 * count)
        return 0

    def kvsnap_restore_blocks_checked(self, sources, blocks, n, offsets, bases, pitches, words, n_spans, programs,
                                      partial, stream):
        """The checked restore: the copy, and (a stand-in for the per-span partials) each record's CRC32C in
        its first partial slot, computed from the record bytes read."""
        self.launches.append(("restore_checked", n))
        spans = self._spans(offsets, bases, pitches, words, n_spans)
        record_bytes = max(offset + 8 * count for offset, _, _, count in spans)
        for i, (source, block) in enumerate(zip(self._int64(sources, n), self._int64(blocks, n))):
            for offset, base, pitch, count in spans:
                C.memmove(base + block * pitch, source + offset, 8 * count)
            C.c_uint32.from_address(partial + 4 * i * n_spans).value = oracle.crc32c(C.string_at(source, record_bytes))
        return 0

    def kvsnap_gather_blocks_checked(self, dests, blocks, n, offsets, bases, pitches, words, n_spans, stage,
                                     stage_pitch, programs, partial, stream):
        """The checked gather: each record to its destination (and to ``stage``), and (as the checked restore's
        stand-in does) its CRC32C in its first partial slot."""
        self.launches.append(("gather_checked", n))
        spans = self._spans(offsets, bases, pitches, words, n_spans)
        record_bytes = max(offset + 8 * count for offset, _, _, count in spans)
        for i, (dest, block) in enumerate(zip(self._int64(dests, n), self._int64(blocks, n))):
            for offset, base, pitch, count in spans:
                C.memmove(dest + offset, base + block * pitch, 8 * count)
                if stage:
                    C.memmove(stage + i * stage_pitch + offset, base + block * pitch, 8 * count)
            C.c_uint32.from_address(partial + 4 * i * n_spans).value = oracle.crc32c(C.string_at(dest, record_bytes))
        return 0

    #: Whether kvsnap_gather_crc32c_fits admits whole-KiB records: off, so hashed saves gather and then take
    #: their CRC32Cs, unless a test turns it on.
    fused = False

    def kvsnap_gather_crc32c_fits(self, record_bytes):
        return int(self.fused and record_bytes % 1024 == 0)

    def kvsnap_gather_crc32c(self, blocks, n, group_bases, group_pitches, record_bytes, out, out_pitch, crcs,
                             stream):
        """The gather with CRC32C: each record from its 1 KiB groups' sources, and its CRC32C."""
        self.launches.append(("gather_crc", n))
        groups = record_bytes // 1024
        bases, pitches = self._int64(group_bases, groups), self._int64(group_pitches, groups)
        for i, block in enumerate(self._int64(blocks, n)):
            for g in range(groups):
                C.memmove(out + i * out_pitch + 1024 * g, bases[g] + block * pitches[g], 1024)
            C.c_uint32.from_address(crcs + 4 * i).value = oracle.crc32c(C.string_at(out + i * out_pitch,
                                                                                    record_bytes))
        return 0

    def kvsnap_crc32c_workspace_bytes(self, record_bytes, n):
        return 16

    def kvsnap_crc32c_records(self, records, record_bytes, pitch, n, prior, out, workspace, work_bytes, stream):
        self.launches.append(("crc32c", n))
        for i in range(n):
            C.c_uint32.from_address(out + 4 * i).value = oracle.crc32c(C.string_at(records + i * pitch, record_bytes),
                                                                       prior)
        return 0

    def kvsnap_restore_checked_crc32c(self, partial, n, offsets, words, n_spans, record_bytes, out, stream):
        self.launches.append(("restore_checked_crc32c", n))
        for i in range(n):
            C.c_uint32.from_address(out + 4 * i).value = C.c_uint32.from_address(partial + 4 * i * n_spans).value
        return 0

    def kvsnap_zero_regions(self, base, starts, lengths, n, stream):
        for start, length in zip(self._int64(starts, n), self._int64(lengths, n)):
            C.memset(base + start, 0, length)
        return 0

    def kvsnap_copy_to_device(self, dst, src, nbytes, stream):
        C.memmove(dst, src, nbytes)
        return 0

    kvsnap_copy_to_host = kvsnap_copy_to_device

    def kvsnap_cuda_error(self):
        return b"host kernels"


class CpuCuda:
    """torch, with the CUDA calls the plane makes answered on the CPU."""

    class Event:
        def record(self, stream=None):
            pass

        def synchronize(self):
            pass

        def query(self):
            return True

    def __init__(self):
        self.cuda = SimpleNamespace(stream=lambda stream: nullcontext(), Event=self.Event,
                                    current_stream=lambda device=None: MagicMock(cuda_stream=0),
                                    ExternalStream=lambda handle, device=None: MagicMock(cuda_stream=handle))

    def __getattr__(self, name):
        return getattr(torch, name)

    @staticmethod
    def _host(kwargs):
        kwargs.pop("pin_memory", None)
        if kwargs.get("device") is CUDA:
            kwargs.pop("device")
        return kwargs

    def empty(self, *args, **kwargs):
        return torch.empty(*args, **self._host(kwargs))

    def zeros(self, *args, **kwargs):
        return torch.zeros(*args, **self._host(kwargs))

    def tensor(self, *args, **kwargs):
        return torch.tensor(*args, **self._host(kwargs))


class OnDevice:
    """A CPU tensor that reports a CUDA device: the few members registration and the span tables read."""

    device = CUDA

    def __init__(self, tensor):
        self.tensor = tensor
        self.shape, self.ndim, self.dtype = tensor.shape, tensor.ndim, tensor.dtype

    def stride(self, *axis):
        return self.tensor.stride(*axis)

    def element_size(self):
        return self.tensor.element_size()

    def data_ptr(self):
        return self.tensor.data_ptr()


class Arena:
    """The pinned pool: one host buffer, allocations carved from it in order."""

    def __init__(self, capacity):
        self.memory = np.zeros(capacity, dtype=np.uint8)
        self.used = 0

    def reserve(self, size):
        if self.used + size > self.memory.size:
            raise MemoryError("arena full")
        allocation = Slab(self, self.memory.ctypes.data + self.used, size)
        self.used += size
        return allocation

    @contextmanager
    def borrow_copy_stream(self):
        yield 7

    @contextmanager
    def operation(self):
        yield

    def close(self):
        pass


class Slab:
    """One allocation of an ``Arena``: device<->host copies are memmoves, counted."""

    def __init__(self, arena, pointer, size):
        self.arena, self.pointer, self.size = arena, pointer, size
        self.closed, self.copies, self.waits = False, 0, 0

    def _open(self):
        if self.closed:
            raise RuntimeError("this slab has been handed back")

    def copy(self, device_ptr, size, offset=0, *, to_host, producer_stream=0):
        self._open()
        if offset < 0 or size < 0 or offset + size > self.size:
            raise ValueError("copy outside the allocation")
        source, target = (device_ptr, self.pointer + offset) if to_host else (self.pointer + offset, device_ptr)
        C.memmove(target, source, size)
        self.copies += 1

    def wait(self):
        self.waits += 1

    def at(self, offset, size):
        return C.string_at(self.pointer + offset, size)

    def fill(self, offset, data):
        C.memmove(self.pointer + offset, data, len(data))


def plane_over(caches, block_size=TOKENS, **options):
    """A plane registered over CPU ``caches``, its pool an Arena and its kernels HostKernels (the restore
    kernel's path unless ``restore_mode`` says otherwise)."""
    options.setdefault("restore_mode", "kernel")
    cpu = CpuCuda()
    with patch.dict(sys.modules, {"torch": cpu}), patch.object(dataplane, "CudaPool", return_value=Arena(1 << 20)):
        plane = TorchBlockDataPlane({name: OnDevice(t) for name, t in caches.items()}, block_size, 1 << 30,
                                    **options)
    plane.torch = cpu
    plane.pool = Arena(64 << 20)
    return plane


def host_tables(*tensors):
    """The launch-table check, for CPU tensors standing in for device ones."""
    for t in tensors:
        assert t.dtype == torch.int64 and t.dim() == 1 and t.is_contiguous()
    return CUDA


@pytest.fixture(autouse=True)
def host_kernels():
    kernels = HostKernels()
    with patch.object(dataplane, "kernel_library", lambda library=None: kernels), \
         patch.object(dataplane, "_int64_device_tensors", host_tables), \
         patch.object(dataplane, "_int32_device_output", lambda t, device, count: None), \
         patch.object(dataplane, "_current_stream_handle", lambda device: 0):
        yield kernels


# ---------------------------------------------------------------- fixture geometry and expectations


def qwen3_8b_caches(blocks, seed=0):
    """The reference fixture's layers: [blocks, H, N, 2D] views of [blocks, N, H, 2D] random bf16 bits."""
    generator = torch.Generator().manual_seed(seed)
    storage = torch.randint(-2**15, 2**15, (LAYERS, blocks, TOKENS, HEADS, WIDTH), dtype=torch.int16,
                            generator=generator).view(torch.bfloat16)
    return {f"model.layers.{i}.self_attn.attn": storage[i].permute(0, 2, 1, 3) for i in range(LAYERS)}


def span_of(view, block):
    """One layer's bytes of ``block`` in storage order (token, head, width), by torch's own indexing."""
    return view[block].permute(1, 0, 2).contiguous().view(torch.int16).numpy().tobytes()


def cache_bits(caches):
    return {name: view.permute(0, 2, 1, 3).contiguous().view(torch.int16).clone() for name, view in caches.items()}


def slabs(plane, count, *, shared):
    """Targets (or sources) for ``count`` records: one shared allocation, or one allocation per record."""
    size = plane.block_bytes
    if shared:
        slab = plane.pool.reserve(count * size)
        return [(slab, i * size) for i in range(count)]
    return [(plane.pool.reserve(size), 0) for _ in range(count)]


@pytest.fixture
def qwen():
    caches = qwen3_8b_caches(12)
    return caches, plane_over(caches), sorted(caches)


# ---------------------------------------------------------------- registration


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
        expected = oracle.register_layout(layer["name"], list(view.shape), list(view.stride()), 2, TOKENS)
        assert {k: layer[k] for k in expected} == expected


# ---------------------------------------------------------------- save


@pytest.mark.parametrize("shared,copies", [(False, 5), (True, 3)])
def test_save_gather_packs_layers_in_name_order_and_zeroes_the_tail(qwen, shared, copies):
    caches, plane, names = qwen
    blocks, tokens = [7, 2, 9, 3, 4], 4 * TOKENS + 5
    before = cache_bits(caches)
    targets = slabs(plane, len(blocks), shared=shared)
    assert plane.save_gather(blocks, targets, tokens, chunk_bytes=2 * plane.block_bytes) == copies
    for i, block in enumerate(blocks):
        slab, offset = targets[i]
        for position, name in enumerate(names):
            want = bytearray(span_of(caches[name], block))
            if i == len(blocks) - 1:                     # token slots 5..15 of the last block
                want[5 * HEADS * WIDTH * 2:] = bytes(len(want) - 5 * HEADS * WIDTH * 2)
            assert slab.at(offset + position * SPAN, SPAN) == bytes(want), (block, name)
    assert all(slab.waits for slab, _ in targets)
    after = cache_bits(caches)
    assert all(torch.equal(after[name], before[name]) for name in names)


def test_save_copies_once_per_run_of_back_to_back_targets(qwen):
    caches, plane, names = qwen
    size = plane.block_bytes
    first = plane.pool.reserve(3 * size)
    second = plane.pool.reserve(2 * size)
    # Runs: first[0..1], first[2] (out of order after it), second[0..1].
    targets = [(first, 0), (first, size), (second, 0), (second, size), (first, 2 * size)]
    assert plane.save_gather([1, 2, 3, 4, 5], targets, 5 * TOKENS) == 3
    assert (first.copies, second.copies) == (2, 1)
    for i, (slab, offset) in enumerate(targets):
        assert slab.at(offset, SPAN) == span_of(caches[names[0]], i + 1)


def test_save_refuses_a_closed_or_short_target_before_any_copy(qwen, host_kernels):
    caches, plane, names = qwen
    size = plane.block_bytes
    closed = plane.pool.reserve(size)
    closed.closed = True
    for targets in ([(plane.pool.reserve(size), 0), (closed, 0)],
                    [(plane.pool.reserve(size), 0), (plane.pool.reserve(size - 8), 0)]):
        with pytest.raises((ValueError, RuntimeError)):
            plane.save_gather([1, 2], targets, 2 * TOKENS)
    assert host_kernels.launches == []


# ---------------------------------------------------------------- restore


@pytest.mark.parametrize("shared", [False, True])
def test_load_scatter_writes_only_the_target_blocks(qwen, shared):
    caches, plane, names = qwen
    blocks = [10, 0, 5, 6, 1]
    size = plane.block_bytes
    sources = slabs(plane, len(blocks), shared=shared)
    records = np.random.default_rng(len(blocks) + shared).integers(0, 256, (len(blocks), size), dtype=np.uint8)
    for (slab, offset), record in zip(sources, records):
        slab.fill(offset, record.tobytes())
    before = cache_bits(caches)
    assert plane.load_scatter(blocks, sources) == 1
    after = cache_bits(caches)
    for position, name in enumerate(names):
        for block in range(12):
            if block in blocks:
                record = records[blocks.index(block)]
                assert span_of(caches[name], block) == record[position * SPAN:(position + 1) * SPAN].tobytes()
            else:
                assert torch.equal(after[name][block], before[name][block])


def test_load_scatter_launches_per_chunk_and_reports_what_is_left(qwen, host_kernels):
    caches, plane, names = qwen
    blocks, size = [3, 8, 1, 0, 6], plane.block_bytes
    sources = slabs(plane, len(blocks), shared=True)
    saved = cache_bits(caches)
    for (slab, offset), block in zip(sources, blocks):
        for position, name in enumerate(names):
            slab.fill(offset + position * SPAN, span_of(caches[name], (block + 2) % 12))
    progress = []
    assert plane.load_scatter(blocks, sources, progress=progress, chunk_bytes=2 * size) == 3
    assert [left for _, left in progress] == [5 * size, 3 * size, size, 0]
    assert progress[0][0] is None and all(event is not None for event, _ in progress[1:])
    assert host_kernels.launches == [("restore", 2), ("restore", 2), ("restore", 1)]
    after = cache_bits(caches)
    for name in names:
        for block in blocks:
            assert torch.equal(after[name][block], saved[name][(block + 2) % 12])


def test_load_scatter_checks_every_source_before_the_launch(qwen, host_kernels):
    caches, plane, names = qwen
    size = plane.block_bytes
    before = cache_bits(caches)
    closed = plane.pool.reserve(size)
    closed.closed = True
    cases = [[(plane.pool.reserve(size), 0), (plane.pool.reserve(size - 8), 0)],       # too short
             [(plane.pool.reserve(size), 0), (closed, 0)],                             # closed
             [(plane.pool.reserve(2 * size), -8), (plane.pool.reserve(size), 0)]]       # negative offset
    for sources in cases:
        with pytest.raises((ValueError, RuntimeError)):
            plane.load_scatter([1, 2], sources)
    assert host_kernels.launches == []
    after = cache_bits(caches)
    assert all(torch.equal(after[name], before[name]) for name in names)


def test_a_failed_launch_drains_the_stream_before_the_sources_can_be_released(qwen):
    caches, plane, names = qwen
    stream = MagicMock(cuda_stream=9)
    plane._copy_stream = stream
    plane._load_tables()
    sources = slabs(plane, 2, shared=True)
    with patch.object(dataplane, "copy_host_blocks", side_effect=RuntimeError("launch failed")):
        with pytest.raises(RuntimeError, match="launch failed"):
            plane.load_scatter([1, 2], sources)
    stream.synchronize.assert_called_once_with()


def test_a_saved_snapshot_restores_into_other_blocks(qwen):
    caches, plane, names = qwen
    saved, restored = [3, 4, 5, 8, 11], [0, 1, 2, 6, 7]
    targets = slabs(plane, len(saved), shared=True)
    expected = {name: [span_of(caches[name], b) for b in saved] for name in names}
    assert plane.save_gather(saved, targets, 5 * TOKENS) == 1
    assert plane.load_scatter(restored, targets) == 1
    for name in names:
        assert [span_of(caches[name], b) for b in restored] == expected[name]


def test_ids_and_counts_are_validated(qwen):
    caches, plane, names = qwen
    for ids in ([12], [-1], [1.0], ["1"]):
        with pytest.raises(ValueError):
            plane.load_scatter(ids, slabs(plane, 1, shared=True))
    with pytest.raises(ValueError):
        plane.load_scatter([1, 2], slabs(plane, 1, shared=True))
    with pytest.raises(ValueError):
        plane.save_gather([1, 2], slabs(plane, 2, shared=True), 33)      # 33 tokens need 3 blocks
    assert plane.save_gather([], [], 0) == 0
    assert plane.load_scatter([], []) == 0


# ---------------------------------------------------------------- other layouts


@pytest.mark.parametrize("strides", [(96, 32, 8, 1), (96, 8, 24, 1), (192, 32, 8, 1), (192, 8, 24, 1)])
def test_tail_zeroing_and_restore_follow_the_actual_strides(strides):
    """The reference's stride permutations (test_scatter_gather.py:291-317): a [5, 3, 4, 8] cache whose
    H and N axes are laid out either way, with blocks packed or interleaved with another layer."""
    heads, tokens, width = 3, 4, 8
    memory = torch.arange(5 * strides[0], dtype=torch.int16)
    cache = memory.view(torch.bfloat16).as_strided((5, heads, tokens, width), strides)
    plane = plane_over({"layer.0": cache}, block_size=tokens)
    original = memory.clone()
    targets = slabs(plane, 2, shared=False)
    plane.save_gather([1, 3], targets, 6)                 # the last block keeps 2 of its 4 tokens
    for i, block in enumerate((1, 3)):
        span = original[block * strides[0]:block * strides[0] + 96].clone()
        if i == 1:
            for head in range(heads):
                for token in (2, 3):
                    at = head * strides[1] + token * strides[2]
                    span[at:at + width] = 0
        assert targets[i][0].at(0, 192) == span.numpy().tobytes()
    assert torch.equal(memory, original)
    plane.load_scatter([0, 4], targets)
    want = original.clone()
    for block, (slab, _) in zip((0, 4), targets):
        want[block * strides[0]:block * strides[0] + 96] = torch.frombuffer(bytearray(slab.at(0, 192)),
                                                                             dtype=torch.int16)
    assert torch.equal(memory, want)


def test_kv_split_layers_pack_k_then_v_and_zero_both_tails():
    generator = torch.Generator().manual_seed(3)
    memory = torch.randint(-2**15, 2**15, (3, 2, 6, 4, 2, 8), dtype=torch.int16, generator=generator)
    caches = {f"layer.{i}": memory[i].view(torch.bfloat16) for i in range(3)}    # [K/V, blocks, N=4, H=2, C=8]
    plane = plane_over(caches, block_size=4)
    assert plane.layers[0]["shape"] == [2, 4, 2, 8] and plane.layers[0]["bytes"] == 256
    assert plane.block_bytes == 3 * 256
    targets = slabs(plane, 2, shared=True)
    plane.save_gather([4, 1], targets, 7)                  # the last block keeps 3 of 4 tokens
    slab = targets[0][0]
    for i, block in enumerate((4, 1)):
        record = slab.at(i * plane.block_bytes, plane.block_bytes)
        for layer in range(3):
            for half in range(2):
                span = bytearray(memory[layer, half, block].numpy().tobytes())
                if i == 1:
                    span[3 * 2 * 8 * 2:] = bytes(len(span) - 3 * 2 * 8 * 2)
                at = layer * 256 + half * 128
                assert record[at:at + 128] == bytes(span), (block, layer, half)
    before = memory.clone()
    plane.load_scatter([0, 5], targets)
    first = torch.frombuffer(bytearray(slab.at(0, plane.block_bytes)), dtype=torch.int16)
    assert torch.equal(memory[:, :, 0].reshape(-1), first)
    assert torch.equal(memory[:, :, 1:5], before[:, :, 1:5])


def test_tail_regions_equal_the_oracle_rule_on_random_records(qwen):
    caches, plane, names = qwen
    rng = np.random.default_rng(0)
    for valid in (1, 5, 15):
        record = rng.integers(0, 256, plane.block_bytes, dtype=np.uint8)
        want = record.copy()
        oracle.zero_tail(want, plane.layers, valid)
        got = record.copy()
        regions = plane._tail_regions(valid)
        for start, length in regions:
            got[start:start + length] = 0
        assert np.array_equal(got, want)
        assert len(regions) == LAYERS    # token-major storage: one merged range per layer


def test_digests_are_returned_in_block_order():
    caches = qwen3_8b_caches(6, seed=2)
    plane = plane_over(caches)
    size = plane.block_bytes

    class OracleHashJob:
        """The oracle in place of the GPU hash job, behind the same interface."""

        def __init__(self, torch_module, records_ptr, record_bytes, record_pitch, n, device, lane, slice_blocks, *,
                     timer=None, keepalive=None, crc=None):
            crcs, shas = oracle.digest_records(records_ptr, record_bytes, record_pitch, n)
            self.crc, self.sha = torch.from_numpy(crcs.astype(np.int64)), torch.from_numpy(shas)

        def query(self):
            return True

        def finished(self, timeout=None):
            return True

        def synchronize(self):
            pass

    targets = slabs(plane, 3, shared=True)
    digests = []
    with patch.object(dataplane, "HashJob", OracleHashJob), \
         patch.object(TorchBlockDataPlane, "_hash_lane", lambda self: MagicMock()):
        plane.save_gather([5, 2, 4], targets, 3 * TOKENS - 2, digests=digests)
    for i, (hexdigest, crc) in enumerate(digests[0].result()):
        record = targets[0][0].at(i * size, size)
        assert crc == oracle.crc32c(record) and hexdigest == oracle.sha256(record).hex()


def test_a_hashed_save_gathers_its_later_records_on_the_lead_stream_and_copies_them_after(host_kernels):
    """The order of a split save's work, stream by stream.  The lead stream starts from where the copy stream
    stood before the first gather.  It gathers every record past the first chunk and zeroes the last one's
    tail.  The copy stream copies the first chunk, then waits for the lead stream before copying the rest.
    The hash lane waits for both gathers."""
    caches = qwen3_8b_caches(12, seed=4)
    plane = plane_over(caches)
    size, log = plane.block_bytes, []
    current = [None]

    class Stream:
        def __init__(self, name, handle):
            self.name, self.cuda_stream = name, handle

        def wait_event(self, event):
            log.append((self.name, "waits", event.label))

        def synchronize(self):
            pass

    class Event:
        count = 0

        def record(self, stream=None):
            Event.count += 1
            self.label = Event.count
            log.append((stream.name, "records", self.label))

        def synchronize(self):
            pass

    @contextmanager
    def on(stream):
        before, current[0] = current[0], stream
        try:
            yield
        finally:
            current[0] = before

    copy, lead, hashes = Stream("copy", 7), Stream("lead", 9), Stream("hash", 11)
    names = {7: "copy", 9: "lead"}
    plane._copy_stream = copy
    plane.torch.cuda.Event, plane.torch.cuda.stream = Event, on
    gather, zero = host_kernels.kvsnap_gather_blocks, host_kernels.kvsnap_zero_regions

    def logged_gather(*args):
        log.append((names[args[-1]], "gathers", args[1]))
        return gather(*args)

    def logged_zero(*args):
        log.append((names[args[-1]], "zeroes", args[3]))
        return zero(*args)

    class Targets(Slab):
        def copy(self, device_ptr, nbytes, offset=0, **kwargs):
            log.append(("copy", "copies", offset // size, nbytes // size))
            super().copy(device_ptr, nbytes, offset, **kwargs)

    arena = Arena(8 * size)
    slab = Targets(arena, arena.memory.ctypes.data, 5 * size)
    blocks, tokens = [7, 2, 9, 3, 4], 4 * TOKENS + 5
    with patch.object(host_kernels, "kvsnap_gather_blocks", logged_gather), \
         patch.object(host_kernels, "kvsnap_zero_regions", logged_zero), \
         patch.object(dataplane, "_current_stream_handle", lambda device: current[0].cuda_stream), \
         patch.object(TorchBlockDataPlane, "_lead_stream", lambda self: lead), \
         patch.object(TorchBlockDataPlane, "_hash_lane", lambda self: SimpleNamespace(stream=hashes)), \
         patch.object(dataplane, "HashJob", MagicMock()):
        copies = plane.save_gather(blocks, [(slab, i * size) for i in range(5)], tokens,
                                   chunk_bytes=2 * size, digests=[])
    assert copies == 2                    # the back-to-back run of targets is cut where the lead's records start
    begun, first, rest, landed = 1, 2, 3, 4       # events in the order recorded
    assert log == [("copy", "records", begun),
                   ("copy", "gathers", 2), ("copy", "records", first),
                   ("lead", "waits", begun), ("lead", "gathers", 3), ("lead", "zeroes", LAYERS),
                   ("lead", "records", rest),
                   ("copy", "copies", 0, 2), ("copy", "waits", rest), ("copy", "copies", 2, 3),
                   ("copy", "records", landed),
                   ("hash", "waits", first), ("hash", "waits", rest)]
    for i, block in enumerate(blocks):
        for position, name in enumerate(sorted(caches)):
            want = bytearray(span_of(caches[name], block))
            if i == len(blocks) - 1:
                want[5 * HEADS * WIDTH * 2:] = bytes(len(want) - 5 * HEADS * WIDTH * 2)
            assert slab.at(i * size + position * SPAN, SPAN) == bytes(want), (block, name)


def test_a_copy_engine_restore_places_chunks_aside_while_the_next_is_copied(host_kernels):
    """The order of a copy-engine restore's work with an aside stream, stream by stream.  Chunks alternate
    between two staging slots.  Each chunk's copies go on the restore stream, its placement on the aside
    stream after them, and a slot is copied into again only once the placement that last read it is done.
    The restore stream waits for the last placement, the progress marks follow the placements, and the
    blocks hold the saved bytes."""
    caches = qwen3_8b_caches(16, seed=6)
    plane = plane_over(caches, restore_mode="dma")
    size, log = plane.block_bytes, []
    current = [None]

    class Stream:
        def __init__(self, name, handle):
            self.name, self.cuda_stream = name, handle

        def wait_event(self, event):
            log.append((self.name, "waits", event.label))

        def synchronize(self):
            pass

    class Event:
        count = 0

        def record(self, stream=None):
            Event.count += 1
            self.label = Event.count
            log.append((stream.name, "records", self.label))

        def synchronize(self):
            pass

        def query(self):
            return True

    @contextmanager
    def on(stream):
        before, current[0] = current[0], stream
        try:
            yield
        finally:
            current[0] = before

    saved, restored = [3, 4, 5, 8, 11], [0, 1, 2, 6, 7]
    targets = slabs(plane, len(saved), shared=True)
    expected = {name: [span_of(caches[name], b) for b in saved] for name in sorted(caches)}
    plane.save_gather(saved, targets, 5 * TOKENS)
    copy, place = Stream("copy", 7), Stream("place", 9)
    names = {7: "copy", 9: "place"}
    plane._copy_stream = copy
    plane.torch.cuda.Event, plane.torch.cuda.stream = Event, on
    to_device, scatter = host_kernels.kvsnap_copy_to_device, host_kernels.kvsnap_scatter_blocks
    slab_at = targets[0][0].pointer

    def logged_copy(dst, src, nbytes, stream):
        if slab_at <= src < slab_at + 5 * size:         # a record copy, not the launch tables' upload
            log.append((names[stream], "copies", (src - slab_at) // size, nbytes // size))
        return to_device(dst, src, nbytes, stream)

    def logged_scatter(*args):
        log.append((names[args[-1]], "places", args[3]))
        return scatter(*args)

    progress = []
    with patch.object(host_kernels, "kvsnap_copy_to_device", logged_copy), \
         patch.object(host_kernels, "kvsnap_scatter_blocks", logged_scatter), \
         patch.object(dataplane, "_current_stream_handle", lambda device: current[0].cuda_stream), \
         patch.object(dataplane, "_drain", lambda torch, stream: None), \
         patch.object(TorchBlockDataPlane, "_place_stream", lambda self: place):
        assert plane.load_scatter(restored, targets, progress=progress, chunk_bytes=2 * size) == 3
    copied0, mark0, placed0, copied1, mark1, placed1, copied2, mark2, placed2 = range(1, 10)
    assert log == [("copy", "copies", 0, 2), ("copy", "records", copied0),
                   ("place", "waits", copied0), ("place", "places", 2), ("place", "records", mark0),
                   ("place", "records", placed0),
                   ("copy", "copies", 2, 2), ("copy", "records", copied1),
                   ("place", "waits", copied1), ("place", "places", 2), ("place", "records", mark1),
                   ("place", "records", placed1),
                   ("copy", "waits", placed0), ("copy", "copies", 4, 1), ("copy", "records", copied2),
                   ("place", "waits", copied2), ("place", "places", 1), ("place", "records", mark2),
                   ("place", "records", placed2),
                   ("copy", "waits", placed2)]
    assert [left for _, left in progress] == [5 * size, 3 * size, size, 0]
    for name in sorted(caches):
        assert [span_of(caches[name], b) for b in restored] == expected[name]


@pytest.mark.parametrize("launches,batches", [(1, [[0]]), (3, [[0], [1], [2]]), (4, [[0], [1], [2], [3]]),
                                               (5, [[0, 1], [2], [3], [4]]), (8, [[0, 1, 2, 3], [4], [5], [6], [7]]),
                                               (19, [[0, 1, 2, 3], [4, 5, 6, 7], [8, 9, 10, 11], [12, 13, 14, 15],
                                                     [16], [17], [18]])])
def test_copy_engine_restores_copy_up_to_four_launches_at_a_time_but_the_last_three(launches, batches):
    bounds = [(28 * k, 28 * k + 28) for k in range(launches)]
    assert TorchBlockDataPlane._copy_batches(bounds, True) == batches
    assert TorchBlockDataPlane._copy_batches(bounds, False) == [[k] for k in range(launches)]


class Shape:
    """Shape and stride arithmetic with no storage, as the reference's layout tests use (test_kv_layout.py)."""

    device = CUDA
    dtype = "torch.bfloat16"

    def __init__(self, shape, strides):
        self.shape, self.strides = tuple(shape), tuple(strides)
        self.ndim = len(shape)

    def stride(self, axis=None):
        return self.strides if axis is None else self.strides[axis]

    def element_size(self):
        return 2


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
    with patch.dict(sys.modules, {"torch": SimpleNamespace()}), \
         patch.object(dataplane, "CudaPool", return_value=MagicMock()):
        if block_bytes is None:
            with pytest.raises(ValueError):
                TorchBlockDataPlane({"layer.0": Shape(shape, strides)}, block_size, 4096)
        else:
            assert TorchBlockDataPlane({"layer.0": Shape(shape, strides)}, block_size, 4096).block_bytes == block_bytes


def test_registration_requires_one_cuda_device():
    with patch.dict(sys.modules, {"torch": SimpleNamespace()}), \
         patch.object(dataplane, "CudaPool", return_value=MagicMock()):
        with pytest.raises(ValueError):
            TorchBlockDataPlane({}, 4, 4096)
        on_cpu = Shape((5, 3, 4, 8), (96, 8, 24, 1))
        on_cpu.device = SimpleNamespace(type="cpu", index=None)
        with pytest.raises(ValueError, match="one and the same CUDA device"):
            TorchBlockDataPlane({"layer.0": on_cpu}, 4, 4096)


def test_restore_mode_is_checked():
    caches = {"layer.0": torch.zeros(4, 2, TOKENS, 8)}
    with pytest.raises(ValueError, match="restore_mode"):
        plane_over(caches, restore_mode="fast")


# ---------------------------------------------------------------- ordering helpers


def test_early_report_follows_the_reference_rule():
    """vllm.py:649-679 as pinned by test_failure_policy.py:180-206."""
    from kvsnap_amd.ordering import EARLY_REPORT_BYTES, copy_left, early_launch_index, early_report
    mib = 1 << 20
    done, pending = MagicMock(query=MagicMock(return_value=True)), MagicMock(query=MagicMock(return_value=False))
    progress = [(None, 300 * mib), (done, 200 * mib), (done, 100 * mib), (pending, 0)]
    assert copy_left(progress) == 100 * mib
    assert early_report(progress) == (100 * mib, pending)
    assert early_report([(None, 300 * mib), (done, 200 * mib), (pending, 100 * mib), (pending, 0)]) is None
    assert copy_left([(None, 300 * mib), (done, 100 * mib), (pending, 50 * mib)]) is None     # still queuing
    assert EARLY_REPORT_BYTES == 128 * mib
    assert early_launch_index(progress) == 1
    # the oracle's restatement of the same rule agrees on the same scenario
    assert oracle.copy_left([(None if e is None else e.query, l) for e, l in progress]) == copy_left(progress)


def test_restore_progress_reaches_the_early_report_threshold_at_the_expected_launch():
    """An 8k-token Qwen3-8B restore: 19 launches of 28 blocks; reportable after the 17th."""
    from kvsnap_amd.ordering import early_launch_index
    size = 36 * 65536
    per_launch = (64 << 20) // size
    progress = [(None, 512 * size)] + [(MagicMock(), (512 - min(512, (k + 1) * per_launch)) * size)
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


# ---------------------------------------------------------------- device staging


class NoDeviceMemory(CpuCuda):
    """CpuCuda whose device allocations above 1 MiB fail as torch's do when the GPU is full."""

    def empty(self, *args, **kwargs):
        if kwargs.get("device") is CUDA:
            count = args[0] if args and isinstance(args[0], int) else 1
            if count > (1 << 20):
                raise torch.OutOfMemoryError("CUDA out of memory. Tried to allocate 504.00 MiB")
        return super().empty(*args, **kwargs)


def test_a_copy_engine_restore_without_device_memory_is_refused_before_any_copy(host_kernels, monkeypatch):
    """With no reserved staging and a full GPU, load_scatter (copy engines) and load_scatter_checked raise
    StagingUnavailable before uploading or copying anything: no launch, no copy, the cache untouched."""
    monkeypatch.setattr(dataplane, "PLACE_ASIDE", False)
    caches = qwen3_8b_caches(12)
    plane = plane_over(caches, restore_mode="dma")
    plane.torch = NoDeviceMemory()
    copies = []
    host_kernels.kvsnap_copy_to_device = lambda *args: copies.append(args) or 0
    sources = slabs(plane, 3, shared=True)
    before = cache_bits(caches)
    with pytest.raises(dataplane.StagingUnavailable, match="out of memory"):
        plane.load_scatter([1, 2, 3], sources)
    with pytest.raises(dataplane.StagingUnavailable):
        plane.load_scatter_checked([1, 2, 3], sources, [0, 0, 0])
    assert copies == [] and host_kernels.launches == []
    after = cache_bits(caches)
    assert all(torch.equal(after[name], before[name]) for name in caches)


def test_restores_take_their_staging_from_the_reserve_and_allocate_nothing(host_kernels, monkeypatch):
    """A plane holding its reserved device staging restores through the copy engines with every device
    allocation failing: the slots are slices of the reserve, and the blocks land."""
    monkeypatch.setattr(dataplane, "PLACE_ASIDE", False)        # copies and placements in turn, one stream
    caches = qwen3_8b_caches(12)
    plane = plane_over(caches, restore_mode="dma")
    assert plane.device_staging_bytes == dataplane.DEVICE_STAGING_BYTES
    plane._reserved_staging = torch.empty(4 * plane.block_bytes + (1 << 20), dtype=torch.uint8)
    plane.torch = NoDeviceMemory()
    size = plane.block_bytes
    sources = slabs(plane, 3, shared=True)
    for i, block in enumerate([4, 5, 6]):
        for position, name in enumerate(sorted(caches)):
            sources[i][0].fill(sources[i][1] + position * SPAN, span_of(caches[name], block))
    assert plane.load_scatter([1, 2, 3], sources, chunk_bytes=size) == 3
    for name in caches:
        for target, block in zip([1, 2, 3], [4, 5, 6]):
            assert span_of(caches[name], target) == span_of(caches[name], block)
    assert plane._reserved_lock.acquire(blocking=False)       # handed back
    plane._reserved_lock.release()


def test_a_batched_checked_copy_engine_restore_keeps_its_slots_and_targets_apart(host_kernels, monkeypatch):
    """load_scatter_checked at its default chunking through the copy engines, with more launches than
    COPY_BATCH + COPY_TAIL (launches of two blocks here): copies grouped four launches at a time but the last
    three, alternating between two device slots; each launch places and checks its blocks from its slot, at
    its own offset, on the aside stream; a slot is copied into again only after the placements that read it.
    Every target block holds its own source's bytes and every CRC32C passes; a wrong one fails that block."""
    caches = qwen3_8b_caches(48, seed=9)
    plane = plane_over(caches, restore_mode="dma")
    plane.pool = Arena(160 << 20)
    size = plane.block_bytes
    monkeypatch.setattr(TorchBlockDataPlane, "_launch_bounds",
                        lambda self, n, chunk_bytes: [(a, min(n, a + 2)) for a in range(0, n, 2)])
    saved = list(range(1, 21))
    restored = list(range(47, 27, -1))
    sources = slabs(plane, 20, shared=True)
    plane.save_gather(saved, sources, 20 * TOKENS)
    crcs = [oracle.crc32c(sources[0][0].at(i * size, size)) for i in range(20)]
    log = []

    class Stream:
        def __init__(self, name, handle):
            self.name, self.cuda_stream = name, handle

        def wait_event(self, event):
            log.append((self.name, "waits", event.label))

        def synchronize(self):
            pass

    class Event:
        count = 0

        def record(self, stream=None):
            Event.count += 1
            self.label = Event.count
            log.append((stream.name, "records", self.label))

        def synchronize(self):
            pass

        def query(self):
            return True

    copy, place = Stream("copy", 7), Stream("place", 9)
    names = {7: "copy", 9: "place"}
    plane._copy_stream = copy
    plane.torch.cuda.Event = Event
    to_device, checked = host_kernels.kvsnap_copy_to_device, host_kernels.kvsnap_restore_blocks_checked
    slab_at = sources[0][0].pointer
    slot_of = {}

    def logged_copy(dst, src, nbytes, stream):
        if slab_at <= src < slab_at + 20 * size:             # a record copy, not a table upload
            first = (src - slab_at) // size
            log.append((names[stream], "copies", first, nbytes // size))
            for j in range(nbytes // size):
                slot_of[first + j] = dst + j * size
        return to_device(dst, src, nbytes, stream)

    def logged_checked(sources_table, blocks, n, *rest):
        reads = list((C.c_int64 * n).from_address(sources_table))
        targets = list((C.c_int64 * n).from_address(blocks))
        first = restored.index(targets[0])
        # every block is read from where its own record was copied, and lands in its own target
        assert reads == [slot_of[first + j] for j in range(n)], first
        assert targets == restored[first:first + n]
        log.append((names[rest[-1]], "checks", first, n))
        return checked(sources_table, blocks, n, *rest)

    with patch.object(host_kernels, "kvsnap_copy_to_device", logged_copy), \
         patch.object(host_kernels, "kvsnap_restore_blocks_checked", logged_checked), \
         patch.object(dataplane, "_drain", lambda torch, stream: None), \
         patch.object(TorchBlockDataPlane, "_place_stream", lambda self: place):
        assert plane.load_scatter_checked(restored, sources, crcs) == 10
    copies = [entry[2:] for entry in log if entry[1] == "copies"]
    assert copies == [(0, 8), (8, 6), (14, 2), (16, 2), (18, 2)]        # launches [0-3], [4-6], 7, 8, 9
    checks = [entry[2:] for entry in log if entry[1] == "checks"]
    assert checks == [(2 * k, 2) for k in range(10)] and all(e[0] == "place" for e in log if e[1] == "checks")
    # the third copy (slot 0 again) waits for the event the place stream recorded after the first batch's checks
    third = log.index(("copy", "copies", 14, 2))
    waited = [e for e in log[:third] if e[0] == "copy" and e[1] == "waits"][-1][2]
    last_check_of_first = max(i for i, e in enumerate(log) if e[:2] == ("place", "checks") and e[2] < 8)
    assert ("place", "records", waited) in log[last_check_of_first:third]
    for name in caches:
        for target, block in zip(restored, saved):
            assert span_of(caches[name], target) == span_of(caches[name], block), (name, target)
    bad = list(crcs)
    bad[5] ^= 1
    with patch.object(dataplane, "_drain", lambda torch, stream: None), \
         patch.object(TorchBlockDataPlane, "_place_stream", lambda self: place):
        with pytest.raises(CorruptSnapshotError, match="first: block 5"):
            plane.load_scatter_checked(restored, sources, bad)


@pytest.mark.parametrize("tokens", [3 * TOKENS, 3 * TOKENS - 5])
def test_a_hashed_direct_save_gathers_records_stage_and_crcs_in_one_pass(host_kernels, tokens):
    """A direct save with digests: the checked gather writes every pinned record and its device copy (the SHA-256
    kernels' input) from one read of the cache and gives the CRC32Cs; the hash job gets those CRC32Cs and
    launches only the SHA-256.  With a partial last block, its tail is zeroed in both copies and its CRC32C is
    taken again: every CRC32C equals the oracle's over the pinned record, and the device copy equals it."""
    caches = qwen3_8b_caches(6, seed=4)
    plane = plane_over(caches, save_mode="direct")
    size = plane.block_bytes
    seen = {}

    class Job:
        def __init__(self, torch_module, records_ptr, record_bytes, record_pitch, n, device, lane, slice_blocks, *,
                     timer=None, keepalive=None, crc=None):
            seen.update(records=C.string_at(records_ptr, n * record_bytes), crc=crc)
            self.crc = crc
            self.sha = torch.zeros((n, 32), dtype=torch.uint8)

        def query(self):
            return True

        def finished(self, timeout=None):
            return True

        def synchronize(self):
            pass

    targets = slabs(plane, 3, shared=True)
    digests = []
    with patch.object(dataplane, "HashJob", Job), \
         patch.object(TorchBlockDataPlane, "_hash_lane", lambda self: MagicMock()):
        assert plane.save_gather([5, 2, 4], targets, tokens, digests=digests) == 1
    assert [kind for kind, _ in host_kernels.launches if kind.startswith("gather")] == ["gather_checked"]
    pinned = targets[0][0].at(0, 3 * size)
    assert seen["records"] == pinned
    for i, block in enumerate([5, 2, 4]):
        assert pinned[i * size:i * size + SPAN] == (span_of(caches[sorted(caches)[0]], block) if i < 2 or
                                                     tokens % TOKENS == 0 else pinned[i * size:i * size + SPAN])
    crcs = [int(c) & 0xFFFFFFFF for c in seen["crc"].view(torch.int32).tolist()]
    assert crcs == [oracle.crc32c(pinned[i * size:(i + 1) * size]) for i in range(3)]
    if tokens % TOKENS:
        want = bytearray(span_of(caches[sorted(caches)[0]], 4))
        want[(tokens % TOKENS) * HEADS * WIDTH * 2:] = bytes(len(want) - (tokens % TOKENS) * HEADS * WIDTH * 2)
        assert pinned[2 * size:2 * size + SPAN] == bytes(want)
        assert ("crc32c", 1) in host_kernels.launches


@pytest.mark.parametrize("tokens", [3 * TOKENS, 3 * TOKENS - 5])
@pytest.mark.parametrize("limit,fused", [(1 << 30, True), (0, False)])
def test_a_small_hashed_staged_save_gathers_records_and_crcs_in_one_pass(host_kernels, monkeypatch, tokens, limit,
                                                                        fused):
    """A staged save with digests of at most GATHER_CRC_MAX_BYTES, over whole-KiB spans: one gather with CRC32C
    packs the device records (the copies' and the SHA-256 kernels' input) and gives their CRC32Cs, and the hash
    job gets them and launches only the SHA-256.  A zeroed tail has its record's CRC32C taken again.  Over the
    limit the save gathers and leaves the CRC32Cs to the hash job.  Either way the pinned records equal the
    device records, and every given CRC32C the oracle's over its pinned record."""
    monkeypatch.setattr(dataplane, "GATHER_CRC_MAX_BYTES", limit)
    host_kernels.fused = True
    caches = qwen3_8b_caches(6, seed=5)
    plane = plane_over(caches)
    size = plane.block_bytes
    seen = {}

    class Job:
        def __init__(self, torch_module, records_ptr, record_bytes, record_pitch, n, device, lane, slice_blocks, *,
                     timer=None, keepalive=None, crc=None):
            seen.update(records=C.string_at(records_ptr, n * record_bytes), crc=crc)
            self.crc = crc
            self.sha = torch.zeros((n, 32), dtype=torch.uint8)

        def query(self):
            return True

        def finished(self, timeout=None):
            return True

        def synchronize(self):
            pass

    targets = slabs(plane, 3, shared=True)
    with patch.object(dataplane, "HashJob", Job), \
         patch.object(TorchBlockDataPlane, "_hash_lane", lambda self: MagicMock()):
        plane.save_gather([5, 2, 4], targets, tokens, digests=[])
    kinds = [kind for kind, _ in host_kernels.launches]
    assert [k for k in kinds if k.startswith("gather")] == (["gather_crc"] if fused else ["gather"])
    pinned = targets[0][0].at(0, 3 * size)
    assert seen["records"] == pinned
    for i, block in enumerate([5, 2, 4]):
        for position, name in enumerate(sorted(caches)):
            want = bytearray(span_of(caches[name], block))
            if i == 2 and tokens % TOKENS:
                cut = (tokens % TOKENS) * HEADS * WIDTH * 2
                want[cut:] = bytes(len(want) - cut)
            assert pinned[i * size + position * SPAN:i * size + (position + 1) * SPAN] == bytes(want), (block, name)
    if fused:
        crcs = [int(c) & 0xFFFFFFFF for c in seen["crc"].view(torch.int32).tolist()]
        assert crcs == [oracle.crc32c(pinned[i * size:(i + 1) * size]) for i in range(3)]
        assert kinds.count("crc32c") == (1 if tokens % TOKENS else 0)   # the zeroed tail's record, taken again
    else:
        assert seen["crc"] is None and "crc32c" not in kinds


def test_the_groups_table_follows_the_spans_and_is_refused_for_spans_that_are_not_whole_kib(host_kernels):
    """For whole-KiB spans, group g of a record comes from its span's base plus (g's KiB within the span), at the
    span's pitch; a layout with a span of another length has no table (its saves gather, then take CRC32Cs)."""
    host_kernels.fused = True
    caches = qwen3_8b_caches(4, seed=1)
    plane = plane_over(caches)
    bases, pitches = plane.group_tables()
    spans = plane.spans()
    assert bases.numel() == pitches.numel() == plane.block_bytes // 1024
    for offset, base, pitch, nbytes in spans:
        for k in range(nbytes // 1024):
            assert (int(bases[offset // 1024 + k]), int(pitches[offset // 1024 + k])) == (base + 1024 * k, pitch)
    storage = torch.zeros((2, 4, 16, 1, 40), dtype=torch.bfloat16)          # 1280-byte spans
    odd = plane_over({f"model.layers.{i}.self_attn.attn": storage[i].permute(0, 2, 1, 3) for i in range(2)})
    assert odd.group_tables() is None
    host_kernels.fused = False
    assert plane_over(caches).group_tables() is None


def test_a_restore_stream_without_a_fast_engine_pair_is_reported(caplog):
    """The copy-engine pick keeps its best candidate either way; when none overlapped the copy stream's engine
    as the fast engines do, the plane says so in a warning (the pair it kept and every candidate's)."""
    accepted = {"candidates": 1, "both_ways_gbps": 96.1, "accepted": True, "tried_both_ways_gbps": [96.1]}
    missed = {"candidates": 4, "both_ways_gbps": 92.5, "accepted": False,
              "tried_both_ways_gbps": [57.7, 92.5, 57.7, 57.7]}
    with caplog.at_level("WARNING", logger="kvsnap_amd.dataplane"):
        assert not dataplane.report_engine_pick(None)
        assert not dataplane.report_engine_pick(accepted)
        assert not caplog.records
        assert dataplane.report_engine_pick(missed)
    (record,) = caplog.records
    assert record.levelname == "WARNING"
    assert "92.5 GB/s" in record.getMessage() and "[57.7, 92.5, 57.7, 57.7]" in record.getMessage()
