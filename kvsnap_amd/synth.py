"""Seeded synthetic KV caches shaped like a model's paged cache (bench and test input).

Two per-layer layouts, both 64 KiB per (layer, block) at Qwen3 shapes in bf16:

* ``"vllm"``: what vLLM 0.31 registers (the reference's fixture,
  tests/connector/test_scatter_gather.py:137-142): storage
  [L, blocks, N, H, 2*D] with K and V side by side, each layer exposed as the
  [blocks, H, N, 2*D] view;
* ``"kv_split"``: [2, blocks, N, H, D] per layer, K and V in separate halves.

Values come from the library's counter-based generator (``kvsnap_synth_fill``),
keyed by (seed, span index, block id, element); the CPU oracle reproduces
them bit for bit.
"""
from __future__ import annotations

import random

from .dataplane import _check, kernel_library

KIND_BF16, KIND_E4M3, KIND_BYTES = 0, 1, 2


def layer_names(layers):
    return [f"model.layers.{i}.self_attn.attn" for i in range(layers)]


def make_caches(layers, num_blocks, *, block_size=16, heads=8, head_dim=128, dtype=None, layout="vllm",
                device="cuda"):
    """Per-layer KV cache views carved from one device allocation (uninitialised)."""
    import torch
    dtype = dtype or torch.bfloat16
    names = layer_names(layers)
    if layout == "vllm":
        backing = torch.empty((layers, num_blocks, block_size, heads, 2 * head_dim), dtype=dtype, device=device)
        return {name: backing[i].permute(0, 2, 1, 3) for i, name in enumerate(names)}, backing
    if layout == "kv_split":
        backing = torch.empty((layers, 2, num_blocks, block_size, heads, head_dim), dtype=dtype, device=device)
        return {name: backing[i] for i, name in enumerate(names)}, backing
    raise ValueError(f"unknown layout {layout}")


def fill(plane, seed, *, kind=KIND_BF16, inv_scales=None, first_block=0, num_blocks=None, stream=None):
    """Fill every span of blocks [first_block, first_block + num_blocks) of a registered plane."""
    import torch
    spans = plane.spans()
    device = next(iter(plane.caches.values())).device
    if num_blocks is None:
        num_blocks = min(plane._num_blocks(t) for t in plane.caches.values()) - first_block
    bases = torch.tensor([s[1] for s in spans], dtype=torch.int64, device=device)
    pitches = torch.tensor([s[2] for s in spans], dtype=torch.int64, device=device)
    words = torch.tensor([s[3] // 8 for s in spans], dtype=torch.int64, device=device)
    for s in spans:
        if s[1] % 16 or s[2] % 16 or s[3] % 16:
            raise ValueError("synthetic fill needs 16-byte aligned spans")
    scales = None
    if inv_scales is not None:
        scales = torch.tensor(list(inv_scales), dtype=torch.float32, device=device)
        if scales.numel() != len(spans):
            raise ValueError("one inverse scale per span")
    lib = kernel_library()
    handle = (stream or torch.cuda.current_stream(device)).cuda_stream
    _check(lib, lib.kvsnap_synth_fill(seed, kind, bases.data_ptr(), pitches.data_ptr(), words.data_ptr(),
                                      scales.data_ptr() if scales is not None else None, len(spans), first_block,
                                      num_blocks, handle))
    return bases, pitches, words, scales   # keep alive until the launch completes


def block_tables(num_blocks, count, *, seed_source=1, seed_target=2):
    """Seeded source and restore-target block ids from [1, num_blocks), disjoint (block 0 is the null block)."""
    source = random.Random(seed_source).sample(range(1, num_blocks), count)
    taken = set(source)
    pool = [b for b in range(1, num_blocks) if b not in taken]
    target = random.Random(seed_target).sample(pool, count)
    return source, target
