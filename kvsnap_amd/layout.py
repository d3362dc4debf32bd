"""KV cache registration: which bytes of each layer one block owns, and the layout identity.

A snapshot record is the concatenation, in sorted layer-name order, of each
layer's per-block bytes copied in physical storage order.  So a layer is
accepted only if one block's elements fill a dense range of its storage,
whatever order the logical axes are laid out in, and blocks do not overlap
(the reference's rule, ``kvsnap/connector/dataplane.py:230-244``, pinned by
its ``tests/connector/test_kv_layout.py`` cases).  The description kept per
layer (name, per-block shape and strides, dtype, bytes) becomes the
snapshot's layout identity (``vllm.py:236``): a snapshot may only be
restored into caches whose identity matches, because two layouts with the
same record size put different elements at the same record offsets.

Two layer shapes are accepted:

* ``[blocks, heads, tokens, width]`` views with contiguous ``width``, the
  reference's only layout (vLLM's ``[blocks, tokens, heads, width]`` storage
  seen as ``[blocks, heads, tokens, width]``); one span per block.
* ``[2, blocks, tokens, heads, width]`` K/V-split caches; each block is a K
  span and a V span, and the layer's part of a record is K then V.
"""
from __future__ import annotations

import json


def dense_extent(axes):
    """Elements one block covers if its (size, stride) axes tile a dense range from its first element,
    else None.  Axes of size 1 take no room and are ignored."""
    covered = 1
    for stride, size in sorted((stride, size) for size, stride in axes if size > 1):
        if stride != covered:
            return None             # a hole below this axis, or an axis overlapping another
        covered *= size
    return covered


def _refuse(name, why):
    raise ValueError(f"KV cache {name!r} has an unsupported layout: {why}")


def _block_major(name, tensor, block_size):
    if tensor.ndim != 4:
        _refuse(name, f"{tensor.ndim} dimensions, expected [blocks, heads, tokens, width]")
    blocks, heads, tokens, width = tensor.shape
    if tokens != block_size:
        _refuse(name, f"{tokens} token slots per block, expected the block size {block_size}")
    if tensor.stride(3) != 1:
        _refuse(name, "the last axis is not contiguous")
    covered = dense_extent([(heads, tensor.stride(1)), (tokens, tensor.stride(2)), (width, 1)])
    if covered is None:
        _refuse(name, "a block's elements do not fill a dense range")
    if tensor.stride(0) < covered:
        _refuse(name, "consecutive blocks overlap")
    return {"name": name, "shape": [heads, tokens, width], "dtype": str(tensor.dtype),
            "stride": [tensor.stride(1), tensor.stride(2), tensor.stride(3)],
            "bytes": heads * tokens * width * tensor.element_size()}


def _kv_split(name, tensor, block_size):
    halves, blocks, tokens, heads, width = tensor.shape
    if halves != 2:
        _refuse(name, "the first axis of a K/V-split cache must have size 2")
    if tokens != block_size:
        _refuse(name, f"{tokens} token slots per block, expected the block size {block_size}")
    if tensor.stride(4) != 1:
        _refuse(name, "the last axis is not contiguous")
    covered = dense_extent([(tokens, tensor.stride(2)), (heads, tensor.stride(3)), (width, 1)])
    if covered is None:
        _refuse(name, "a block's K (or V) elements do not fill a dense range")
    # The K/V axis and the block axis, by stride: the inner one must clear a span, the outer one all of them.
    (inner_stride, inner_count), (outer_stride, _) = sorted([(tensor.stride(0), 2), (tensor.stride(1), blocks)])
    if inner_stride < covered or outer_stride < inner_stride * inner_count:
        _refuse(name, "K and V spans or consecutive blocks overlap")
    return {"name": name, "shape": [2, tokens, heads, width], "dtype": str(tensor.dtype),
            "stride": [tensor.stride(0), tensor.stride(2), tensor.stride(3), tensor.stride(4)],
            "bytes": 2 * tokens * heads * width * tensor.element_size()}


def describe_layer(name, tensor, block_size):
    """The identity entry of one layer, or ValueError if its layout cannot be snapshotted."""
    if tensor.ndim == 5:
        return _kv_split(name, tensor, block_size)
    return _block_major(name, tensor, block_size)


def layout_identity(layers):
    """The snapshot identity string of registered ``layers`` (the reference's kv_layout, vllm.py:236)."""
    return json.dumps(layers, sort_keys=True, separators=(",", ":"))


class LayoutMismatch(ValueError):
    """A snapshot's recorded KV layout is not the registered caches' layout; nothing may be copied."""


def require_layout(snapshot, identity):
    """Refuse ``snapshot`` unless it was taken under layout ``identity`` (reference ``vllm.py:438-444``).

    Two layouts can share a record size (a K/V-split and a vLLM-layout cache
    of one model both make 2,359,296-byte Qwen3-8B records) while putting
    different elements at the same offsets, so the sizes agreeing proves
    nothing: the identity strings must be equal.
    """
    recorded = snapshot.get("kv_layout")
    if recorded is None:
        raise LayoutMismatch("the snapshot records no KV layout")
    if recorded != identity:
        raise LayoutMismatch("the snapshot's KV layout differs from the registered caches' layout")
