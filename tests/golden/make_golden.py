"""Write tests/golden/golden.json from sources independent of the oracle.

    make -f oracle/ref.mk && python tests/golden/make_golden.py

* CRC32C: the reference's own csrc/dataplane/io.cpp, compiled from the
  read-only reference tree into oracle/_ref/libkvsnap_io_ref.so, over seeded
  bytes of many lengths (including extend-from-a-prior cases).
* SHA-256: hashlib (OpenSSL), over the same bytes.
* Records: the reference's Qwen3-8B fixture geometry
  (tests/connector/test_scatter_gather.py:3-13, 137-158): 36 layers of
  [blocks, 8 heads, 16 tokens, 256] bf16 views over [blocks, 16, 8, 256]
  storage, filled with seeded random 16-bit patterns; each record is built
  with torch's own strided indexing (view[block].permute(1, 0, 2)), in sorted
  layer-name order, and the tail of the last block zeroed as that test expects
  (:197-204).  Stored as SHA-256 + CRC32C per record.
* Layout accept/reject: tests/connector/test_kv_layout.py:60-80.

The inputs are regenerated from numpy's PCG64 with the stated seeds.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import json
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
OUT = Path(__file__).resolve().parent / "golden.json"
REF_IO = ROOT / "oracle" / "_ref" / "libkvsnap_io_ref.so"

CRC_LENGTHS = [0, 1, 2, 3, 4, 7, 8, 9, 15, 16, 17, 31, 63, 64, 65, 127, 128, 1023, 4095, 4096, 4097,
               12287, 12288, 12289, 65536, 100003]
LAYERS, HEADS, BLOCK_SIZE, WIDTH = 36, 8, 16, 256


def random_bytes(seed, n):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8).tobytes()


def fixture_storage(blocks, seed=7):
    """[LAYERS, blocks, 16 tokens, 8 heads, 256] int16 patterns (the fixture's backing)."""
    return np.random.default_rng(seed).integers(-2**15, 2**15, (LAYERS, blocks, BLOCK_SIZE, HEADS, WIDTH),
                                                dtype=np.int16)


def main():
    ref = C.CDLL(str(REF_IO))
    ref.kvsnap_crc32c_extend.argtypes = [C.c_char_p, C.c_size_t, C.c_uint32]
    ref.kvsnap_crc32c_extend.restype = C.c_uint32
    crc = []
    for length in CRC_LENGTHS:
        data = random_bytes(1000 + length, length)
        for prior in (0, 0xE3069283):
            crc.append({"seed": 1000 + length, "length": length, "prior": prior,
                        "crc32c": int(ref.kvsnap_crc32c_extend(data, length, prior))})
    sha = [{"seed": 1000 + length, "length": length, "sha256": hashlib.sha256(random_bytes(1000 + length, length)).hexdigest()}
           for length in CRC_LENGTHS]

    import torch
    blocks = 6
    backing = torch.from_numpy(fixture_storage(blocks)).view(torch.bfloat16)
    names = sorted(f"model.layers.{i}.self_attn.attn" for i in range(LAYERS))
    views = {f"model.layers.{i}.self_attn.attn": backing[i].permute(0, 2, 1, 3) for i in range(LAYERS)}
    block_ids, tokens = [5, 0, 3, 1], 3 * BLOCK_SIZE + 5
    records = []
    for index, block in enumerate(block_ids):
        parts = []
        for name in names:
            span = bytearray(views[name][block].permute(1, 0, 2).contiguous().view(torch.int16).numpy().tobytes())
            if index == len(block_ids) - 1:
                span[5 * HEADS * WIDTH * 2:] = bytes((BLOCK_SIZE - 5) * HEADS * WIDTH * 2)
            parts.append(bytes(span))
        record = b"".join(parts)
        records.append({"block": block, "bytes": len(record), "sha256": hashlib.sha256(record).hexdigest(),
                        "crc32c": int(ref.kvsnap_crc32c_extend(record, len(record), 0))})

    layouts = [
        {"shape": [5, 3, 4, 8], "stride": [96, 8, 24, 1], "block_size": 4, "block_bytes": 192},
        {"shape": [5, 3, 4, 8], "stride": [192, 32, 8, 1], "block_size": 4, "block_bytes": 192},
        {"shape": [5, 3, 4, 8], "stride": [96, 8, 8, 1], "block_size": 4, "block_bytes": None},
        {"shape": [5, 3, 4, 8], "stride": [48, 32, 8, 1], "block_size": 4, "block_bytes": None},
    ]
    golden = {
        "crc32c": crc,
        "sha256": sha,
        "records": {"geometry": "qwen3-8b fixture, 36 layers [B,8,16,256] over [B,16,8,256] bf16",
                    "storage_seed": 7, "blocks": blocks, "block_ids": block_ids, "num_kv_tokens": tokens,
                    "records": records},
        "layouts": layouts,
    }
    OUT.write_text(json.dumps(golden, indent=1) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
