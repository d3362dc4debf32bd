"""MI355X-native KV snapshot dataplane (drop-in for kvsnap's save/restore path).

``dataplane``  pinned pool binding, ``TorchBlockDataPlane``, restore/gather launches
``native_io``  host CRC32C and pread/pwrite pool binding
``crc32c``     incremental host CRC32C
``blobs``      snapshot blob header format and disk-staged reads
``synth``      seeded synthetic KV caches (bench and test input)
``build``      builds ``_native/`` in-tree for gfx950
"""
