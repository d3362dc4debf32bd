/*
 * Host snapshot I/O: C-ABI version 1, built into kvsnap_amd/_native/libkvsnap_io.so.
 *
 * Replaces the reference's csrc/dataplane/io.cpp (simon-jd/kvsnap), bound by
 * kvsnap/store/native_io.py:59-68.  Same symbols and error contract: the I/O
 * entries return 0 or an errno value (never -1).
 */
#ifndef KVSNAP_IO_H
#define KVSNAP_IO_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* CRC32C of `size` bytes extending `prior` (0 starts a new checksum).  io.cpp:39-44 */
uint32_t kvsnap_crc32c_extend(const void* data, size_t size, uint32_t prior);
/* kvsnap_crc32c_extend(data, size, 0).  io.cpp:45-47 */
uint32_t kvsnap_crc32c(const void* data, size_t size);
/* Always 1.  io.cpp:48 */
int kvsnap_io_abi_version(void);

/* Write all `size` bytes at `offset`, retrying EINTR and short writes; a
 * zero-byte write is EIO; `durable` adds fdatasync.  io.cpp:51-69 */
int kvsnap_pwrite_all(int fd, const void* data, size_t size, int64_t offset, int durable);
/* Read exactly `size` bytes at `offset`; end of file is EIO.  io.cpp:71-81 */
int kvsnap_pread_all(int fd, void* data, size_t size, int64_t offset);

/* A pool of 1..64 worker threads with a budget of `max_bytes` in flight, or
 * NULL.  io.cpp:130-133 */
void* kvsnap_io_pool_create(size_t workers, size_t max_bytes);
/* Stops the workers after the queued transfers.  io.cpp:134 */
void kvsnap_io_pool_destroy(void* pool);
/* One pread (write=0) or pwrite (write=1) on a worker, waited for; EMSGSIZE
 * above the budget, ECANCELED while stopping.  io.cpp:135-154 */
int kvsnap_io_pool_transfer(void* pool, int fd, void* data, size_t size, int64_t offset, int write, int durable);

/* The blob ring reader: the disk stage of a restore (replaces the read
 * threads of read_prepared_into, kvsnap/store/store.py:686-723, and their
 * per-block kvsnap_io_pool_transfer calls, io.cpp:135-154).  `threads` native
 * threads (1..64) take blocks 0..n_blocks-1 in order; block i is the payload
 * range [payload_offsets[i], + block_bytes) of the blob file paths[i] (32-byte
 * header "<8sIQI8s": "KVSBLOB1", version 1, payload length, CRC32C, 8 zero
 * bytes), pread into the ring of `slots` slots of `per_chunk` blocks at
 * ring + ((i / per_chunk) % slots) * per_chunk * block_bytes
 * + (i % per_chunk) * block_bytes.  A block of chunk k >= slots waits for
 * kvsnap_blob_reader_release(k - slots).  With `verify`, each block's
 * CRC32C must equal crcs[i].  Paths and tables are copied; the ring is
 * borrowed until kvsnap_blob_reader_finish returns.  NULL on bad arguments. */
void* kvsnap_blob_reader_start(const char* const* paths, const uint64_t* payload_offsets, const uint32_t* crcs,
                               int64_t n_blocks, uint64_t block_bytes, void* ring, int64_t per_chunk, int64_t slots,
                               int threads, int verify);
/* 0 once every block of chunk `chunk` is in its slot; else the error of the
 * first failed block at or before the chunk's end (an errno from open/pread,
 * EIO for a short file, EBADMSG for a bad header, ERANGE for a block past the
 * payload, EILSEQ for a CRC32C mismatch), its index in *failed_block.  The
 * first failure stops the reader.  EINVAL for a chunk out of range. */
int kvsnap_blob_reader_wait(void* reader, int64_t chunk, int64_t* failed_block);
/* Chunk `chunk`'s slot may be refilled. */
int kvsnap_blob_reader_release(void* reader, int64_t chunk);
/* Stops the threads, waits for them and frees the reader; returns the first
 * failure (as kvsnap_blob_reader_wait) or 0. */
int kvsnap_blob_reader_finish(void* reader, int64_t* failed_block);

#ifdef __cplusplus
}
#endif

#endif /* KVSNAP_IO_H */
