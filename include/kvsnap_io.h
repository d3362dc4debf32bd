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

#ifdef __cplusplus
}
#endif

#endif /* KVSNAP_IO_H */
