/*
 * Pinned snapshot pool: C-ABI version 2, built into kvsnap_amd/_native/libkvsnap_hip.so.
 *
 * Replaces the reference's csrc/dataplane/cuda_pool.cpp (simon-jd/kvsnap),
 * bound by kvsnap/connector/dataplane.py:47-66 and :122-126.  Same symbols,
 * argument meaning and error contract: every int entry returns 0 on success
 * (kvsnap_pool_ready: 1 ready / 0 not ready) and -1 on failure with a
 * thread-local message from kvsnap_cuda_error(); a reservation that cannot fit
 * fails with a message containing "pinned capacity exhausted" and copies
 * nothing.  Copies run on the pool's one non-blocking HIP stream; completion
 * of an allocation's copies is tracked by its event, and release blocks until
 * that completion is proven (otherwise the allocation stays reserved).
 */
#ifndef KVSNAP_POOL_H
#define KVSNAP_POOL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Last error of the calling thread.  cuda_pool.cpp:50 */
const char* kvsnap_cuda_error(void);
/* Same slot under this library's own name (no reference counterpart). */
const char* kvsnap_hip_error(void);

/* Always 2.  cuda_pool.cpp:52 */
int kvsnap_pool_abi_version(void);

/* A pool of `capacity` pinned bytes on `device` (hipHostMalloc, portable and
 * mapped at its host address), or NULL.  cuda_pool.cpp:53-62 */
void* kvsnap_pool_create(size_t capacity, int device);

/* Frees the pool, unless its stream cannot be drained (then the memory is
 * left allocated).  cuda_pool.cpp:63 */
void kvsnap_pool_destroy(void* pool);

/* Drain the copy stream, then free; on failure the pool stays valid for a
 * retry.  cuda_pool.cpp:66-74 */
int kvsnap_pool_close_checked(void* pool);

/* The copy stream (a hipStream_t) as a borrowed handle.  cuda_pool.cpp:78-85 */
int kvsnap_pool_copy_stream(void* pool, uintptr_t* stream);

/* First-fit reservation of `size` bytes: its id and host address.
 * cuda_pool.cpp:86-104 */
int kvsnap_pool_reserve(void* pool, size_t size, uint64_t* id, void** ptr);

/* `size` bytes between allocation `id` at `host_offset` and `device_ptr`
 * (to_host: D2H after fencing `producer_stream`).  cuda_pool.cpp:107-133 */
int kvsnap_pool_copy(void* pool, uint64_t id, size_t host_offset, void* device_ptr, size_t size, int to_host,
                     uintptr_t producer_stream);

/* `height` rows of `width` bytes, host rows `host_pitch` apart, device rows
 * `device_pitch` apart.  cuda_pool.cpp:139-169 */
int kvsnap_pool_copy_2d(void* pool, uint64_t id, size_t host_offset, size_t host_pitch, void* device_ptr,
                        size_t device_pitch, size_t width, size_t height, int to_host, uintptr_t producer_stream);

/* Block until the allocation's copies complete.  cuda_pool.cpp:170-177 */
int kvsnap_pool_wait(void* pool, uint64_t id);

/* 1 when the allocation's copies have completed, 0 if not yet, -1 on error.
 * cuda_pool.cpp:178-189 */
int kvsnap_pool_ready(void* pool, uint64_t id);

/* Wait for the allocation's copies, then return its bytes to the pool.
 * cuda_pool.cpp:190-199 */
int kvsnap_pool_release(void* pool, uint64_t id);

/* Host address of a live allocation (no reference counterpart: the reference
 * returns it only from reserve). */
int kvsnap_pool_pointer(void* pool, uint64_t id, void** ptr);

#ifdef __cplusplus
}
#endif

#endif /* KVSNAP_POOL_H */
