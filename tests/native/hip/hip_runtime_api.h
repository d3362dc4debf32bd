// Test-only stand-in for the subset of the HIP runtime API that the pinned
// pool (kvsnap_amd/csrc/pool.cpp) calls, so the CPU tests can build the pool
// with g++ and drive its error paths.  Copies are memcpy; completion is a
// pending counter; faults are injected through the kvsnap_test_* hooks.
// Proves control flow only, never GPU behaviour.
#pragma once
#include <cstddef>
#include <cstdint>

typedef int hipError_t;
typedef void* hipStream_t;
typedef void* hipEvent_t;
typedef int hipMemcpyKind;

constexpr hipError_t hipSuccess = 0, hipErrorNotReady = 600, hipErrorUnknown = 999;
constexpr unsigned hipHostMallocPortable = 0x1, hipHostMallocMapped = 0x2;
constexpr unsigned hipHostMallocCoherent = 0x40000000u, hipHostMallocNonCoherent = 0x80000000u;
constexpr unsigned hipStreamNonBlocking = 0x1, hipEventDisableTiming = 0x2;
constexpr hipMemcpyKind hipMemcpyHostToDevice = 1, hipMemcpyDeviceToHost = 2;

extern "C" {
const char* hipGetErrorString(hipError_t);
hipError_t hipSetDevice(int);
hipError_t hipHostMalloc(void**, std::size_t, unsigned);
hipError_t hipHostFree(void*);
hipError_t hipHostGetDevicePointer(void**, void*, unsigned);
hipError_t hipStreamCreateWithFlags(hipStream_t*, unsigned);
hipError_t hipStreamSynchronize(hipStream_t);
hipError_t hipStreamQuery(hipStream_t);
hipError_t hipStreamDestroy(hipStream_t);
hipError_t hipStreamWaitEvent(hipStream_t, hipEvent_t, unsigned);
hipError_t hipEventCreateWithFlags(hipEvent_t*, unsigned);
hipError_t hipEventRecord(hipEvent_t, hipStream_t);
hipError_t hipEventSynchronize(hipEvent_t);
hipError_t hipEventQuery(hipEvent_t);
hipError_t hipEventDestroy(hipEvent_t);
hipError_t hipMemcpyAsync(void*, const void*, std::size_t, hipMemcpyKind, hipStream_t);
hipError_t hipMemcpy2DAsync(void*, std::size_t, const void*, std::size_t, std::size_t, std::size_t, hipMemcpyKind,
                            hipStream_t);
void kvsnap_test_fail_next_record();
void kvsnap_test_fail_next_stream_sync();
void kvsnap_test_fail_next_host_alloc();
void kvsnap_test_map_elsewhere(int enable);
int kvsnap_test_pending();
int kvsnap_test_live_events();
std::uintptr_t kvsnap_test_last_copy_stream();
unsigned kvsnap_test_last_host_flags();
}
