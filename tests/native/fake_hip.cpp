// Fault-injecting CPU implementation of tests/native/hip/hip_runtime_api.h.
// A copy happens at once and leaves one "pending" unit of work; a stream sync,
// or a sync on an event recorded after it, clears the pending work; a query
// reports not-ready while work is pending.
#include "hip/hip_runtime_api.h"

#include <cstdlib>
#include <cstring>

namespace {
struct Event {
    bool recorded = false;
};
bool fail_record = false, fail_sync = false, fail_host_alloc = false, map_elsewhere = false;
int pending = 0, live_events = 0;
hipStream_t last_copy_stream = nullptr;
unsigned last_host_flags = 0;
}  // namespace

extern "C" {
const char* hipGetErrorString(hipError_t) { return "injected HIP error"; }
hipError_t hipSetDevice(int) { return hipSuccess; }
hipError_t hipHostMalloc(void** p, std::size_t size, unsigned flags) {
    last_host_flags = flags;
    if (fail_host_alloc) {
        fail_host_alloc = false;
        return hipErrorUnknown;
    }
    *p = std::malloc(size);
    return *p ? hipSuccess : hipErrorUnknown;
}
hipError_t hipHostFree(void* p) {
    std::free(p);
    return hipSuccess;
}
hipError_t hipHostGetDevicePointer(void** device, void* host, unsigned) {
    *device = map_elsewhere ? static_cast<char*>(host) + 4096 : host;
    return hipSuccess;
}
hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned) {
    *s = std::malloc(1);
    return hipSuccess;
}
hipError_t hipStreamSynchronize(hipStream_t) {
    if (fail_sync) {
        fail_sync = false;
        return hipErrorUnknown;
    }
    pending = 0;
    return hipSuccess;
}
hipError_t hipStreamQuery(hipStream_t) { return pending ? hipErrorNotReady : hipSuccess; }
hipError_t hipStreamDestroy(hipStream_t s) {
    std::free(s);
    return hipSuccess;
}
hipError_t hipStreamWaitEvent(hipStream_t, hipEvent_t, unsigned) { return hipSuccess; }
hipError_t hipEventCreateWithFlags(hipEvent_t* e, unsigned) {
    *e = new Event();
    ++live_events;
    return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t e, hipStream_t) {
    if (fail_record) {
        fail_record = false;
        return hipErrorUnknown;
    }
    static_cast<Event*>(e)->recorded = true;
    return hipSuccess;
}
hipError_t hipEventSynchronize(hipEvent_t e) {
    if (static_cast<Event*>(e)->recorded) pending = 0;
    return hipSuccess;
}
hipError_t hipEventQuery(hipEvent_t e) {
    return static_cast<Event*>(e)->recorded && pending ? hipErrorNotReady : hipSuccess;
}
hipError_t hipEventDestroy(hipEvent_t e) {
    delete static_cast<Event*>(e);
    --live_events;
    return hipSuccess;
}
hipError_t hipMemcpyAsync(void* to, const void* from, std::size_t size, hipMemcpyKind, hipStream_t s) {
    last_copy_stream = s;
    std::memcpy(to, from, size);
    ++pending;
    return hipSuccess;
}
hipError_t hipMemcpy2DAsync(void* to, std::size_t to_pitch, const void* from, std::size_t from_pitch,
                            std::size_t width, std::size_t height, hipMemcpyKind, hipStream_t s) {
    last_copy_stream = s;
    for (std::size_t r = 0; r < height; ++r)
        std::memcpy(static_cast<char*>(to) + r * to_pitch, static_cast<const char*>(from) + r * from_pitch, width);
    ++pending;
    return hipSuccess;
}
void kvsnap_test_fail_next_record() { fail_record = true; }
void kvsnap_test_fail_next_stream_sync() { fail_sync = true; }
void kvsnap_test_fail_next_host_alloc() { fail_host_alloc = true; }
void kvsnap_test_map_elsewhere(int enable) { map_elsewhere = enable != 0; }
int kvsnap_test_pending() { return pending; }
int kvsnap_test_live_events() { return live_events; }
std::uintptr_t kvsnap_test_last_copy_stream() { return reinterpret_cast<std::uintptr_t>(last_copy_stream); }
unsigned kvsnap_test_last_host_flags() { return last_host_flags; }
}
