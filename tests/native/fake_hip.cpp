// A CPU model of the HIP runtime calls that kvsnap_amd/csrc/pool.cpp makes, so
// tests/test_pool.py can build the pool with g++ and drive its error paths.
//
// Each stream is a queue of deferred work: a copy is recorded when it is
// issued and runs only when something waits for it (a stream synchronize, a
// synchronize on an event recorded after it, or another stream waiting on
// such an event).  An event remembers how much of its stream's queue had been
// issued when it was recorded.  So the tests see what the pool would read or
// write before its waits, not only after.  Faults are armed by the
// kvsnap_test_* hooks and fire once.  This proves control flow only, never
// GPU behaviour.
#include "hip/hip_runtime_api.h"

#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <functional>
#include <set>

namespace {

struct Queue {
    std::deque<std::function<void()>> work;
    std::uint64_t issued = 0, finished = 0;

    void issue(std::function<void()> job) {
        work.push_back(std::move(job));
        ++issued;
    }
    void run_until(std::uint64_t mark) {
        while (finished < mark && !work.empty()) {
            work.front()();
            work.pop_front();
            ++finished;
        }
    }
    void run_all() { run_until(issued); }
};

struct Mark {
    Queue* queue = nullptr;
    std::uint64_t at = 0;
};

Queue null_queue;            // work issued on stream 0
std::set<Queue*> queues;     // streams made by hipStreamCreateWithFlags
int marks_alive = 0;

struct Armed {
    bool record = false, sync = false, host_alloc = false;
} armed;
bool mapped_elsewhere = false;
hipStream_t last_copy_on = nullptr;
unsigned last_host_flags = 0;

Queue& queue_of(hipStream_t stream) { return stream ? *static_cast<Queue*>(stream) : null_queue; }

bool fire(bool& fault) {
    const bool fired = fault;
    fault = false;
    return fired;
}

}  // namespace

extern "C" {

const char* hipGetErrorString(hipError_t) { return "fault injected by the HIP stand-in"; }

hipError_t hipSetDevice(int) { return hipSuccess; }

hipError_t hipHostMalloc(void** out, std::size_t bytes, unsigned flags) {
    last_host_flags = flags;
    if (fire(armed.host_alloc)) return hipErrorUnknown;
    *out = std::calloc(1, bytes ? bytes : 1);
    return *out ? hipSuccess : hipErrorUnknown;
}

hipError_t hipHostFree(void* memory) {
    std::free(memory);
    return hipSuccess;
}

hipError_t hipHostGetDevicePointer(void** device, void* host, unsigned) {
    // The pool requires pinned memory mapped at its own host address; the hook breaks that on purpose.
    *device = mapped_elsewhere ? static_cast<char*>(host) + 4096 : host;
    return hipSuccess;
}

hipError_t hipStreamCreateWithFlags(hipStream_t* stream, unsigned) {
    Queue* queue = new Queue();
    queues.insert(queue);
    *stream = queue;
    return hipSuccess;
}

hipError_t hipStreamSynchronize(hipStream_t stream) {
    if (fire(armed.sync)) return hipErrorUnknown;
    queue_of(stream).run_all();
    return hipSuccess;
}

hipError_t hipStreamQuery(hipStream_t stream) {
    const Queue& queue = queue_of(stream);
    return queue.finished == queue.issued ? hipSuccess : hipErrorNotReady;
}

hipError_t hipStreamDestroy(hipStream_t stream) {
    Queue* queue = static_cast<Queue*>(stream);
    queue->run_all();  // a destroyed stream still completes its work
    queues.erase(queue);
    delete queue;
    return hipSuccess;
}

hipError_t hipEventCreateWithFlags(hipEvent_t* event, unsigned) {
    *event = new Mark();
    ++marks_alive;
    return hipSuccess;
}

hipError_t hipEventRecord(hipEvent_t event, hipStream_t stream) {
    if (fire(armed.record)) return hipErrorUnknown;
    Mark* mark = static_cast<Mark*>(event);
    mark->queue = &queue_of(stream);
    mark->at = mark->queue->issued;
    return hipSuccess;
}

hipError_t hipEventSynchronize(hipEvent_t event) {
    const Mark* mark = static_cast<Mark*>(event);
    if (mark->queue) mark->queue->run_until(mark->at);
    return hipSuccess;
}

hipError_t hipEventQuery(hipEvent_t event) {
    const Mark* mark = static_cast<Mark*>(event);
    return !mark->queue || mark->queue->finished >= mark->at ? hipSuccess : hipErrorNotReady;
}

hipError_t hipEventDestroy(hipEvent_t event) {
    delete static_cast<Mark*>(event);
    --marks_alive;
    return hipSuccess;
}

hipError_t hipStreamWaitEvent(hipStream_t, hipEvent_t event, unsigned) {
    // The waiting stream's later work may not start before the event: in this model, finish it now.
    return hipEventSynchronize(event);
}

hipError_t hipMemcpyAsync(void* to, const void* from, std::size_t bytes, hipMemcpyKind, hipStream_t stream) {
    last_copy_on = stream;
    queue_of(stream).issue([=] { std::memcpy(to, from, bytes); });
    return hipSuccess;
}

hipError_t hipMemcpy2DAsync(void* to, std::size_t to_pitch, const void* from, std::size_t from_pitch,
                            std::size_t width, std::size_t rows, hipMemcpyKind, hipStream_t stream) {
    last_copy_on = stream;
    queue_of(stream).issue([=] {
        for (std::size_t row = 0; row < rows; ++row)
            std::memcpy(static_cast<char*>(to) + row * to_pitch, static_cast<const char*>(from) + row * from_pitch,
                        width);
    });
    return hipSuccess;
}

// ---- hooks for the tests

void kvsnap_test_fail_next_record() { armed.record = true; }
void kvsnap_test_fail_next_stream_sync() { armed.sync = true; }
void kvsnap_test_fail_next_host_alloc() { armed.host_alloc = true; }
void kvsnap_test_map_elsewhere(int enable) { mapped_elsewhere = enable != 0; }

int kvsnap_test_pending() {
    std::uint64_t waiting = null_queue.issued - null_queue.finished;
    for (const Queue* queue : queues) waiting += queue->issued - queue->finished;
    return static_cast<int>(waiting);
}

int kvsnap_test_live_events() { return marks_alive; }
std::uintptr_t kvsnap_test_last_copy_stream() { return reinterpret_cast<std::uintptr_t>(last_copy_on); }
unsigned kvsnap_test_last_host_flags() { return last_host_flags; }

}  // extern "C"
