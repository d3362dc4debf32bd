// Test-only syscall faults for kvsnap_amd/csrc/io.cpp, linked with
// -Wl,--wrap=pwrite,--wrap=pread,--wrap=fdatasync.  Per syscall kind
// (0 pwrite, 1 pread, 2 fdatasync): a number of leading EINTRs, a cap on bytes
// per call (short transfers), a one-shot zero-byte result, a sticky errno, and
// a hold that parks calls until released.  Counts every call.
#include <atomic>
#include <cerrno>
#include <cstddef>
#include <thread>

#include <sys/types.h>
#include <unistd.h>

extern "C" {
ssize_t __real_pwrite(int, const void*, size_t, off_t);
ssize_t __real_pread(int, void*, size_t, off_t);
int __real_fdatasync(int);
}

namespace {
struct Fault {
    std::atomic<int> calls{0}, eintr{0}, fail_errno{0}, zero_once{0}, hold{0};
    std::atomic<size_t> short_max{0};
};
Fault faults[3];

// Returns -1 with errno set, 0 for a zero transfer, or 1 to proceed (size may shrink).
int inject(int kind, size_t* size) {
    Fault& f = faults[kind];
    f.calls.fetch_add(1);
    while (f.hold.load()) std::this_thread::yield();
    if (f.eintr.load() > 0) {
        f.eintr.fetch_sub(1);
        errno = EINTR;
        return -1;
    }
    if (f.zero_once.exchange(0)) return 0;
    if (int e = f.fail_errno.load()) {
        errno = e;
        return -1;
    }
    const size_t cap = f.short_max.load();
    if (size && cap && *size > cap) *size = cap;
    return 1;
}
}  // namespace

extern "C" {
ssize_t __wrap_pwrite(int fd, const void* data, size_t size, off_t offset) {
    int rc = inject(0, &size);
    return rc <= 0 ? rc : __real_pwrite(fd, data, size, offset);
}
ssize_t __wrap_pread(int fd, void* data, size_t size, off_t offset) {
    int rc = inject(1, &size);
    return rc <= 0 ? rc : __real_pread(fd, data, size, offset);
}
int __wrap_fdatasync(int fd) {
    int rc = inject(2, nullptr);
    return rc < 0 ? rc : __real_fdatasync(fd);
}
void kvsnap_test_io_reset() {
    for (auto& f : faults) {
        f.calls = 0;
        f.eintr = 0;
        f.fail_errno = 0;
        f.zero_once = 0;
        f.hold = 0;
        f.short_max = 0;
    }
}
void kvsnap_test_io_fault(int kind, int eintr, size_t short_max, int fail_errno, int zero_once) {
    faults[kind].eintr = eintr;
    faults[kind].short_max = short_max;
    faults[kind].fail_errno = fail_errno;
    faults[kind].zero_once = zero_once;
}
int kvsnap_test_io_calls(int kind) { return faults[kind].calls.load(); }
void kvsnap_test_io_hold(int kind, int hold) { faults[kind].hold = hold; }
}
