// Shared by the pool and the kernel launchers: one thread-local error slot,
// read through kvsnap_cuda_error().
#pragma once
#include <string>

namespace kvsnap {
void set_error(const std::string& message);
}
