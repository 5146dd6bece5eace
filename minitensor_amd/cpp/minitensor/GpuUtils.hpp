// GpuUtils.hpp -- HIP error handling and the launch-stream contract.
//
// Contract kept from the reference (include/GpuUtils.hpp:47-73):
//   * every launch goes to the thread-local active_stream() (nullptr = the
//     legacy default stream), so graph capture can redirect it;
//   * HIP failures throw std::runtime_error; launches recorded during stream
//     capture are not reported as errors;
//   * the C ABI's MT_ERR_INVALID becomes std::invalid_argument, every other
//     status std::runtime_error.
#pragma once

#include <hip/hip_runtime.h>

#include <stdexcept>
#include <string>

#include "mtgemm.h"

namespace mt_detail {

[[noreturn]] inline void hip_fail(hipError_t e, const char* file, int line) {
    throw std::runtime_error(std::string("HIP Error: ") + hipGetErrorString(e) + " at " + file +
                             ":" + std::to_string(line));
}

}  // namespace mt_detail

#define GPU_CHECK(call)                                                   \
    do {                                                                  \
        hipError_t mt_err_ = (call);                                      \
        if (mt_err_ != hipSuccess) mt_detail::hip_fail(mt_err_, __FILE__, __LINE__); \
    } while (0)

inline hipStream_t& active_stream() {
    thread_local hipStream_t s = nullptr;
    return s;
}

inline hipError_t get_last_error_capture_safe() {
    hipError_t e = hipGetLastError();
    return e == hipErrorStreamCaptureUnsupported ? hipSuccess : e;
}

// Throws the reference's exception type for a non-zero mt_status.
inline void mt_check_status(int rc, const char* what) {
    if (rc == MT_OK) return;
    std::string msg = std::string(what) + ": " + mt_strerror(rc);
    if (rc == MT_ERR_INVALID) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

// Sets a stream as active_stream() for the lifetime of the guard.
class ActiveStreamGuard {
public:
    explicit ActiveStreamGuard(hipStream_t s) : prev_(active_stream()) { active_stream() = s; }
    ~ActiveStreamGuard() { active_stream() = prev_; }
    ActiveStreamGuard(const ActiveStreamGuard&) = delete;
    ActiveStreamGuard& operator=(const ActiveStreamGuard&) = delete;

private:
    hipStream_t prev_;
};
