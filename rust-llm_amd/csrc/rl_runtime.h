// Host-side helpers shared by the library's translation units: status returns
// with a per-thread message, and a scoped device selection.
#pragma once
#include <hip/hip_runtime.h>

#include <string>

#include "rl_error.h"
#include "rl_sampler.h"

namespace rl {

inline int fail(int code, const std::string &msg) {
    set_last_error(msg);
    return code;
}

inline int hip_fail(hipError_t e, const char *what) {
    return fail(RL_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

// Makes `dev` current for the scope and restores the caller's device after.
struct DeviceGuard {
    int prev = -1;
    bool ok = true;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) ok = hipSetDevice(dev) == hipSuccess;
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

}  // namespace rl
