// Internal declarations shared by the library's translation units.
#pragma once
#include <hip/hip_runtime.h>

#include <string>

#include "mg/capi.h"

namespace mg {

// Sets this thread's last error message; returns `code` for tail calls.
int set_error(int code, const char* fmt, ...);
void clear_error();

// Wraps a HIP call: on failure records "<what>: <hip error string>" and returns MG_ERR_HIP.
#define MG_HIP(call, what)                                                                   \
    do {                                                                                     \
        hipError_t mg_e_ = (call);                                                           \
        if (mg_e_ != hipSuccess) return ::mg::set_error(MG_ERR_HIP, "%s: %s", what, hipGetErrorString(mg_e_)); \
    } while (0)

#define MG_CHECK(cond, code, ...)                                 \
    do {                                                          \
        if (!(cond)) return ::mg::set_error(code, __VA_ARGS__);   \
    } while (0)

// Translates an env launcher's return (0, positive hipError_t, negative MG_ERR_*).
int launcher_status(int rc, const char* what);

// Kernel timing (mg_timing_*): when enabled, begin/end record HIP events on
// `stream` around a launch and the durations are accumulated lazily.
struct TimedLaunch {
    TimedLaunch(int kernel, hipStream_t stream);
    ~TimedLaunch();
    int kernel_;
    hipStream_t stream_;
    void* start_;
};

// Device allocation with error reporting.
int device_alloc(void** p, size_t bytes, const char* what);

}  // namespace mg

struct mg_gym {
    const mg_env_desc* env;
    uint32_t n;
    uint32_t seed;
    hipStream_t stream;
    void* state;
    void* actions;
    float* obs;
    float* reward;
    uint8_t* done;
    uint32_t* rng;
};
