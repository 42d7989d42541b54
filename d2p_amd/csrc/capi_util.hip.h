// capi_util.hip.h -- error plumbing for the extern "C" entry points.
// Entry points return D2P_OK (0) or a non-zero code; the message of the last
// failure on the calling thread is available from d2p_last_error().
#pragma once
#include <hip/hip_runtime.h>
#include <stdio.h>

namespace d2p_amd {
void set_last_error(const char* fmt, ...);

// Kernel timing hooks (see d2p_profile_enable): when enabled, every launch of
// this library is bracketed by HIP events recorded on the launch stream.
bool profiling_enabled();
void profile_begin(hipStream_t stream, hipEvent_t* start);
void profile_end(const char* name, hipStream_t stream, hipEvent_t start);

// Compute units of the current device (cached per device; 0 if unknown).
int device_cus();

// A new nonzero launch epoch (tags the progress words of split elements).
uint32_t next_epoch();
}

// Launches `kernel` and, when profiling is on, times it with events on `stream`.
#define D2P_LAUNCH(name, kernel, grid, block, lds, stream, ...)                  \
    do {                                                                         \
        hipEvent_t ev0_ = nullptr;                                               \
        const bool prof_ = d2p_amd::profiling_enabled();                         \
        if (prof_) d2p_amd::profile_begin((stream), &ev0_);                     \
        hipLaunchKernelGGL(kernel, grid, block, lds, stream, __VA_ARGS__);       \
        if (prof_) d2p_amd::profile_end(name, (stream), ev0_);                   \
    } while (0)

#define D2P_OK 0
#define D2P_ERR_ARG 1
#define D2P_ERR_HIP 2

#define D2P_REQUIRE(cond, msg)                                                   \
    do {                                                                         \
        if (!(cond)) {                                                           \
            d2p_amd::set_last_error("%s", msg);                                  \
            return D2P_ERR_ARG;                                                  \
        }                                                                        \
    } while (0)

#define D2P_HIP(expr)                                                            \
    do {                                                                         \
        hipError_t e_ = (expr);                                                  \
        if (e_ != hipSuccess) {                                                  \
            d2p_amd::set_last_error("%s failed: %s", #expr, hipGetErrorString(e_)); \
            return D2P_ERR_HIP;                                                  \
        }                                                                        \
    } while (0)

// Returns from the enclosing entry point when a launch step fails.
#define D2P_TRY(...)                    \
    do {                                \
        const int rc_ = (__VA_ARGS__);  \
        if (rc_ != D2P_OK) return rc_;  \
    } while (0)
