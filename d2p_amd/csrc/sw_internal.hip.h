// sw_internal.hip.h -- linear-gap soft Smith-Waterman pieces shared between the
// first-order (sw_linear.hip) and second-order (sw_second.hip) entry points.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>

namespace d2p_amd {
namespace sw {

// Floats of one skewed alpha-like table plus the last rows of every stripe
// (B * stripes * stored_steps * (64 + 1)).
size_t table_floats(int B, int max_L1, int max_L2);

// Workspace prefix of every linear-gap entry point: per-element status words, the
// trash line, then one alpha table with its last rows.
struct Layout {
    int* status;
    float* trash;
    float* alpha_sk;
    float* brow;
    size_t bytes;   // bytes of this prefix
};
Layout layout(void* workspace, int B, int max_L1, int max_L2);

// Checks shared by the entry points (sizes, LDS budget); D2P_OK or an error code.
int check_shape(int B, int max_L1, int max_L2, float temperature);

// Forward sweep: alpha table, last rows and partition[B] (status words reset).
int launch_forward(const float* scores, const int* lengths, int B, int max_L1, int max_L2,
                   float gap, float T, const Layout& ws, float* partition, hipStream_t st);

// Reverse sweep: marginals, dS/dgap and dS/dT per element, from a forward's table.
// precise: sum dS/dgap and dS/dT in double (for the second-order paths).
int launch_backward(const float* scores, const int* lengths, int B, int max_L1, int max_L2,
                    float gap, float T, const Layout& ws, const float* partition,
                    float* marginals, float* grad_gap, float* grad_T, hipStream_t st,
                    bool precise = false);

}  // namespace sw
}  // namespace d2p_amd
