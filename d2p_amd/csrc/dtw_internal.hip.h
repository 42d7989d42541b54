// dtw_internal.hip.h -- soft-DTW pieces shared between the first-order (dtw.hip) and
// second-order (dtw_second.hip) entry points.
#pragma once
#include <hip/hip_runtime.h>

#include "wavefront.hip.h"

namespace d2p_amd {
namespace dtw {

using Layout = wf::Layout;

// Checks shared by the entry points (sizes, LDS budget); D2P_OK or an error code.
int check_shape(int B, int max_L1, int max_L2, float temperature);

// Forward sweep: alpha table, last rows and value[B] (status words reset).
int launch_forward(const float* costs, const int* lengths, int B, int max_L1, int max_L2,
                   float T, int bandwidth, const Layout& ws, float* value, hipStream_t st);

// Reverse sweep: marginals and dvalue/dT per element, from a forward's table.
int launch_backward(const float* costs, const int* lengths, int B, int max_L1, int max_L2,
                    float T, int bandwidth, const Layout& ws, float* marginals, float* grad_T,
                    hipStream_t st);

}  // namespace dtw
}  // namespace d2p_amd
