// swa_internal.hip.h -- affine-gap soft Smith-Waterman pieces shared between the
// first-order (sw_affine.hip) and second-order (swa_second.hip) entry points.
#pragma once
#include <hip/hip_runtime.h>

#include "wavefront.hip.h"

namespace d2p_amd {
namespace swa {

using Layout = wf::Layout;   // three planes (M, I, D)

int check_shape(int B, int max_L1, int max_L2, float temperature);

// The first-order workspace prefix; split: with the split-element areas (the flows
// area holds a float4 and a float2 per stripe and step).
Layout affine_layout(void* workspace, int B, int max_L1, int max_L2, bool split);

// Forward sweep: (M, I, D) tables, last rows and partition[B] (status words reset).
// nwa: global alignment (soft NW with affine gaps): partition[b] is the value.
int launch_forward(const float* scores, const int* lengths, int B, int max_L1, int max_L2,
                   float go, float ge, float T, const Layout& ws, float* partition,
                   hipStream_t st, bool nwa = false);

// Reverse sweep: marginals and dS/d(open, ext, T) per element, from a forward's tables.
int launch_backward(const float* scores, const int* lengths, int B, int max_L1, int max_L2,
                    float go, float ge, float T, const Layout& ws, const float* partition,
                    float* marginals, float* grad_open, float* grad_ext, float* grad_T,
                    hipStream_t st, bool nwa = false);

}  // namespace swa
}  // namespace d2p_amd
