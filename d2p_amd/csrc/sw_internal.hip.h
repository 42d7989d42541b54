// sw_internal.hip.h -- linear-gap soft Smith-Waterman pieces shared between the
// first-order (sw_linear.hip) and second-order (sw_second.hip) entry points.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>

#include "wavefront.hip.h"

namespace d2p_amd {
namespace sw {

using Layout = wf::Layout;

using Split = wf::Split;
using wf::choose_split;

// Checks shared by the entry points (sizes, LDS budget); D2P_OK or an error code.
int check_shape(int B, int max_L1, int max_L2, float temperature);

// Forward sweep: alpha table, last rows and partition[B] (status words reset).
// global: soft Needleman-Wunsch (gap boundary rows, no sky term); partition[B] then
// receives the value alpha[L1, L2].
// ckpt: store only the checkpoint rows a recomputing reverse sweep starts from (where
// helper waves write the table; otherwise the whole table, which holds them too).
int launch_forward(const float* scores, const int* lengths, int B, int max_L1, int max_L2,
                   float gap, float T, const Layout& ws, float* partition, hipStream_t st,
                   bool global = false, bool ckpt = false);

// The forward sweep and the HVP's forward tangent sweep along V in one pass: the
// alpha table, last rows and partition as launch_forward, the tangent table and its
// last rows, and sdot[B], the value's tangent.  wpart: [B][parts] scratch for split
// elements (at least B * stripes floats).
int launch_forward_tangent(const float* scores, const float* V, const int* lengths, int B,
                           int max_L1, int max_L2, float gap, float T, const Layout& ws,
                           float* partition, float* tan_sk, float* tan_brow, float* sdot,
                           float* wpart, hipStream_t st, bool global = false);

// Whether a first-order call recomputes alpha in its reverse sweep (and so runs the
// forward in checkpoint mode).
bool recompute_alpha(int B, int max_L1, int max_L2, const Layout& ws);

// Reverse sweep: marginals, dS/dgap and dS/dT per element, from a forward's table.
// precise: sum dS/dgap and dS/dT in double (for the second-order paths).
// global: soft Needleman-Wunsch, from a global forward's table and value.
// poison_value: when the call's last sweep is this one, the value array; if the
// sweep runs unsplit, its epilogue writes NaN into all outputs of elements whose
// status word is set (value included) and *poisoned comes back true, so that the
// caller needs no separate poison pass.
int launch_backward(const float* scores, const int* lengths, int B, int max_L1, int max_L2,
                    float gap, float T, const Layout& ws, const float* partition,
                    float* marginals, float* grad_gap, float* grad_T, hipStream_t st,
                    bool precise = false, bool global = false, float* poison_value = nullptr,
                    bool* poisoned = nullptr, bool recompute = false);

}  // namespace sw
}  // namespace d2p_amd
