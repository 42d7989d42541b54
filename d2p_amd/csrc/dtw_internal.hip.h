// dtw_internal.hip.h -- soft-DTW pieces shared between the first-order (dtw.hip) and
// second-order (dtw_second.hip) entry points.
#pragma once
#include <hip/hip_runtime.h>

#include "wavefront.hip.h"

namespace d2p_amd {
namespace dtw {

using Layout = wf::Layout;

constexpr int PF = 16;   // steps per chunk of the forward and tangent sweeps

// i*L2/L1 of (1-based) row i in float, as the reference's band test computes it
// (/root/reference/src/dtw/kernels_cpu.cpp:24-29).
__device__ __forceinline__ float band_centre(int i, int L1, int L2) {
    return L1 > 0 ? (float)((long long)i * L2) / (float)L1 : 0.0f;
}

// Cell (row centre ej, 1-based column j) lies in the band (bandwidth < 0: no band).
__device__ __forceinline__ bool in_band(float ej, int j, float bw) {
    return bw < 0.0f || fabsf((float)j - ej) <= bw;
}

// ------------------------------------------------------------ banded tables
//
// With a Sakoe-Chiba band every stripe sweeps only its window: the steps that can
// hold an in-band cell of its rows.  The skewed tables keep, per stripe, APAD steps
// of boundary values before the window's first forward chunk, the window's chunks
// and one chunk of boundary values after them, at a per-element stripe stride
// band_stride().  Cells outside the window are out of the band: alpha (and the
// tangent) there are never read, beta and the marginals are zero.

// Widths above 2^20 cover every table (L2 < 2^18): clamped so the sums stay in int.
__host__ __device__ inline int band_cap(int bandwidth) {
    return bandwidth < (1 << 20) ? bandwidth : (1 << 20);
}

// Table steps a stripe needs beyond the centre line's run across its rows: the band
// on both sides, the 63-step skew, the rounding to chunks and the two pads.
__host__ __device__ inline int band_margin(int bandwidth) { return 2 * band_cap(bandwidth) + 160; }

// Steps [lo, hi] of stripe s whose cells may lie in the band (lo > hi: none).  A
// superset: the columns j of row i with |j - ej(i)| <= bw lie in
// [floor(ej) - bw - 1, ceil(ej) + bw + 1] even after the float rounding of j - ej
// (bw + 1 is exact in float), and ej grows with i, so the first row bounds the low
// end and the last row the high end.
__device__ __forceinline__ void band_window(int s, int L1, int L2, float bw, int& lo, int& hi) {
    if (bw < 0.0f) {
        lo = 0;
        hi = L2 + 62;
        return;
    }
    const int i0 = s * 64;
    const int rows = min(64, L1 - i0);
    const int bwi = band_cap(bw >= 1048576.0f ? (1 << 20) : (int)bw);
    const int c_lo = max((int)floorf(band_centre(i0 + 1, L1, L2)) - bwi - 2, 0);
    const int c_hi = min((int)ceilf(band_centre(i0 + rows, L1, L2)) + bwi, L2 - 1);
    lo = c_lo;
    hi = c_hi + rows - 1;
}

// Table steps per stripe of an element (NT without a band).  A stripe's window spans
// at most ceil((rows - 1) * L2 / L1) + 2*bw + 68 steps (the float error of the row
// centres stays below 1/8 for L2 < 2^18); APAD, the rounding to PF-step chunks and
// the trailing chunk add at most APAD + 3*PF - 1.
__device__ __forceinline__ int band_stride(int L1, int L2, float bw, int NT) {
    if (bw < 0.0f || L1 <= 0) return NT;
    const int bwi = bw >= 1048576.0f ? (1 << 20) : (int)bw;
    const int r = min(64, L1) - 1;
    const int span = (int)(((long long)r * L2 + L1 - 1) / L1);
    return min(NT, band_margin(bwi) + span);
}

// Table steps per element the host reserves for a bandwidth: at least
// stripes * band_stride() of every element shape within (max_L1, max_L2).  With
// L1 <= 64 that is one stride, at most band_margin + L2; above, the spans of
// ceil(L1/64) strides of ceil(63*L2/L1) add up to less than 2*L2 plus one step each.
__host__ inline size_t band_elem_steps(int max_L1, int max_L2, int bandwidth) {
    const size_t ns = ((size_t)max_L1 + 63) / 64;
    const size_t full = ns * (size_t)wf::stored_steps(max_L2);
    if (bandwidth < 0) return full;
    const size_t banded = ns * (size_t)(band_margin(bandwidth) + 1) + 2 * (size_t)max_L2;
    return banded < full ? banded : full;
}

// Address of the first stored step of stripe s (a table step -APAD without a band).
// A stripe whose window starts at forward chunk k_lo stores steps from
// k_lo*PF - APAD on: table step t sits at the result + (t - k_lo*PF + APAD) * 64.
// Plain pointer arithmetic from the table pointer, so the compiler keeps the
// accesses in the global address space.
__device__ __forceinline__ float* band_stripe(float* table, int b, size_t elem_steps, int s,
                                              int stride) {
    return table + ((size_t)b * elem_steps + (size_t)s * stride) * 64;
}
__device__ __forceinline__ const float* band_stripe(const float* table, int b, size_t elem_steps,
                                                    int s, int stride) {
    return table + ((size_t)b * elem_steps + (size_t)s * stride) * 64;
}

// Checks shared by the entry points (sizes, LDS budget); D2P_OK or an error code.
int check_shape(int B, int max_L1, int max_L2, float temperature);

// Forward sweep: alpha table, last rows and value[B] (status words reset).
int launch_forward(const float* costs, const int* lengths, int B, int max_L1, int max_L2,
                   float T, int bandwidth, const Layout& ws, float* value, hipStream_t st);

// Reverse sweep: marginals and dvalue/dT per element, from a forward's table alone
// (the costs are not needed).  With poison_value (the forward's value[B]) and an unsplit
// element, the sweep itself puts NaN in the outputs of an element whose waits gave up,
// and *poisoned reports that no separate poison pass is needed.
int launch_backward(const int* lengths, int B, int max_L1, int max_L2, float T,
                    int bandwidth, const Layout& ws, float* marginals, float* grad_T,
                    hipStream_t st, float* poison_value = nullptr, bool* poisoned = nullptr);

}  // namespace dtw
}  // namespace d2p_amd
