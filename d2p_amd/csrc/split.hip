// split.hip -- host policy and small kernels shared by the sweeps that divide an
// element's stripes among several workgroups ("parts"; wavefront.hip.h).

#include <stdlib.h>

#include "wavefront.hip.h"
#include "capi_util.hip.h"

namespace d2p_amd {
namespace wf {

namespace {

// Status words and progress words of split elements start at zero.
__global__ void split_reset_kernel(int* __restrict__ status, uint64_t* __restrict__ fflag,
                                   uint64_t* __restrict__ bflag, int B, int G) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < B) status[i] = 0;
    if (i < B * G) {
        store_flag(fflag + i, 0);
        store_flag(bflag + i, 0);
    }
}

// partition[b] of a split element: the parts' (max, scaled sum) and the cell (0,0).
__global__ void partition_merge_kernel(const float2* __restrict__ fpart,
                                       float* __restrict__ partition, int B, int G, float T) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    const float c = kLog2e / T;
    OnlineLSE tot;
    tot.m = 0.0f;
    tot.z = 1.0f;
    for (int g = 0; g < G; ++g) {
        const float2 v = fpart[(size_t)b * G + g];
        tot.merge(v.x, v.y, c);
    }
    partition[b] = tot.m + T * kLn2 * fast_log2(tot.z);
}

// Sum of the parts' partial results of a split element.
__global__ void sum_parts_kernel(const float* __restrict__ spart, float* __restrict__ out, int B,
                                 int G) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    float t = 0.0f;
    for (int g = 0; g < G; ++g) t += spart[(size_t)b * G + g];
    out[b] = t;
}

}  // namespace

int launch_sum_parts(const float* spart, float* out, int B, int G, hipStream_t st) {
    D2P_LAUNCH("sum_parts", sum_parts_kernel, dim3((B + 255) / 256), dim3(256), 0, st, spart, out,
               B, G);
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

Split choose_split(int B, int max_L1, const Layout& ws, int max_spw) {
    const int ns = (max_L1 + 63) / 64;
    Split sp{1, ns > 0 ? ns : 1};
    if (ws.fflag == nullptr || ns <= 1) return sp;
    int G = 0;
    if (const char* e = getenv("D2P_AMD_SPLIT")) G = atoi(e);
    if (G <= 0 && ns > 4) {
        // Parts of 4 stripes (one wave per SIMD: the pipeline's per-step latency is
        // lowest when a wave has its SIMD to itself) if the whole grid is resident at
        // once; else parts of 8 (one stripe per wave), or as few parts as fit.
        const int cus = device_cus();
        G = (ns + 3) / 4;
        if (split_grid(B, G) > cus) {
            G = (ns + NW - 1) / NW;
            while (G > 1 && split_grid(B, G) > cus) --G;
        }
    }
    // an unsplit element whose rings do not fit in LDS: parts of at most max_spw
    // stripes, whatever the device or the environment asks for
    if (max_spw > 0 && ns > max_spw) {
        const int g_min = (ns + max_spw - 1) / max_spw;
        G = G > g_min ? G : g_min;
    }
    G = G < ns ? G : ns;
    if (G <= 1) return sp;
    sp.SPW = (ns + G - 1) / G;
    sp.G = (ns + sp.SPW - 1) / sp.SPW;   // no part without stripes
    return sp;
}

int launch_split_reset(const Layout& ws, int B, int G, hipStream_t st) {
    D2P_LAUNCH("split_reset", split_reset_kernel, dim3((B * G + 255) / 256), dim3(256), 0, st,
               ws.status, ws.fflag, ws.bflag, B, G);
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

int launch_partition_merge(const Layout& ws, float* partition, int B, int G, float T,
                           hipStream_t st) {
    D2P_LAUNCH("partition_merge", partition_merge_kernel, dim3((B + 255) / 256), dim3(256), 0,
               st, ws.fpart, partition, B, G, T);
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

}  // namespace wf
}  // namespace d2p_amd
