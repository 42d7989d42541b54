// split.hip -- host policy and small kernels shared by the sweeps that divide an
// element's stripes among several workgroups ("parts"; wavefront.hip.h).

#include <stdlib.h>

#include <vector>

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

__global__ void flag_reset_kernel(uint64_t* __restrict__ flags, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) store_flag(flags + i, 0);
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

__global__ void partition_dot_merge_kernel(const float2* __restrict__ fpart,
                                           const float* __restrict__ wpart,
                                           float* __restrict__ partition,
                                           float* __restrict__ sdot, int B, int G, float T) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    const float c = kLog2e / T;
    OnlineLSEDot tot;
    tot.m = 0.0f;
    tot.z = 1.0f;
    tot.w = 0.0f;
    for (int g = 0; g < G; ++g) {
        const float2 v = fpart[(size_t)b * G + g];
        tot.merge(v.x, v.y, wpart[(size_t)b * G + g], c);
    }
    // the cells' weights 2^((alpha - S) c) with S rounded to fp32 (not w / z)
    const float S = tot.m + T * kLn2 * fast_log2(tot.z);
    partition[b] = S;
    sdot[b] = tot.w * fast_exp2((tot.m - S) * c);
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

// NaN into every output of an element whose status word is set; one workgroup per
// element (a clean element reads its word and returns).
__global__ void __launch_bounds__(256)
poison_kernel(const int* __restrict__ status, int B, long long n, float* __restrict__ m0,
              float* __restrict__ m1, float* __restrict__ v0, float* __restrict__ v1,
              float* __restrict__ v2, float* __restrict__ v3) {
    const int b = blockIdx.x;
    if (b >= B || __builtin_amdgcn_readfirstlane(status[b]) == 0) return;
    const float nan = __builtin_nanf("");
    if (threadIdx.x == 0) {
        if (v0) v0[b] = nan;
        if (v1) v1[b] = nan;
        if (v2) v2[b] = nan;
        if (v3) v3[b] = nan;
    }
    for (long long i = threadIdx.x; i < n; i += blockDim.x) {
        if (m0) m0[(size_t)b * n + i] = nan;
        if (m1) m1[(size_t)b * n + i] = nan;
    }
}

}  // namespace

std::vector<int (*)(int)>& spin_setters() {
    static std::vector<int (*)(int)> setters;
    return setters;
}

void register_spin_setter(int (*setter)(int)) { spin_setters().push_back(setter); }

int launch_poison(const int* status, int B, long long per_elem, float* mat0, float* mat1,
                  float* vec0, float* vec1, float* vec2, float* vec3, hipStream_t st) {
    if (B <= 0) return D2P_OK;
    D2P_LAUNCH("poison", poison_kernel, dim3(B), dim3(256), 0, st, status, B, per_elem, mat0,
               mat1, vec0, vec1, vec2, vec3);
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

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

int launch_flag_reset(uint64_t* flags, int n, hipStream_t st) {
    if (n <= 0) return D2P_OK;
    D2P_LAUNCH("flag_reset", flag_reset_kernel, dim3((n + 255) / 256), dim3(256), 0, st, flags, n);
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

int launch_partition_dot_merge(const Layout& ws, const float* wpart, float* partition,
                               float* sdot, int B, int G, float T, hipStream_t st) {
    D2P_LAUNCH("partition_merge", partition_dot_merge_kernel, dim3((B + 255) / 256), dim3(256),
               0, st, ws.fpart, wpart, partition, sdot, B, G, T);
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

}  // namespace wf
}  // namespace d2p_amd

extern "C" int d2p_set_spin_limit(int spins) {
    D2P_REQUIRE(spins >= 1, "spin limit must be positive");
    for (auto setter : d2p_amd::wf::spin_setters())
        D2P_REQUIRE(setter(spins) == 0, "hipMemcpyToSymbol of the spin limit failed");
    return D2P_OK;
}
