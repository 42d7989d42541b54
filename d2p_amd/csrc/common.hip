// common.hip -- error state and batch-scaling kernel of the C ABI.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "capi_util.hip.h"
#include "dp_common.hip.h"
#include "../../include/d2p_amd.h"

namespace d2p_amd {

static thread_local char g_last_error[512] = "";

void set_last_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

// ---------------------------------------------------------------------------
// kernel timing registry
// ---------------------------------------------------------------------------
namespace {
struct PendingLaunch {
    std::string name;
    hipEvent_t start, end;
};
struct KernelStats {
    long long count = 0;
    double total_ms = 0.0, min_ms = 1e30, max_ms = 0.0;
};
std::mutex g_prof_mu;
bool g_prof_on = false;
std::vector<PendingLaunch> g_pending;
std::map<std::string, KernelStats> g_stats;

void resolve_pending_locked() {
    for (auto& p : g_pending) {
        hipEventSynchronize(p.end);
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, p.start, p.end) == hipSuccess) {
            KernelStats& k = g_stats[p.name];
            k.count += 1;
            k.total_ms += ms;
            k.min_ms = ms < k.min_ms ? ms : k.min_ms;
            k.max_ms = ms > k.max_ms ? ms : k.max_ms;
        }
        hipEventDestroy(p.start);
        hipEventDestroy(p.end);
    }
    g_pending.clear();
}
}  // namespace

bool profiling_enabled() { return g_prof_on; }

uint32_t next_epoch() {
    static std::atomic<uint32_t> epoch{0};
    const uint32_t e = ++epoch;
    return e != 0 ? e : ++epoch;
}

int device_cus() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return 0;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

void profile_begin(hipStream_t stream, hipEvent_t* start) {
    if (hipEventCreate(start) != hipSuccess) { *start = nullptr; return; }
    hipEventRecord(*start, stream);
}

void profile_end(const char* name, hipStream_t stream, hipEvent_t start) {
    if (!start) return;
    hipEvent_t end;
    if (hipEventCreate(&end) != hipSuccess) { hipEventDestroy(start); return; }
    hipEventRecord(end, stream);
    std::lock_guard<std::mutex> lk(g_prof_mu);
    g_pending.push_back({name, start, end});
}

// dst = g[b] * src over [B, n]; float4 body when the row length allows it.  Batch
// rows run along blockIdx.y (stepping by gridDim.y), so the row factor is loaded once
// per row and no index is divided.
__global__ void __launch_bounds__(256)
scale_by_batch_kernel(const float* __restrict__ src, const float* __restrict__ g,
                      long long g_stride, float* __restrict__ dst, int B, long long n, int vec) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    const long long first = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    typedef float v4f __attribute__((ext_vector_type(4)));
    for (int b = blockIdx.y; b < B; b += gridDim.y) {
        const float gb = g[(size_t)b * g_stride];
        if (vec) {
            const long long n4 = n >> 2;
            const v4f* s4 = reinterpret_cast<const v4f*>(src) + (size_t)b * n4;
            v4f* d4 = reinterpret_cast<v4f*>(dst) + (size_t)b * n4;
            for (long long i = first; i < n4; i += stride)
                __builtin_nontemporal_store(__builtin_nontemporal_load(s4 + i) * gb, d4 + i);
        } else {
            const float* s1 = src + (size_t)b * n;
            float* d1 = dst + (size_t)b * n;
            for (long long i = first; i < n; i += stride) d1[i] = gb * s1[i];
        }
    }
}

// The same for [B, max_L1, max_L2] tensors that are zero outside each element's
// lengths (the marginals): cells inside the lengths are scaled as above; the others
// are written as g[b] * 0 without being read (the same bits as g[b] * src where src
// is +0, NaN where g[b] is not finite).  A workgroup handles whole rows of one element
// (rows along x, elements along y); vec: 16-byte quads (max_L2 a multiple of 4 and
// both bases 16-byte aligned).
__global__ void __launch_bounds__(256)
scale_by_batch_lengths_kernel(const float* __restrict__ src, const float* __restrict__ g,
                              long long g_stride, float* __restrict__ dst,
                              const int* __restrict__ lengths, int B, int L1max, int L2max,
                              int vec) {
    typedef float v4f __attribute__((ext_vector_type(4)));
    for (int b = blockIdx.y; b < B; b += gridDim.y) {
        const float gb = g[(size_t)b * g_stride];
        const float z = gb * 0.0f;
        const int L1 = min(max(lengths[2 * b], 0), L1max);
        const int L2 = min(max(lengths[2 * b + 1], 0), L2max);
        for (int i = blockIdx.x; i < L1max; i += gridDim.x) {
            const size_t row = ((size_t)b * L1max + i) * (size_t)L2max;
            const int lim = i < L1 ? L2 : 0;   // columns read in this row
            if (vec) {
                const v4f* s4 = reinterpret_cast<const v4f*>(src + row);
                v4f* d4 = reinterpret_cast<v4f*>(dst + row);
                for (int q = threadIdx.x; q < (L2max >> 2); q += blockDim.x) {
                    const int c0 = 4 * q;
                    v4f v = {z, z, z, z};
                    if (c0 < lim) {
                        const v4f x = __builtin_nontemporal_load(s4 + q);
                        v.x = x.x * gb;
                        v.y = c0 + 1 < lim ? x.y * gb : z;
                        v.z = c0 + 2 < lim ? x.z * gb : z;
                        v.w = c0 + 3 < lim ? x.w * gb : z;
                    }
                    __builtin_nontemporal_store(v, d4 + q);
                }
            } else {
                for (int j = threadIdx.x; j < L2max; j += blockDim.x)
                    dst[row + j] = j < lim ? src[row + j] * gb : z;
            }
        }
    }
}

}  // namespace d2p_amd

extern "C" const char* d2p_last_error(void) { return d2p_amd::g_last_error; }

extern "C" int d2p_abi_version(void) { return 1; }

extern "C" int d2p_profile_enable(int on) {
    std::lock_guard<std::mutex> lk(d2p_amd::g_prof_mu);
    d2p_amd::g_prof_on = on != 0;
    return D2P_OK;
}

extern "C" void d2p_profile_reset(void) {
    std::lock_guard<std::mutex> lk(d2p_amd::g_prof_mu);
    d2p_amd::resolve_pending_locked();
    d2p_amd::g_stats.clear();
}

extern "C" int d2p_profile_report(char* buf, size_t len) {
    std::lock_guard<std::mutex> lk(d2p_amd::g_prof_mu);
    d2p_amd::resolve_pending_locked();
    std::string out;
    char line[256];
    for (auto& kv : d2p_amd::g_stats) {
        const auto& k = kv.second;
        snprintf(line, sizeof(line), "%s %lld %.6f %.6f %.6f\n", kv.first.c_str(), k.count,
                 k.total_ms, k.min_ms, k.max_ms);
        out += line;
    }
    D2P_REQUIRE(buf != nullptr && len > out.size(), "report buffer too small");
    memcpy(buf, out.c_str(), out.size() + 1);
    return D2P_OK;
}

extern "C" int d2p_scale_by_batch(const float* src, const float* g, float* dst, int B,
                                  long long per_batch, void* stream) {
    return d2p_scale_by_batch_strided(src, g, 1, dst, B, per_batch, stream);
}

extern "C" int d2p_scale_by_batch_strided(const float* src, const float* g, long long g_stride,
                                          float* dst, int B, long long per_batch, void* stream) {
    D2P_REQUIRE(B >= 0 && per_batch >= 0, "negative size");
    D2P_REQUIRE(g_stride >= 0, "negative factor stride");
    if (B == 0 || per_batch == 0) return D2P_OK;
    D2P_REQUIRE(src && g && dst, "null pointer argument");
    const bool vec = (per_batch % 4 == 0) && (((uintptr_t)src | (uintptr_t)dst) % 16 == 0);
    // about 32768 workgroups in all (measured on [256, 512 x 512]: 82 us against 85
    // with 16384 and 92 with 8192): rows along y, each row's elements along x
    const long long row_work = vec ? per_batch / 4 : per_batch;
    const int by = B < 65535 ? B : 65535;
    long long bx = (row_work + 255) / 256;
    const long long cap = 32768 / by > 1 ? 32768 / by : 1;
    if (bx > cap) bx = cap;
    D2P_LAUNCH("scale_by_batch", d2p_amd::scale_by_batch_kernel,
               dim3((unsigned)bx, (unsigned)by), dim3(256), 0, (hipStream_t)stream, src, g,
               g_stride, dst, B, per_batch, vec ? 1 : 0);
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

extern "C" int d2p_scale_by_batch_lengths(const float* src, const float* g, long long g_stride,
                                          const int* lengths, float* dst, int B, int max_L1,
                                          int max_L2, void* stream) {
    D2P_REQUIRE(B >= 0 && max_L1 >= 0 && max_L2 >= 0, "negative size");
    D2P_REQUIRE(g_stride >= 0, "negative factor stride");
    if (B == 0 || max_L1 == 0 || max_L2 == 0) return D2P_OK;
    if (lengths == nullptr)
        return d2p_scale_by_batch_strided(src, g, g_stride, dst, B,
                                          (long long)max_L1 * max_L2, stream);
    D2P_REQUIRE(src && g && dst, "null pointer argument");
    const bool vec = (max_L2 % 4 == 0) && (((uintptr_t)src | (uintptr_t)dst) % 16 == 0);
    // about 32768 workgroups in all, as the flat form: elements along y, rows along x
    const int by = B < 65535 ? B : 65535;
    const int cap = 32768 / by > 1 ? 32768 / by : 1;
    const int bx = max_L1 < cap ? max_L1 : cap;
    D2P_LAUNCH("scale_by_batch", d2p_amd::scale_by_batch_lengths_kernel, dim3(bx, by),
               dim3(256), 0, (hipStream_t)stream, src, g, g_stride, dst, lengths, B, max_L1,
               max_L2, vec ? 1 : 0);
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}
