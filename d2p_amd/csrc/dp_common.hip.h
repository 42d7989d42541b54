// dp_common.hip.h -- device helpers shared by the soft-DP wavefront kernels
// (gfx950 / CDNA4, wave64).
//
// Numeric contract (restating /root/reference/src/common/numerics.h:23-105):
//   * sentinels NINF = -1e30 and PINF = +1e30 stand for -inf/+inf;
//   * a soft-max of terms v_k is  m + T*log(sum_k exp((v_k - m)/T))  with m the
//     largest term, so the DP value stays on the same fp32 rounding grid as the
//     reference (alpha = m + small correction).  The correction is computed with
//     the native base-2 transcendentals: exp((x-m)/T) = exp2((x-m)*log2(e)/T)
//     and T*log(s) = (T*ln2)*log2(s).
// Only the rounding of the small correction differs from the reference, which
// moves alpha by at most one ulp in rare cells.

#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace d2p_amd {

constexpr float kNINF = -1e30f;
constexpr float kPINF = 1e30f;
constexpr float kLog2e = 1.44269504088896341f;
constexpr float kLn2 = 0.69314718055994531f;

// Native v_exp_f32 / v_log_f32 (base 2).  exp2 of a very negative argument is 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// Whole-wave lane shifts through DPP (no LDS round trip).  The boundary lane
// receives 0 (bound_ctrl: one instruction, no fill register); the sweeps use these
// where the boundary lane's value is 0 or is never read.
// wave_shr1: lane r receives lane r-1's value, lane 0 receives 0.
__device__ __forceinline__ float wave_shr1(float v) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x138, 0xf, 0xf, true));
}
// wave_shl1: lane r receives lane r+1's value, lane 63 receives 0.
__device__ __forceinline__ float wave_shl1(float v) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x130, 0xf, 0xf, true));
}

// DPP shifts whose boundary lane takes its value from `old` (per lane) instead of a
// constant: with these, lane 0 / lane 63 read a neighbour value staged in a register
// with no extra select.
__device__ __forceinline__ float wave_shr1_or(float v, float old) {
    return __int_as_float(__builtin_amdgcn_update_dpp(
        __float_as_int(old), __float_as_int(v), 0x138, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_shl1_or(float v, float old) {
    return __int_as_float(__builtin_amdgcn_update_dpp(
        __float_as_int(old), __float_as_int(v), 0x130, 0xf, 0xf, false));
}

// max(max(a, b), max(c, d)) as one v_max_f32 and one v_max3_f32.  Through fmaxf the
// compiler first quiets (canonicalises) each operand that is not the result of
// arithmetic, e.g. a score read from LDS: one more instruction per use.  A quiet NaN
// operand gives the other operands' max, as fmaxf; a signalling NaN gives a NaN.
__device__ __forceinline__ float max4_raw(float a, float b, float c, float d) {
    float t, m;
    __asm__("v_max_f32 %0, %1, %2" : "=v"(t) : "v"(c), "v"(d));
    __asm__("v_max3_f32 %0, %1, %2, %3" : "=v"(m) : "v"(a), "v"(b), "v"(t));
    return m;
}

__device__ __forceinline__ float lane_bcast(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Completes this wave's outstanding LDS operations and stops the compiler from
// moving memory accesses across this point.  LDS is one in-order memory per CU, so
// this orders the wave's LDS writes before its later LDS reads (of any lane) and
// before a flag write that other waves poll.  Unlike a C++ fence it does not wait
// for outstanding global loads/stores (vmcnt), so HBM prefetches stay in flight.
__device__ __forceinline__ void wave_lds_sync() {
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// Online log-sum-exp accumulator in natural units with the exp2 scale c = log2(e)/T:
// keeps (m, z) with  LSE = m + T*ln(z).
// Sum of a[0..N) in a balanced tree (short dependency chain; N a power of two).
template <int N, typename T>
__device__ __forceinline__ T tree_sum(const T* a) {
    if constexpr (N == 1) {
        return a[0];
    } else {
        return tree_sum<N / 2>(a) + tree_sum<N / 2>(a + N / 2);
    }
}

struct OnlineLSE {
    float m, z;
    __device__ __forceinline__ void init() { m = kNINF; z = 0.0f; }
    // Starting state that lets add() take NINF (invalid) cells without a branch:
    // they can only accumulate at the NINF scale, which the first finite cell
    // wipes out (its d is huge, so z restarts at 1), and merge() drops a state
    // whose m is still <= NINF.
    __device__ __forceinline__ void init_open() { m = -3.0e38f; z = 0.0f; }
    __device__ __forceinline__ void add(float x, float c) {
        float d = (x - m) * c;
        float e = fast_exp2(-fabsf(d));
        bool up = d > 0.0f;
        z = up ? fmaf(z, e, 1.0f) : z + e;
        m = up ? x : m;
    }
    // Adds N values at once: one rescale to the block's max, then N independent
    // exp2 terms summed in a balanced tree (no serial chain through m and z).
    template <int N>
    __device__ __forceinline__ void add_block(const float* x, float c) {
        float mx[N];
#pragma unroll
        for (int i = 0; i < N; ++i) mx[i] = x[i];
#pragma unroll
        for (int w = N / 2; w >= 1; w /= 2)
#pragma unroll
            for (int i = 0; i < w; ++i) mx[i] = fmaxf(mx[i], mx[i + w]);
        const float M = fmaxf(m, mx[0]);
        float e[N];
#pragma unroll
        for (int i = 0; i < N; ++i) e[i] = fast_exp2((x[i] - M) * c);
        z = z * fast_exp2((m - M) * c) + tree_sum<N>(e);
        m = M;
    }
    // add_block with the block's max already known: bmax, the max of the values
    // (and of -1e20, so that cells at the -1e30 sentinel add exact zeros), tracked by
    // the caller as the values were made.
    template <int N>
    __device__ __forceinline__ void add_block_max(const float* x, float bmax, float c) {
        const float M = fmaxf(m, bmax);
        float e[N];
#pragma unroll
        for (int i = 0; i < N; ++i) e[i] = fast_exp2((x[i] - M) * c);
        z = fmaf(z, fast_exp2((m - M) * c), tree_sum<N>(e));
        m = M;
    }
    __device__ __forceinline__ void merge(float m2, float z2, float c) {
        float M = fmaxf(m, m2);
        float za = (m <= kNINF) ? 0.0f : z * fast_exp2((m - M) * c);
        float zb = (m2 <= kNINF) ? 0.0f : z2 * fast_exp2((m2 - M) * c);
        m = M;
        z = za + zb;
    }
};

// OnlineLSE that also carries w = sum_i 2^((x_i - m) c) y_i for a companion value y_i
// of each x_i: w / z is then the softmax-weighted mean of the y_i (the value's
// tangent from the cells' tangents, with the partition's own weights).
struct OnlineLSEDot {
    float m, z, w;
    __device__ __forceinline__ void init_open() { m = -3.0e38f; z = 0.0f; w = 0.0f; }
    template <int N>
    __device__ __forceinline__ void add_block_max(const float* x, const float* y, float bmax,
                                                  float c) {
        // (products and sums as explicit fmas: a contraction left to the compiler
        // can differ between instantiations, and so would the bits)
        static_assert(N % 2 == 0, "pairs of values");
        const float M = fmaxf(m, bmax);
        const float r = fast_exp2((m - M) * c);
        float e[N], ey[N / 2];
#pragma unroll
        for (int i = 0; i < N; ++i) e[i] = fast_exp2((x[i] - M) * c);
#pragma unroll
        for (int i = 0; i < N / 2; ++i) ey[i] = fmaf(e[2 * i], y[2 * i], e[2 * i + 1] * y[2 * i + 1]);
        z = fmaf(z, r, tree_sum<N>(e));
        w = fmaf(w, r, tree_sum<N / 2>(ey));
        m = M;
    }
    __device__ __forceinline__ void merge(float m2, float z2, float w2, float c) {
        const float M = fmaxf(m, m2);
        const float ra = (m <= kNINF) ? 0.0f : fast_exp2((m - M) * c);
        const float rb = (m2 <= kNINF) ? 0.0f : fast_exp2((m2 - M) * c);
        m = M;
        z = fmaf(z2, rb, z * ra);
        w = fmaf(w2, rb, w * ra);
    }
};

template <typename Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = op(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
    return wave_reduce(v, [](float a, float b) { return a + b; });
}

__device__ __forceinline__ double wave_sum(double v) {
    return wave_reduce(v, [](double a, double b) { return a + b; });
}

// Combines per-lane OnlineLSE states across the wave; result valid in every lane.
__device__ __forceinline__ void wave_merge_lse(OnlineLSE& s, float c) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        float m2 = __shfl_xor(s.m, off, 64);
        float z2 = __shfl_xor(s.z, off, 64);
        s.merge(m2, z2, c);
    }
}
__device__ __forceinline__ void wave_merge_lse(OnlineLSEDot& s, float c) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        float m2 = __shfl_xor(s.m, off, 64);
        float z2 = __shfl_xor(s.z, off, 64);
        float w2 = __shfl_xor(s.w, off, 64);
        s.merge(m2, z2, w2, c);
    }
}

}  // namespace d2p_amd
