// sw_linear.hip -- linear-gap soft Smith-Waterman on gfx950.
//
// Reference behaviour restated (not translated):
//   forward   /root/reference/src/sw/kernels_cpu.cpp:70-148
//   backward  /root/reference/src/sw/kernels_cpu.cpp:154-271
// DP:  alpha[i,j] = LSE_T( alpha[i-1,j-1]+s[i,j] (i>1,j>1), alpha[i-1,j]+gap (i>1),
//                          alpha[i,j-1]+gap (j>1), s[i,j] )
//      alpha[0,0] = 0, rest of row/col 0 = NINF,  S = LSE_T over cells 0..L1 x 0..L2.
//
// Mapping (one workgroup per batch element, NW wave64s):
//   * rows are cut into 64-row stripes; lane r of the wave that owns stripe s
//     holds DP row 64*s+r+1 and sweeps the columns with a one-column skew per lane
//     (lane r works on column t-r at step t), so the 64 cells a wave computes at a
//     step lie on one anti-diagonal;
//   * the up / diagonal neighbours come from lane r-1 through a DPP wave shift;
//     lane 0 gets them from the stripe above through an LDS ring written by that
//     stripe's lane 63;
//   * stripes form a software pipeline: stripe s runs `lag` chunks of P steps
//     behind stripe s-1; all waves meet at a workgroup barrier after every chunk;
//   * scores (and, in the backward, marginals) are staged per chunk through a
//     padded LDS tile so every HBM access is a contiguous row segment;
//   * the forward stores alpha in a skewed layout alpha_sk[b][stripe][t][lane],
//     one contiguous 256-byte vector per wave step, which the backward streams back
//     in reverse.
// The backward is the reverse sweep of the reference (scatter form, no atomics):
// every cell receives its successors' contributions from the DPP neighbour or its
// own previous step, in the reference's accumulation order
//   beta = ((beta_init + from(i+1,j+1)) + from(i,j+1)) + from(i+1,j).

#include "dp_common.hip.h"
#include "../../include/d2p_amd.h"
#include "capi_util.hip.h"

namespace d2p_amd {
namespace sw {

constexpr int NW = 8;      // waves per workgroup
constexpr int PF = 32;     // steps per chunk, forward sweep
constexpr int PB = 16;     // steps per chunk, backward sweep (holds more state per step)

// Chunks of lag between consecutive stripes: lane 63 of stripe s-1 produces
// column c at step c+63 and lane 0 of stripe s consumes it at step c, so the
// producer's chunk must precede the consumer's (63/P + 2 chunks); and a wave's
// next stripe must start only after its previous one ended, (NW-1)*lag >= nch,
// which also keeps the LDS rings free of overlap between pipeline generations.
template <int P>
__host__ __device__ inline int stripe_lag(int nch) {
    const int lagmin = 63 / P + 2;
    int l = (nch + NW - 2) / (NW - 1);
    return l > lagmin ? l : lagmin;
}

template <int P>
__host__ inline int ring_len_for(int L2max) {
    int nch = (L2max + 63 + P - 1) / P;
    int need = (stripe_lag<P>(nch) + 2) * P;
    int r = 64;
    while (r < need) r <<= 1;
    return r;
}

// Stripe scheduled at global chunk gc for this wave, or -1.  Stripe order q runs
// 0..NS-1 and starts at chunk q*lag; stripes of one wave never overlap in time.
__device__ __forceinline__ int stripe_at(int gc, int wave, int lag, int nch, int NS, int* k) {
    int qmax = gc / lag;
    if (qmax > NS - 1) qmax = NS - 1;
    if (qmax < wave) return -1;
    int q = qmax - ((qmax - wave) % NW);
    int kk = gc - q * lag;
    if (kk >= nch) return -1;
    *k = kk;
    return q;
}

// Steps stored per stripe in the skewed alpha table: whole forward chunks plus the
// two leading steps t = -2, -1 (always NINF), so every chunk stores unconditionally.
__host__ __device__ inline int stored_steps(int L2max) {
    return ((L2max + 63 + PF - 1) / PF) * PF + 2;
}

// Shift registers that gather one lane's per-step value across a chunk of P steps:
// push_from_top: lane 63 inserts, everything moves down one lane per step, so after
//   the chunk lane 64-P+u holds step u's value;
// push_from_bottom: lane 0 inserts, everything moves up one lane per step, so lane
//   P-1-u holds step u's value.
__device__ __forceinline__ float push_from_top(float reg, float v, int lane) {
    const float moved = wave_shl1(reg, 0.0f);
    return lane == 63 ? v : moved;
}
__device__ __forceinline__ float push_from_bottom(float reg, float v, int lane) {
    const float moved = wave_shr1(reg, 0.0f);
    return lane == 0 ? v : moved;
}

template <int P>
__global__ void __launch_bounds__(NW * 64)
sw_forward_kernel(const float* __restrict__ scores, const int* __restrict__ lengths,
                  float* __restrict__ alpha_sk, float* __restrict__ partition,
                  int L1max, int L2max, int NSmax, float gap, float T, int ring_len) {
    extern __shared__ float smem[];
    __shared__ float red_m[NW], red_z[NW];
    const int b = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    float* tile = smem + wave * 64 * (P + 1);
    float* rings = smem + NW * 64 * (P + 1);
    const int rmask = ring_len - 1;

    const int L1 = min(max(lengths[2 * b], 0), L1max);
    const int L2 = min(max(lengths[2 * b + 1], 0), L2max);
    const float c = kLog2e / T;
    const float tl = T * kLn2;
    const int NS = (L1 + 63) >> 6;
    const int nsteps = L2 + 63;
    const int nch = (nsteps + P - 1) / P;
    const int lag = stripe_lag<P>(nch);
    const int total = (NS > 0 && L2 > 0) ? (NS - 1) * lag + nch : 0;
    const size_t NT = (size_t)stored_steps(L2max);
    const float* sbase = scores + (size_t)b * L1max * L2max;

    OnlineLSE acc;
    acc.init_open();
    float cur = kNINF, up_prev = kNINF;
    float nxt[P];

    for (int gc = 0; gc < total; ++gc) {
        int k = 0;
        const int s = stripe_at(gc, wave, lag, nch, NS, &k);
        if (s >= 0) {
            const int i0 = s * 64;
            const bool row_ok = i0 + lane < L1;
            const int t0 = k * P;
            if (k == 0) {
                // first chunk of a stripe: stage its scores now, reset the row state
                cur = kNINF;
                up_prev = kNINF;
#pragma unroll
                for (int q = 0; q < P; ++q) {
                    const int rl = q * (64 / P) + lane / P, u = lane % P;
                    const int col = t0 + u - rl, grow = i0 + rl;
                    float v = 0.0f;
                    if (grow < L1 && col >= 0 && col < L2) v = sbase[(size_t)grow * L2max + col];
                    tile[rl * (P + 1) + u] = v;
                }
            }
            const bool has_next = (k + 1) < nch;
            if (has_next) {  // prefetch the next chunk's scores into registers
#pragma unroll
                for (int q = 0; q < P; ++q) {
                    const int rl = q * (64 / P) + lane / P, u = lane % P;
                    const int col = t0 + P + u - rl, grow = i0 + rl;
                    float v = 0.0f;
                    if (grow < L1 && col >= 0 && col < L2) v = sbase[(size_t)grow * L2max + col];
                    nxt[q] = v;
                }
            }
            float* out = alpha_sk + ((size_t)b * NSmax + s) * NT * 64 + lane;
            if (k == 0) { out[0] = kNINF; out[64] = kNINF; }  // steps t = -2, -1
            // lane 0's up values for this chunk (bottom row of the stripe above):
            // lane u of `ring_vals` holds column t0 + u
            float ring_vals = kNINF;
            if (s > 0 && lane < P)
                ring_vals = rings[((wave + NW - 1) % NW) * ring_len + ((t0 + lane) & rmask)];
            wave_lds_sync();
            float sv[P];
#pragma unroll
            for (int u = 0; u < P; ++u) sv[u] = tile[lane * (P + 1) + u];
            float bottom = kNINF;  // gathers lane 63's alpha of every step (push_from_top)
#pragma unroll
            for (int u = 0; u < P; ++u) {
                const int t = t0 + u;
                const int col = t - lane;
                const bool ok = row_ok && (unsigned)col < (unsigned)L2;
                float up = wave_shr1(cur, kNINF);
                const float r0 = lane_bcast(ring_vals, u);
                up = (lane == 0) ? r0 : up;
                const float diag = up_prev;
                up_prev = up;
                // out-of-table neighbours are NINF, so no i>1 / j>1 guards are needed
                const float vd = diag + sv[u];
                const float vu = up + gap;
                const float vl = cur + gap;
                const float m = fmaxf(fmaxf(vd, vu), fmaxf(vl, sv[u]));
                const float sum = fast_exp2((vd - m) * c) + fast_exp2((vu - m) * c) +
                                  fast_exp2((vl - m) * c) + fast_exp2((sv[u] - m) * c);
                const float a = m + tl * fast_log2(sum);
                cur = ok ? a : kNINF;
                out[(size_t)(t + 2) * 64] = cur;
                bottom = push_from_top(bottom, cur, lane);
                acc.add(cur, c);
            }
            // publish lane 63's row for the stripe below: lane 64-P+u holds step u,
            // whose lane-63 column is t0+u-63
            if (lane >= 64 - P) {
                const int col = t0 + (lane - (64 - P)) - 63;
                if (col >= 0 && col < L2) rings[wave * ring_len + (col & rmask)] = bottom;
            }
            if (has_next) {
#pragma unroll
                for (int q = 0; q < P; ++q) {
                    const int rl = q * (64 / P) + lane / P, u = lane % P;
                    tile[rl * (P + 1) + u] = nxt[q];
                }
            }
        }
        __syncthreads();
    }

    // partition: merge lanes, waves, and the cell (0,0) whose alpha is 0
    wave_merge_lse(acc, c);
    if (lane == 0) { red_m[wave] = acc.m; red_z[wave] = acc.z; }
    __syncthreads();
    if (threadIdx.x == 0) {
        OnlineLSE tot;
        tot.m = 0.0f;
        tot.z = 1.0f;
        for (int w = 0; w < NW; ++w) tot.merge(red_m[w], red_z[w], c);
        partition[b] = tot.m + tl * fast_log2(tot.z);
    }
}

template <int P>
__global__ void __launch_bounds__(NW * 64)
sw_backward_kernel(const float* __restrict__ scores, const int* __restrict__ lengths,
                   const float* __restrict__ alpha_sk, const float* __restrict__ partition,
                   float* __restrict__ post, float* __restrict__ grad_gap,
                   float* __restrict__ grad_T, int L1max, int L2max, int NSmax, float gap,
                   float T, int ring_len) {
    extern __shared__ float smem[];
    __shared__ float red_g[NW], red_p[NW];
    const int b = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    float* tile = smem + wave * 64 * (P + 1);
    float* ringU = smem + NW * 64 * (P + 1);
    float* ringD = ringU + NW * ring_len;
    const int rmask = ring_len - 1;

    const int L1 = min(max(lengths[2 * b], 0), L1max);
    const int L2 = min(max(lengths[2 * b + 1], 0), L2max);
    const float c = kLog2e / T;
    const float S = partition[b];
    const int NS = (L1 + 63) >> 6;
    const int nsteps = L2 + 63;
    const int nch = (nsteps + P - 1) / P;
    const int lag = stripe_lag<P>(nch);
    const int total = (NS > 0 && L2 > 0) ? (NS - 1) * lag + nch : 0;
    const size_t NT = (size_t)stored_steps(L2max);
    const float* sbase = scores + (size_t)b * L1max * L2max;
    float* pbase = post + (size_t)b * L1max * L2max;

    // zero the padded part of the marginal matrix
    if (L1 < L1max || L2 < L2max) {
        for (size_t idx = threadIdx.x; idx < (size_t)L1max * L2max; idx += NW * 64) {
            const int r = (int)(idx / L2max), cc = (int)(idx % L2max);
            if (r >= L1 || cc >= L2) pbase[idx] = 0.0f;
        }
    }

    float g_acc = 0.0f, p_acc = 0.0f;
    float A[P + 2], nA[P], Bv = kNINF, nBv = kNINF, nxt[P];
    float in_left = 0.0f, in_up = 0.0f, in_diag = 0.0f, in_diag_next = 0.0f;

    for (int gc = 0; gc < total; ++gc) {
        int k = 0;
        const int q = stripe_at(gc, wave, lag, nch, NS, &k);
        if (q >= 0) {
            const int s = NS - 1 - q;
            const int i0 = s * 64;
            const bool row_ok = i0 + lane < L1;
            const int t_hi = nsteps - 1 - k * P;
            const float* abase = alpha_sk + ((size_t)b * NSmax + s) * NT * 64 + lane;
            const float* aup = alpha_sk + ((size_t)b * NSmax + (s > 0 ? s - 1 : 0)) * NT * 64 + 63;
            if (k == 0) {
                in_left = in_up = in_diag = in_diag_next = 0.0f;
#pragma unroll
                for (int qq = 0; qq < P; ++qq) {
                    const int rl = qq * (64 / P) + lane / P, u = lane % P;
                    const int col = t_hi - u - rl, grow = i0 + rl;
                    float v = 0.0f;
                    if (grow < L1 && col >= 0 && col < L2) v = sbase[(size_t)grow * L2max + col];
                    tile[rl * (P + 1) + u] = v;
                }
#pragma unroll
                for (int qq = 0; qq < P + 2; ++qq) {
                    const int t = t_hi - qq;
                    A[qq] = (t >= -2) ? abase[(size_t)(t + 2) * 64] : kNINF;
                }
                Bv = kNINF;
                if (s > 0 && lane <= P) {
                    const int t = t_hi - lane + 63;
                    if (t <= nsteps - 1) Bv = aup[(size_t)(t + 2) * 64];
                }
            }
            const bool has_next = (k + 1) < nch;
            if (has_next) {  // prefetch scores, own alpha and the row above for the next chunk
                const int th2 = t_hi - P;
#pragma unroll
                for (int qq = 0; qq < P; ++qq) {
                    const int rl = qq * (64 / P) + lane / P, u = lane % P;
                    const int col = th2 - u - rl, grow = i0 + rl;
                    float v = 0.0f;
                    if (grow < L1 && col >= 0 && col < L2) v = sbase[(size_t)grow * L2max + col];
                    nxt[qq] = v;
                }
#pragma unroll
                for (int qq = 0; qq < P; ++qq) {
                    const int t = th2 - 2 - qq;
                    nA[qq] = (t >= -2) ? abase[(size_t)(t + 2) * 64] : kNINF;
                }
                nBv = kNINF;
                if (s > 0 && lane <= P) {
                    const int t = th2 - lane + 63;
                    if (t <= nsteps - 1) nBv = aup[(size_t)(t + 2) * 64];
                }
            }
            // contributions from the stripe below for lane 63, columns t_hi-u-63 (up)
            // and t_hi-u-62 (diagonal): lane u of preU / preD holds step u's value
            const bool below = (s + 1) < NS;
            float preU = 0.0f, preD = 0.0f;
            if (below && lane < P) {
                const int tt = t_hi - lane;
                preU = ringU[wave * ring_len + ((tt - 63) & rmask)];
                preD = ringD[wave * ring_len + ((tt - 62) & rmask)];
            }
            wave_lds_sync();
            float sv[P];
#pragma unroll
            for (int u = 0; u < P; ++u) sv[u] = tile[lane * (P + 1) + u];
            float topU = 0.0f, topD = 0.0f;  // gather lane 0's outputs (push_from_bottom)
#pragma unroll
            for (int u = 0; u < P; ++u) {
                const int t = t_hi - u;
                const int col = t - lane;
                const bool ok = row_ok && (unsigned)col < (unsigned)L2;
                const float a0 = A[u], a1 = A[u + 1];
                float upa = wave_shr1(a1, kNINF);
                float dga = wave_shr1(A[u + 2], kNINF);
                const float bu0 = lane_bcast(Bv, u);
                const float bd0 = lane_bcast(Bv, u + 1);
                upa = (lane == 0) ? bu0 : upa;
                dga = (lane == 0) ? bd0 : dga;
                const float ru = lane_bcast(preU, u);
                const float rd = lane_bcast(preD, u);
                in_up = (lane == 63) ? ru : in_up;
                in_diag = (lane == 63) ? rd : in_diag;

                // out-of-table predecessors are NINF: no i>1 / j>1 guards needed
                const float vd = dga + sv[u];
                const float vu = upa + gap;
                const float vl = a1 + gap;
                const float m = fmaxf(fmaxf(vd, vu), fmaxf(vl, sv[u]));
                const float e0 = fast_exp2((vd - m) * c), e1 = fast_exp2((vu - m) * c);
                const float e2 = fast_exp2((vl - m) * c), e3 = fast_exp2((sv[u] - m) * c);
                const float rin = fast_rcp(((e0 + e1) + e2) + e3);
                const float w0 = e0 * rin, w1 = e1 * rin, w2 = e2 * rin, w3 = e3 * rin;
                float lp = (a0 - S) * c;
                lp = lp < 0.0f ? lp : 0.0f;
                const float binit = fast_exp2(lp);
                // reference accumulation order: init, diagonal, left, up successor
                float beta = ((binit + in_diag) + in_left) + in_up;
                const bool live = ok && (beta != 0.0f) && (fabsf(beta) <= 3.0e38f);
                beta = live ? beta : 0.0f;
                const float pv = live ? beta * (w0 + w3) : 0.0f;
                const float od = live ? beta * w0 : 0.0f;
                const float ou = live ? beta * w1 : 0.0f;
                const float ol = live ? beta * w2 : 0.0f;
                tile[lane * (P + 1) + u] = pv;
                g_acc += ou;
                g_acc += ol;
                p_acc += pv * sv[u];
                topU = push_from_bottom(topU, ou, lane);
                topD = push_from_bottom(topD, od, lane);
                in_left = ol;
                in_up = wave_shl1(ou, 0.0f);
                in_diag = in_diag_next;
                in_diag_next = wave_shl1(od, 0.0f);
            }
            // hand lane 0's up / diagonal contributions to the stripe above: lane P-1-u
            // holds step u, whose lane-0 column is t_hi-u
            if (lane < P) {
                const int tt = t_hi - (P - 1 - lane);
                const int slot = ((wave + 1) % NW) * ring_len + (tt & rmask);
                ringU[slot] = topU;
                ringD[slot] = topD;
            }
            wave_lds_sync();
            // write this chunk's marginals (contiguous row segments)
#pragma unroll
            for (int qq = 0; qq < P; ++qq) {
                const int rl = qq * (64 / P) + lane / P, u = lane % P;
                const int col = t_hi - u - rl, grow = i0 + rl;
                if (grow < L1 && col >= 0 && col < L2)
                    pbase[(size_t)grow * L2max + col] = tile[rl * (P + 1) + u];
            }
            wave_lds_sync();
            if (has_next) {
#pragma unroll
                for (int qq = 0; qq < P; ++qq) {
                    const int rl = qq * (64 / P) + lane / P, u = lane % P;
                    tile[rl * (P + 1) + u] = nxt[qq];
                }
                A[0] = A[P];
                A[1] = A[P + 1];
#pragma unroll
                for (int qq = 0; qq < P; ++qq) A[qq + 2] = nA[qq];
                Bv = nBv;
            }
        }
        __syncthreads();
    }

    g_acc = wave_sum(g_acc);
    p_acc = wave_sum(p_acc);
    if (lane == 0) { red_g[wave] = g_acc; red_p[wave] = p_acc; }
    __syncthreads();
    if (threadIdx.x == 0) {
        float g = 0.0f, p = 0.0f;
        for (int w = 0; w < NW; ++w) { g += red_g[w]; p += red_p[w]; }
        grad_gap[b] = g;
        grad_T[b] = (S - (p + g * gap)) / T;
    }
}

}  // namespace sw
}  // namespace d2p_amd

using namespace d2p_amd;

extern "C" size_t d2p_sw_workspace_bytes(int B, int max_L1, int max_L2) {
    if (B <= 0 || max_L1 <= 0 || max_L2 <= 0) return 0;
    const size_t ns = ((size_t)max_L1 + 63) / 64;
    return (size_t)B * ns * (size_t)sw::stored_steps(max_L2) * 64 * sizeof(float);
}

extern "C" int d2p_sw_forward_marginals(const float* scores, const int* lengths, int B,
                                        int max_L1, int max_L2, float gap, float temperature,
                                        float* partition, float* marginals, float* grad_gap,
                                        float* grad_T, void* workspace,
                                        size_t workspace_bytes, void* stream) {
    D2P_REQUIRE(B >= 0 && max_L1 >= 0 && max_L2 >= 0, "negative dimension");
    D2P_REQUIRE(temperature > 0.0f, "temperature must be positive");
    if (B == 0) return D2P_OK;
    D2P_REQUIRE(scores && lengths && partition && marginals && grad_gap && grad_T,
                "null pointer argument");
    const size_t need = d2p_sw_workspace_bytes(B, max_L1, max_L2);
    D2P_REQUIRE(need == 0 || (workspace && workspace_bytes >= need), "workspace too small");
    hipStream_t st = (hipStream_t)stream;
    const int ns = (max_L1 + 63) / 64;
    const int ring_f = sw::ring_len_for<sw::PF>(max_L2);
    const int ring_b = sw::ring_len_for<sw::PB>(max_L2);
    const size_t lds_f = (size_t)sw::NW * 64 * (sw::PF + 1) * 4 + (size_t)sw::NW * ring_f * 4;
    const size_t lds_b = (size_t)sw::NW * 64 * (sw::PB + 1) * 4 + 2 * (size_t)sw::NW * ring_b * 4;
    D2P_REQUIRE(lds_f <= 150 * 1024 && lds_b <= 150 * 1024,
                "max_L2 too large for the LDS stripe rings");
    D2P_HIP(hipFuncSetAttribute((const void*)sw::sw_forward_kernel<sw::PF>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_f));
    D2P_HIP(hipFuncSetAttribute((const void*)sw::sw_backward_kernel<sw::PB>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_b));
    float* alpha_sk = (float*)workspace;
    D2P_LAUNCH("sw_forward", sw::sw_forward_kernel<sw::PF>, dim3(B), dim3(sw::NW * 64), lds_f,
               st, scores, lengths, alpha_sk, partition, max_L1, max_L2, ns, gap, temperature,
               ring_f);
    D2P_HIP(hipGetLastError());
    D2P_LAUNCH("sw_backward", sw::sw_backward_kernel<sw::PB>, dim3(B), dim3(sw::NW * 64),
               lds_b, st, scores, lengths, alpha_sk, partition, marginals, grad_gap, grad_T,
               max_L1, max_L2, ns, gap, temperature, ring_b);
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}
