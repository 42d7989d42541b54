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
    const size_t NT = (size_t)L2max + 65;

    OnlineLSE acc;
    acc.init();
    float cur = kNINF, up_prev = kNINF;
    float nxt[P];

    for (int gc = 0; gc < total; ++gc) {
        int k = 0;
        const int s = stripe_at(gc, wave, lag, nch, NS, &k);
        if (s >= 0) {
            const int i0 = s * 64;
            const int row = i0 + lane;
            const bool row_ok = row < L1;
            const int t0 = k * P;
            const float* srow = scores + (size_t)b * L1max * L2max;
            // stage this chunk's score parallelogram (first chunk of a stripe only;
            // later chunks were prefetched during the previous chunk)
            if (k == 0) {
                cur = kNINF;
                up_prev = kNINF;
#pragma unroll
                for (int q = 0; q < P; ++q) {
                    const int rl = q * (64 / P) + lane / P, u = lane % P;
                    const int col = t0 + u - rl, grow = i0 + rl;
                    float v = 0.0f;
                    if (grow < L1 && col >= 0 && col < L2) v = srow[(size_t)grow * L2max + col];
                    tile[rl * (P + 1) + u] = v;
                }
            }
            // prefetch the next chunk
            const bool has_next = (k + 1) < nch;
            if (has_next) {
#pragma unroll
                for (int q = 0; q < P; ++q) {
                    const int rl = q * (64 / P) + lane / P, u = lane % P;
                    const int col = t0 + P + u - rl, grow = i0 + rl;
                    float v = 0.0f;
                    if (grow < L1 && col >= 0 && col < L2) v = srow[(size_t)grow * L2max + col];
                    nxt[q] = v;
                }
            }
            wave_lds_sync();
            float* out = alpha_sk + ((size_t)b * NSmax + s) * NT * 64 + lane;
            if (k == 0) { out[0] = kNINF; out[64] = kNINF; }  // steps t = -2, -1
            const float* ring_up = rings + ((wave + NW - 1) % NW) * ring_len;
            float* ring_me = rings + wave * ring_len;
            const int i = row + 1;
#pragma unroll
            for (int u = 0; u < P; ++u) {
                const int t = t0 + u;
                const int col = t - lane;
                const bool ok = row_ok && col >= 0 && col < L2;
                const float sv = tile[lane * (P + 1) + u];
                float up = wave_shr1(cur, kNINF);
                const float rv = (s > 0) ? ring_up[t & rmask] : kNINF;
                if (lane == 0) up = rv;
                const float diag = up_prev;
                up_prev = up;
                const int j = col + 1;
                const float vd = (i > 1 && j > 1) ? diag + sv : kNINF;
                const float vu = (i > 1) ? up + gap : kNINF;
                const float vl = (j > 1) ? cur + gap : kNINF;
                const float m = fmaxf(fmaxf(vd, vu), fmaxf(vl, sv));
                const float sum = fast_exp2((vd - m) * c) + fast_exp2((vu - m) * c) +
                                  fast_exp2((vl - m) * c) + fast_exp2((sv - m) * c);
                const float a = m + tl * fast_log2(sum);
                cur = ok ? a : kNINF;
                if (t < nsteps) out[(size_t)(t + 2) * 64] = cur;
                if (lane == 63 && ok) ring_me[col & rmask] = cur;
                if (ok) acc.add(cur, c);
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
    const size_t NT = (size_t)L2max + 65;
    const float* srow = scores + (size_t)b * L1max * L2max;
    float* prow = post + (size_t)b * L1max * L2max;

    // zero the padded part of the marginal matrix
    if (L1 < L1max || L2 < L2max) {
        for (size_t idx = threadIdx.x; idx < (size_t)L1max * L2max; idx += NW * 64) {
            const int r = (int)(idx / L2max), cc = (int)(idx % L2max);
            if (r >= L1 || cc >= L2) prow[idx] = 0.0f;
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
            const int row = i0 + lane;
            const bool row_ok = row < L1;
            const int t_hi = nsteps - 1 - k * P;
            const float* abase = alpha_sk + ((size_t)b * NSmax + s) * NT * 64 + lane;
            const float* aup = alpha_sk + ((size_t)b * NSmax + (s - 1)) * NT * 64 + 63;
            if (k == 0) {
                in_left = in_up = in_diag = in_diag_next = 0.0f;
#pragma unroll
                for (int qq = 0; qq < P; ++qq) {
                    const int rl = qq * (64 / P) + lane / P, u = lane % P;
                    const int col = t_hi - u - rl, grow = i0 + rl;
                    float v = 0.0f;
                    if (grow < L1 && col >= 0 && col < L2) v = srow[(size_t)grow * L2max + col];
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
            if (has_next) {
                const int th2 = t_hi - P;
#pragma unroll
                for (int qq = 0; qq < P; ++qq) {
                    const int rl = qq * (64 / P) + lane / P, u = lane % P;
                    const int col = th2 - u - rl, grow = i0 + rl;
                    float v = 0.0f;
                    if (grow < L1 && col >= 0 && col < L2) v = srow[(size_t)grow * L2max + col];
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
            wave_lds_sync();
            const float* rU_in = ringU + wave * ring_len;            // from stripe s+1
            const float* rD_in = ringD + wave * ring_len;
            float* rU_out = ringU + ((wave + 1) % NW) * ring_len;   // to stripe s-1
            float* rD_out = ringD + ((wave + 1) % NW) * ring_len;
            const bool below = (s + 1) < NS;
            const int i = row + 1;
#pragma unroll
            for (int u = 0; u < P; ++u) {
                const int t = t_hi - u;
                const int col = t - lane;
                const int j = col + 1;
                const bool ok = row_ok && col >= 0 && col < L2;
                const float sv = tile[lane * (P + 1) + u];
                const float a0 = A[u], a1 = A[u + 1];
                float upa = wave_shr1(a1, kNINF);
                float dga = wave_shr1(A[u + 2], kNINF);
                const float bu0 = lane_bcast(Bv, u);
                const float bd0 = lane_bcast(Bv, u + 1);
                if (lane == 0) { upa = bu0; dga = bd0; }
                // contributions from the stripe below reach lane 63 through the ring
                const float ru = below ? rU_in[(t - 63) & rmask] : 0.0f;
                const float rd = below ? rD_in[(t - 62) & rmask] : 0.0f;
                if (lane == 63) { in_up = ru; in_diag = rd; }

                const float vd = (i > 1 && j > 1) ? dga + sv : kNINF;
                const float vu = (i > 1) ? upa + gap : kNINF;
                const float vl = (j > 1) ? a1 + gap : kNINF;
                const float m = fmaxf(fmaxf(vd, vu), fmaxf(vl, sv));
                const float e0 = fast_exp2((vd - m) * c), e1 = fast_exp2((vu - m) * c);
                const float e2 = fast_exp2((vl - m) * c), e3 = fast_exp2((sv - m) * c);
                const float rin = fast_rcp(((e0 + e1) + e2) + e3);
                const float w0 = e0 * rin, w1 = e1 * rin, w2 = e2 * rin, w3 = e3 * rin;
                float lp = (a0 - S) * c;
                lp = lp < 0.0f ? lp : 0.0f;
                const float binit = fast_exp2(lp);
                float beta = ((binit + in_diag) + in_left) + in_up;
                const bool live = ok && (beta != 0.0f) && (fabsf(beta) <= 3.0e38f);
                beta = live ? beta : 0.0f;
                const float pv = live ? beta * (w0 + w3) : 0.0f;
                if (ok) tile[lane * (P + 1) + u] = pv;
                const float od = live ? beta * w0 : 0.0f;
                const float ou = live ? beta * w1 : 0.0f;
                const float ol = live ? beta * w2 : 0.0f;
                g_acc += ou;
                g_acc += ol;
                p_acc += pv * sv;
                // lane 0 hands its up/diag contributions to the stripe above
                if (lane == 0) { rU_out[t & rmask] = ou; rD_out[t & rmask] = od; }
                in_left = ol;
                in_up = wave_shl1(ou, 0.0f);
                in_diag = in_diag_next;
                in_diag_next = wave_shl1(od, 0.0f);
            }
            wave_lds_sync();
            // write this chunk's marginals (contiguous row segments)
#pragma unroll
            for (int qq = 0; qq < P; ++qq) {
                const int rl = qq * (64 / P) + lane / P, u = lane % P;
                const int col = t_hi - u - rl, grow = i0 + rl;
                if (grow < L1 && col >= 0 && col < L2)
                    prow[(size_t)grow * L2max + col] = tile[rl * (P + 1) + u];
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
    return (size_t)B * ns * ((size_t)max_L2 + 65) * 64 * sizeof(float);
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
