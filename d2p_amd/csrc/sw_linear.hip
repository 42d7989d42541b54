// sw_linear.hip -- linear-gap soft Smith-Waterman on gfx950.
//
// Reference behaviour restated (not translated):
//   forward   /root/reference/src/sw/kernels_cpu.cpp:70-148
//   backward  /root/reference/src/sw/kernels_cpu.cpp:154-271
// DP:  alpha[i,j] = LSE_T( alpha[i-1,j-1]+s[i,j] (i>1,j>1), alpha[i-1,j]+gap (i>1),
//                          alpha[i,j-1]+gap (j>1), s[i,j] )
//      alpha[0,0] = 0, rest of row/col 0 = NINF,  S = LSE_T over cells 0..L1 x 0..L2.
//
// Mapping: the stripe pipeline of wavefront.hip.h.  The forward keeps each lane's
// alpha in a register, takes the up / diagonal neighbours from lane r-1 by DPP (lane 0
// from the ring of the stripe above, staged in the DPP "old" operand), stores alpha
// in the skewed table alpha_sk[b][stripe][step][lane] and each stripe's last row by
// step, and folds every cell into a per-lane online LSE for the partition.
// The backward is the reverse sweep of the reference (scatter form, no atomics): each
// cell receives its successors' contributions from the DPP neighbour or from its own
// previous step, in the reference's accumulation order
//   beta = ((beta_init + from(i+1,j+1)) + from(i,j+1)) + from(i+1,j).

#include <type_traits>
#include <vector>

#include "wavefront.hip.h"
#include "../../include/d2p_amd.h"
#include "capi_util.hip.h"
#include "sw_internal.hip.h"

namespace d2p_amd {
namespace sw {

using namespace wf;

constexpr int PF = 16;               // steps per chunk, forward sweep
constexpr int DUMMY = 64 + PF;       // per-wave LDS sink for the lanes that do not publish

__global__ void __launch_bounds__(NW * 64)
sw_forward_kernel(const float* __restrict__ scores, const int* __restrict__ lengths,
                  float* __restrict__ alpha_sk, float* __restrict__ brow,
                  float* __restrict__ partition,
                  int* __restrict__ status, int L1max, int L2max, int NSmax, float gap, float T,
                  int R) {
    constexpr int P = PF;
    extern __shared__ float smem[];
    __shared__ int prog[NW];
    __shared__ float red_m[NW], red_z[NW];
    const int b = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const unsigned ul4 = (unsigned)lane * 4u;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    using Tile = QuadTile<P>;
    float* tiles = smem + wave * 2 * Tile::FLOATS;         // double-buffered score chunk
    float* rings = smem + NW * 2 * Tile::FLOATS;           // [NW][R]
    float* sink = rings + NW * R + wave * DUMMY;       // per-wave write sink
    int* st = status + b;

    if (lane == 0) prog[wave] = -1;
    if (threadIdx.x == 0) *st = 0;
    __syncthreads();

    const int L1 = min(max(lengths[2 * b], 0), L1max);
    const int L2 = min(max(lengths[2 * b + 1], 0), L2max);
    const float c = kLog2e / T;
    const float tl = T * kLn2;
    const int NS = L2 > 0 ? (L1 + 63) >> 6 : 0;
    const int nsteps = L2 + 63;
    const int nch = (nsteps + P - 1) / P;
    const size_t NT = (size_t)stored_steps(L2max);
    const float* sbase = scores + (size_t)b * L1max * L2max;

    OnlineLSE acc;
    acc.init_open();

    for (int s = wave; s < NS; s += NW) {
        set_pipeline_priority(s % NW);
        const int i0 = s * 64;
        const int L2eff = (i0 + lane < L1) ? L2 : 0;   // rows past L1 are never valid
        const float* ring_in = ring_from(rings, s, R);
        float* ring_out = ring_of(rings, s, R);
        // wave-uniform base (step 0) + 32-bit lane offset: scalar-base stores
        float* out = alpha_sk + (((size_t)b * NSmax + s) * NT + APAD) * 64;
        float* brow_s = brow + ((size_t)b * NSmax + s) * NT;   // last row, by step
#pragma unroll
        for (int t = -APAD; t < 0; ++t) lane_store(out + t * 64, ul4, kNINF);
        wave_lds_sync();   // the previous stripe's tile reads are complete
        const uint32_t tile_lds = lds_address(tiles);
        dma_quads<P, 1>(tile_lds, sbase, i0, L1max, L2max, lane, 0);
        float cur = kNINF, up_prev = kNINF;

        for (int k = 0; k < nch; ++k) {
            const int t0 = k * P;
            chunk_waits<P>(prog, s, NS, k, nch, R, st);
            // this chunk's scores: loaded one chunk ago, followed by the P + 1 stores of
            // that chunk (the first chunk's load is the last issued)
            if (k == 0) wait_vmcnt<0>(); else wait_vmcnt<P>();
            const float* tile = tiles + (k & 1) * Tile::FLOATS;
            float sv[P], av[P];
            read_quads<P, 1>(tile, lane, sv);
            // lane 0's up values: column t0+j sits in lane j (ring slot = producer step)
            float rreg = kNINF;
            if (s > 0 && lane < P) rreg = ring_in[ring_index(t0 + lane + 63, R)];
            if (k + 1 < nch)
                dma_quads<P, 1>(tile_lds + ((k + 1) & 1) * Tile::FLOATS * 4, sbase, i0, L1max,
                                  L2max, lane, t0 + P);
            // lane 63 publishes its alpha of step u into ring slot (t0+u) % R; the
            // other lanes write into the sink (R is a multiple of P: no wrap in a chunk)
            float* pub = (lane == 63) ? ring_out + ring_index(t0, R) : sink + lane;
            float* outc = out + (size_t)t0 * 64;
            // FULL: every cell of the chunk lies inside the element, no validity masks
            auto steps = [&](auto full) {
                constexpr bool FULL = decltype(full)::value;
#pragma unroll
                for (int u = 0; u < P; ++u) {
                    const int t = t0 + u;
                    const float up = wave_shr1_or(cur, rreg);   // lane 0: stripe above
                    rreg = wave_shl1(rreg, kNINF);
                    const float diag = up_prev;
                    up_prev = up;
                    // out-of-table neighbours are NINF, so no i>1 / j>1 guards are needed
                    const float vd = diag + sv[u];
                    const float vu = up + gap;
                    const float vl = cur + gap;
                    const float m = fmaxf(fmaxf(vd, vu), fmaxf(vl, sv[u]));
                    const float sum = (fast_exp2((vd - m) * c) + fast_exp2((vu - m) * c)) +
                                      (fast_exp2((vl - m) * c) + fast_exp2((sv[u] - m) * c));
                    const float a = m + tl * fast_log2(sum);
                    if (FULL) {
                        cur = a;
                    } else {
                        const bool ok = (unsigned)(t - lane) < (unsigned)L2eff;
                        cur = ok ? a : kNINF;
                    }
                    lane_store(outc + u * 64, ul4, cur);
                    pub[u] = cur;
                    av[u] = cur;
                }
            };
            if (i0 + 63 < L1 && t0 >= 63 && t0 + P <= L2) steps(std::true_type{});
            else steps(std::false_type{});
            acc.add_block<P>(av, c);
            // the stripe's last row (lane 63) by step, contiguous, for the reverse sweep
            // of the stripe below; one store instruction
            wave_lds_sync();
            if (lane < P) lane_store(brow_s, (unsigned)(t0 + lane) * 4u, ring_out[t0 % R + lane]);
            publish(prog, wave, s * PROG_STRIDE + k + 1);
        }
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

// PRECISE: accumulate dS/dgap and dS/dT per lane in double (second-order callers,
// whose Jacobians amplify errors in these sums).
template <int P, bool PRECISE = false>
__global__ void __launch_bounds__(NW * 64)
sw_backward_kernel(const float* __restrict__ scores, const int* __restrict__ lengths,
                   const float* __restrict__ alpha_sk, const float* __restrict__ brow,
                   const float* __restrict__ partition,
                   float* __restrict__ post, float* __restrict__ grad_gap,
                   float* __restrict__ grad_T, int* __restrict__ status, float* __restrict__ trash,
                   int L1max, int L2max, int NSmax, float gap, float T, int R) {
        extern __shared__ float smem[];
    __shared__ int prog[NW];
    using Acc = typename std::conditional<PRECISE, double, float>::type;
    __shared__ Acc red_g[NW], red_p[NW];
    const int b = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const unsigned ul4 = (unsigned)lane * 4u;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Per wave, two chunk buffers, each: the score tile (then the chunk's marginals),
    // P alpha rows (steps t_hi-2 .. t_hi-P-1, 64 lanes each) and one row of values from
    // the stripe above.  All three arrive by direct-to-LDS loads one chunk ahead.
    using Tile = QuadTile<P>;
    constexpr int ABUF = Tile::FLOATS;            // alpha rows
    constexpr int RBUF = ABUF + P * 64;           // row above
    constexpr int BUF = RBUF + 64;
    float* bufs = smem + wave * 2 * BUF;
    float2* rings = reinterpret_cast<float2*>(smem + NW * 2 * BUF);  // [NW][R] (up, diag)
    float2* sink = rings + NW * R + wave * DUMMY;
    int* st = status + b;
    // the chunk's marginals go to an output tile laid over its own buffer, whose
    // inputs are all in registers by then (the next chunk loads into the other one)
    using OutTile = ChunkTile<P>;
    static_assert(OutTile::FLOATS <= BUF, "output tile fits the chunk buffer");
    const int obase_lane = OutTile::read_base(lane);

    if (lane == 0) prog[wave] = -1;
    __syncthreads();

    const int L1 = min(max(lengths[2 * b], 0), L1max);
    const int L2 = min(max(lengths[2 * b + 1], 0), L2max);
    const float c = kLog2e / T;
    const float S = partition[b];
    const int NS = L2 > 0 ? (L1 + 63) >> 6 : 0;
    const int nsteps = L2 + 63;
    const int nch = (nsteps + P - 1) / P;
    const size_t NT = (size_t)stored_steps(L2max);
    const float* sbase = scores + (size_t)b * L1max * L2max;
    float* pbase = post + (size_t)b * L1max * L2max;

    zero_padding(pbase, L1, L2, L1max, L2max, NW * 64);

    Acc g_acc = 0, p_acc = 0;
    float A[P + 2];

    // Stripes run bottom-up: order q = 0..NS-1 handles stripe NS-1-q, on wave q % NW.
    for (int q = wave; q < NS; q += NW) {
        set_pipeline_priority(q % NW);
        const int s = NS - 1 - q;
        const int i0 = s * 64;
        const int L2eff = (i0 + lane < L1) ? L2 : 0;
        // alpha tables of this stripe and of the one above, from step -APAD
        const float* astripe = alpha_sk + ((size_t)b * NSmax + s) * NT * 64;
        const float* bup = brow + ((size_t)b * NSmax + (s > 0 ? s - 1 : 0)) * NT;
        const float2* ring_in = ring_from(rings, q, R);   // from stripe s+1
        float2* ring_out = ring_of(rings, q, R);          // to stripe s-1
        const bool below = q > 0;

        // Loads of chunk k (t_hi = nsteps-1-kP) into buffer k&1: the score quad tile, P
        // alpha rows (steps t_hi-2 .. t_hi-P-1, four per load), and the row-above values
        // (lane j <= P: the alpha of the last row of the stripe above at step
        // t_hi - j + 63, clamped to the last step; lanes past P repeat lane P's address).
        auto issue_chunk = [&](int k) {
            const int th = nsteps - 1 - k * P;
            const uint32_t buf = lds_address(bufs + (k & 1) * BUF);
            dma_quads<P, -1>(buf, sbase, i0, L1max, L2max, lane, th);
            dma_rows4<P, -1>(buf + ABUF * 4, astripe, th - 2, ul4);
            uint32_t roff = (uint32_t)min(th - min(lane, P) + 63, nsteps - 1) * 4u;
            uint32_t rl = buf + RBUF * 4;
            lds_dma_dword<0>(bup, roff, rl, 0u);
        };

        // the first two alphas of chunk 0 (steps nsteps-1, nsteps-2); later chunks
        // carry them over from the previous chunk
        A[P] = lane_load(astripe + (size_t)(nsteps - 1 + APAD) * 64, ul4);
        A[P + 1] = lane_load(astripe + (size_t)(nsteps - 2 + APAD) * 64, ul4);
        __asm__ volatile("" ::"v"(A[P]), "v"(A[P + 1]));   // completes the two loads here
        wave_lds_sync();   // the previous stripe's buffer reads are complete
        issue_chunk(0);
        float in_left = 0.0f, in_up = 0.0f, in_diag = 0.0f, in_diag_next = 0.0f;

        for (int k = 0; k < nch; ++k) {
            const int t_hi = nsteps - 1 - k * P;
            chunk_waits<P>(prog, q, NS, k, nch, R, st);
            // this chunk's loads were issued one chunk ago and followed by exactly the P
            // marginal stores of that chunk (the first chunk's are the last issued)
            if (k == 0) wait_vmcnt<0>(); else wait_vmcnt<P>();
            float* buf = bufs + (k & 1) * BUF;
            float sv[P];
            read_quads<P, -1>(buf, lane, sv);
            A[0] = A[P];
            A[1] = A[P + 1];
#pragma unroll
            for (int j = 0; j < P; ++j) A[j + 2] = buf[ABUF + rows_row<P, -1>(j) * 64 + lane];
            // lane j: alpha of the row above at lane-63 step t_hi - j + 63
            float bv = buf[RBUF + lane];
            bv = (s > 0 && lane <= P && t_hi - lane + 63 <= nsteps - 1) ? bv : kNINF;
            // Contributions from the stripe below for lane 63.  The producer (lane 0 of
            // stripe s+1) wrote the pair for its column c into slot (nsteps-1-c) % R;
            // lane 63 at step u needs column t_hi-u-63 (up) and t_hi-u-62 (diagonal),
            // i.e. slots kP+u+63 and kP+u+62.  Lane 63-j holds step j; the register is
            // shifted up one lane per step so lane 63 sees the step it needs next.
            float pre_u = 0.0f, pre_d = 0.0f;
            if (below && lane >= 64 - P) {
                const int j = 63 - lane;
                pre_u = ring_in[ring_index(k * P + j + 63, R)].x;
                pre_d = ring_in[ring_index(k * P + j + 62, R)].y;
            }
            if (k + 1 < nch) issue_chunk(k + 1);
            // lane 0 publishes (up, diag) of step u into slot (kP+u) % R
            float2* pub = (lane == 0) ? ring_out + ring_index(k * P, R) : sink + lane;
            // lane 63 starts the chunk with the ring's values for steps 0 and 1
            {
                const float u0 = lane_bcast(pre_u, 63), d0 = lane_bcast(pre_d, 63);
                const float d1 = lane_bcast(pre_d, 62);
                if (lane == 63) { in_up = u0; in_diag = d0; in_diag_next = d1; }
            }
            Acc gs[P], ps[P];
            float pre_d2 = wave_shr1(pre_d, 0.0f);   // lane 63 = step 1 (then shifted on)
            pre_d2 = wave_shr1(pre_d2, 0.0f);        // lane 63 = step 2
            // FULL: every cell of the chunk lies inside the element, no validity masks
            auto steps = [&](auto full) {
            constexpr bool FULL = decltype(full)::value;
#pragma unroll
            for (int u = 0; u < P; ++u) {
                const int t = t_hi - u;
                const bool ok = FULL || (unsigned)(t - lane) < (unsigned)L2eff;
                // cells outside the element hold arbitrary tensor data: neutralise them
                const float sc = ok ? sv[u] : kNINF;
                const float a0 = A[u], a1 = A[u + 1];
                // up / diagonal alphas from lane r-1; lane 0 takes the row above
                const float bv_next = wave_shl1(bv, kNINF);
                const float upa = wave_shr1_or(a1, bv);
                const float dga = wave_shr1_or(A[u + 2], bv_next);
                bv = bv_next;
                const float vd = dga + sc;
                const float vu = upa + gap;
                const float vl = a1 + gap;
                const float m = fmaxf(fmaxf(vd, vu), fmaxf(vl, sc));
                const float e0 = fast_exp2((vd - m) * c), e1 = fast_exp2((vu - m) * c);
                const float e2 = fast_exp2((vl - m) * c), e3 = fast_exp2((sc - m) * c);
                const float rin = fast_rcp(((e0 + e1) + e2) + e3);
                float lp = (a0 - S) * c;   // subtract first: exact for nearby values
                lp = lp < 0.0f ? lp : 0.0f;
                const float binit = fast_exp2(lp);
                // reference accumulation order: init, diagonal, left, up successor
                const float beta = ((binit + in_diag) + in_left) + in_up;
                const bool live = ok && (beta <= 3.0e38f);    // skips inf / NaN like the reference
                const float br = live ? beta * rin : 0.0f;
                const float od = br * e0, ou = br * e1, ol = br * e2;
                const float pv = br * (e0 + e3);
                buf[obase_lane + u] = pv;
                gs[u] = (Acc)ou + (Acc)ol;
                ps[u] = (Acc)(pv * sc);
                pub[u] = make_float2(ou, od);
                // successor contributions for the next steps; lane 63 takes the ring
                pre_u = wave_shr1(pre_u, 0.0f);
                in_left = ol;
                in_up = wave_shl1_or(ou, pre_u);
                in_diag = in_diag_next;
                in_diag_next = wave_shl1_or(od, pre_d2);
                pre_d2 = wave_shr1(pre_d2, 0.0f);
            }
            };
            if (i0 + 63 < L1 && t_hi - P - 62 >= 0 && t_hi < L2) steps(std::true_type{});
            else steps(std::false_type{});

            // the chunk's parameter-gradient terms: balanced sums, then one add each
            g_acc += tree_sum<P>(gs);
            p_acc += tree_sum<P>(ps);
            wave_lds_sync();
            // write this chunk's marginals back over the cells the scores came from:
            // exactly P stores (cells outside the element's lengths go to the trash
            // line in boundary chunks, and carry 0 in inside chunks)
            write_tile<P, -1>(buf, pbase, trash, i0, L1, L2, L1max, L2max, lane, t_hi);
            publish(prog, wave, q * PROG_STRIDE + k + 1);
        }
    }

    g_acc = wave_sum(g_acc);
    p_acc = wave_sum(p_acc);
    if (lane == 0) { red_g[wave] = g_acc; red_p[wave] = p_acc; }
    __syncthreads();
    if (threadIdx.x == 0) {
        Acc g = 0, p = 0;
        for (int w = 0; w < NW; ++w) { g += red_g[w]; p += red_p[w]; }
        grad_gap[b] = (float)g;
        grad_T[b] = (float)(((Acc)S - (p + g * (Acc)gap)) / (Acc)T);
    }
}

}  // namespace sw
}  // namespace d2p_amd

namespace d2p_amd {
namespace sw {

namespace {
constexpr size_t kLdsLimit = 160 * 1024 - 256;

size_t lds_forward(int max_L1, int max_L2) {
    const int R = wf::ring_len(max_L1, max_L2, 256);
    return (size_t)wf::NW * 2 * 64 * PF * sizeof(float) +
           ((size_t)wf::NW * R + wf::NW * DUMMY) * sizeof(float);
}

size_t lds_backward(int max_L1, int max_L2, int P) {
    const int R = wf::ring_len(max_L1, max_L2, 128);
    return (size_t)wf::NW * 2 * (64 * P + 64 * P + 64) * sizeof(float) +
           ((size_t)wf::NW * R + wf::NW * DUMMY) * sizeof(float2);
}

// backward: 16-step chunks when they fit in LDS, else 8-step chunks (long rows need
// long rings)
int backward_chunk(int max_L1, int max_L2) {
    return lds_backward(max_L1, max_L2, 16) <= kLdsLimit ? 16 : 8;
}
}  // namespace

int check_shape(int B, int max_L1, int max_L2, float temperature) {
    D2P_REQUIRE(B >= 0 && max_L1 >= 0 && max_L2 >= 0, "negative dimension");
    D2P_REQUIRE(temperature > 0.0f, "temperature must be positive");
    D2P_REQUIRE(max_L2 + 63 < (1 << 16) * 4, "max_L2 too large");
    // per-lane byte offsets within one batch element are 32-bit
    D2P_REQUIRE((size_t)max_L1 * max_L2 < ((size_t)1 << 30), "DP table too large");
    D2P_REQUIRE(lds_forward(max_L1, max_L2) <= kLdsLimit &&
                    lds_backward(max_L1, max_L2, backward_chunk(max_L1, max_L2)) <= kLdsLimit,
                "sequence too long for the LDS stripe rings");
    return D2P_OK;
}

int launch_forward(const float* scores, const int* lengths, int B, int max_L1, int max_L2,
                   float gap, float T, const Layout& ws, float* partition, hipStream_t st) {
    const int ns = (max_L1 + 63) / 64;
    const int R = wf::ring_len(max_L1, max_L2, 256);
    const size_t lds = lds_forward(max_L1, max_L2);
    D2P_HIP(hipFuncSetAttribute((const void*)sw_forward_kernel,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    D2P_LAUNCH("sw_forward", sw_forward_kernel, dim3(B), dim3(wf::NW * 64), lds, st, scores,
               lengths, ws.alpha_sk, ws.brow, partition, ws.status, max_L1, max_L2, ns, gap, T, R);
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

template <int P, bool PRECISE>
int launch_backward_p(const float* scores, const int* lengths, int B, int max_L1, int max_L2,
                      float gap, float T, const Layout& ws, const float* partition,
                      float* marginals, float* grad_gap, float* grad_T, hipStream_t st) {
    const int ns = (max_L1 + 63) / 64;
    const int R = wf::ring_len(max_L1, max_L2, 128);
    const size_t lds = lds_backward(max_L1, max_L2, P);
    D2P_HIP(hipFuncSetAttribute((const void*)sw_backward_kernel<P, PRECISE>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    D2P_LAUNCH("sw_backward", (sw_backward_kernel<P, PRECISE>), dim3(B), dim3(wf::NW * 64), lds,
               st, scores, lengths, ws.alpha_sk, ws.brow, partition, marginals, grad_gap, grad_T,
               ws.status, ws.trash, max_L1, max_L2, ns, gap, T, R);
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

int launch_backward(const float* scores, const int* lengths, int B, int max_L1, int max_L2,
                    float gap, float T, const Layout& ws, const float* partition,
                    float* marginals, float* grad_gap, float* grad_T, hipStream_t st,
                    bool precise) {
    const int P = backward_chunk(max_L1, max_L2);
    if (P == 16)
        return precise ? launch_backward_p<16, true>(scores, lengths, B, max_L1, max_L2, gap, T, ws,
                                                     partition, marginals, grad_gap, grad_T, st)
                       : launch_backward_p<16, false>(scores, lengths, B, max_L1, max_L2, gap, T,
                                                      ws, partition, marginals, grad_gap, grad_T, st);
    return precise ? launch_backward_p<8, true>(scores, lengths, B, max_L1, max_L2, gap, T, ws,
                                                partition, marginals, grad_gap, grad_T, st)
                   : launch_backward_p<8, false>(scores, lengths, B, max_L1, max_L2, gap, T, ws,
                                                 partition, marginals, grad_gap, grad_T, st);
}

}  // namespace sw
}  // namespace d2p_amd

using namespace d2p_amd;

extern "C" size_t d2p_sw_workspace_bytes(int B, int max_L1, int max_L2) {
    if (B <= 0 || max_L1 < 0 || max_L2 < 0) return 0;
    // status words | trash line | skewed alpha table | last row of every stripe
    return wf::layout(nullptr, B, max_L1, max_L2).bytes;
}

extern "C" int d2p_sw_status(const void* workspace, int B, int* status, void* stream) {
    D2P_REQUIRE(status != nullptr, "null status pointer");
    *status = 0;
    if (B <= 0 || workspace == nullptr) return D2P_OK;
    std::vector<int> host(B);
    D2P_HIP(hipMemcpyAsync(host.data(), workspace, sizeof(int) * B, hipMemcpyDeviceToHost,
                           (hipStream_t)stream));
    D2P_HIP(hipStreamSynchronize((hipStream_t)stream));
    for (int v : host) *status |= v;
    return D2P_OK;
}

extern "C" int d2p_sw_forward_marginals(const float* scores, const int* lengths, int B,
                                        int max_L1, int max_L2, float gap, float temperature,
                                        float* partition, float* marginals, float* grad_gap,
                                        float* grad_T, void* workspace,
                                        size_t workspace_bytes, void* stream) {
    const int rc = sw::check_shape(B, max_L1, max_L2, temperature);
    if (rc != D2P_OK) return rc;
    if (B == 0) return D2P_OK;
    D2P_REQUIRE(scores && lengths && partition && marginals && grad_gap && grad_T,
                "null pointer argument");
    const size_t need = d2p_sw_workspace_bytes(B, max_L1, max_L2);
    D2P_REQUIRE(workspace && workspace_bytes >= need, "workspace too small");
    hipStream_t st = (hipStream_t)stream;
    const wf::Layout ws = wf::layout(workspace, B, max_L1, max_L2);
    int r = sw::launch_forward(scores, lengths, B, max_L1, max_L2, gap, temperature, ws,
                               partition, st);
    if (r != D2P_OK) return r;
    return sw::launch_backward(scores, lengths, B, max_L1, max_L2, gap, temperature, ws,
                               partition, marginals, grad_gap, grad_T, st);
}
