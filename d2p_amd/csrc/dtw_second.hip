// dtw_second.hip -- second-order quantities of soft DTW on gfx950: Hessian-vector
// products and the Jacobian of the alignment marginals with respect to temperature.
//
// Reference behaviour restated (not translated):
//   HVP          /root/reference/src/dtw/kernels_cpu.cpp:229-377
//   param grad   /root/reference/src/dtw/kernels_cpu.cpp:383-534 (temperature only)
// With w the softmin weights of a cell over its predecessors (diag, up, left) and
// x their tangents (0 outside the table and the band):
//   tangent   HVP   x[i,j] = V[i,j] + sum_k w_k x_k
//             T     x[i,j] = (softmin - E_w[alpha_pred]) / T + sum_k w_k x_k
//   reverse   beta and a second channel g both start at the terminal cell (beta 1,
//             g 0) and flow to the predecessors: beta_k += beta w_k,
//             g_k += g w_k + beta dw_k with
//             HVP   dw_k = w_k (E_w[x] - x_k) / T
//             T     dw_k = w_k ((E_w[x] - x_k) / T + (alpha_k - E_w[alpha]) / T^2);
//             the output of a cell is g.
// Mapping: the stripe pipeline of wavefront.hip.h, as in sw_second.hip: the tangent
// sweep reads the primal table like the reverse sweep and passes its tangent like
// the forward; the reverse sweep carries (beta, g) pairs.

#include <vector>

#include "wavefront.hip.h"
#include "../../include/d2p_amd.h"
#include "capi_util.hip.h"
#include "dtw_internal.hip.h"

namespace d2p_amd {
namespace dtw2 {

using namespace wf;

enum Mode { HVP = 0, TEMP = 1 };

using dtw::band_centre;
using dtw::band_stride;
using dtw::band_stripe;
using dtw::band_window;
using dtw::in_band;
using dtw::PF;

template <int MODE, int P>
__global__ void __launch_bounds__(NW * 64)
dtw_tangent_kernel(const float* __restrict__ input, const int* __restrict__ lengths,
                   const float* __restrict__ alpha_sk, const float* __restrict__ brow,
                   float* __restrict__ tan_sk, float* __restrict__ tan_brow,
                   int* __restrict__ status, uint64_t* __restrict__ tflag, int B, int L1max,
                   int L2max, int NSmax, size_t elem_steps, float T, int bandwidth, int R, int G,
                   int SPW, uint32_t epoch) {
    static_assert(P == PF, "the tangent table shares the primal table's chunks");
    using Tile = ChunkTile<P>;
    constexpr int AR = Tile::FLOATS;      // P alpha rows after the input tile
    constexpr int RR = AR + P * 64;       // row above
    constexpr int TR = RR + 64;           // tangent row of the part above
    constexpr int BUF = TR + 64;
    constexpr int SINK = 64 + P;
    extern __shared__ __align__(16) float smem[];
    __shared__ int prog[NW];
    // parts as in the primal forward: part p > 0 takes its first stripe's tangent row
    // above from part p - 1 through tan_brow
    int b, part;
    split_decode(blockIdx.x, G, b, part);
    if (b >= B) return;
    const int lane = threadIdx.x & 63;
    const unsigned ul4 = (unsigned)lane * 4u;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    float* buf = smem + wave * BUF;
    __shared__ float fslot[64];   // progress word prefetched by wave 0, the only wave whose
                                  // stripe borders another part
    const uint32_t fslot_lds = lds_address(fslot);
    float* rings = smem + NW * BUF;
    float* sink = rings + NW * R + wave * SINK;
    int* st = status + b;
    const int tbase = Tile::read_base(lane);

    if (lane == 0) prog[wave] = -1;
    __syncthreads();

    const int L1 = lengths ? min(max(lengths[2 * b], 0), L1max) : L1max;
    const int L2 = lengths ? min(max(lengths[2 * b + 1], 0), L2max) : L2max;
    const float c = kLog2e / T;
    const float rT = 1.0f / T;
    const float bw = (bandwidth < 0 || L1 == 0 || L2 == 0) ? -1.0f : (float)bandwidth;
    const int NS = L2 > 0 ? (L1 + 63) >> 6 : 0;
    const int nsteps = L2 + 63;
    const int nch = (nsteps + P - 1) / P;
    const size_t NT = (size_t)stored_steps(L2max);
    const float* ibase = input + (size_t)b * L1max * L2max;   // V (HVP) or costs (T)
    const uint32_t in_lds = lds_address(buf);
    const int s_begin = part * SPW;
    const int NL = max(min(NS, s_begin + SPW) - s_begin, 0);   // stripes of this part
    const bool has_next = s_begin + NL < NS;
    const uint64_t* flag_in = tflag + (size_t)b * G + (part > 0 ? part - 1 : 0);
    uint64_t* flag_out = tflag + (size_t)b * G + part;
    const int stride = band_stride(L1, L2, bw, (int)NT);   // table steps per stripe
    if ((size_t)NS * stride > elem_steps) {   // never: the host reserves enough
        if (threadIdx.x == 0) atomicOr(st, 2);
        return;
    }

    for (int l = wave; l < NL; l += NW) {
        const int s = s_begin + l;
        const int i0 = s * 64;
        const int L2eff = (i0 + lane < L1) ? L2 : 0;
        const float ej = band_centre(i0 + lane + 1, L1, L2);
        // the chunks [k_lo, k_end) of the stripe's band window, and the steps
        // [up_lo, up_end) the stripe above computed
        int t_lo, t_hi;
        band_window(s, L1, L2, bw, t_lo, t_hi);
        const int k_lo = __builtin_amdgcn_readfirstlane(t_lo <= t_hi ? min(t_lo / P, nch) : nch);
        const int k_end = __builtin_amdgcn_readfirstlane(t_lo <= t_hi ? t_hi / P + 1 : nch);
        int up_lo = 0, up_end = 0;
        if (s > 0) {
            band_window(s - 1, L1, L2, bw, t_lo, t_hi);
            up_lo = t_lo <= t_hi ? (t_lo / P) * P : nch * P;
            up_end = t_lo <= t_hi ? (t_hi / P + 1) * P : nch * P;
        }
        // table step t of this stripe at astripe + (t - sh + APAD) * 64, tout + (t - sh) * 64
        const int sh = k_lo * P;
        const float* astripe = band_stripe(alpha_sk, b, elem_steps, s, stride);
        const float* bup = brow + ((size_t)b * NSmax + (s > 0 ? s - 1 : 0)) * NT;
        float* tout = band_stripe(tan_sk, b, elem_steps, s, stride) + APAD * 64;
        float* tb_s = tan_brow + ((size_t)b * NSmax + s) * NT;
        const float* tb_up = tan_brow + ((size_t)b * NSmax + (s > 0 ? s - 1 : 0)) * NT;
        const float* ring_in = ring_from(rings, l, R);
        float* ring_out = ring_of(rings, l, R);
        const bool x_in = l == 0 && part > 0;        // tangent row above from part - 1
        const bool x_out = l == NL - 1 && has_next;  // tangent row feeds part + 1
        int seen = -1;       // chunks of the previous part known to be complete

        auto issue_chunk = [&](int k) {
            const int t0 = k * P;
            dma_tile<P, 1>(in_lds, ibase, i0, L1max, L2max, lane, t0);
            dma_rows<P, 1>(in_lds + AR * 4, astripe, t0 - sh, ul4);
            uint32_t roff = (uint32_t)min(t0 + 62 + min(lane, P), nsteps - 1) * 4u;
            uint32_t rl = in_lds + RR * 4;
            lds_dma_dword<0>(bup, roff, rl, 0u);
            if (x_in) {
                // lane j < P: the tangent of the last row above at step t0 + 63 + j
                uint32_t toff = (uint32_t)min(t0 + 63 + min(lane, P - 1), nsteps - 1) * 4u;
                uint32_t tl = in_lds + TR * 4;
                lds_dma_dword_sys<0>(tb_up, toff, tl, 0u);
            }
        };

        // tangents of the APAD steps before the window and of the chunk after it: 0
        // (column 0 and off the band)
#pragma unroll
        for (int t = -APAD; t < 0; ++t) lane_store(tout + t * 64, ul4, 0.0f);
        if (k_end < nch) {
#pragma unroll
            for (int t = 0; t < P; ++t) lane_store(tout + (k_end * P - sh + t) * 64, ul4, 0.0f);
        }
        // so are the last row's tangents outside the window
        for (int t = lane; t < k_lo * P; t += 64) {
            if (x_out) store_sys(tb_s + t, 0.0f);
            else tb_s[t] = 0.0f;
        }
        for (int t = k_end * P + lane; t < nch * P; t += 64) {
            if (x_out) store_sys(tb_s + t, 0.0f);
            else tb_s[t] = 0.0f;
        }
        publish(prog, wave, l * PROG_STRIDE + k_lo);   // nothing to do before the window
        wave_lds_sync();
        if (k_lo < k_end) {
            if (x_in) seen = wait_part(flag_in, epoch, min(k_lo + lead(P), nch), st);
            issue_chunk(k_lo);
        }
        float Aw[P + 2];
        Aw[P] = kPINF;   // alpha at the two steps before the window: column 0 or off band
        Aw[P + 1] = kPINF;
        float cur = 0.0f, up_prev = 0.0f;

        for (int k = k_lo; k < k_end; ++k) {
            const int t0 = k * P;
            chunk_waits<P>(prog, l, NL, k, nch, R, st, k_lo);
            // this chunk's loads, followed by at least the P + 1 stores of the previous
            // chunk
            if (k == k_lo) wait_vmcnt<0>(); else wait_vmcnt<P>();
            if (x_in && k > k_lo) {
                // its progress word, loaded one chunk ago before those stores
                const int got = flag_chunks_lds(fslot, epoch);
                seen = got > seen ? got : seen;
            }
            float iv[P];
#pragma unroll
            for (int u = 0; u < P; ++u) iv[u] = buf[tbase + u];
            Aw[0] = Aw[P];
            Aw[1] = Aw[P + 1];
#pragma unroll
            for (int j = 0; j < P; ++j) Aw[j + 2] = buf[AR + j * 64 + lane];
            float bv = buf[RR + lane];
            bv = (s > 0 && lane <= P && t0 + 62 + lane <= nsteps - 1) ? bv : kPINF;
            // tangents of the row above (0 at the steps the stripe above did not compute)
            float rreg = 0.0f;
            if (s > 0 && lane < P) {
                const int tu = t0 + lane + 63;
                if (x_in) rreg = buf[TR + lane];
                else if (tu >= up_lo && tu < up_end) rreg = ring_in[ring_index(tu, R)];
            }
            wave_lds_sync();
            if (k + 1 < k_end) {
                if (x_in) {
                    const int need = min(k + 1 + lead(P), nch);
                    if (seen < need) seen = wait_part(flag_in, epoch, need, st);
                }
                issue_chunk(k + 1);
                if (x_in) flag_load_lds(flag_in, fslot_lds, lane);
            }
            float* pub = (lane == 63) ? ring_out + ring_index(t0, R) : sink + lane;
            float* toutc = tout + (size_t)(t0 - sh) * 64;
#pragma unroll
            for (int u = 0; u < P; ++u) {
                const int t = t0 + u;
                const int col = t - lane;
                const bool ok = (unsigned)col < (unsigned)L2eff && in_band(ej, col + 1, bw);
                const float a0 = Aw[u + 2], a1 = Aw[u + 1];
                const float dga = wave_shr1_or(Aw[u], bv);
                const float bvn = wave_shl1(bv);
                const float upa = wave_shr1_or(a1, bvn);
                bv = bvn;
                const float tu = wave_shr1_or(cur, rreg);
                rreg = wave_shl1(rreg);
                const float td = up_prev;
                up_prev = tu;
                const float tl = cur;
                const float m = fminf(fminf(dga, upa), a1);
                const float ed = fast_exp2((m - dga) * c), eu = fast_exp2((m - upa) * c);
                const float el = fast_exp2((m - a1) * c);
                const float rin = m < kPINF ? fast_rcp((ed + eu) + el) : 0.0f;
                const float wsum = ((ed * td + eu * tu) + el * tl) * rin;
                float x;
                if (MODE == HVP) {
                    x = iv[u] + wsum;
                } else {
                    // softmin - E_w[alpha], both relative to the smallest predecessor m:
                    // the alphas grow with the path length, and the weights' sum
                    // differs from 1 by an ulp or two, so E_w[alpha] taken whole would
                    // carry that ulp times |alpha| into every cell.  Without a finite
                    // predecessor (cell (1,1), whose alpha[0,0] = 0 this sweep does not
                    // read, and unreachable cells) the weights are 0 and the term is
                    // alpha - cost, as in the reference.
                    const float mp = m < kPINF ? m : 0.0f;
                    const float ea = ((ed * (dga - mp) + eu * (upa - mp)) + el * (a1 - mp)) * rin;
                    x = (((a0 - iv[u]) - mp) - ea) * rT + wsum;
                }
                cur = ok ? x : 0.0f;
                lane_store(toutc + u * 64, ul4, cur);
                pub[u] = cur;
            }
            wave_lds_sync();
            if (lane < P) {
                const float v = ring_out[t0 % R + lane];
                if (x_out) store_sys(tb_s + t0 + lane, v);
                else lane_store(tb_s, (unsigned)(t0 + lane) * 4u, v);
            }
            publish(prog, wave, l * PROG_STRIDE + k + 1);
            if (x_out && k >= 2) {
                // at least P + P/4 + 1 loads and 2P + 2 stores follow the row store of
                // chunk k - 2: it (and everything before) is complete
                wait_vmcnt<3 * P + P / 4 + 3>();
                if (lane == 0) store_flag(flag_out, progress_word(epoch, k - 1));
            }
        }
        publish(prog, wave, l * PROG_STRIDE + nch);   // nothing to do after the window
        if (x_out) {
            wait_vmcnt<0>();
            if (lane == 0) store_flag(flag_out, progress_word(epoch, nch));
        }
    }
}

// DOT: accumulate <V, output> into dot[b] instead of writing the output.
template <int MODE, int P, bool DOT>
__global__ void __launch_bounds__(NW * 64)
dtw_dual_kernel(const float* __restrict__ V, const int* __restrict__ lengths,
                const float* __restrict__ alpha_sk, const float* __restrict__ brow,
                const float* __restrict__ tan_sk, const float* __restrict__ tan_brow,
                float* __restrict__ out, float* __restrict__ dot, int* __restrict__ status,
                float* __restrict__ trash, uint64_t* __restrict__ dflag,
                float4* __restrict__ flows4, float* __restrict__ spart, int B, int L1max,
                int L2max, int NSmax, size_t elem_steps, float T, int bandwidth, int R, int G,
                int SPW, uint32_t epoch) {
    using Tile = ChunkTile<P>;
    constexpr int AR = DOT ? Tile::FLOATS : 0;   // P alpha rows (after the V tile)
    constexpr int XR = AR + P * 64;
    constexpr int RA = XR + P * 64;
    constexpr int RX = RA + 64;
    constexpr int OT = RX + 64;
    constexpr int FB = OT + (DOT ? 0 : Tile::FLOATS);   // flows from the part below
    constexpr int BUF = FB + 64;
    static_assert(4 * P <= 64, "boundary flows fit their buffer");
    constexpr int SINK = 64 + P;
    extern __shared__ __align__(16) float smem[];
    __shared__ int prog[NW];
    __shared__ float red[NW];
    // parts run bottom-up as in the primal backward; the last stripe of a part below
    // the first hands its flows to the part above through flows4
    int b, dpart;
    split_decode(blockIdx.x, G, b, dpart);
    if (b >= B) return;
    const int part = G - 1 - dpart;
    const int lane = threadIdx.x & 63;
    const unsigned ul4 = (unsigned)lane * 4u;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    float* buf = smem + wave * BUF;
    float* otile = buf + OT;
    __shared__ float fslot[64];   // progress word prefetched by wave 0, the only wave whose
                                  // stripe borders another part
    const uint32_t fslot_lds = lds_address(fslot);
    float4* rings = reinterpret_cast<float4*>(smem + NW * BUF);
    float4* sink = rings + NW * R + wave * SINK;
    int* st = status + b;
    const int tbase = Tile::read_base(lane);

    if (lane == 0) prog[wave] = -1;
    __syncthreads();

    const int L1 = lengths ? min(max(lengths[2 * b], 0), L1max) : L1max;
    const int L2 = lengths ? min(max(lengths[2 * b + 1], 0), L2max) : L2max;
    const float c = kLog2e / T;
    const float rT = 1.0f / T;
    const float bw = (bandwidth < 0 || L1 == 0 || L2 == 0) ? -1.0f : (float)bandwidth;
    const int NS = L2 > 0 ? (L1 + 63) >> 6 : 0;
    const int nsteps = L2 + 63;
    const int nch = (nsteps + P - 1) / P;
    const size_t NT = (size_t)stored_steps(L2max);
    const float* vbase = DOT ? V + (size_t)b * L1max * L2max : nullptr;
    float* obase = DOT ? nullptr : out + (size_t)b * L1max * L2max;
    const uint32_t in_lds = lds_address(buf);

    if (!DOT) {   // each part zeroes its share of the rows' padding
        const int rows = (L1max + G - 1) / G;
        zero_padding(obase, L1, L2, L1max, L2max, NW * 64, part * rows,
                     min(L1max, part * rows + rows));
    }

    float dacc = 0.0f;
    float A[P + 2], X[P + 2];
    const int s_begin = part * SPW;
    const int NL = max(min(NS, s_begin + SPW) - s_begin, 0);   // stripes of this part
    const bool has_next = s_begin + NL < NS;
    const uint64_t* flag_in = dflag + (size_t)b * G + (part + 1 < G ? part + 1 : part);
    uint64_t* flag_out = dflag + (size_t)b * G + part;
    const int stride = band_stride(L1, L2, bw, (int)NT);   // table steps per stripe
    if ((size_t)NS * stride > elem_steps) {   // never: the host reserves enough
        if (threadIdx.x == 0) atomicOr(st, 2);
        return;
    }

    for (int q = wave; q < NL; q += NW) {
        const int s = s_begin + NL - 1 - q;
        const int i0 = s * 64;
        const int L2eff = (i0 + lane < L1) ? L2 : 0;
        const float ej = band_centre(i0 + lane + 1, L1, L2);
        const int term_step = (i0 + lane == L1 - 1) ? L2 - 1 + lane : -1000000;
        // the stripe's band window as reverse chunks [k_lo, k_end), its tables from
        // forward chunk kf_lo, and the reverse slots [dn_lo, dn_end) the stripe below
        // computed
        int t_lo, t_hi;
        band_window(s, L1, L2, bw, t_lo, t_hi);
        const bool none = t_lo > t_hi;
        const int k_lo = __builtin_amdgcn_readfirstlane(none ? nch : (nsteps - 1 - t_hi) / P);
        const int k_end = __builtin_amdgcn_readfirstlane(none ? nch : (nsteps - 1 - t_lo) / P + 1);
        const int kf_lo = __builtin_amdgcn_readfirstlane(none ? 0 : t_lo / PF);
        int dn_lo = 0, dn_end = 0;
        if (s + 1 < NS) {
            band_window(s + 1, L1, L2, bw, t_lo, t_hi);
            dn_lo = t_lo <= t_hi ? ((nsteps - 1 - t_hi) / P) * P : nch * P;
            dn_end = t_lo <= t_hi ? ((nsteps - 1 - t_lo) / P + 1) * P : nch * P;
        }
        const size_t ub = ((size_t)b * NSmax + (s > 0 ? s - 1 : 0)) * NT;
        // table step t of this stripe at astripe / xstripe + (t - sh + APAD) * 64
        const int sh = kf_lo * PF;
        const float* astripe = band_stripe(alpha_sk, b, elem_steps, s, stride);
        const float* xstripe = band_stripe(tan_sk, b, elem_steps, s, stride);
        const float* bup = brow + ub;
        const float* xup = tan_brow + ub;
        const float4* ring_in = ring_from(rings, q, R);
        float4* ring_out = ring_of(rings, q, R);
        const bool x_in = q == 0 && has_next;             // flows from the part below
        const bool x_out = q == NL - 1 && part > 0;       // flows to the part above
        const bool below = q > 0 || x_in;
        // boundary flows by producer step: written by stripe s (x_out), read from s + 1
        float4* flows_out = flows4 + ((size_t)b * NSmax + s) * NT;
        const float* flows_in = reinterpret_cast<const float*>(
            flows4 + ((size_t)b * NSmax + (x_in ? s + 1 : s)) * NT);
        int seen = -1;       // chunks of the part below known to be complete

        auto issue_chunk = [&](int k) {
            const int th = nsteps - 1 - k * P;
            if (DOT) dma_tile<P, -1>(in_lds, vbase, i0, L1max, L2max, lane, th);
            dma_rows<P, -1>(in_lds + AR * 4, astripe, th - 2 - sh, ul4);
            dma_rows<P, -1>(in_lds + XR * 4, xstripe, th - 2 - sh, ul4);
            const uint32_t roff = (uint32_t)min(th - min(lane, P) + 63, nsteps - 1) * 4u;
            uint32_t o = roff, l = in_lds + RA * 4;
            lds_dma_dword<0>(bup, o, l, 0u);
            o = roff;
            l = in_lds + RX * 4;
            lds_dma_dword<0>(xup, o, l, 0u);
            if (x_in) {
                // flows of producer slots kP+62 .. kP+62+P (float4 each), from .z of the
                // first to .y of the last: float f of that range in lane f, clamped to
                // the last slot
                o = (uint32_t)min((k * P + 62) * 4 + 2 + min(lane, 4 * P - 1), (nsteps - 1) * 4 + 3) * 4u;
                l = in_lds + FB * 4;
                lds_dma_dword_sys<0>(flows_in, o, l, 0u);
            }
        };

        if (!DOT && bw >= 0.0f) {
            // cells of the stripe's rows at steps outside the window: off the band, zero
            const int a_end = nsteps - k_end * P;   // steps below are not swept
            const int b_beg = nsteps - k_lo * P;    // nor are steps from here on
            const int rows = min(64, L1 - i0);
            for (int r = 0; r < rows; ++r) {
                float* row = obase + (size_t)(i0 + r) * L2max;
                const int c1 = min(L2, a_end - r);
                for (int cc = lane; cc < c1; cc += 64) row[cc] = 0.0f;
                for (int cc = max(0, b_beg - r) + lane; cc < L2; cc += 64) row[cc] = 0.0f;
            }
        }
        publish(prog, wave, q * PROG_STRIDE + k_lo);   // nothing to do before the window
        if (k_lo == k_end) {
            publish(prog, wave, q * PROG_STRIDE + nch);
            if (x_out) {
                if (lane == 0) store_flag(flag_out, progress_word(epoch, nch));
            }
            continue;
        }
        {
            const int th0 = nsteps - 1 - k_lo * P;   // the window's first step
            const float* a0p = astripe + (size_t)(th0 - sh + APAD) * 64;
            const float* x0p = xstripe + (size_t)(th0 - sh + APAD) * 64;
            A[P] = lane_load(a0p, ul4);
            A[P + 1] = lane_load(a0p - 64, ul4);
            X[P] = lane_load(x0p, ul4);
            X[P + 1] = lane_load(x0p - 64, ul4);
            __asm__ volatile("" ::"v"(A[P]), "v"(A[P + 1]), "v"(X[P]), "v"(X[P + 1]));
        }
        wave_lds_sync();
        if (x_in) seen = wait_part(flag_in, epoch, min(k_lo + lead(P), nch), st);
        issue_chunk(k_lo);
        float lb = 0.0f, lg = 0.0f, ubt = 0.0f, ug = 0.0f;
        float db = 0.0f, dg = 0.0f, db2 = 0.0f, dg2 = 0.0f;

        for (int k = k_lo; k < k_end; ++k) {
            const int t_hi = nsteps - 1 - k * P;
            chunk_waits<P>(prog, q, NL, k, nch, R, st, k_lo);
            // this chunk's loads, followed by at least the P output stores of the
            // previous chunk (none when accumulating a dot product)
            if (k == k_lo || DOT) wait_vmcnt<0>(); else wait_vmcnt<P>();
            if (x_in && k > k_lo) {
                // its progress word, loaded one chunk ago before those stores
                const int got = flag_chunks_lds(fslot, epoch);
                seen = got > seen ? got : seen;
            }
            float vv[P];
#pragma unroll
            for (int u = 0; u < P; ++u) vv[u] = DOT ? buf[tbase + u] : 0.0f;
            A[0] = A[P];
            A[1] = A[P + 1];
            X[0] = X[P];
            X[1] = X[P + 1];
#pragma unroll
            for (int j = 0; j < P; ++j) {
                A[j + 2] = buf[AR + rows_row<P, -1>(j) * 64 + lane];
                X[j + 2] = buf[XR + rows_row<P, -1>(j) * 64 + lane];
            }
            const bool row_ok = s > 0 && lane <= P && t_hi - lane + 63 <= nsteps - 1;
            float bA = row_ok ? buf[RA + lane] : kPINF;
            float bX = row_ok ? buf[RX + lane] : 0.0f;
            float qub = 0.0f, qug = 0.0f, qdb = 0.0f, qdg = 0.0f;
            if (below && lane >= 64 - P) {
                // slots the stripe below did not compute carry no flow (off the band)
                const int j = 63 - lane;
                const int su = k * P + j + 63, sd = su - 1;
                const bool ou = su >= dn_lo && su < dn_end, od = sd >= dn_lo && sd < dn_end;
                if (x_in) {
                    // .z, .w of slot kP+62+j and .x, .y of slot kP+63+j
                    qdb = od ? buf[FB + 4 * j] : 0.0f;
                    qdg = od ? buf[FB + 4 * j + 1] : 0.0f;
                    qub = ou ? buf[FB + 4 * j + 2] : 0.0f;
                    qug = ou ? buf[FB + 4 * j + 3] : 0.0f;
                } else {
                    if (ou) {
                        const float4 ru = ring_in[ring_index(su, R)];
                        qub = ru.x;
                        qug = ru.y;
                    }
                    if (od) {
                        const float4 rd = ring_in[ring_index(sd, R)];
                        qdb = rd.z;
                        qdg = rd.w;
                    }
                }
            }
            wave_lds_sync();
            if (k + 1 < k_end) {
                if (x_in) {
                    const int need = min(k + 1 + lead(P), nch);
                    if (seen < need) seen = wait_part(flag_in, epoch, need, st);
                }
                issue_chunk(k + 1);
                if (x_in) flag_load_lds(flag_in, fslot_lds, lane);
            }
            float4* pub = (lane == 0) ? ring_out + ring_index(k * P, R) : sink + lane;
            {
                const float u0b = lane_bcast(qub, 63), u0g = lane_bcast(qug, 63);
                const float d0b = lane_bcast(qdb, 63), d0g = lane_bcast(qdg, 63);
                const float d1b = lane_bcast(qdb, 62), d1g = lane_bcast(qdg, 62);
                if (lane == 63) {
                    ubt = u0b; ug = u0g;
                    db = d0b; dg = d0g;
                    db2 = d1b; dg2 = d1g;
                }
            }
            qdb = wave_shr1(wave_shr1(qdb));
            qdg = wave_shr1(wave_shr1(qdg));
#pragma unroll
            for (int u = 0; u < P; ++u) {
                const int t = t_hi - u;
                const int col = t - lane;
                const bool ok = (unsigned)col < (unsigned)L2eff && in_band(ej, col + 1, bw);
                const float a1 = A[u + 1], x1 = X[u + 1];
                const float nA = wave_shl1(bA), nX = wave_shl1(bX);
                const float upa = wave_shr1_or(a1, bA), upx = wave_shr1_or(x1, bX);
                const float dga = wave_shr1_or(A[u + 2], nA), dgx = wave_shr1_or(X[u + 2], nX);
                bA = nA;
                bX = nX;
                const float m = fminf(fminf(dga, upa), a1);
                const float ed = fast_exp2((m - dga) * c), eu = fast_exp2((m - upa) * c);
                const float el = fast_exp2((m - a1) * c);
                const float rin = m < kPINF ? fast_rcp((ed + eu) + el) : 0.0f;
                const float wd = ed * rin, wu = eu * rin, wl = el * rin;
                // E_w[x] - x_k and (for the temperature) alpha_k - E_w[alpha], with the
                // means taken relative to the predecessor of the smallest alpha m (the
                // largest weight; finite whenever any weight is not 0): the weights' sum
                // differs from 1 by an ulp or two, which must not multiply tangents and
                // alphas that grow with the path length.  Predecessors of weight 0 may
                // carry any finite tangent; their products with the weight are 0.
                const float xp = a1 <= m ? x1 : (upa <= m ? upx : dgx);
                const float pdx = dgx - xp, pux = upx - xp, plx = x1 - xp;
                const float ex = (wd * pdx + wu * pux) + wl * plx;   // E_w[x] - xp
                float dwd = wd * (ex - pdx) * rT, dwu = wu * (ex - pux) * rT;
                float dwl = wl * (ex - plx) * rT;
                if (MODE == TEMP) {
                    const float pda = dga - m, pua = upa - m, pla = a1 - m;
                    const float ea = (wd * pda + wu * pua) + wl * pla;   // E_w[alpha] - m
                    const float rT2 = rT * rT;
                    dwd += wd * (pda - ea) * rT2;
                    dwu += wu * (pua - ea) * rT2;
                    dwl += wl * (pla - ea) * rT2;
                }
                // reference accumulation order: init, diagonal, left, up successor
                const float binit = t == term_step ? 1.0f : 0.0f;
                const float beta = ((binit + db) + lb) + ubt;
                const float g = ((dg + lg) + ug);
                const bool live = MODE == HVP ? (ok && beta != 0.0f)
                                              : (ok && !(beta == 0.0f && fabsf(g) < 1e-20f));
                const float bl = live ? beta : 0.0f;
                const float gl = live ? g : 0.0f;
                if (DOT) dacc += gl * (ok ? vv[u] : 0.0f);
                else otile[tbase + u] = gl;
                const float obd = bl * wd, obu = bl * wu, obl = bl * wl;
                const float ogd = gl * wd + bl * dwd, ogu = gl * wu + bl * dwu;
                const float ogl = gl * wl + bl * dwl;
                pub[u] = make_float4(obu, ogu, obd, ogd);
                qub = wave_shr1(qub);
                qug = wave_shr1(qug);
                lb = obl;
                lg = ogl;
                ubt = wave_shl1_or(obu, qub);
                ug = wave_shl1_or(ogu, qug);
                db = db2;
                dg = dg2;
                db2 = wave_shl1_or(obd, qdb);
                dg2 = wave_shl1_or(ogd, qdg);
                qdb = wave_shr1(qdb);
                qdg = wave_shr1(qdg);
            }
            wave_lds_sync();
            if (!DOT) write_tile<P, -1>(otile, obase, trash, i0, L1, L2, L1max, L2max, lane, t_hi);
            publish(prog, wave, q * PROG_STRIDE + k + 1);
            if (x_out) {
                // this chunk's flows to the part above, by producer step
                if (lane < P) store_sys4(flows_out + k * P + lane, ring_out[ring_index(k * P, R) + lane]);
                if (k >= 2) {
                    // at least P/2 + 2 (DOT: + P) loads, 2 flow stores and (DOT: none,
                    // else 2P) output stores follow the flow store of chunk k - 2
                    wait_vmcnt<(DOT ? P + P / 2 + 4 : 2 * P + P / 2 + 4)>();
                    if (lane == 0) store_flag(flag_out, progress_word(epoch, k - 1));
                }
            }
        }
        publish(prog, wave, q * PROG_STRIDE + nch);   // nothing to do after the window
        if (x_out) {
            wait_vmcnt<0>();
            if (lane == 0) store_flag(flag_out, progress_word(epoch, nch));
        }
    }

    if (DOT) {
        dacc = wave_sum(dacc);
        if (lane == 0) red[wave] = dacc;
        __syncthreads();
        if (threadIdx.x == 0) {
            float t = 0.0f;
            for (int w = 0; w < NW; ++w) t += red[w];
            if (G == 1) dot[b] = t;
            else spart[(size_t)b * G + part] = t;
        }
    }
}

// ------------------------------------------------------------------ host side

// dynamic LDS bound: 160 KiB less the kernels' static arrays (progress words,
// reductions, the prefetched progress-word slot)
constexpr size_t kLdsLimit = 160 * 1024 - 512;
constexpr int PT = 16;

// LDS of one workgroup whose stripe boundaries use rings of R columns
size_t lds_tangent_r(int R) {
    return (size_t)NW * (65 * PT + PT * 64 + 64 + 64) * sizeof(float) +
           ((size_t)NW * R + NW * (64 + PT)) * sizeof(float);
}
size_t lds_tangent(int L1, int L2) { return lds_tangent_r(ring_len(L1, L2, 256)); }

size_t lds_dual_r(bool dot, int P, int R) {
    const int buf = (dot ? 65 * P : 0) + 2 * P * 64 + 128 + (dot ? 0 : 65 * P) + 64;
    return (size_t)NW * buf * sizeof(float) + ((size_t)NW * R + NW * (64 + P)) * sizeof(float4);
}

// Largest reverse-sweep chunk (16, 8 or 4 steps) whose buffers and rings fit in LDS,
// for a workgroup that runs `rows` rows of stripes.
int dual_chunk(bool dot, int rows, int L2) {
    const int R = ring_len(rows, L2, 128);
    if (lds_dual_r(dot, 16, R) <= kLdsLimit) return 16;
    if (lds_dual_r(dot, 8, R) <= kLdsLimit) return 8;
    if (lds_dual_r(dot, 4, R) <= kLdsLimit) return 4;
    return 0;
}

// Workspace after the primal layout: tangent table + last rows, [B] scalars, then for
// split elements the parts' partial sums and the reverse sweep's boundary flows
// (float4 by step).
struct Second {
    Layout prim;
    float* tan_sk;
    float* tan_brow;
    float* value;
    float* scratch;
    float* spart;     // [B][stripe]
    float4* flows4;   // [B][stripe][step]
    size_t bytes;
};

// bandwidth >= 0: banded primal and tangent tables (the windows of the band)
Second second_layout(void* ws, int B, int L1, int L2, int bandwidth) {
    Second w;
    const size_t es = dtw::band_elem_steps(L1, L2, bandwidth);
    w.prim = layout(ws, B, L1, L2, 1, true, 8, es);
    char* p = (char*)ws + round256(w.prim.bytes);
    const size_t ns = ((size_t)L1 + 63) / 64;
    w.tan_sk = (float*)p;
    w.tan_brow = w.tan_sk + (size_t)B * es * 64;
    p += round256(table_floats(B, L1, L2, 1, es) * sizeof(float));
    w.value = (float*)p;
    w.scratch = w.value + B;
    p += round256((size_t)2 * B * sizeof(float));
    const size_t parts = (size_t)B * (ns > 0 ? ns : 1);
    w.spart = (float*)p;
    p += round256(parts * sizeof(float));
    w.flows4 = (float4*)p;
    p += round256(parts * (size_t)stored_steps(L2) * sizeof(float4));
    w.bytes = (size_t)(p - (char*)ws);
    return w;
}

template <int MODE>
int launch_tangent(const float* input, const int* lengths, int B, int L1, int L2, float T,
                   int bw, const Second& w, hipStream_t st) {
    const int ns = (L1 + 63) / 64;
    // rings of an unsplit element that do not fit: parts of at most NW stripes
    const Split sp = choose_split(B, L1, w.prim, lds_tangent(L1, L2) <= kLdsLimit ? 0 : NW);
    const int R = ring_len(sp.G > 1 ? sp.SPW * 64 : L1, L2, 256);
    const size_t lds = lds_tangent_r(R);
    D2P_REQUIRE(lds <= kLdsLimit, "sequence too long for the LDS stripe rings");
    auto kern = dtw_tangent_kernel<MODE, PT>;
    if (sp.G > 1) D2P_TRY(launch_flag_reset(w.prim.fflag, B * sp.G, st));
    D2P_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds));
    D2P_LAUNCH("dtw_tangent", kern, dim3(split_grid(B, sp.G)), dim3(NW * 64), lds, st, input,
               lengths, w.prim.alpha_sk, w.prim.brow, w.tan_sk, w.tan_brow, w.prim.status,
               w.prim.fflag, B, L1, L2, ns, w.prim.elem_steps, T, bw, R, sp.G, sp.SPW,
               next_epoch());
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

template <int MODE, bool DOT>
int launch_dual(const float* V, const int* lengths, int B, int L1, int L2, float T, int bw,
                const Second& w, float* out, float* dot, hipStream_t st) {
    const int ns = (L1 + 63) / 64;
    const Split sp = choose_split(B, L1, w.prim, dual_chunk(DOT, L1, L2) > 0 ? 0 : NW);
    const int rows = sp.G > 1 ? sp.SPW * 64 : L1;
    const int R = ring_len(rows, L2, 128);
    const int P = dual_chunk(DOT, rows, L2);
    D2P_REQUIRE(P > 0, "sequence too long for the LDS stripe rings");
    const size_t lds = lds_dual_r(DOT, P, R);
    auto k16 = dtw_dual_kernel<MODE, 16, DOT>;
    auto k8 = dtw_dual_kernel<MODE, 8, DOT>;
    auto k4 = dtw_dual_kernel<MODE, 4, DOT>;
    auto kern = P == 16 ? k16 : (P == 8 ? k8 : k4);
    if (sp.G > 1) D2P_TRY(launch_flag_reset(w.prim.bflag, B * sp.G, st));
    D2P_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds));
    D2P_LAUNCH("dtw_dual", kern, dim3(split_grid(B, sp.G)), dim3(NW * 64), lds, st, V, lengths,
               w.prim.alpha_sk, w.prim.brow, w.tan_sk, w.tan_brow, out, dot, w.prim.status,
               w.prim.trash, w.prim.bflag, w.flows4, w.spart, B, L1, L2, ns, w.prim.elem_steps,
               T, bw, R, sp.G, sp.SPW, next_epoch());
    if (DOT && sp.G > 1 && launch_sum_parts(w.spart, dot, B, sp.G, st) != D2P_OK)
        return D2P_ERR_HIP;
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

// rings that do not fit for an unsplit element force parts of at most NW stripes
int check(int B, int L1, int L2, float T) { return dtw::check_shape(B, L1, L2, T); }

}  // namespace dtw2
}  // namespace d2p_amd

using namespace d2p_amd;

extern "C" size_t d2p_dtw_second_workspace_bytes_banded(int B, int max_L1, int max_L2,
                                                         int bandwidth) {
    if (B <= 0 || max_L1 < 0 || max_L2 < 0) return 0;
    return dtw2::second_layout(nullptr, B, max_L1, max_L2, bandwidth).bytes;
}

extern "C" size_t d2p_dtw_second_workspace_bytes(int B, int max_L1, int max_L2) {
    return d2p_dtw_second_workspace_bytes_banded(B, max_L1, max_L2, -1);
}

extern "C" int d2p_dtw_hvp(const float* costs, const float* tangent, const int* lengths, int B,
                           int max_L1, int max_L2, float temperature, int bandwidth, float* hvp,
                           void* workspace, size_t workspace_bytes, void* stream) {
    D2P_TRY(dtw2::check(B, max_L1, max_L2, temperature));
    if (B == 0) return D2P_OK;
    D2P_REQUIRE(costs && tangent && hvp, "null pointer argument");
    D2P_REQUIRE(workspace && workspace_bytes >=
                                 d2p_dtw_second_workspace_bytes_banded(B, max_L1, max_L2,
                                                                       bandwidth),
                "workspace too small");
    hipStream_t st = (hipStream_t)stream;
    const dtw2::Second w = dtw2::second_layout(workspace, B, max_L1, max_L2, bandwidth);
    D2P_TRY(dtw::launch_forward(costs, lengths, B, max_L1, max_L2, temperature, bandwidth, w.prim,
                                w.value, st));
    D2P_TRY(dtw2::launch_tangent<dtw2::HVP>(tangent, lengths, B, max_L1, max_L2, temperature,
                                            bandwidth, w, st));
    D2P_TRY(dtw2::launch_dual<dtw2::HVP, false>(nullptr, lengths, B, max_L1, max_L2, temperature,
                                                bandwidth, w, hvp, nullptr, st));
    return wf::launch_poison(w.prim.status, B, (long long)max_L1 * max_L2, hvp, nullptr, nullptr,
                             nullptr, nullptr, nullptr, st);
}

extern "C" int d2p_dtw_param_jacobian(const float* costs, const int* lengths, int B, int max_L1,
                                      int max_L2, float temperature, int bandwidth,
                                      float* jacobian, void* workspace, size_t workspace_bytes,
                                      void* stream) {
    D2P_TRY(dtw2::check(B, max_L1, max_L2, temperature));
    if (B == 0) return D2P_OK;
    D2P_REQUIRE(costs && jacobian, "null pointer argument");
    D2P_REQUIRE(workspace && workspace_bytes >=
                                 d2p_dtw_second_workspace_bytes_banded(B, max_L1, max_L2,
                                                                       bandwidth),
                "workspace too small");
    hipStream_t st = (hipStream_t)stream;
    const dtw2::Second w = dtw2::second_layout(workspace, B, max_L1, max_L2, bandwidth);
    D2P_TRY(dtw::launch_forward(costs, lengths, B, max_L1, max_L2, temperature, bandwidth, w.prim,
                                w.value, st));
    D2P_TRY(dtw2::launch_tangent<dtw2::TEMP>(costs, lengths, B, max_L1, max_L2, temperature,
                                             bandwidth, w, st));
    D2P_TRY(dtw2::launch_dual<dtw2::TEMP, false>(nullptr, lengths, B, max_L1, max_L2,
                                                 temperature, bandwidth, w, jacobian, nullptr, st));
    return wf::launch_poison(w.prim.status, B, (long long)max_L1 * max_L2, jacobian, nullptr,
                             nullptr, nullptr, nullptr, nullptr, st);
}

extern "C" int d2p_dtw_backward_full(const float* costs, const float* grad_alignment,
                                     const int* lengths, int B, int max_L1, int max_L2,
                                     float temperature, int bandwidth, float* grad_costs,
                                     float* grad_T, void* workspace, size_t workspace_bytes,
                                     void* stream) {
    D2P_TRY(dtw2::check(B, max_L1, max_L2, temperature));
    if (B == 0) return D2P_OK;
    D2P_REQUIRE(costs && grad_alignment && grad_costs && grad_T,
                "null pointer argument");
    D2P_REQUIRE(workspace && workspace_bytes >=
                                 d2p_dtw_second_workspace_bytes_banded(B, max_L1, max_L2,
                                                                       bandwidth),
                "workspace too small");
    hipStream_t st = (hipStream_t)stream;
    const dtw2::Second w = dtw2::second_layout(workspace, B, max_L1, max_L2, bandwidth);
    D2P_TRY(dtw::launch_forward(costs, lengths, B, max_L1, max_L2, temperature, bandwidth, w.prim,
                                w.value, st));
    D2P_TRY(dtw2::launch_tangent<dtw2::HVP>(grad_alignment, lengths, B, max_L1, max_L2,
                                            temperature, bandwidth, w, st));
    D2P_TRY(dtw2::launch_dual<dtw2::HVP, false>(nullptr, lengths, B, max_L1, max_L2, temperature,
                                                bandwidth, w, grad_costs, nullptr, st));
    D2P_TRY(dtw2::launch_tangent<dtw2::TEMP>(costs, lengths, B, max_L1, max_L2, temperature,
                                             bandwidth, w, st));
    D2P_TRY(dtw2::launch_dual<dtw2::TEMP, true>(grad_alignment, lengths, B, max_L1, max_L2,
                                                temperature, bandwidth, w, nullptr, grad_T, st));
    return wf::launch_poison(w.prim.status, B, (long long)max_L1 * max_L2, grad_costs, nullptr,
                             grad_T, nullptr, nullptr, nullptr, st);
}
