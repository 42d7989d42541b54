// swa_second.hip -- second-order quantities of affine-gap soft Smith-Waterman on
// gfx950: Hessian-vector products and Jacobians of the marginals with respect to
// gap_open, gap_ext and temperature.
//
// Reference behaviour restated (not translated):
//   HVP          /root/reference/src/sw_affine/kernels_cpu.cpp:362-631
//   param grad   /root/reference/src/sw_affine/kernels_cpu.cpp:643-921 (0 open, 1 ext, 2 T)
// Each of the three states X in {M, I, D} has softmax weights over its candidates:
//   M: (M, I, D)[i-1,j-1] + s and s;  I: M[i-1,j] + open, I[i-1,j] + ext;
//   D: M[i,j-1] + open, D[i,j-1] + ext  (no weights when every candidate is NINF).
// The tangent sweep gives x_X = sum_k w_k d_k (+ (X - E_w[v]) / T for the
// temperature) with d the candidates' tangents:
//   HVP  d_M = (x_M + V, x_I + V, x_D + V, V) at the diagonal, d_I, d_D plain;
//   open / ext: +1 on the open / extend candidates of I and D.
// The reverse sweep carries beta and a second channel g per state, with
//   g_pred += g w_k + beta dw_k,  dw_k = w_k (d_k - E_w[d]) / T
//   (+ w_k (E_w[v] - v_k) / T^2 for the temperature),
// started from beta_init (x - dS) / T (HVP: first in the accumulation; param: last,
// with - beta_init (X - S) / T^2 for the temperature).  Output per cell: HVP
// g_M (sum w_M) + beta_M (sum dw_M); param g_M.
//
// Mapping: the stripe pipeline of wavefront.hip.h.  The tangent sweep carries the
// (x_M, x_I, x_D) triple across stripes in a float4 ring; the reverse sweep sends
// (beta, g) flows upward in three rings: up flows to (M, I), diagonal flows to
// (M, I) and to D.  Only the edge lane writes these rings (exec-masked stores), so
// they need no per-lane sinks.

#include <vector>

#include "wavefront.hip.h"
#include "../../include/d2p_amd.h"
#include "capi_util.hip.h"
#include "swa_internal.hip.h"

namespace d2p_amd {
namespace swa2 {

using namespace wf;

enum Mode { HVP = 0, OPEN = 1, EXT = 2, TEMP = 3 };

// Softmax weights w of three candidate values v (none when all are NINF) and their
// tangents dw_k = w_k (d_k - E_w[d]) / T for candidate tangents d; the parameter
// modes take the differences relative to the largest candidate's tangent (the
// weights' sum differs from 1 by an ulp or two), and the temperature adds
// w_k (E_w[v] - v_k) / T^2.
template <int MODE>
__device__ __forceinline__ void softmax3_tangent(const float (&v)[3], const float (&d)[3],
                                                 float c, float rT, float (&w)[3],
                                                 float (&dw)[3]) {
    const float m = fmaxf(fmaxf(v[0], v[1]), v[2]);
    const float e0 = fast_exp2((v[0] - m) * c), e1 = fast_exp2((v[1] - m) * c);
    const float e2 = fast_exp2((v[2] - m) * c);
    const float r = m > kNINF ? fast_rcp((e0 + e1) + e2) : 0.0f;
    w[0] = e0 * r;
    w[1] = e1 * r;
    w[2] = e2 * r;
    if (MODE == HVP) {
        const float E = (w[0] * d[0] + w[1] * d[1]) + w[2] * d[2];
#pragma unroll
        for (int k = 0; k < 3; ++k) dw[k] = w[k] * (d[k] - E) * rT;
    } else {
        const float p = v[0] >= m ? d[0] : (v[1] >= m ? d[1] : d[2]);
        const float q0 = d[0] - p, q1 = d[1] - p, q2 = d[2] - p;
        const float E = (w[0] * q0 + w[1] * q1) + w[2] * q2;
        dw[0] = w[0] * (q0 - E) * rT;
        dw[1] = w[1] * (q1 - E) * rT;
        dw[2] = w[2] * (q2 - E) * rT;
        if (MODE == TEMP) {
            const float rT2 = rT * rT;
            const float p0 = v[0] - m, p1 = v[1] - m, p2 = v[2] - m;
            const float Ev = (w[0] * p0 + w[1] * p1) + w[2] * p2;
            dw[0] += w[0] > 0.0f ? w[0] * (Ev - p0) * rT2 : 0.0f;
            dw[1] += w[1] > 0.0f ? w[1] * (Ev - p1) * rT2 : 0.0f;
            dw[2] += w[2] > 0.0f ? w[2] * (Ev - p2) * rT2 : 0.0f;
        }
    }
}

// ------------------------------------------------------------------ tangent sweep

// NWA: global alignment with affine gaps (/root/reference/src/nw_affine/kernels_cpu.cpp:
// 353-613 and 619-1002): each state has three candidates (M: the diagonal states, no
// start; I: M, I, D above; D: M, I, D to the left); the HVP tangent of M adds V to
// the weighted diagonal tangents; the boundary chains I[i,0], D[0,j] carry the
// tangents 1 (open) or i-1 / j-1 (ext).  The value's tangent is taken at the terminal
// cell by the reverse sweep, so no per-cell sum is formed here.
template <int MODE, int P, bool NWA = false>
__global__ void __launch_bounds__(NW * 64)
swa_tangent_kernel(const float* __restrict__ scores, const float* __restrict__ V,
                   const int* __restrict__ lengths, const float* __restrict__ alpha_sk,
                   const float* __restrict__ brow, const float* __restrict__ partition,
                   float* __restrict__ tan_sk, float* __restrict__ tan_brow,
                   float* __restrict__ sdot, int* __restrict__ status,
                   uint64_t* __restrict__ tflag, float* __restrict__ spart, int B, int L1max,
                   int L2max, int NSmax, float go, float ge, float T, int R, int G, int SPW,
                   uint32_t epoch) {
    constexpr bool HAS_V = MODE == HVP;
    using Tile = ChunkTile<P>;
    constexpr int VT = Tile::FLOATS;
    constexpr int AR = VT + (HAS_V ? Tile::FLOATS : 0);   // 3 planes x P alpha rows
    constexpr int RR = AR + 3 * P * 64;                   // 3 planes x row above
    constexpr int TR = RR + 3 * 64;                       // 3 tangent rows of the part above
    constexpr int BUF = TR + 3 * 64;
    constexpr int SINK = 64 + P;
    extern __shared__ __align__(16) float smem[];
    __shared__ int prog[NW];
    __shared__ float red[NW];
    // parts as in the primal forward: part p > 0 takes its first stripe's tangent rows
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
    const float S = partition[b];
    const int NS = L2 > 0 ? (L1 + 63) >> 6 : 0;
    const int nsteps = L2 + 63;
    const int nch = (nsteps + P - 1) / P;
    const size_t NT = (size_t)stored_steps(L2max);
    const size_t PL = NT * 64;
    const float* sbase = scores + (size_t)b * L1max * L2max;
    const float* vbase = HAS_V ? V + (size_t)b * L1max * L2max : nullptr;
    const uint32_t in_lds = lds_address(buf);
    float sacc = 0.0f;
    const int s_begin = part * SPW;
    const int NL = max(min(NS, s_begin + SPW) - s_begin, 0);   // stripes of this part
    const bool has_next = s_begin + NL < NS;
    const uint64_t* flag_in = tflag + (size_t)b * G + (part > 0 ? part - 1 : 0);
    uint64_t* flag_out = tflag + (size_t)b * G + part;

    for (int l = wave; l < NL; l += NW) {
        const int s = s_begin + l;
        const int i0 = s * 64;
        const int L2eff = (i0 + lane < L1) ? L2 : 0;
        const float* astripe = alpha_sk + ((size_t)b * NSmax + s) * 3 * PL;
        const float* bup = brow + ((size_t)b * NSmax + (s > 0 ? s - 1 : 0)) * 3 * NT;
        float* tout = tan_sk + ((size_t)b * NSmax + s) * 3 * PL + APAD * 64;
        float* tb_s = tan_brow + ((size_t)b * NSmax + s) * 3 * NT;
        const float* tb_up = tan_brow + ((size_t)b * NSmax + (s > 0 ? s - 1 : 0)) * 3 * NT;
        const float4* ring_in = ring_from(rings, l, R);
        float4* ring_out = ring_of(rings, l, R);
        const bool x_in = l == 0 && part > 0;        // tangent rows above from part - 1
        const bool x_out = l == NL - 1 && has_next;  // tangent rows feed part + 1
        int seen = -1;       // chunks of the previous part known to be complete

        auto issue_chunk = [&](int k) {
            const int t0 = k * P;
            dma_tile<P, 1>(in_lds, sbase, i0, L1max, L2max, lane, t0);
            if (HAS_V) dma_tile<P, 1>(in_lds + VT * 4, vbase, i0, L1max, L2max, lane, t0);
#pragma unroll
            for (int pl = 0; pl < 3; ++pl)
                dma_rows<P, 1>(in_lds + (AR + pl * P * 64) * 4, astripe + pl * PL, t0, ul4);
            const uint32_t roff = (uint32_t)min(t0 + 62 + min(lane, P), nsteps - 1) * 4u;
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) {
                uint32_t o = roff, la = in_lds + (RR + pl * 64) * 4;
                lds_dma_dword<0>(bup + pl * NT, o, la, 0u);
            }
            if (x_in) {
                // lane j < P: the tangents of the last row above at step t0 + 63 + j
                const uint32_t toff = (uint32_t)min(t0 + 63 + min(lane, P - 1), nsteps - 1) * 4u;
#pragma unroll
                for (int pl = 0; pl < 3; ++pl) {
                    uint32_t o = toff, la = in_lds + (TR + pl * 64) * 4;
                    lds_dma_dword_sys<0>(tb_up + pl * NT, o, la, 0u);
                }
            }
        };

        // NWA: the boundary I[i,0] of this lane's row, its value and tangent
        const bool rowv = NWA && i0 + lane < L1;
        const float bndI = rowv ? go + (float)(i0 + lane) * ge : kNINF;
        const float xbI = rowv ? (MODE == OPEN ? 1.0f : (MODE == EXT ? (float)(i0 + lane) : 0.0f))
                               : 0.0f;
#pragma unroll
        for (int t = -APAD; t < 0; ++t)
#pragma unroll
            for (int pl = 0; pl < 3; ++pl)
                lane_store(tout + pl * PL + t * 64, ul4, pl == 1 ? xbI : 0.0f);
        wave_lds_sync();
        if (x_in) seen = wait_part(flag_in, epoch, min(lead(P), nch), st);
        issue_chunk(0);
        float AM[P + 2], AI[P + 2], AD[P + 2];
        AM[P] = AM[P + 1] = AD[P] = AD[P + 1] = kNINF;
        AI[P] = AI[P + 1] = bndI;
        float cM = 0.0f, cI = xbI, cD = 0.0f;       // tangents at the previous step
        float pM = 0.0f, pI = 0.0f, pD = 0.0f;      // their up values
        if (NWA && lane == 0 && s > 0)   // lane 0's first diagonal: I[i0, 0]
            pI = MODE == OPEN ? 1.0f : (MODE == EXT ? (float)(i0 - 1) : 0.0f);

        for (int k = 0; k < nch; ++k) {
            const int t0 = k * P;
            chunk_waits<P>(prog, l, NL, k, nch, R, st);
            // this chunk's loads, followed by at least the 3P + 3 stores of the previous
            // chunk
            if (k == 0) wait_vmcnt<0>(); else wait_vmcnt<3 * P>();
            if (x_in && k > 0) {
                // its progress word, loaded one chunk ago before those stores
                const int got = flag_chunks_lds(fslot, epoch);
                seen = got > seen ? got : seen;
            }
            float sv[P], vv[P];
#pragma unroll
            for (int u = 0; u < P; ++u) {
                sv[u] = buf[tbase + u];
                vv[u] = HAS_V ? buf[VT + tbase + u] : 0.0f;
            }
            AM[0] = AM[P]; AM[1] = AM[P + 1];
            AI[0] = AI[P]; AI[1] = AI[P + 1];
            AD[0] = AD[P]; AD[1] = AD[P + 1];
#pragma unroll
            for (int j = 0; j < P; ++j) {
                AM[j + 2] = buf[AR + j * 64 + lane];
                AI[j + 2] = buf[AR + P * 64 + j * 64 + lane];
                AD[j + 2] = buf[AR + 2 * P * 64 + j * 64 + lane];
            }
            const bool row_ok = s > 0 && lane <= P && t0 + 62 + lane <= nsteps - 1;
            float bM = row_ok ? buf[RR + lane] : kNINF;
            float bI = row_ok ? buf[RR + 64 + lane] : kNINF;
            float bD = row_ok ? buf[RR + 128 + lane] : kNINF;
            float rM = 0.0f, rI = 0.0f, rD = 0.0f;
            if (NWA && s == 0) {
                // row 0: lane j <= P the values at column t0 - 1 + j (0-based; -1 is
                // the start cell), lane j < P the tangents at column t0 + j
                const int c0 = t0 - 1 + lane;
                if (lane <= P) {
                    bM = c0 == -1 ? 0.0f : kNINF;
                    bD = c0 >= 0 ? go + (float)c0 * ge : kNINF;
                }
                if (lane < P)
                    rD = MODE == OPEN ? 1.0f : (MODE == EXT ? (float)(t0 + lane) : 0.0f);
            }
            if (s > 0 && lane < P) {
                if (x_in) {
                    rM = buf[TR + lane];
                    rI = buf[TR + 64 + lane];
                    rD = buf[TR + 128 + lane];
                } else {
                    const float4 r = ring_in[ring_index(t0 + lane + 63, R)];
                    rM = r.x;
                    rI = r.y;
                    rD = r.z;
                }
            }
            wave_lds_sync();
            if (k + 1 < nch) {
                if (x_in) {
                    const int need = min(k + 1 + lead(P), nch);
                    if (seen < need) seen = wait_part(flag_in, epoch, need, st);
                }
                issue_chunk(k + 1);
                if (x_in) flag_load_lds(flag_in, fslot_lds, lane);
            }
            float4* pub = (lane == 63) ? ring_out + ring_index(t0, R) : sink + lane;
            float* toutc = tout + (size_t)t0 * 64;
#pragma unroll
            for (int u = 0; u < P; ++u) {
                const int t = t0 + u;
                const bool ok = (unsigned)(t - lane) < (unsigned)L2eff;
                const float sc = ok ? sv[u] : kNINF;
                const float vd = ok ? vv[u] : 0.0f;
                // primal predecessors
                const float dM = wave_shr1_or(AM[u], bM), dI = wave_shr1_or(AI[u], bI),
                            dD = wave_shr1_or(AD[u], bD);
                const float nbM = wave_shl1(bM), nbI = wave_shl1(bI),
                            nbD = wave_shl1(bD);
                const float uM = wave_shr1_or(AM[u + 1], nbM), uI = wave_shr1_or(AI[u + 1], nbI);
                const float uD = NWA ? wave_shr1_or(AD[u + 1], nbD) : kNINF;
                bM = nbM;
                bI = nbI;
                bD = nbD;
                const float lM = AM[u + 1], lI = AI[u + 1], lD = AD[u + 1];
                // tangent predecessors
                const float tuM = wave_shr1_or(cM, rM), tuI = wave_shr1_or(cI, rI),
                            tuD = wave_shr1_or(cD, rD);
                rM = wave_shl1(rM);
                rI = wave_shl1(rI);
                rD = wave_shl1(rD);
                const float tdM = pM, tdI = pI, tdD = pD;
                pM = tuM;
                pI = tuI;
                pD = tuD;
                float xM, xI, xD;
                if constexpr (NWA) {
                    const float ao = MODE == OPEN ? 1.0f : 0.0f, ae = MODE == EXT ? 1.0f : 0.0f;
                    // M over the diagonal states
                    const float m3 = fmaxf(fmaxf(dM, dI), dD);
                    const float e0 = fast_exp2((dM - m3) * c), e1 = fast_exp2((dI - m3) * c);
                    const float e2 = fast_exp2((dD - m3) * c);
                    const float r3 = m3 > kNINF ? fast_rcp((e0 + e1) + e2) : 0.0f;
                    // I over M + open, I + ext, D + open above
                    const float i0v = uM + go, i1v = uI + ge, i2v = uD + go;
                    const float mi = fmaxf(fmaxf(i0v, i1v), i2v);
                    const float f0 = fast_exp2((i0v - mi) * c), f1 = fast_exp2((i1v - mi) * c);
                    const float f2 = fast_exp2((i2v - mi) * c);
                    const float ri = mi > kNINF ? fast_rcp((f0 + f1) + f2) : 0.0f;
                    // D over M + open, D + ext, I + open to the left
                    const float d0v = lM + go, d1v = lD + ge, d2v = lI + go;
                    const float md = fmaxf(fmaxf(d0v, d1v), d2v);
                    const float g0 = fast_exp2((d0v - md) * c), g1 = fast_exp2((d1v - md) * c);
                    const float g2 = fast_exp2((d2v - md) * c);
                    const float rd = md > kNINF ? fast_rcp((g0 + g1) + g2) : 0.0f;
                    const float di0 = tuM + ao, di1 = tuI + ae, di2 = tuD + ao;
                    const float dd0 = cM + ao, dd1 = cD + ae, dd2 = cI + ao;
                    if (MODE == HVP) {
                        xM = r3 > 0.0f ? vd + ((e0 * tdM + e1 * tdI) + e2 * tdD) * r3 : 0.0f;
                        xI = ((f0 * di0 + f1 * di1) + f2 * di2) * ri;
                        xD = ((g0 * dd0 + g1 * dd1) + g2 * dd2) * rd;
                    } else {
                        // E_w[d] as the largest candidate's tangent plus the weighted
                        // differences (see the linear-gap kernel)
                        const float pm = dM >= m3 ? tdM : (dI >= m3 ? tdI : tdD);
                        xM = r3 > 0.0f
                                 ? pm + ((e0 * (tdM - pm) + e1 * (tdI - pm)) + e2 * (tdD - pm)) * r3
                                 : 0.0f;
                        const float pi = i0v >= mi ? di0 : (i1v >= mi ? di1 : di2);
                        xI = ri > 0.0f
                                 ? pi + ((f0 * (di0 - pi) + f1 * (di1 - pi)) + f2 * (di2 - pi)) * ri
                                 : 0.0f;
                        const float pd = d0v >= md ? dd0 : (d1v >= md ? dd1 : dd2);
                        xD = rd > 0.0f
                                 ? pd + ((g0 * (dd0 - pd) + g1 * (dd1 - pd)) + g2 * (dd2 - pd)) * rd
                                 : 0.0f;
                        if (MODE == TEMP) {
                            // alpha - E_w[v] per state, relative to the largest candidate
                            // (M: alpha - s - E_w[diagonal])
                            const float E3 =
                                ((e0 * (dM - m3) + e1 * (dI - m3)) + e2 * (dD - m3)) * r3;
                            const float E3i =
                                ((f0 * (i0v - mi) + f1 * (i1v - mi)) + f2 * (i2v - mi)) * ri;
                            const float E3d =
                                ((g0 * (d0v - md) + g1 * (d1v - md)) + g2 * (d2v - md)) * rd;
                            xM += r3 > 0.0f ? ((AM[u + 2] - sc - m3) - E3) * rT : 0.0f;
                            xI += ri > 0.0f ? ((AI[u + 2] - mi) - E3i) * rT : 0.0f;
                            xD += rd > 0.0f ? ((AD[u + 2] - md) - E3d) * rT : 0.0f;
                        }
                    }
                } else {
                // M
                const float v0 = dM + sc, v1 = dI + sc, v2 = dD + sc;
                const float m4 = fmaxf(fmaxf(v0, v1), fmaxf(v2, sc));
                const float e0 = fast_exp2((v0 - m4) * c), e1 = fast_exp2((v1 - m4) * c);
                const float e2 = fast_exp2((v2 - m4) * c), e3 = fast_exp2((sc - m4) * c);
                const float r4 = fast_rcp(((e0 + e1) + e2) + e3);
                // I
                const float i0v = uM + go, i1v = uI + ge;
                const float mi = fmaxf(i0v, i1v);
                const float f0 = fast_exp2((i0v - mi) * c), f1 = fast_exp2((i1v - mi) * c);
                const float ri = mi > kNINF ? fast_rcp(f0 + f1) : 0.0f;
                // D
                const float d0v = lM + go, d1v = lD + ge;
                const float md = fmaxf(d0v, d1v);
                const float g0 = fast_exp2((d0v - md) * c), g1 = fast_exp2((d1v - md) * c);
                const float rd = md > kNINF ? fast_rcp(g0 + g1) : 0.0f;
                if (MODE == HVP) {
                    xM = (((e0 * (tdM + vd) + e1 * (tdI + vd)) + e2 * (tdD + vd)) + e3 * vd) * r4;
                    xI = (f0 * tuM + f1 * tuI) * ri;
                    xD = (g0 * cM + g1 * cD) * rd;
                } else {
                    // The parameter tangents pass E_w[d] on as the candidate of the
                    // largest value plus the weighted differences (two candidates:
                    // d_0 + w_1 (d_1 - d_0)): the weights' sum differs from 1 by an ulp
                    // or two, and taken whole that factor would compound along the
                    // alignment into tangents that grow with its length (the Jacobian
                    // subtracts dS/dtheta from them).
                    const float ao = MODE == OPEN ? 1.0f : 0.0f, ae = MODE == EXT ? 1.0f : 0.0f;
                    const float pM = v0 >= m4 ? tdM : (v1 >= m4 ? tdI : (v2 >= m4 ? tdD : 0.0f));
                    xM = pM + (((e0 * (tdM - pM) + e1 * (tdI - pM)) + e2 * (tdD - pM)) - e3 * pM) * r4;
                    const float di0 = tuM + ao, di1 = tuI + ae;
                    xI = ri > 0.0f ? di0 + f1 * ri * (di1 - di0) : 0.0f;
                    const float dd0 = cM + ao, dd1 = cD + ae;
                    xD = rd > 0.0f ? dd0 + g1 * rd * (dd1 - dd0) : 0.0f;
                    if (MODE == TEMP) {
                        // alpha - E_w[v] of each state, both relative to its largest
                        // candidate (the weights' sum differs from 1 by an ulp or two)
                        const float E4 =
                            (((e0 * (v0 - m4) + e1 * (v1 - m4)) + e2 * (v2 - m4)) + e3 * (sc - m4)) *
                            r4;
                        const float E2i = (f0 * (i0v - mi) + f1 * (i1v - mi)) * ri;
                        const float E2d = (g0 * (d0v - md) + g1 * (d1v - md)) * rd;
                        xM += ((AM[u + 2] - m4) - E4) * rT;
                        xI += ri > 0.0f ? ((AI[u + 2] - mi) - E2i) * rT : 0.0f;
                        xD += rd > 0.0f ? ((AD[u + 2] - md) - E2d) * rT : 0.0f;
                    }
                }
                }
                cM = ok ? xM : 0.0f;
                cI = ok ? xI : (NWA && t < lane ? xbI : 0.0f);   // NWA: left of column 0
                cD = ok ? xD : 0.0f;
                lane_store(toutc + u * 64, ul4, cM);
                lane_store(toutc + PL + u * 64, ul4, cI);
                lane_store(toutc + 2 * PL + u * 64, ul4, cD);
                pub[u] = make_float4(cM, cI, cD, 0.0f);
                if (MODE == HVP && !NWA) {
                    float lp;
                    lp = (AM[u + 2] - S) * c;
                    sacc += fast_exp2(lp < 0.0f ? lp : 0.0f) * cM;
                    lp = (AI[u + 2] - S) * c;
                    sacc += fast_exp2(lp < 0.0f ? lp : 0.0f) * cI;
                    lp = (AD[u + 2] - S) * c;
                    sacc += fast_exp2(lp < 0.0f ? lp : 0.0f) * cD;
                }
            }
            wave_lds_sync();
            if (lane < P) {
                const float4 r = ring_out[t0 % R + lane];
                if (x_out) {
                    store_sys(tb_s + t0 + lane, r.x);
                    store_sys(tb_s + NT + t0 + lane, r.y);
                    store_sys(tb_s + 2 * NT + t0 + lane, r.z);
                } else {
                    const unsigned o = (unsigned)(t0 + lane) * 4u;
                    lane_store(tb_s, o, r.x);
                    lane_store(tb_s + NT, o, r.y);
                    lane_store(tb_s + 2 * NT, o, r.z);
                }
            }
            publish(prog, wave, l * PROG_STRIDE + k + 1);
            if (x_out && k >= 2) {
                // at least P + 3P/4 + 3 loads and 6P + 6 stores follow the row stores of
                // chunk k - 2 (more than the counter holds): those are complete
                wait_vmcnt<63>();
                if (lane == 0) store_flag(flag_out, progress_word(epoch, k - 1));
            }
        }
        if (x_out) {
            wait_vmcnt<0>();
            if (lane == 0) store_flag(flag_out, progress_word(epoch, nch));
        }
    }

    if (MODE == HVP && !NWA) {
        sacc = wave_sum(sacc);
        if (lane == 0) red[wave] = sacc;
        __syncthreads();
        if (threadIdx.x == 0) {
            float t = 0.0f;
            for (int w = 0; w < NW; ++w) t += red[w];
            if (G == 1) sdot[b] = t;
            else spart[(size_t)b * G + part] = t;
        }
    }
}

// ------------------------------------------------------------------ reverse sweep

// NWA: global alignment: beta and g start at the terminal cell only, beta_X = w_X and
// g_X = w_X (x_X - E_w[x]) / T (+ w_X (E_w[a] - a_X) / T^2 for the temperature) over
// its three states, computed there from the tables; a state passes flow when beta >
// 1e-20 or |g| > 1e-20; the output is g_M (the marginal is beta_M).  The third ring
// carries (diagonal D, up D) (beta, g) pairs.
template <int MODE, int P, bool DOT, bool NWA = false>
__global__ void __launch_bounds__(NW * 64)
swa_dual_kernel(const float* __restrict__ scores, const float* __restrict__ V,
                const int* __restrict__ lengths, const float* __restrict__ alpha_sk,
                const float* __restrict__ brow, const float* __restrict__ tan_sk,
                const float* __restrict__ tan_brow, const float* __restrict__ partition,
                const float* __restrict__ dS, float* __restrict__ out, float* __restrict__ dot,
                int* __restrict__ status, float* __restrict__ trash,
                uint64_t* __restrict__ dflag, float4* __restrict__ fU, float4* __restrict__ fD,
                float2* __restrict__ fE, float* __restrict__ spart, int B, int L1max,
                int L2max, int NSmax, float go, float ge, float T, int R, int G, int SPW,
                uint32_t epoch) {
    constexpr bool HAS_V = MODE == HVP || DOT;
    using Tile = ChunkTile<P>;
    constexpr int VT = Tile::FLOATS;
    constexpr int AR = VT + (HAS_V ? Tile::FLOATS : 0);   // 3 x P alpha rows
    constexpr int XR = AR + 3 * P * 64;                   // 3 x P tangent rows
    constexpr int RA = XR + 3 * P * 64;                   // 3 alpha rows above
    constexpr int RX = RA + 3 * 64;                       // 3 tangent rows above
    constexpr int OT = RX + 3 * 64;
    // flows from the part below: up (float4), diagonal (float4), diagonal to D (float2)
    constexpr int FBU = OT + (DOT ? 0 : Tile::FLOATS);
    constexpr int FBD = FBU + 64;
    constexpr int FBE = FBD + 64;
    constexpr int BUF = FBE + 64;
    static_assert(4 * P + 4 <= 64, "boundary flows fit their buffers");
    using FE = std::conditional_t<NWA, float4, float2>;
    extern __shared__ __align__(16) float smem[];
    __shared__ int prog[NW];
    __shared__ float red[NW];
    // parts run bottom-up as in the primal backward; the last stripe of a part below
    // the first hands its flows to the part above through fU / fD / fE
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
    // rings [NW][R]: (beta, g) up flows to (M, I); diagonal flows to (M, I); to D
    float4* ringU = reinterpret_cast<float4*>(smem + NW * BUF);
    float4* ringD = ringU + NW * R;
    FE* ringE = reinterpret_cast<FE*>(ringD + NW * R);
    FE* fEx = reinterpret_cast<FE*>(fE);
    int* st = status + b;
    const int tbase = Tile::read_base(lane);

    if (lane == 0) prog[wave] = -1;
    __syncthreads();

    const int L1 = lengths ? min(max(lengths[2 * b], 0), L1max) : L1max;
    const int L2 = lengths ? min(max(lengths[2 * b + 1], 0), L2max) : L2max;
    const float c = kLog2e / T;
    const float rT = 1.0f / T;
    const float S = partition[b];
    const float dSb = dS[b];
    const int NS = L2 > 0 ? (L1 + 63) >> 6 : 0;
    const int nsteps = L2 + 63;
    const int nch = (nsteps + P - 1) / P;
    const size_t NT = (size_t)stored_steps(L2max);
    const size_t PL = NT * 64;
    const float* sbase = scores + (size_t)b * L1max * L2max;
    const float* vbase = HAS_V ? V + (size_t)b * L1max * L2max : nullptr;
    float* obase = DOT ? nullptr : out + (size_t)b * L1max * L2max;
    const uint32_t in_lds = lds_address(buf);

    if (!DOT) {   // each part zeroes its share of the rows' padding
        const int rows = (L1max + G - 1) / G;
        zero_padding(obase, L1, L2, L1max, L2max, NW * 64, part * rows,
                     min(L1max, part * rows + rows));
    }

    float dacc = 0.0f;
    float AM[P + 2], AI[P + 2], AD[P + 2], XM[P + 2], XI[P + 2], XD[P + 2];
    const int s_begin = part * SPW;
    const int NL = max(min(NS, s_begin + SPW) - s_begin, 0);   // stripes of this part
    const bool has_next = s_begin + NL < NS;
    const uint64_t* flag_in = dflag + (size_t)b * G + (part + 1 < G ? part + 1 : part);
    uint64_t* flag_out = dflag + (size_t)b * G + part;

    for (int q = wave; q < NL; q += NW) {
        const int s = s_begin + NL - 1 - q;
        const int i0 = s * 64;
        const int L2eff = (i0 + lane < L1) ? L2 : 0;
        const size_t sb = ((size_t)b * NSmax + s) * 3;
        const size_t ub = ((size_t)b * NSmax + (s > 0 ? s - 1 : 0)) * 3;
        const float* astripe = alpha_sk + sb * PL;
        const float* xstripe = tan_sk + sb * PL;
        const float* bupA = brow + ub * NT;
        const float* bupX = tan_brow + ub * NT;
        const float4* inU = ring_from(ringU, q, R);
        const float4* inD = ring_from(ringD, q, R);
        const FE* inE = ring_from(ringE, q, R);
        float4* outU = ring_of(ringU, q, R);
        float4* outD = ring_of(ringD, q, R);
        FE* outE = ring_of(ringE, q, R);
        const bool x_in = q == 0 && has_next;             // flows from the part below
        const bool x_out = q == NL - 1 && part > 0;       // flows to the part above
        const bool below = q > 0 || x_in;
        // boundary flows by producer step: written by stripe s (x_out), read from s + 1
        const size_t fo = ((size_t)b * NSmax + s) * NT;
        const size_t fi = ((size_t)b * NSmax + (x_in ? s + 1 : s)) * NT;
        int seen = -1;       // chunks of the part below known to be complete

        auto issue_chunk = [&](int k) {
            const int th = nsteps - 1 - k * P;
            dma_tile<P, -1>(in_lds, sbase, i0, L1max, L2max, lane, th);
            if (HAS_V) dma_tile<P, -1>(in_lds + VT * 4, vbase, i0, L1max, L2max, lane, th);
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) {
                dma_rows<P, -1>(in_lds + (AR + pl * P * 64) * 4, astripe + pl * PL, th - 2, ul4);
                dma_rows<P, -1>(in_lds + (XR + pl * P * 64) * 4, xstripe + pl * PL, th - 2, ul4);
            }
            const uint32_t roff = (uint32_t)min(th - min(lane, P) + 63, nsteps - 1) * 4u;
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) {
                uint32_t o = roff, l = in_lds + (RA + pl * 64) * 4;
                lds_dma_dword<0>(bupA + pl * NT, o, l, 0u);
                o = roff;
                l = in_lds + (RX + pl * 64) * 4;
                lds_dma_dword<0>(bupX + pl * NT, o, l, 0u);
            }
            if (x_in) {
                // up flows of producer slots kP+63 .. kP+62+P, diagonal flows of slots
                // kP+62 .. kP+61+P: float f of each range in lane f, clamped to the last
                // slot
                const int last = nsteps - 1;
                uint32_t o = (uint32_t)min((k * P + 63) * 4 + min(lane, 4 * P - 1), last * 4 + 3) * 4u;
                uint32_t l = in_lds + FBU * 4;
                lds_dma_dword_sys<0>(reinterpret_cast<const float*>(fU + fi), o, l, 0u);
                o = (uint32_t)min((k * P + 62) * 4 + min(lane, 4 * P - 1), last * 4 + 3) * 4u;
                l = in_lds + FBD * 4;
                lds_dma_dword_sys<0>(reinterpret_cast<const float*>(fD + fi), o, l, 0u);
                // NWA: (diagonal D, up D) quads of slots kP+62 .. kP+62+P
                o = NWA ? (uint32_t)min((k * P + 62) * 4 + min(lane, 4 * P + 3), last * 4 + 3) * 4u
                        : (uint32_t)min((k * P + 62) * 2 + min(lane, 2 * P - 1), last * 2 + 1) * 4u;
                l = in_lds + FBE * 4;
                lds_dma_dword_sys<0>(reinterpret_cast<const float*>(fEx + fi), o, l, 0u);
            }
        };

        {
            const size_t o0 = (size_t)(nsteps - 1 + APAD) * 64, o1 = o0 - 64;
            AM[P] = lane_load(astripe + o0, ul4);
            AM[P + 1] = lane_load(astripe + o1, ul4);
            AI[P] = lane_load(astripe + PL + o0, ul4);
            AI[P + 1] = lane_load(astripe + PL + o1, ul4);
            AD[P] = lane_load(astripe + 2 * PL + o0, ul4);
            AD[P + 1] = lane_load(astripe + 2 * PL + o1, ul4);
            XM[P] = lane_load(xstripe + o0, ul4);
            XM[P + 1] = lane_load(xstripe + o1, ul4);
            XI[P] = lane_load(xstripe + PL + o0, ul4);
            XI[P + 1] = lane_load(xstripe + PL + o1, ul4);
            XD[P] = lane_load(xstripe + 2 * PL + o0, ul4);
            XD[P + 1] = lane_load(xstripe + 2 * PL + o1, ul4);
            __asm__ volatile("" ::"v"(AM[P]), "v"(AM[P + 1]), "v"(AI[P]), "v"(AI[P + 1]),
                             "v"(AD[P]), "v"(AD[P + 1]), "v"(XM[P]), "v"(XM[P + 1]),
                             "v"(XI[P]), "v"(XI[P + 1]), "v"(XD[P]), "v"(XD[P + 1]));
        }
        wave_lds_sync();
        if (x_in) seen = wait_part(flag_in, epoch, min(lead(P), nch), st);
        issue_chunk(0);
        // pending successor flows (beta b*, channel g*): from (i, j+1) to M and D; from
        // (i+1, j) to M and I; from (i+1, j+1) to M, I, D (this step and the next)
        float lbM = 0, lgM = 0, lbD = 0, lgD = 0;
        float ubM = 0, ugM = 0, ubI = 0, ugI = 0;
        float lbI = 0, lgI = 0, ubD = 0, ugD = 0;          // NWA: left to I, up to D
        // NWA: the terminal cell's step on this lane
        const int term_step = (NWA && i0 + lane == L1 - 1) ? L2 - 1 + lane : -1000000;
        float dbM = 0, dgM = 0, dbI = 0, dgI = 0, dbD = 0, dgD = 0;
        float ebM = 0, egM = 0, ebI = 0, egI = 0, ebD = 0, egD = 0;

        for (int k = 0; k < nch; ++k) {
            const int t_hi = nsteps - 1 - k * P;
            chunk_waits<P>(prog, q, NL, k, nch, R, st);
            // this chunk's loads, followed by at least the P output stores of the
            // previous chunk (none when accumulating a dot product)
            if (k == 0 || DOT) wait_vmcnt<0>(); else wait_vmcnt<P>();
            if (x_in && k > 0) {
                // its progress word, loaded one chunk ago before those stores
                const int got = flag_chunks_lds(fslot, epoch);
                seen = got > seen ? got : seen;
            }
            float sv[P], vv[P];
#pragma unroll
            for (int u = 0; u < P; ++u) {
                sv[u] = buf[tbase + u];
                vv[u] = HAS_V ? buf[VT + tbase + u] : 0.0f;
            }
            AM[0] = AM[P]; AM[1] = AM[P + 1];
            AI[0] = AI[P]; AI[1] = AI[P + 1];
            AD[0] = AD[P]; AD[1] = AD[P + 1];
            XM[0] = XM[P]; XM[1] = XM[P + 1];
            XI[0] = XI[P]; XI[1] = XI[P + 1];
            XD[0] = XD[P]; XD[1] = XD[P + 1];
#pragma unroll
            for (int j = 0; j < P; ++j) {
                const int r = rows_row<P, -1>(j) * 64 + lane;
                AM[j + 2] = buf[AR + r];
                AI[j + 2] = buf[AR + P * 64 + r];
                AD[j + 2] = buf[AR + 2 * P * 64 + r];
                XM[j + 2] = buf[XR + r];
                XI[j + 2] = buf[XR + P * 64 + r];
                XD[j + 2] = buf[XR + 2 * P * 64 + r];
            }
            const bool row_ok = s > 0 && lane <= P && t_hi - lane + 63 <= nsteps - 1;
            float bAM = row_ok ? buf[RA + lane] : kNINF;
            float bAI = row_ok ? buf[RA + 64 + lane] : kNINF;
            float bAD = row_ok ? buf[RA + 128 + lane] : kNINF;
            float bXM = row_ok ? buf[RX + lane] : 0.0f;
            float bXI = row_ok ? buf[RX + 64 + lane] : 0.0f;
            float bXD = row_ok ? buf[RX + 128 + lane] : 0.0f;
            if (NWA && s == 0 && lane <= P) {
                // row 0 at column t_hi - lane (0-based; -1 is the start cell)
                const int c0 = t_hi - lane;
                bAM = c0 == -1 ? 0.0f : kNINF;
                bAD = c0 >= 0 ? go + (float)c0 * ge : kNINF;
                bXD = c0 >= 0 ? (MODE == OPEN ? 1.0f : (MODE == EXT ? (float)c0 : 0.0f)) : 0.0f;
            }
            // flows from the stripe below for lane 63: lane 63-j holds step j
            float4 qU = make_float4(0, 0, 0, 0), qD = make_float4(0, 0, 0, 0);
            float2 qE = make_float2(0, 0), qEu = make_float2(0, 0);
            if (below && lane >= 64 - P) {
                const int j = 63 - lane;
                if (x_in) {
                    qU = make_float4(buf[FBU + 4 * j], buf[FBU + 4 * j + 1], buf[FBU + 4 * j + 2],
                                     buf[FBU + 4 * j + 3]);
                    qD = make_float4(buf[FBD + 4 * j], buf[FBD + 4 * j + 1], buf[FBD + 4 * j + 2],
                                     buf[FBD + 4 * j + 3]);
                    if (NWA) {
                        qE = make_float2(buf[FBE + 4 * j], buf[FBE + 4 * j + 1]);
                        qEu = make_float2(buf[FBE + 4 * (j + 1) + 2], buf[FBE + 4 * (j + 1) + 3]);
                    } else {
                        qE = make_float2(buf[FBE + 2 * j], buf[FBE + 2 * j + 1]);
                    }
                } else {
                    const int iu = ring_index(k * P + j + 63, R);
                    qU = inU[iu];
                    const int id = ring_index(k * P + j + 62, R);
                    qD = inD[id];
                    if constexpr (NWA) {
                        const float4 e = inE[id], eu = inE[iu];
                        qE = make_float2(e.x, e.y);
                        qEu = make_float2(eu.z, eu.w);
                    } else {
                        qE = inE[id];
                    }
                }
            }
            wave_lds_sync();
            if (k + 1 < nch) {
                if (x_in) {
                    const int need = min(k + 1 + lead(P), nch);
                    if (seen < need) seen = wait_part(flag_in, epoch, need, st);
                }
                issue_chunk(k + 1);
                if (x_in) flag_load_lds(flag_in, fslot_lds, lane);
            }
            const int slot0 = ring_index(k * P, R);
            {
                const float a0 = lane_bcast(qU.x, 63), a1 = lane_bcast(qU.y, 63);
                const float a2 = lane_bcast(qU.z, 63), a3 = lane_bcast(qU.w, 63);
                const float d0 = lane_bcast(qD.x, 63), d1 = lane_bcast(qD.y, 63);
                const float d2 = lane_bcast(qD.z, 63), d3 = lane_bcast(qD.w, 63);
                const float d4 = lane_bcast(qE.x, 63), d5 = lane_bcast(qE.y, 63);
                const float n0 = lane_bcast(qD.x, 62), n1 = lane_bcast(qD.y, 62);
                const float n2 = lane_bcast(qD.z, 62), n3 = lane_bcast(qD.w, 62);
                const float n4 = lane_bcast(qE.x, 62), n5 = lane_bcast(qE.y, 62);
                if (NWA) {
                    const float a4 = lane_bcast(qEu.x, 63), a5 = lane_bcast(qEu.y, 63);
                    if (lane == 63) { ubD = a4; ugD = a5; }
                }
                if (lane == 63) {
                    ubM = a0; ugM = a1; ubI = a2; ugI = a3;
                    dbM = d0; dgM = d1; dbI = d2; dgI = d3; dbD = d4; dgD = d5;
                    ebM = n0; egM = n1; ebI = n2; egI = n3; ebD = n4; egD = n5;
                }
            }
            float qdb0 = wave_shr1(wave_shr1(qD.x));
            float qdg0 = wave_shr1(wave_shr1(qD.y));
            float qdb1 = wave_shr1(wave_shr1(qD.z));
            float qdg1 = wave_shr1(wave_shr1(qD.w));
            float qdb2 = wave_shr1(wave_shr1(qE.x));
            float qdg2 = wave_shr1(wave_shr1(qE.y));
            float qub0 = qU.x, qug0 = qU.y, qub1 = qU.z, qug1 = qU.w;
            float qub2 = qEu.x, qug2 = qEu.y;
            // NWA: one cell of the reverse sweep and the flows' shifts after it
            auto nwa_cell = [&](int u, int t, bool ok, float vd, float sc, float dgAM, float dgAI,
                                float dgAD, float dxM, float dxI, float dxD, float upM,
                                float upI, float upD, float uxM, float uxI, float uxD, float lfM,
                                float lfI, float lfD, float lxM, float lxI, float lxD) {
                (void)sc;
                const float ao = MODE == OPEN ? 1.0f : 0.0f, ae = MODE == EXT ? 1.0f : 0.0f;
                // M over the diagonal states; I over (M + open, I + ext, D + open) above;
                // D over (M + open, D + ext, I + open) to the left
                float w[3], dw[3], wi[3], dwi[3], wd[3], dwd[3];
                softmax3_tangent<MODE>({dgAM, dgAI, dgAD}, {dxM, dxI, dxD}, c, rT, w, dw);
                softmax3_tangent<MODE>({upM + go, upI + ge, upD + go}, {uxM + ao, uxI + ae, uxD + ao},
                                       c, rT, wi, dwi);
                softmax3_tangent<MODE>({lfM + go, lfD + ge, lfI + go}, {lxM + ao, lxD + ae, lxI + ao},
                                       c, rT, wd, dwd);
                // the terminal cell seeds both channels with its states' softmax weights,
                // normalised from the states themselves: exp((X - S) / T) with the
                // rounded value S sums to 1 only within ulp(S) / T, an error that the
                // tangents (of the alignment length's size) would carry into every entry
                float biM = 0.0f, biI = 0.0f, biD = 0.0f, giM = 0.0f, giI = 0.0f, giD = 0.0f;
                if (t == term_step) {
                    float wt[3], dwt[3];
                    softmax3_tangent<MODE>({AM[u], AI[u], AD[u]}, {XM[u], XI[u], XD[u]}, c, rT,
                                           wt, dwt);
                    biM = wt[0]; biI = wt[1]; biD = wt[2];
                    giM = dwt[0]; giI = dwt[1]; giD = dwt[2];
                }
                const float bM = ((biM + dbM) + lbM) + ubM;
                const float bI = ((biI + dbI) + ubI) + lbI;
                const float bD = ((biD + dbD) + lbD) + ubD;
                const float gM = ((giM + dgM) + lgM) + ugM;
                const float gI = ((giI + dgI) + ugI) + lgI;
                const float gD = ((giD + dgD) + lgD) + ugD;
                // a state passes flow only when beta > 1e-20 or |g| > 1e-20
                const bool pM_ = ok && (bM > 1e-20f || fabsf(gM) > 1e-20f);
                const bool pI_ = ok && (bI > 1e-20f || fabsf(gI) > 1e-20f);
                const bool pD_ = ok && (bD > 1e-20f || fabsf(gD) > 1e-20f);
                const float BM = pM_ ? bM : 0.0f, BI = pI_ ? bI : 0.0f, BD = pD_ ? bD : 0.0f;
                const float GM = pM_ ? gM : 0.0f, GI = pI_ ? gI : 0.0f, GD = pD_ ? gD : 0.0f;
                if (DOT) dacc += GM * vd;
                else otile[tbase + u] = GM;
                const float obM0 = BM * w[0], obI0 = BM * w[1], obD0 = BM * w[2];
                const float ogM0 = GM * w[0] + BM * dw[0], ogI0 = GM * w[1] + BM * dw[1];
                const float ogD0 = GM * w[2] + BM * dw[2];
                const float obMu = BI * wi[0], obIu = BI * wi[1], obDu = BI * wi[2];
                const float ogMu = GI * wi[0] + BI * dwi[0], ogIu = GI * wi[1] + BI * dwi[1];
                const float ogDu = GI * wi[2] + BI * dwi[2];
                const float obMl = BD * wd[0], obDl = BD * wd[1], obIl = BD * wd[2];
                const float ogMl = GD * wd[0] + BD * dwd[0], ogDl = GD * wd[1] + BD * dwd[1];
                const float ogIl = GD * wd[2] + BD * dwd[2];
                if (lane == 0) {
                    outU[slot0 + u] = make_float4(obMu, ogMu, obIu, ogIu);
                    outD[slot0 + u] = make_float4(obM0, ogM0, obI0, ogI0);
                    if constexpr (NWA) outE[slot0 + u] = make_float4(obD0, ogD0, obDu, ogDu);
                }
                qub0 = wave_shr1(qub0);
                qug0 = wave_shr1(qug0);
                qub1 = wave_shr1(qub1);
                qug1 = wave_shr1(qug1);
                qub2 = wave_shr1(qub2);
                qug2 = wave_shr1(qug2);
                lbM = obMl; lgM = ogMl; lbD = obDl; lgD = ogDl; lbI = obIl; lgI = ogIl;
                ubM = wave_shl1_or(obMu, qub0);
                ugM = wave_shl1_or(ogMu, qug0);
                ubI = wave_shl1_or(obIu, qub1);
                ugI = wave_shl1_or(ogIu, qug1);
                ubD = wave_shl1_or(obDu, qub2);
                ugD = wave_shl1_or(ogDu, qug2);
                dbM = ebM; dgM = egM; dbI = ebI; dgI = egI; dbD = ebD; dgD = egD;
                ebM = wave_shl1_or(obM0, qdb0);
                egM = wave_shl1_or(ogM0, qdg0);
                ebI = wave_shl1_or(obI0, qdb1);
                egI = wave_shl1_or(ogI0, qdg1);
                ebD = wave_shl1_or(obD0, qdb2);
                egD = wave_shl1_or(ogD0, qdg2);
                qdb0 = wave_shr1(qdb0);
                qdg0 = wave_shr1(qdg0);
                qdb1 = wave_shr1(qdb1);
                qdg1 = wave_shr1(qdg1);
                qdb2 = wave_shr1(qdb2);
                qdg2 = wave_shr1(qdg2);
            };
#pragma unroll
            for (int u = 0; u < P; ++u) {
                const int t = t_hi - u;
                const bool ok = (unsigned)(t - lane) < (unsigned)L2eff;
                const float sc = ok ? sv[u] : kNINF;
                const float vd = ok ? vv[u] : 0.0f;
                // primal and tangent predecessors
                const float nAM = wave_shl1(bAM), nAI = wave_shl1(bAI),
                            nAD = wave_shl1(bAD);
                const float nXM = wave_shl1(bXM), nXI = wave_shl1(bXI),
                            nXD = wave_shl1(bXD);
                const float upM = wave_shr1_or(AM[u + 1], bAM), upI = wave_shr1_or(AI[u + 1], bAI);
                const float uxM = wave_shr1_or(XM[u + 1], bXM), uxI = wave_shr1_or(XI[u + 1], bXI);
                const float upD = NWA ? wave_shr1_or(AD[u + 1], bAD) : kNINF;
                const float uxD = NWA ? wave_shr1_or(XD[u + 1], bXD) : 0.0f;
                const float dgAM = wave_shr1_or(AM[u + 2], nAM), dgAI = wave_shr1_or(AI[u + 2], nAI),
                            dgAD = wave_shr1_or(AD[u + 2], nAD);
                const float dxM = wave_shr1_or(XM[u + 2], nXM), dxI = wave_shr1_or(XI[u + 2], nXI),
                            dxD = wave_shr1_or(XD[u + 2], nXD);
                bAM = nAM; bAI = nAI; bAD = nAD;
                bXM = nXM; bXI = nXI; bXD = nXD;
                const float lfM = AM[u + 1], lfD = AD[u + 1], lxM = XM[u + 1], lxD = XD[u + 1];
                const float lfI = AI[u + 1], lxI = XI[u + 1];
                if constexpr (NWA) {
                    nwa_cell(u, t, ok, vd, sc, dgAM, dgAI, dgAD, dxM, dxI, dxD, upM, upI, upD,
                             uxM, uxI, uxD, lfM, lfI, lfD, lxM, lxI, lxD);
                    continue;
                }
                // M: weights over (M, I, D) diagonal + s, and s
                const float v0 = dgAM + sc, v1 = dgAI + sc, v2 = dgAD + sc;
                const float m4 = fmaxf(fmaxf(v0, v1), fmaxf(v2, sc));
                const float e0 = fast_exp2((v0 - m4) * c), e1 = fast_exp2((v1 - m4) * c);
                const float e2 = fast_exp2((v2 - m4) * c), e3 = fast_exp2((sc - m4) * c);
                const float r4 = fast_rcp(((e0 + e1) + e2) + e3);
                const float w0 = e0 * r4, w1 = e1 * r4, w2 = e2 * r4, w3 = e3 * r4;
                // I: open from M above, extend from I above
                const float i0v = upM + go, i1v = upI + ge;
                const float mi = fmaxf(i0v, i1v);
                const float f0 = fast_exp2((i0v - mi) * c), f1 = fast_exp2((i1v - mi) * c);
                const float ri = mi > kNINF ? fast_rcp(f0 + f1) : 0.0f;
                const float wi0 = f0 * ri, wi1 = f1 * ri;
                // D: open from M left, extend from D left
                const float d0v = lfM + go, d1v = lfD + ge;
                const float md = fmaxf(d0v, d1v);
                const float g0 = fast_exp2((d0v - md) * c), g1 = fast_exp2((d1v - md) * c);
                const float rd = md > kNINF ? fast_rcp(g0 + g1) : 0.0f;
                const float wd0 = g0 * rd, wd1 = g1 * rd;
                // candidate tangents
                const float ao = MODE == OPEN ? 1.0f : 0.0f, ae = MODE == EXT ? 1.0f : 0.0f;
                const float vt = MODE == HVP ? vd : 0.0f;
                const float dm0 = dxM + vt, dm1 = dxI + vt, dm2 = dxD + vt, dm3 = vt;
                const float di0 = uxM + ao, di1 = uxI + ae;
                const float dd0 = lxM + ao, dd1 = lxD + ae;
                float dw0, dw1, dw2, dw3, dwi0, dwi1, dwd0, dwd1;
                if (MODE == HVP) {
                    const float mM = ((w0 * dm0 + w1 * dm1) + w2 * dm2) + w3 * dm3;
                    const float mI = wi0 * di0 + wi1 * di1;
                    const float mD = wd0 * dd0 + wd1 * dd1;
                    dw0 = w0 * (dm0 - mM) * rT;
                    dw1 = w1 * (dm1 - mM) * rT;
                    dw2 = w2 * (dm2 - mM) * rT;
                    dw3 = w3 * (dm3 - mM) * rT;
                    dwi0 = wi0 * (di0 - mI) * rT;
                    dwi1 = wi1 * (di1 - mI) * rT;
                    dwd0 = wd0 * (dd0 - mD) * rT;
                    dwd1 = wd1 * (dd1 - mD) * rT;
                } else {
                    // The parameter Jacobians take E_w[d] - d_k (and E_w[v] - v_k)
                    // relative to the candidate of the largest value: the weights' sum
                    // differs from 1 by an ulp or two, which must not multiply tangents
                    // and values that grow with the alignment length.  With two
                    // candidates, E_w[d] - d_0 = w_1 (d_1 - d_0) exactly.
                    const float p = v0 >= m4 ? dm0 : (v1 >= m4 ? dm1 : (v2 >= m4 ? dm2 : dm3));
                    const float q0 = dm0 - p, q1 = dm1 - p, q2 = dm2 - p, q3 = dm3 - p;
                    const float mM = ((w0 * q0 + w1 * q1) + w2 * q2) + w3 * q3;
                    dw0 = w0 * (q0 - mM) * rT;
                    dw1 = w1 * (q1 - mM) * rT;
                    dw2 = w2 * (q2 - mM) * rT;
                    dw3 = w3 * (q3 - mM) * rT;
                    const float wwi = wi0 * wi1 * rT, wwd = wd0 * wd1 * rT;
                    dwi0 = wwi * (di0 - di1);
                    dwi1 = -dwi0;
                    dwd0 = wwd * (dd0 - dd1);
                    dwd1 = -dwd0;
                    if (MODE == TEMP) {
                        const float rT2 = rT * rT;
                        const float p0 = v0 - m4, p1 = v1 - m4, p2 = v2 - m4, p3 = sc - m4;
                        const float E4 = ((w0 * p0 + w1 * p1) + w2 * p2) + w3 * p3;
                        dw0 += w0 * (E4 - p0) * rT2;
                        dw1 += w1 * (E4 - p1) * rT2;
                        dw2 += w2 * (E4 - p2) * rT2;
                        dw3 += w3 * (E4 - p3) * rT2;
                        // w_0 (E - v_0) = w_0 w_1 (v_1 - v_0); 0 when either is impossible
                        const float ti = wi1 > 0.0f ? wi0 * wi1 * (i1v - i0v) * rT2 : 0.0f;
                        const float td = wd1 > 0.0f ? wd0 * wd1 * (d1v - d0v) * rT2 : 0.0f;
                        dwi0 += ti;
                        dwi1 -= ti;
                        dwd0 += td;
                        dwd1 -= td;
                    }
                }
                // initial values of the two channels
                float lp;
                lp = (AM[u] - S) * c;
                const float biM = fast_exp2(lp < 0.0f ? lp : 0.0f);
                lp = (AI[u] - S) * c;
                const float biI = fast_exp2(lp < 0.0f ? lp : 0.0f);
                lp = (AD[u] - S) * c;
                const float biD = fast_exp2(lp < 0.0f ? lp : 0.0f);
                const float giM = biM * (XM[u] - dSb) * rT;
                const float giI = biI * (XI[u] - dSb) * rT;
                const float giD = biD * (XD[u] - dSb) * rT;
                // channels in the reference's accumulation order (init first for the
                // HVP; last for the parameter Jacobians, then the temperature term of
                // reachable states)
                const float bM = ((biM + dbM) + lbM) + ubM;
                const float bI = (biI + dbI) + ubI;
                const float bD = (biD + dbD) + lbD;
                float gM, gI, gD;
                if (MODE == HVP) {
                    gM = ((giM + dgM) + lgM) + ugM;
                    gI = (giI + dgI) + ugI;
                    gD = (giD + dgD) + lgD;
                } else {
                    gM = ((dgM + lgM) + ugM) + giM;
                    gI = (dgI + ugI) + giI;
                    gD = (dgD + lgD) + giD;
                    if (MODE == TEMP) {
                        const float rT2 = rT * rT;
                        if (AM[u] > kNINF) gM -= biM * (AM[u] - S) * rT2;
                        if (AI[u] > kNINF) gI -= biI * (AI[u] - S) * rT2;
                        if (AD[u] > kNINF) gD -= biD * (AD[u] - S) * rT2;
                    }
                }
                const float BM = ok ? bM : 0.0f, BI = ok ? bI : 0.0f, BD = ok ? bD : 0.0f;
                const float GM = ok ? gM : 0.0f, GI = ok ? gI : 0.0f, GD = ok ? gD : 0.0f;
                const float o = MODE == HVP
                                    ? GM * (((w0 + w1) + w2) + w3) + BM * (((dw0 + dw1) + dw2) + dw3)
                                    : GM;
                if (DOT) dacc += o * vd;
                else otile[tbase + u] = o;
                // flows to the predecessors
                const float obM0 = BM * w0, obI0 = BM * w1, obD0 = BM * w2;
                const float ogM0 = GM * w0 + BM * dw0, ogI0 = GM * w1 + BM * dw1;
                const float ogD0 = GM * w2 + BM * dw2;
                const float obMu = BI * wi0, obIu = BI * wi1;
                const float ogMu = GI * wi0 + BI * dwi0, ogIu = GI * wi1 + BI * dwi1;
                const float obMl = BD * wd0, obDl = BD * wd1;
                const float ogMl = GD * wd0 + BD * dwd0, ogDl = GD * wd1 + BD * dwd1;
                if (lane == 0) {
                    outU[slot0 + u] = make_float4(obMu, ogMu, obIu, ogIu);
                    outD[slot0 + u] = make_float4(obM0, ogM0, obI0, ogI0);
                    if constexpr (!NWA) outE[slot0 + u] = make_float2(obD0, ogD0);
                }
                // successor flows for the next steps; lane 63 takes the rings
                qub0 = wave_shr1(qub0);
                qug0 = wave_shr1(qug0);
                qub1 = wave_shr1(qub1);
                qug1 = wave_shr1(qug1);
                lbM = obMl; lgM = ogMl; lbD = obDl; lgD = ogDl;
                ubM = wave_shl1_or(obMu, qub0);
                ugM = wave_shl1_or(ogMu, qug0);
                ubI = wave_shl1_or(obIu, qub1);
                ugI = wave_shl1_or(ogIu, qug1);
                dbM = ebM; dgM = egM; dbI = ebI; dgI = egI; dbD = ebD; dgD = egD;
                ebM = wave_shl1_or(obM0, qdb0);
                egM = wave_shl1_or(ogM0, qdg0);
                ebI = wave_shl1_or(obI0, qdb1);
                egI = wave_shl1_or(ogI0, qdg1);
                ebD = wave_shl1_or(obD0, qdb2);
                egD = wave_shl1_or(ogD0, qdg2);
                qdb0 = wave_shr1(qdb0);
                qdg0 = wave_shr1(qdg0);
                qdb1 = wave_shr1(qdb1);
                qdg1 = wave_shr1(qdg1);
                qdb2 = wave_shr1(qdb2);
                qdg2 = wave_shr1(qdg2);
            }
            wave_lds_sync();
            if (!DOT) write_tile<P, -1>(otile, obase, trash, i0, L1, L2, L1max, L2max, lane, t_hi);
            publish(prog, wave, q * PROG_STRIDE + k + 1);
            if (x_out) {
                // this chunk's flows to the part above, by producer step
                if (lane < P) {
                    const int sl = slot0 + lane;
                    store_sys4(fU + fo + k * P + lane, outU[sl]);
                    store_sys4(fD + fo + k * P + lane, outD[sl]);
                    if constexpr (NWA) store_sys4(fEx + fo + k * P + lane, outE[sl]);
                    else store_sys2(fE + fo + k * P + lane, outE[sl]);
                }
                if (k >= 2) {
                    // at least P + 3P/2 + 6 loads, 6 flow stores and (DOT: none, else 2P)
                    // output stores follow the flow stores of chunk k - 2: complete
                    wait_vmcnt<(DOT ? P + 3 * P / 2 + 12 : 3 * P + 3 * P / 2 + 12)>();
                    if (lane == 0) store_flag(flag_out, progress_word(epoch, k - 1));
                }
            }
        }
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
constexpr int PT = 8;   // tangent sweep chunk
constexpr int PD = 4;   // reverse sweep chunk

// LDS of one workgroup whose stripe boundaries use rings of R columns
size_t lds_tangent_r(bool has_v, int R) {
    const int buf = 65 * PT * (has_v ? 2 : 1) + 3 * PT * 64 + 3 * 64 + 3 * 64;
    return (size_t)NW * buf * sizeof(float) + ((size_t)NW * R + NW * (64 + PT)) * sizeof(float4);
}
size_t lds_tangent(bool has_v, int L1, int L2) { return lds_tangent_r(has_v, ring_len(L1, L2, 256)); }

size_t lds_dual_r(bool has_v, bool dot, int R, bool nwa) {
    const int buf = 65 * PD * (has_v ? 2 : 1) + 6 * PD * 64 + 6 * 64 + (dot ? 0 : 65 * PD) + 3 * 64;
    return (size_t)NW * buf * sizeof(float) +
           (size_t)NW * R * (2 * sizeof(float4) + (nwa ? sizeof(float4) : sizeof(float2)));
}
size_t lds_dual(bool has_v, bool dot, int L1, int L2, bool nwa) {
    return lds_dual_r(has_v, dot, ring_len(L1, L2, 128), nwa);
}

// Workspace after the primal layout: tangent tables + last rows, [B] scalars, then for
// split elements the parts' partial sums and the reverse sweep's boundary flows by
// step (up and diagonal (beta, g) pairs to M and I, float4 each; diagonal pair to D,
// and for global alignment the up pair to D beside it: a float4 slot).
struct Second {
    Layout prim;
    float* tan_sk;
    float* tan_brow;
    float* sdot;
    float* part;
    float* dS[3];   // dS/dopen, dS/dext, dS/dT
    float* spart;   // [B][stripe]
    float4* fU;     // [B][stripe][step]
    float4* fD;
    float2* fE;
    size_t bytes;
};

Second second_layout(void* ws, int B, int L1, int L2) {
    Second w;
    w.prim = swa::affine_layout(ws, B, L1, L2, true);
    char* p = (char*)ws + round256(w.prim.bytes);
    const size_t ns = ((size_t)L1 + 63) / 64;
    w.tan_sk = (float*)p;
    w.tan_brow = w.tan_sk + (size_t)B * ns * 3 * stored_steps(L2) * 64;
    p += round256(table_floats(B, L1, L2, 3) * sizeof(float));
    w.sdot = (float*)p;
    w.part = w.sdot + B;
    w.dS[0] = w.part + B;
    w.dS[1] = w.dS[0] + B;
    w.dS[2] = w.dS[1] + B;
    p += round256((size_t)5 * B * sizeof(float));
    const size_t parts = (size_t)B * (ns > 0 ? ns : 1);
    const size_t slots = parts * (size_t)stored_steps(L2);
    w.spart = (float*)p;
    p += round256(parts * sizeof(float));
    w.fU = (float4*)p;
    p += round256(slots * sizeof(float4));
    w.fD = (float4*)p;
    p += round256(slots * sizeof(float4));
    w.fE = (float2*)p;
    p += round256(slots * sizeof(float4));
    w.bytes = (size_t)(p - (char*)ws);
    return w;
}

template <int MODE, bool NWA = false>
int launch_tangent(const float* scores, const float* V, const int* lengths, int B, int L1, int L2,
                   float go, float ge, float T, const Second& w, float* sdot, hipStream_t st) {
    const int ns = (L1 + 63) / 64;
    constexpr bool has_v = MODE == HVP;
    // rings of an unsplit element that do not fit: parts of at most NW stripes
    const Split sp = choose_split(B, L1, w.prim, lds_tangent(has_v, L1, L2) <= kLdsLimit ? 0 : NW);
    const int R = ring_len(sp.G > 1 ? sp.SPW * 64 : L1, L2, 256);
    const size_t lds = lds_tangent_r(has_v, R);
    D2P_REQUIRE(lds <= kLdsLimit, "sequence too long for the LDS stripe rings");
    auto kern = swa_tangent_kernel<MODE, PT, NWA>;
    if (sp.G > 1) D2P_TRY(launch_flag_reset(w.prim.fflag, B * sp.G, st));
    D2P_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds));
    D2P_LAUNCH(NWA ? "nwa_tangent" : "swa_tangent", kern, dim3(split_grid(B, sp.G)), dim3(NW * 64), lds, st, scores, V,
               lengths, w.prim.alpha_sk, w.prim.brow, w.part, w.tan_sk, w.tan_brow, sdot,
               w.prim.status, w.prim.fflag, w.spart, B, L1, L2, ns, go, ge, T, R, sp.G, sp.SPW,
               next_epoch());
    if (MODE == HVP && !NWA && sp.G > 1 && launch_sum_parts(w.spart, sdot, B, sp.G, st) != D2P_OK)
        return D2P_ERR_HIP;
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

// dS: the value's tangent (or dS/dtheta) per element, seeding every cell; global
// alignment seeds the terminal cell from the tables instead and ignores it.
template <int MODE, bool DOT, bool NWA = false>
int launch_dual(const float* scores, const float* V, const int* lengths, int B, int L1, int L2,
                float go, float ge, float T, const Second& w, const float* dS, float* out,
                float* dot, hipStream_t st) {
    const int ns = (L1 + 63) / 64;
    constexpr bool has_v = MODE == HVP || DOT;
    const Split sp =
        choose_split(B, L1, w.prim, lds_dual(has_v, DOT, L1, L2, NWA) <= kLdsLimit ? 0 : NW);
    const int R = ring_len(sp.G > 1 ? sp.SPW * 64 : L1, L2, 128);
    const size_t lds = lds_dual_r(has_v, DOT, R, NWA);
    D2P_REQUIRE(lds <= kLdsLimit, "sequence too long for the LDS stripe rings");
    auto kern = swa_dual_kernel<MODE, PD, DOT, NWA>;
    if (sp.G > 1) D2P_TRY(launch_flag_reset(w.prim.bflag, B * sp.G, st));
    D2P_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds));
    D2P_LAUNCH(NWA ? "nwa_dual" : "swa_dual", kern, dim3(split_grid(B, sp.G)), dim3(NW * 64), lds, st, scores, V,
               lengths, w.prim.alpha_sk, w.prim.brow, w.tan_sk, w.tan_brow, w.part, dS, out, dot,
               w.prim.status, w.prim.trash, w.prim.bflag, w.fU, w.fD, w.fE, w.spart, B, L1, L2,
               ns, go, ge, T, R, sp.G, sp.SPW, next_epoch());
    if (DOT && sp.G > 1 && launch_sum_parts(w.spart, dot, B, sp.G, st) != D2P_OK)
        return D2P_ERR_HIP;
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

template <int MODE, bool DOT, bool NWA = false>
int param_pass(const float* scores, const float* ga, const int* lengths, int B, int L1, int L2,
               float go, float ge, float T, const Second& w, float* out, float* dot,
               hipStream_t st) {
    const int rc = launch_tangent<MODE, NWA>(scores, nullptr, lengths, B, L1, L2, go, ge, T, w,
                                             nullptr, st);
    if (rc != D2P_OK) return rc;
    return launch_dual<MODE, DOT, NWA>(scores, ga, lengths, B, L1, L2, go, ge, T, w,
                                       w.dS[MODE - 1], out, dot, st);
}

// rings that do not fit for an unsplit element force parts of at most NW stripes
int check(int B, int L1, int L2, float T) { return swa::check_shape(B, L1, L2, T); }

}  // namespace swa2
}  // namespace d2p_amd

using namespace d2p_amd;

extern "C" size_t d2p_swa_second_workspace_bytes(int B, int max_L1, int max_L2) {
    if (B <= 0 || max_L1 < 0 || max_L2 < 0) return 0;
    return swa2::second_layout(nullptr, B, max_L1, max_L2).bytes;
}

extern "C" int d2p_swa_hvp(const float* scores, const float* tangent, const int* lengths, int B,
                           int max_L1, int max_L2, float gap_open, float gap_ext,
                           float temperature, float* hvp, void* workspace,
                           size_t workspace_bytes, void* stream) {
    D2P_TRY(swa2::check(B, max_L1, max_L2, temperature));
    if (B == 0) return D2P_OK;
    D2P_REQUIRE(scores && tangent && hvp, "null pointer argument");
    D2P_REQUIRE(workspace && workspace_bytes >= d2p_swa_second_workspace_bytes(B, max_L1, max_L2),
                "workspace too small");
    hipStream_t st = (hipStream_t)stream;
    const swa2::Second w = swa2::second_layout(workspace, B, max_L1, max_L2);
    D2P_TRY(swa::launch_forward(scores, lengths, B, max_L1, max_L2, gap_open, gap_ext,
                                temperature, w.prim, w.part, st));
    D2P_TRY(swa2::launch_tangent<swa2::HVP>(scores, tangent, lengths, B, max_L1, max_L2, gap_open,
                                            gap_ext, temperature, w, w.sdot, st));
    D2P_TRY(swa2::launch_dual<swa2::HVP, false>(scores, tangent, lengths, B, max_L1, max_L2,
                                                gap_open, gap_ext, temperature, w, w.sdot, hvp,
                                                nullptr, st));
    return wf::launch_poison(w.prim.status, B, (long long)max_L1 * max_L2, hvp, nullptr, nullptr,
                             nullptr, nullptr, nullptr, st);
}

extern "C" int d2p_swa_param_jacobian(const float* scores, int param_type, const int* lengths,
                                      int B, int max_L1, int max_L2, float gap_open,
                                      float gap_ext, float temperature, float* jacobian,
                                      void* workspace, size_t workspace_bytes, void* stream) {
    D2P_TRY(swa2::check(B, max_L1, max_L2, temperature));
    D2P_REQUIRE(param_type >= 0 && param_type <= 2, "param_type must be 0, 1 or 2");
    if (B == 0) return D2P_OK;
    D2P_REQUIRE(scores && jacobian, "null pointer argument");
    D2P_REQUIRE(workspace && workspace_bytes >= d2p_swa_second_workspace_bytes(B, max_L1, max_L2),
                "workspace too small");
    hipStream_t st = (hipStream_t)stream;
    const swa2::Second w = swa2::second_layout(workspace, B, max_L1, max_L2);
    D2P_TRY(swa::launch_forward(scores, lengths, B, max_L1, max_L2, gap_open, gap_ext,
                                temperature, w.prim, w.part, st));
    // dS/dtheta from the marginal backward (marginals into the output, overwritten below)
    D2P_TRY(swa::launch_backward(scores, lengths, B, max_L1, max_L2, gap_open, gap_ext,
                                 temperature, w.prim, w.part, jacobian, w.dS[0], w.dS[1], w.dS[2],
                                 st));
    switch (param_type) {
        case 0:
            D2P_TRY(swa2::param_pass<swa2::OPEN, false>(scores, nullptr, lengths, B, max_L1,
                                                        max_L2, gap_open, gap_ext, temperature, w,
                                                        jacobian, nullptr, st));
            break;
        case 1:
            D2P_TRY(swa2::param_pass<swa2::EXT, false>(scores, nullptr, lengths, B, max_L1, max_L2,
                                                       gap_open, gap_ext, temperature, w, jacobian,
                                                       nullptr, st));
            break;
        default:
            D2P_TRY(swa2::param_pass<swa2::TEMP, false>(scores, nullptr, lengths, B, max_L1,
                                                        max_L2, gap_open, gap_ext, temperature, w,
                                                        jacobian, nullptr, st));
    }
    return wf::launch_poison(w.prim.status, B, (long long)max_L1 * max_L2, jacobian, nullptr,
                             nullptr, nullptr, nullptr, nullptr, st);
}

extern "C" int d2p_swa_backward_full(const float* scores, const float* grad_alignment,
                                     const int* lengths, int B, int max_L1, int max_L2,
                                     float gap_open, float gap_ext, float temperature,
                                     float* grad_scores, float* grad_open, float* grad_ext,
                                     float* grad_T, void* workspace, size_t workspace_bytes,
                                     void* stream) {
    D2P_TRY(swa2::check(B, max_L1, max_L2, temperature));
    if (B == 0) return D2P_OK;
    D2P_REQUIRE(scores && grad_alignment && grad_scores && grad_open && grad_ext &&
                    grad_T,
                "null pointer argument");
    D2P_REQUIRE(workspace && workspace_bytes >= d2p_swa_second_workspace_bytes(B, max_L1, max_L2),
                "workspace too small");
    hipStream_t st = (hipStream_t)stream;
    const swa2::Second w = swa2::second_layout(workspace, B, max_L1, max_L2);
    const float* ga = grad_alignment;
    D2P_TRY(swa::launch_forward(scores, lengths, B, max_L1, max_L2, gap_open, gap_ext,
                                temperature, w.prim, w.part, st));
    D2P_TRY(swa::launch_backward(scores, lengths, B, max_L1, max_L2, gap_open, gap_ext,
                                 temperature, w.prim, w.part, grad_scores, w.dS[0], w.dS[1],
                                 w.dS[2], st));
    D2P_TRY(swa2::launch_tangent<swa2::HVP>(scores, ga, lengths, B, max_L1, max_L2, gap_open,
                                            gap_ext, temperature, w, w.sdot, st));
    D2P_TRY(swa2::launch_dual<swa2::HVP, false>(scores, ga, lengths, B, max_L1, max_L2, gap_open,
                                                gap_ext, temperature, w, w.sdot, grad_scores,
                                                nullptr, st));
    D2P_TRY(swa2::param_pass<swa2::OPEN, true>(scores, ga, lengths, B, max_L1, max_L2, gap_open,
                                               gap_ext, temperature, w, nullptr, grad_open, st));
    D2P_TRY(swa2::param_pass<swa2::EXT, true>(scores, ga, lengths, B, max_L1, max_L2, gap_open,
                                              gap_ext, temperature, w, nullptr, grad_ext, st));
    D2P_TRY(swa2::param_pass<swa2::TEMP, true>(scores, ga, lengths, B, max_L1, max_L2, gap_open,
                                               gap_ext, temperature, w, nullptr, grad_T, st));
    return wf::launch_poison(w.prim.status, B, (long long)max_L1 * max_L2, grad_scores, nullptr,
                             grad_open, grad_ext, grad_T, nullptr, st);
}

// ------------------------------------------------------------------ global alignment
// soft_nw_affine's second-order entry points (reference: src/nw_affine/torch_cuda.cpp):
// the NW mode of the same sweeps.  Neither the HVP nor the Jacobians need the marginal
// backward: the reverse sweep seeds the terminal cell from the tables.

extern "C" size_t d2p_nwa_second_workspace_bytes(int B, int max_L1, int max_L2) {
    return d2p_swa_second_workspace_bytes(B, max_L1, max_L2);
}

extern "C" int d2p_nwa_hvp(const float* scores, const float* tangent, const int* lengths, int B,
                           int max_L1, int max_L2, float gap_open, float gap_ext,
                           float temperature, float* hvp, void* workspace,
                           size_t workspace_bytes, void* stream) {
    D2P_TRY(swa2::check(B, max_L1, max_L2, temperature));
    if (B == 0) return D2P_OK;
    D2P_REQUIRE(scores && tangent && hvp, "null pointer argument");
    D2P_REQUIRE(workspace && workspace_bytes >= d2p_nwa_second_workspace_bytes(B, max_L1, max_L2),
                "workspace too small");
    hipStream_t st = (hipStream_t)stream;
    const swa2::Second w = swa2::second_layout(workspace, B, max_L1, max_L2);
    D2P_TRY(swa::launch_forward(scores, lengths, B, max_L1, max_L2, gap_open, gap_ext,
                                temperature, w.prim, w.part, st, true));
    D2P_TRY((swa2::launch_tangent<swa2::HVP, true>(scores, tangent, lengths, B, max_L1, max_L2,
                                                   gap_open, gap_ext, temperature, w, w.sdot,
                                                   st)));
    D2P_TRY((swa2::launch_dual<swa2::HVP, false, true>(scores, tangent, lengths, B, max_L1,
                                                       max_L2, gap_open, gap_ext, temperature, w,
                                                       w.sdot, hvp, nullptr, st)));
    return wf::launch_poison(w.prim.status, B, (long long)max_L1 * max_L2, hvp, nullptr, nullptr,
                             nullptr, nullptr, nullptr, st);
}

extern "C" int d2p_nwa_param_jacobian(const float* scores, int param_type, const int* lengths,
                                      int B, int max_L1, int max_L2, float gap_open,
                                      float gap_ext, float temperature, float* jacobian,
                                      void* workspace, size_t workspace_bytes, void* stream) {
    D2P_TRY(swa2::check(B, max_L1, max_L2, temperature));
    D2P_REQUIRE(param_type >= 0 && param_type <= 2, "param_type must be 0, 1 or 2");
    if (B == 0) return D2P_OK;
    D2P_REQUIRE(scores && jacobian, "null pointer argument");
    D2P_REQUIRE(workspace && workspace_bytes >= d2p_nwa_second_workspace_bytes(B, max_L1, max_L2),
                "workspace too small");
    hipStream_t st = (hipStream_t)stream;
    const swa2::Second w = swa2::second_layout(workspace, B, max_L1, max_L2);
    D2P_TRY(swa::launch_forward(scores, lengths, B, max_L1, max_L2, gap_open, gap_ext,
                                temperature, w.prim, w.part, st, true));
    switch (param_type) {
        case 0:
            D2P_TRY((swa2::param_pass<swa2::OPEN, false, true>(scores, nullptr, lengths, B, max_L1,
                                                               max_L2, gap_open, gap_ext,
                                                               temperature, w, jacobian, nullptr,
                                                               st)));
            break;
        case 1:
            D2P_TRY((swa2::param_pass<swa2::EXT, false, true>(scores, nullptr, lengths, B, max_L1,
                                                              max_L2, gap_open, gap_ext,
                                                              temperature, w, jacobian, nullptr,
                                                              st)));
            break;
        default:
            D2P_TRY((swa2::param_pass<swa2::TEMP, false, true>(scores, nullptr, lengths, B, max_L1,
                                                               max_L2, gap_open, gap_ext,
                                                               temperature, w, jacobian, nullptr,
                                                               st)));
    }
    return wf::launch_poison(w.prim.status, B, (long long)max_L1 * max_L2, jacobian, nullptr,
                             nullptr, nullptr, nullptr, nullptr, st);
}

extern "C" int d2p_nwa_backward_full(const float* scores, const float* grad_alignment,
                                     const int* lengths, int B, int max_L1, int max_L2,
                                     float gap_open, float gap_ext, float temperature,
                                     float* grad_scores, float* grad_open, float* grad_ext,
                                     float* grad_T, void* workspace, size_t workspace_bytes,
                                     void* stream) {
    D2P_TRY(swa2::check(B, max_L1, max_L2, temperature));
    if (B == 0) return D2P_OK;
    D2P_REQUIRE(scores && grad_alignment && grad_scores && grad_open && grad_ext && grad_T,
                "null pointer argument");
    D2P_REQUIRE(workspace && workspace_bytes >= d2p_nwa_second_workspace_bytes(B, max_L1, max_L2),
                "workspace too small");
    hipStream_t st = (hipStream_t)stream;
    const swa2::Second w = swa2::second_layout(workspace, B, max_L1, max_L2);
    const float* ga = grad_alignment;
    D2P_TRY(swa::launch_forward(scores, lengths, B, max_L1, max_L2, gap_open, gap_ext,
                                temperature, w.prim, w.part, st, true));
    D2P_TRY((swa2::launch_tangent<swa2::HVP, true>(scores, ga, lengths, B, max_L1, max_L2,
                                                   gap_open, gap_ext, temperature, w, w.sdot,
                                                   st)));
    D2P_TRY((swa2::launch_dual<swa2::HVP, false, true>(scores, ga, lengths, B, max_L1, max_L2,
                                                       gap_open, gap_ext, temperature, w, w.sdot,
                                                       grad_scores, nullptr, st)));
    D2P_TRY((swa2::param_pass<swa2::OPEN, true, true>(scores, ga, lengths, B, max_L1, max_L2,
                                                      gap_open, gap_ext, temperature, w, nullptr,
                                                      grad_open, st)));
    D2P_TRY((swa2::param_pass<swa2::EXT, true, true>(scores, ga, lengths, B, max_L1, max_L2,
                                                     gap_open, gap_ext, temperature, w, nullptr,
                                                     grad_ext, st)));
    D2P_TRY((swa2::param_pass<swa2::TEMP, true, true>(scores, ga, lengths, B, max_L1, max_L2,
                                                      gap_open, gap_ext, temperature, w, nullptr,
                                                      grad_T, st)));
    return wf::launch_poison(w.prim.status, B, (long long)max_L1 * max_L2, grad_scores, nullptr,
                             grad_open, grad_ext, grad_T, nullptr, st);
}
