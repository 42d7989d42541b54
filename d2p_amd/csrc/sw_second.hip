// sw_second.hip -- second-order quantities of linear-gap soft Smith-Waterman on
// gfx950: Hessian-vector products and Jacobians of the marginals with respect to
// gap and temperature.
//
// Reference behaviour restated (not translated):
//   HVP          /root/reference/src/sw/kernels_cpu.cpp:279-477
//   param grad   /root/reference/src/sw/kernels_cpu.cpp:491-710 (0 = gap, 1 = T)
// Both are a forward tangent sweep followed by a two-channel reverse sweep.  With
// w the softmax weights of a cell over its candidates v = (diag + s, up + gap,
// left + gap, s) and d the candidates' tangents:
//   tangent      x[i,j] = sum_k w_k d_k (+ (alpha - E_w[v]) / T for the temperature)
//                d = (x_diag + V, x_up, x_left, V)             HVP (V = direction)
//                d = (x_diag, x_up + 1, x_left + 1, 0)         d/dgap
//                d = (x_diag, x_up, x_left, 0)                 d/dT
//   reverse      beta as in the marginal backward; a second channel g with
//                g_pred += g w_k + beta dw_k,  dw_k = w_k (d_k - E_w[d]) / T
//                (+ w_k (E_w[v] - v_k) / T^2 for the temperature), started from
//                beta_init (x - dS) / T  (HVP: first; param: last, with
//                - beta_init (alpha - S) / T^2 for the temperature), and the output
//                of a cell is g (w_diag + w_sky) + beta (dw_diag + dw_sky).
// For the HVP dS = sum_cells beta_init x (computed by the tangent sweep); for a
// parameter it is dS/dtheta from the marginal backward.
//
// Mapping: the stripe pipeline of wavefront.hip.h.  The tangent sweep runs like the
// forward (its tangent crosses stripes through a float ring) and reads the primal
// alpha table like the backward; the reverse sweep is the backward with a second
// flow channel (float4 ring: beta and g towards the up and diagonal neighbours).
// Inputs arrive by direct-to-LDS loads one chunk ahead into one buffer per wave,
// copied to registers at the start of each chunk before the next chunk's loads.

#include <cstdlib>
#include <type_traits>
#include <vector>

#include "wavefront.hip.h"
#include "../../include/d2p_amd.h"
#include "capi_util.hip.h"
#include "sw_internal.hip.h"

namespace d2p_amd {
namespace sw2 {

using namespace wf;

enum Mode { HVP = 0, GAP = 1, TEMP = 2 };

// ------------------------------------------------------------------ tangent sweep

// HELP (parts of at most NW/2 stripes): wave NW/2 + l loads stripe l's inputs (score
// and direction quads, alpha rows, the row above) one chunk ahead, publishing
// hprog[l] = chunks loaded.  Chunk k's buffer is wave l's own for even k and the
// helper's for odd k, and the helper refills it with chunk k + 2 once wave l has
// finished chunk k (prog[l]).  Wave l keeps only the tangent row of the part above.
template <int MODE, int P, bool NWG = false, bool HELP = false>
__global__ void __launch_bounds__(NW * 64)
sw_tangent_kernel(const float* __restrict__ scores, const float* __restrict__ V,
                  const int* __restrict__ lengths, const float* __restrict__ alpha_sk,
                  const float* __restrict__ brow, const float* __restrict__ partition,
                  float* __restrict__ tan_sk, float* __restrict__ tan_brow,
                  float* __restrict__ sdot, int* __restrict__ status,
                  uint64_t* __restrict__ tflag, float* __restrict__ spart, int B, int L1max,
                  int L2max, int NSmax, float gap, float T, int R, int G, int SPW,
                  uint32_t epoch) {
    constexpr bool HAS_V = MODE == HVP;
    using Tile = QuadTile<P>;                                // 16-byte score/direction loads
    constexpr int VT = Tile::FLOATS;                         // direction tile
    constexpr int AR = VT + (HAS_V ? Tile::FLOATS : 0);      // P alpha rows
    constexpr int RR = AR + P * 64;                          // row above
    constexpr int TR = RR + 64;                              // tangent row of the part above
    constexpr int BUF = TR + 64;
    constexpr int SINK = 64 + P;
    extern __shared__ __align__(16) float smem[];
    __shared__ int prog[NW];
    __shared__ int hprog[NW];     // HELP: chunks of stripe l loaded by its helper
    __shared__ float red[NW];
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
    float* rings = smem + NW * BUF;                          // [NW][R] tangent of lane 63
    float* sink = rings + NW * R + wave * SINK;
    int* st = status + b;

    if (lane == 0) {
        prog[wave] = -1;
        hprog[wave] = -1;
    }
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
    const float* sbase = scores + (size_t)b * L1max * L2max;
    const float* vbase = HAS_V ? V + (size_t)b * L1max * L2max : nullptr;
    const uint32_t in_lds = lds_address(buf);
    float sacc = 0.0f;   // sum of beta_init * tangent (HVP)
    const int s_begin = part * SPW;
    const int NL = max(min(NS, s_begin + SPW) - s_begin, 0);   // stripes of this part
    const bool has_next = s_begin + NL < NS;
    const uint64_t* flag_in = tflag + (size_t)b * G + (part > 0 ? part - 1 : 0);
    uint64_t* flag_out = tflag + (size_t)b * G + part;
    // HELP: chunk k's input buffer (wave l's for even k, its helper's for odd k)
    auto kbuf = [&](int l, int k) { return smem + ((k & 1) ? l + NW / 2 : l) * BUF; };

    if constexpr (HELP) {
        if (NL > NW / 2) {   // never: the host picks HELP for parts of at most NW/2 stripes
            if (threadIdx.x == 0) atomicOr(st, 2);
            return;
        }
        const int l = wave - NW / 2;
        if (l >= 0 && l < NL) {
            const int s = s_begin + l;
            const int i0 = s * 64;
            const float* astripe = alpha_sk + ((size_t)b * NSmax + s) * NT * 64;
            const float* bup = brow + ((size_t)b * NSmax + (s > 0 ? s - 1 : 0)) * NT;
            auto load = [&](int k) {
                const int t0 = k * P;
                const uint32_t base = lds_address(kbuf(l, k));
                dma_quads<P, 1>(base, sbase, i0, L1max, L2max, lane, t0);
                if (HAS_V) dma_quads<P, 1>(base + VT * 4, vbase, i0, L1max, L2max, lane, t0);
                dma_rows<P, 1>(base + AR * 4, astripe, t0, ul4);
                uint32_t roff = (uint32_t)min(t0 + 62 + min(lane, P), nsteps - 1) * 4u;
                uint32_t rl = base + RR * 4;
                lds_dma_dword<0>(bup, roff, rl, 0u);
            };
            if (nch > 0) {
                load(0);
                wait_vmcnt<0>();
                publish(hprog, l, 1);
                if (nch > 1) load(1);
            }
            for (int k = 0; k < nch; ++k) {
                if (k + 1 < nch) {
                    // chunk k + 1's loads are the last issued
                    wait_vmcnt<0>();
                    publish(hprog, l, k + 2);
                }
                // once wave l has finished chunk k, its buffer takes chunk k + 2
                wait_for(prog, l, l * PROG_STRIDE + k + 1, st);
                if (k + 2 < nch) load(k + 2);
            }
        }
    }

    for (int l = wave; l < NL; l += NW) {
        const int s = s_begin + l;
        const int i0 = s * 64;
        const int L2eff = (i0 + lane < L1) ? L2 : 0;
        const float* astripe = alpha_sk + ((size_t)b * NSmax + s) * NT * 64;   // step -APAD
        const float* bup = brow + ((size_t)b * NSmax + (s > 0 ? s - 1 : 0)) * NT;
        float* tout = tan_sk + (((size_t)b * NSmax + s) * NT + APAD) * 64;
        float* tb_s = tan_brow + ((size_t)b * NSmax + s) * NT;
        const float* tb_up = tan_brow + ((size_t)b * NSmax + (s > 0 ? s - 1 : 0)) * NT;
        const float* ring_in = ring_from(rings, l, R);
        float* ring_out = ring_of(rings, l, R);
        const bool x_in = l == 0 && part > 0;        // tangent row above from part - 1
        const bool x_out = l == NL - 1 && has_next;  // tangent row feeds part + 1
        int seen = -1;       // chunks of the previous part known to be complete

        // Loads of chunk k (steps t0 .. t0+P-1): the score (and direction) tiles, the
        // P alpha rows, and for lane j <= P the last row of the stripe above at step
        // t0 + 62 + j (clamped; lanes past P repeat lane P).
        // (HELP: the helper issues all but the tangent row above, into buffer kbuf)
        auto issue_chunk = [&](int k) {
            const int t0 = k * P;
            const uint32_t base = HELP ? lds_address(kbuf(l, k)) : in_lds;
            if (!HELP) {
                dma_quads<P, 1>(base, sbase, i0, L1max, L2max, lane, t0);
                if (HAS_V) dma_quads<P, 1>(base + VT * 4, vbase, i0, L1max, L2max, lane, t0);
                dma_rows<P, 1>(base + AR * 4, astripe, t0, ul4);
                uint32_t roff = (uint32_t)min(t0 + 62 + min(lane, P), nsteps - 1) * 4u;
                uint32_t rl = base + RR * 4;
                lds_dma_dword<0>(bup, roff, rl, 0u);
            }
            if (x_in) {
                // lane j < P: the tangent of the last row above at step t0 + 63 + j
                uint32_t toff = (uint32_t)min(t0 + 63 + min(lane, P - 1), nsteps - 1) * 4u;
                uint32_t tl = base + TR * 4;
                lds_dma_dword_sys<0>(tb_up, toff, tl, 0u);
            }
        };

        // NWG: the cells left of column 0 hold the row's boundary alpha i*gap, whose
        // tangent is i for the gap Jacobian and 0 otherwise (SW: NINF and 0)
        const float aleft = NWG ? (float)(i0 + lane + 1) * gap : kNINF;
        const float xleft = (NWG && MODE == GAP) ? (float)(i0 + lane + 1) : 0.0f;
        const int term_step = (NWG && i0 + lane == L1 - 1) ? L2 - 1 + lane : -1000000;
        // tangents of the column-0 boundary
#pragma unroll
        for (int t = -APAD; t < 0; ++t) lane_store(tout + t * 64, ul4, xleft);
        wave_lds_sync();
        if (x_in) seen = wait_part(flag_in, epoch, min(lead(P), nch), st);
        issue_chunk(0);
        float Aw[P + 2];
        Aw[P] = aleft;        // alpha at steps -2, -1: column-0 boundary
        Aw[P + 1] = aleft;
        // tangents: previous step, its up value (NWG gap Jacobian: the boundary's)
        float cur = xleft, up_prev = (NWG && MODE == GAP) ? (float)(i0 + lane) : 0.0f;

        for (int k = 0; k < nch; ++k) {
            const int t0 = k * P;
            chunk_waits<P>(prog, l, NL, k, nch, R, st);
            // this chunk's loads, followed by at least the P + 1 stores of the previous
            // chunk (the first chunk's loads are the last issued)
            if (k == 0) wait_vmcnt<0>(); else wait_vmcnt<P>();
            if (HELP) wait_for(hprog, l, k + 1, st);   // the helper's loads of chunk k
            if (x_in && k > 0) {
                // its progress word, loaded one chunk ago before those stores
                const int got = flag_chunks_lds(fslot, epoch);
                seen = got > seen ? got : seen;
            }
            float* buf = HELP ? kbuf(l, k) : smem + wave * BUF;
            float sv[P], vv[P];
            read_quads<P, 1>(buf, lane, sv);
            if (HAS_V) {
                read_quads<P, 1>(buf + VT, lane, vv);
            } else {
#pragma unroll
                for (int u = 0; u < P; ++u) vv[u] = 0.0f;
            }
            Aw[0] = Aw[P];
            Aw[1] = Aw[P + 1];
#pragma unroll
            for (int j = 0; j < P; ++j) Aw[j + 2] = buf[AR + j * 64 + lane];
            // lane j: alpha of the last row above at step t0 + 62 + j (row 0: NINF, or
            // for NWG alpha[0, t0+j] = (t0+j)*gap)
            float bv = buf[RR + lane];
            bv = (s > 0 && lane <= P && t0 + 62 + lane <= nsteps - 1) ? bv : kNINF;
            if (NWG && s == 0) bv = lane <= P ? (float)(t0 + lane) * gap : kNINF;
            // lane 0's up tangents: column t0+j sits in lane j (row 0: 0, or for the
            // NWG gap Jacobian the boundary's t0+j+1 gaps)
            float rreg = 0.0f;
            if (s > 0 && lane < P)
                rreg = x_in ? buf[TR + lane] : ring_in[ring_index(t0 + lane + 63, R)];
            else if (NWG && MODE == GAP && s == 0 && lane < P)
                rreg = (float)(t0 + lane + 1);
            wave_lds_sync();   // every read of the input buffer is complete
            if (k + 1 < nch) {
                if (x_in) {
                    const int need = min(k + 1 + lead(P), nch);
                    if (seen < need) seen = wait_part(flag_in, epoch, need, st);
                }
                issue_chunk(k + 1);
                if (x_in) flag_load_lds(flag_in, fslot_lds, lane);
            }
            float* pub = (lane == 63) ? ring_out + ring_index(t0, R) : sink + lane;
            float* toutc = tout + (size_t)t0 * 64;
            // (HVP, SW) beta_init = 2^min((alpha - S) c, 0) is exactly 0 below 2^-150: a
            // chunk none of whose alphas comes within 150 c^-1 of S skips its share of the
            // value's tangent (most chunks: alpha grows along the anti-diagonals towards S)
            bool inits = true;
            if constexpr (MODE == HVP && !NWG) {
                float amax = Aw[2];
#pragma unroll
                for (int u = 1; u < P; ++u) amax = fmaxf(amax, Aw[u + 2]);
                inits = __builtin_amdgcn_ballot_w64((amax - S) * c >= -151.0f) != 0;
            }
            auto steps = [&](auto init) {
            constexpr bool INIT = decltype(init)::value;
#pragma unroll
            for (int u = 0; u < P; ++u) {
                const int t = t0 + u;
                const bool ok = (unsigned)(t - lane) < (unsigned)L2eff;
                const float sc = ok ? sv[u] : kNINF;
                const float vd = ok ? vv[u] : 0.0f;
                // primal predecessors: left = own previous step, up / diagonal = lane
                // r-1 one / two steps back (lane 0: the last row above)
                const float a0 = Aw[u + 2], a1 = Aw[u + 1];
                const float dga = wave_shr1_or(Aw[u], bv);
                const float bvn = wave_shl1(bv);
                const float upa = wave_shr1_or(a1, bvn);
                bv = bvn;
                // tangent predecessors
                const float tu = wave_shr1_or(cur, rreg);
                rreg = wave_shl1(rreg);
                const float td = up_prev;
                up_prev = tu;
                const float tl = cur;
                const float v0 = dga + sc, v1 = upa + gap, v2 = a1 + gap;
                // NWG: no restart candidate
                const float m = NWG ? fmaxf(fmaxf(v0, v1), v2) : fmaxf(fmaxf(v0, v1), fmaxf(v2, sc));
                const float e0 = fast_exp2((v0 - m) * c), e1 = fast_exp2((v1 - m) * c);
                const float e2 = fast_exp2((v2 - m) * c);
                const float e3 = NWG ? 0.0f : fast_exp2((sc - m) * c);
                const float rin = fast_rcp(((e0 + e1) + e2) + e3);
                float x;
                if (MODE == HVP) {
                    x = (((e0 * (td + vd) + e1 * tu) + e2 * tl) + e3 * vd) * rin;
                } else {
                    // The parameter tangents pass E_w[d] on as the candidate of the
                    // largest value plus the weighted differences: the weights' sum
                    // differs from 1 by an ulp or two, and taken whole that factor
                    // would compound along the alignment into tangents that grow with
                    // its length (the Jacobian subtracts dS/dtheta from them).
                    const float d1 = MODE == GAP ? tu + 1.0f : tu;
                    const float d2 = MODE == GAP ? tl + 1.0f : tl;
                    const float pd = v0 >= m ? td : (v1 >= m ? d1 : (v2 >= m ? d2 : 0.0f));
                    x = pd + (((e0 * (td - pd) + e1 * (d1 - pd)) + e2 * (d2 - pd)) - e3 * pd) * rin;
                    if (MODE == TEMP) {
                        // alpha - E_w[v], both relative to the largest value m
                        const float ev =
                            (((e0 * (v0 - m) + e1 * (v1 - m)) + e2 * (v2 - m)) + e3 * (sc - m)) *
                            rin;
                        x += ((a0 - m) - ev) * rT;
                    }
                }
                cur = ok ? x : ((NWG && t - lane < 0) ? xleft : 0.0f);
                lane_store(toutc + u * 64, ul4, cur);
                pub[u] = cur;
                if (MODE == HVP) {
                    if (NWG) {
                        // the value's tangent is the terminal cell's
                        if (t == term_step) sacc += cur;
                    } else if (INIT) {
                        float lp = (a0 - S) * c;
                        lp = lp < 0.0f ? lp : 0.0f;
                        sacc += fast_exp2(lp) * cur;
                    }
                }
            }
            };
            if (inits) steps(std::true_type{});
            else steps(std::false_type{});
            // the stripe's last row of tangents by step: one store instruction
            wave_lds_sync();
            if (lane < P) {
                const float v = ring_out[t0 % R + lane];
                if (x_out) store_sys(tb_s + t0 + lane, v);
                else lane_store(tb_s, (unsigned)(t0 + lane) * 4u, v);
            }
            publish(prog, wave, l * PROG_STRIDE + k + 1);
            if (x_out && k >= 2) {
                // at least P/4 + P/4 + 1 loads and 2P + 2 stores follow the row store
                // of chunk k - 2 (HELP: the 2P + 2 stores): it (and everything before)
                // is complete
                if constexpr (HELP) wait_vmcnt<2 * P + 2>();
                else wait_vmcnt<2 * P + Tile::NQ + P / 4 + 3>();
                if (lane == 0) store_flag(flag_out, progress_word(epoch, k - 1));
            }
        }
        if (x_out) {
            wait_vmcnt<0>();
            if (lane == 0) store_flag(flag_out, progress_word(epoch, nch));
        }
    }

    if (MODE == HVP) {
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

// DOT: instead of writing the per-cell output, accumulate its dot product with the
// matrix passed as V (the marginal cotangent) into dot[b].
// HELP (quad tiles, per-cell output, parts of at most NW/2 stripes): wave NW/2 + q
// moves stripe order q's data.  Chunk k's buffer is the k % 3-th of three: wave q's
// own, the helper's, and one of NW/2 more after the waves' buffers.  The helper loads
// a chunk's scores, direction, alpha and tangent rows and rows above into its buffer
// (publishing hprog[q] = chunks loaded), writes the chunk's output tile out once wave
// q has finished the chunk (prog[q]), and then loads chunk k + 3 into that buffer: its
// loads have two chunks of time.  Wave q loads only a part's flows from below.
template <int MODE, int P, bool DOT, bool NWG = false, bool HELP = false>
__global__ void __launch_bounds__(NW * 64)
sw_dual_kernel(const float* __restrict__ scores, const float* __restrict__ V,
               const int* __restrict__ lengths, const float* __restrict__ alpha_sk,
               const float* __restrict__ brow, const float* __restrict__ tan_sk,
               const float* __restrict__ tan_brow, const float* __restrict__ partition,
               const float* __restrict__ dS, float* __restrict__ out, float* __restrict__ dot,
               int* __restrict__ status, float* __restrict__ trash,
               uint64_t* __restrict__ dflag, float4* __restrict__ flows4,
               float* __restrict__ spart, int B, int L1max, int L2max, int NSmax, float gap,
               float T, int R, int G, int SPW, uint32_t epoch) {
    constexpr bool HAS_V = MODE == HVP || DOT;
    // QT (8- and 16-step chunks): score, direction and output tiles move as 16-byte
    // quads (P/4 instructions each); 4-step chunks keep dword tiles
    constexpr bool QT = P == 8 || P == 16;
    static_assert(!HELP || (QT && !DOT), "helper waves move quad tiles and write the output");
    using Tile = typename std::conditional<QT, QuadTile<(QT ? P : 8)>, ChunkTile<P>>::type;
    constexpr int NQ = P / 4;
    constexpr int NSTORE = DOT ? 0 : (QT ? NQ : P);         // output stores, inside chunk
    constexpr int VT = Tile::FLOATS;
    constexpr int AR = VT + (HAS_V ? Tile::FLOATS : 0);     // P alpha rows
    constexpr int XR = AR + P * 64;                         // P tangent rows
    constexpr int RA = XR + P * 64;                         // alpha row above
    constexpr int RX = RA + 64;                             // tangent row above
    constexpr int OT = RX + 64;                             // output tile
    constexpr int FB = OT + (DOT ? 0 : Tile::FLOATS);       // flows from the part below
    constexpr int BUF = FB + 64;
    static_assert(4 * P + 2 <= 64, "boundary flows fit their buffer");
    constexpr int SINK = 64 + P;
    extern __shared__ __align__(16) float smem[];
    __shared__ int prog[NW];
    __shared__ int hprog[NW];     // HELP: chunks of stripe order q loaded by its helper
    __shared__ float red[NW];
    // parts as in the primal backward: bottom-up, part p < G - 1 takes its last
    // stripe's flows from below from part p + 1 through flows4
    int b, dpart;
    split_decode(blockIdx.x, G, b, dpart);
    if (b >= B) return;
    const int part = G - 1 - dpart;
    const int lane = threadIdx.x & 63;
    const unsigned ul4 = (unsigned)lane * 4u;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    float* wbuf = smem + wave * BUF;   // this wave's chunk buffer
    __shared__ float fslot[64];   // progress word prefetched by wave 0, the only wave whose
                                  // stripe borders another part
    const uint32_t fslot_lds = lds_address(fslot);
    // (HELP: NW/2 more chunk buffers, then the rings)
    float4* rings = reinterpret_cast<float4*>(smem + (HELP ? NW + NW / 2 : NW) * BUF);  // [NW][R]
    float4* sink = rings + NW * R + wave * SINK;
    int* st = status + b;
    const int tbase = ChunkTile<P>::read_base(lane);   // dword tiles (4-step chunks)

    if (lane == 0) {
        prog[wave] = -1;
        hprog[wave] = -1;
    }
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
    const float* sbase = scores + (size_t)b * L1max * L2max;
    const float* vbase = HAS_V ? V + (size_t)b * L1max * L2max : nullptr;
    float* obase = DOT ? nullptr : out + (size_t)b * L1max * L2max;

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

    if constexpr (HELP) {
        if (NL > NW / 2) {   // never: the host picks HELP for parts of at most NW/2 stripes
            if (threadIdx.x == 0) atomicOr(st, 2);
            return;
        }
        const int q = wave - NW / 2;
        if (q >= 0 && q < NL) {
            const int s = s_begin + NL - 1 - q;
            const int i0 = s * 64;
            const size_t sb = ((size_t)b * NSmax + s) * NT;
            const float* astripe = alpha_sk + sb * 64;
            const float* xstripe = tan_sk + sb * 64;
            const size_t ub = ((size_t)b * NSmax + (s > 0 ? s - 1 : 0)) * NT;
            const float* bup = brow + ub;
            const float* xup = tan_brow + ub;
            // chunk k's buffer: wave q's own, this wave's, or the extra one
            auto cbuf = [&](int k) {
                const int r = k % 3;
                return smem + (r == 0 ? q : (r == 1 ? wave : NW + q)) * BUF;
            };
            // the loads of a chunk: at least NLD instructions (more in a chunk that
            // reaches past the element, whose quads load as dwords)
            constexpr int NLD = NQ * (HAS_V ? 2 : 1) + 2 * (P / 4) + 2;
            auto load = [&](int k) {
                const int th = nsteps - 1 - k * P;
                const uint32_t in = lds_address(cbuf(k));
                dma_quads<P, -1>(in, sbase, i0, L1max, L2max, lane, th);
                if (HAS_V) dma_quads<P, -1>(in + VT * 4, vbase, i0, L1max, L2max, lane, th);
                dma_rows<P, -1>(in + AR * 4, astripe, th - 2, ul4);
                dma_rows<P, -1>(in + XR * 4, xstripe, th - 2, ul4);
                // lane j <= P: the last rows above (alpha, tangent) at step th - j + 63
                const uint32_t roff = (uint32_t)min(th - min(lane, P) + 63, nsteps - 1) * 4u;
                uint32_t o = roff, l = in + RA * 4;
                lds_dma_dword<0>(bup, o, l, 0u);
                o = roff;
                l = in + RX * 4;
                lds_dma_dword<0>(xup, o, l, 0u);
            };
            // whole row segments of the output where rows start aligned (write_aligned)
            const bool aligned = (L2max & (P - 1)) == 0;
            AlignedCarry<P> carry;
            carry.clear();
            if (nch > 0) {
                load(0);
                wait_vmcnt<0>();
                publish(hprog, q, 1);
                if (nch > 1) load(1);
                if (nch > 2) load(2);
            }
            for (int k = 0; k < nch; ++k) {
                if (k + 1 < nch) {
                    // chunk k + 1's loads, followed by chunk k + 2's (if any) and, from
                    // k = 1 on, by chunk k - 1's NQ output stores
                    if (k == 0) {
                        if (nch > 2) wait_vmcnt<NLD>(); else wait_vmcnt<0>();
                    } else {
                        if (k + 2 < nch) wait_vmcnt<NQ + NLD>(); else wait_vmcnt<NQ>();
                    }
                    publish(hprog, q, k + 2);   // also completes this wave's LDS reads
                }
                // once wave q has finished chunk k, its output tile leaves and the
                // buffer takes chunk k + 3 (the stores have read the tile: their data
                // dependence waits for the reads)
                wait_for(prog, q, q * PROG_STRIDE + k + 1, st);
                if (aligned)
                    write_aligned<P, true>(cbuf(k) + OT, obase, trash, carry, i0, L1max, L2max,
                                           lane, nsteps - 1 - k * P);
                else
                    write_quads<P, -1>(cbuf(k) + OT, obase, trash, i0, L1, L2, L1max, L2max,
                                       lane, nsteps - 1 - k * P);
                if (k + 3 < nch) load(k + 3);
            }
        }
    }

    for (int q = wave; q < NL; q += NW) {
        const int s = s_begin + NL - 1 - q;
        const int i0 = s * 64;
        const int L2eff = (i0 + lane < L1) ? L2 : 0;
        // NWG: beta starts at 1 in the terminal cell only (and its tangent at 0)
        const int term_step = (NWG && i0 + lane == L1 - 1) ? L2 - 1 + lane : -1000000;
        const size_t sb = ((size_t)b * NSmax + s) * NT;
        const size_t ub = ((size_t)b * NSmax + (s > 0 ? s - 1 : 0)) * NT;
        const float* astripe = alpha_sk + sb * 64;
        const float* xstripe = tan_sk + sb * 64;
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

        // chunk k's buffer: this wave's own, or (HELP) the k % 3-th of its three
        auto kbuf = [&](int k) {
            if (!HELP) return wbuf;
            const int r = k % 3;
            return smem + (r == 0 ? wave : (r == 1 ? wave + NW / 2 : NW + wave)) * BUF;
        };
        // x_in: the flows of chunk k from the part below, producer slots kP+62 ..
        // kP+62+P (float4 each): float f of the range in lane f, clamped to the last
        // slot (HELP: two chunks ahead, into chunk k's buffer; else one chunk ahead)
        auto issue_flows = [&](int k) {
            uint32_t foff = (uint32_t)min((k * P + 62) * 4 + min(lane, 4 * P + 1),
                                          (nsteps - 1) * 4 + 3) * 4u;
            uint32_t fdst = lds_address(kbuf(k)) + FB * 4;
            lds_dma_dword_sys<0>(flows_in, foff, fdst, 0u);
        };
        auto issue_chunk = [&](int k) {
            const int th = nsteps - 1 - k * P;
            const uint32_t in = lds_address(kbuf(k));
            if constexpr (HELP) {
                // (the helper loads the tiles and rows)
            } else if constexpr (QT) {
                dma_quads<P, -1>(in, sbase, i0, L1max, L2max, lane, th);
                if (HAS_V) dma_quads<P, -1>(in + VT * 4, vbase, i0, L1max, L2max, lane, th);
            } else {
                dma_tile<P, -1>(in, sbase, i0, L1max, L2max, lane, th);
                if (HAS_V) dma_tile<P, -1>(in + VT * 4, vbase, i0, L1max, L2max, lane, th);
            }
            if constexpr (!HELP) {
                dma_rows<P, -1>(in + AR * 4, astripe, th - 2, ul4);
                dma_rows<P, -1>(in + XR * 4, xstripe, th - 2, ul4);
                const uint32_t roff = (uint32_t)min(th - min(lane, P) + 63, nsteps - 1) * 4u;
                uint32_t o = roff, l = in + RA * 4;
                lds_dma_dword<0>(bup, o, l, 0u);
                o = roff;
                l = in + RX * 4;
                lds_dma_dword<0>(xup, o, l, 0u);
            }
            if (!HELP && x_in) issue_flows(k);
        };

        {
            const float* a0p = astripe + (size_t)(nsteps - 1 + APAD) * 64;
            const float* x0p = xstripe + (size_t)(nsteps - 1 + APAD) * 64;
            A[P] = lane_load(a0p, ul4);
            A[P + 1] = lane_load(a0p - 64, ul4);
            X[P] = lane_load(x0p, ul4);
            X[P + 1] = lane_load(x0p - 64, ul4);
            __asm__ volatile("" ::"v"(A[P]), "v"(A[P + 1]), "v"(X[P]), "v"(X[P + 1]));
        }
        wave_lds_sync();
        if (x_in) seen = wait_part(flag_in, epoch, min(lead(P) + (HELP ? 1 : 0), nch), st);
        issue_chunk(0);
        if (HELP && x_in) {
            issue_flows(0);
            if (nch > 1) issue_flows(1);
        }
        // successor flows: (beta, g) from the left successor, up successor, diagonal
        float lb = 0.0f, lg = 0.0f, ubt = 0.0f, ug = 0.0f;
        float db = 0.0f, dg = 0.0f, db2 = 0.0f, dg2 = 0.0f;

        for (int k = 0; k < nch; ++k) {
            const int t_hi = nsteps - 1 - k * P;
            chunk_waits<P>(prog, q, NL, k, nch, R, st);
            // this chunk's loads, followed by at least the NSTORE output stores of the
            // previous chunk (none when accumulating a dot product; the first chunk's
            // loads are the last issued).  HELP: the helper loads the tiles and rows;
            // this wave's own loads (a part's flows from below) are followed by
            // nothing, or by the previous chunk's flow store (x_out); other stripes
            // wait for no memory operation of their own
            if constexpr (HELP) {
                // x_in: chunk k's flows (loaded two chunks ago) and the progress word
                // loaded one chunk ago, followed by chunk k + 1's flows (k + 1 < nch)
                // and the previous chunk's flow store (x_out)
                if (x_in) {
                    if (k == 0) wait_vmcnt<0>();
                    else if (x_out && k + 1 < nch) wait_vmcnt<2>();
                    else if (x_out || k + 1 < nch) wait_vmcnt<1>();
                    else wait_vmcnt<0>();
                }
                wait_for(hprog, q, k + 1, st);
            } else {
                if (k == 0 || DOT) wait_vmcnt<0>(); else wait_vmcnt<NSTORE>();
            }
            float* buf = kbuf(k);
            float* otile = buf + OT;
            if (x_in && k > 0) {
                // its progress word, loaded one chunk ago before those stores
                const int got = flag_chunks_lds(fslot, epoch);
                seen = got > seen ? got : seen;
            }
            float sv[P], vv[P];
            if constexpr (QT) {
                read_quads<P, -1>(buf, lane, sv);
                if (HAS_V) {
                    read_quads<P, -1>(buf + VT, lane, vv);
                } else {
#pragma unroll
                    for (int u = 0; u < P; ++u) vv[u] = 0.0f;
                }
            } else {
#pragma unroll
                for (int u = 0; u < P; ++u) {
                    sv[u] = buf[tbase + u];
                    vv[u] = HAS_V ? buf[VT + tbase + u] : 0.0f;
                }
            }
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
            float bA = row_ok ? buf[RA + lane] : kNINF;
            float bX = row_ok ? buf[RX + lane] : 0.0f;
            if (NWG && s == 0) {
                // row 0 above the first stripe: alpha (col+1)*gap at column t_hi - lane,
                // tangent col+1 for the gap Jacobian
                const int jc = t_hi - lane + 1;
                const bool in = lane <= P && jc >= 0;
                bA = in ? (float)jc * gap : kNINF;
                bX = (in && MODE == GAP) ? (float)jc : 0.0f;
            }
            // flows from the stripe below for lane 63 (see the marginal backward):
            // lane 63-j holds step j; up flows from slot kP+j+63, diagonal kP+j+62
            float qub = 0.0f, qug = 0.0f, qdb = 0.0f, qdg = 0.0f;
            if (below && lane >= 64 - P) {
                const int j = 63 - lane;
                if (x_in) {
                    qub = buf[FB + 4 * (j + 1)];
                    qug = buf[FB + 4 * (j + 1) + 1];
                    qdb = buf[FB + 4 * j + 2];
                    qdg = buf[FB + 4 * j + 3];
                } else {
                    const float4 ru = ring_in[ring_index(k * P + j + 63, R)];
                    const float4 rd = ring_in[ring_index(k * P + j + 62, R)];
                    qub = ru.x;
                    qug = ru.y;
                    qdb = rd.z;
                    qdg = rd.w;
                }
            }
            wave_lds_sync();   // every read of the input buffer is complete
            if (k + 1 < nch) {
                if constexpr (HELP) {
                    // the progress word, then (once the part below has published enough
                    // chunks) chunk k + 2's flows
                    if (x_in) {
                        flag_load_lds(flag_in, fslot_lds, lane);
                        if (k + 2 < nch) {
                            const int need = min(k + 2 + lead(P), nch);
                            if (seen < need) seen = wait_part(flag_in, epoch, need, st);
                            issue_flows(k + 2);
                        }
                    }
                } else {
                    if (x_in) {
                        const int need = min(k + 1 + lead(P), nch);
                        if (seen < need) seen = wait_part(flag_in, epoch, need, st);
                    }
                    issue_chunk(k + 1);
                    if (x_in) flag_load_lds(flag_in, fslot_lds, lane);
                }
            }
            float4* pub = (lane == 0) ? ring_out + ring_index(k * P, R) : sink + lane;
            {
                // lane 63 starts from step 0's flows (its own) and step 1's diagonal
                // flows (lane 62's, one DPP shift)
                const float d1b = wave_shr1(qdb), d1g = wave_shr1(qdg);
                if (lane == 63) {
                    ubt = qub; ug = qug;
                    db = qdb; dg = qdg;
                    db2 = d1b; dg2 = d1g;
                }
                qdb = wave_shr1(d1b);
                qdg = wave_shr1(d1g);
            }
            // QT: the output quad being filled, memory-column order (step 4q + 3 - e in
            // element e); one 16-byte LDS write per four steps
            float4 quad = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            // (SW) beta_init = 2^min((alpha - S) c, 0) is exactly 0 below 2^-150: a chunk
            // none of whose alphas comes within 150 c^-1 of S skips those exponentials
            // (most chunks: alpha grows along the anti-diagonals towards S)
            bool inits = true;
            if constexpr (!NWG) {
                float amax = A[0];
#pragma unroll
                for (int u = 1; u < P; ++u) amax = fmaxf(amax, A[u]);
                inits = __builtin_amdgcn_ballot_w64((amax - S) * c >= -151.0f) != 0;
            }
            // INIT: some cell of the chunk may have beta_init > 0 (else the initial terms
            // are left out: adding their exact zeros changes no bit); FULL: every cell
            // of the chunk lies inside the element (no validity masks; the raw max)
            auto steps = [&](auto init, auto full) {
            constexpr bool INIT = decltype(init)::value;
            constexpr bool FULL = decltype(full)::value;
#pragma unroll
            for (int u = 0; u < P; ++u) {
                const int t = t_hi - u;
                const bool ok = FULL || (unsigned)(t - lane) < (unsigned)L2eff;
                const float sc = FULL ? sv[u] : (ok ? sv[u] : kNINF);
                const float vd = FULL ? vv[u] : (ok ? vv[u] : 0.0f);
                // primal and tangent predecessors
                const float a0 = A[u], a1 = A[u + 1], x0 = X[u], x1 = X[u + 1];
                const float nA = wave_shl1(bA), nX = wave_shl1(bX);
                const float upa = wave_shr1_or(a1, bA), upx = wave_shr1_or(x1, bX);
                const float dga = wave_shr1_or(A[u + 2], nA), dgx = wave_shr1_or(X[u + 2], nX);
                bA = nA;
                bX = nX;
                const float v0 = dga + sc, v1 = upa + gap, v2 = a1 + gap;
                // NWG: no restart candidate.  (FULL HVP: the cell's own alpha, which the
                // forward formed from these operands as m + T ln(sum) >= m, takes the
                // max's place: every exponent is at most 0, the largest term at least
                // 1/4, and the shift cancels in the normalisation.  The parameter
                // Jacobians use m itself below.)
                const float m = NWG ? fmaxf(fmaxf(v0, v1), v2)
                                    : (FULL ? (MODE == HVP ? a0 : max4_raw(v0, v1, v2, sc))
                                            : fmaxf(fmaxf(v0, v1), fmaxf(v2, sc)));
                const float e0 = fast_exp2((v0 - m) * c), e1 = fast_exp2((v1 - m) * c);
                const float e2 = fast_exp2((v2 - m) * c);
                const float e3 = NWG ? 0.0f : fast_exp2((sc - m) * c);
                const float rin = fast_rcp(((e0 + e1) + e2) + e3);
                const float w0 = e0 * rin, w1 = e1 * rin, w2 = e2 * rin, w3 = e3 * rin;
                // candidate tangents and the weight tangents
                float d0, d1, d2, d3;
                if (MODE == HVP) {
                    d0 = dgx + vd; d1 = upx; d2 = x1; d3 = vd;
                } else if (MODE == GAP) {
                    d0 = dgx; d1 = upx + 1.0f; d2 = x1 + 1.0f; d3 = 0.0f;
                } else {
                    d0 = dgx; d1 = upx; d2 = x1; d3 = 0.0f;
                }
                float dw0, dw1, dw2, dw3;
                float mean_hvp = 0.0f;
                if (MODE == HVP) {
                    const float mean = ((w0 * d0 + w1 * d1) + w2 * d2) + w3 * d3;
                    mean_hvp = mean;
                    dw0 = w0 * (d0 - mean) * rT;
                    dw1 = w1 * (d1 - mean) * rT;
                    dw2 = w2 * (d2 - mean) * rT;
                    dw3 = w3 * (d3 - mean) * rT;
                } else {
                    // the parameter Jacobians take E_w[d] - d_k and E_w[v] - v_k relative
                    // to the candidate of the largest value: the weights' sum differs
                    // from 1 by an ulp or two, which must not multiply tangents and
                    // values that grow with the alignment length
                    const float p = v0 >= m ? d0 : (v1 >= m ? d1 : (v2 >= m ? d2 : d3));
                    const float q0 = d0 - p, q1 = d1 - p, q2 = d2 - p, q3 = d3 - p;
                    const float mean = ((w0 * q0 + w1 * q1) + w2 * q2) + w3 * q3;
                    dw0 = w0 * (q0 - mean) * rT;
                    dw1 = w1 * (q1 - mean) * rT;
                    dw2 = w2 * (q2 - mean) * rT;
                    dw3 = w3 * (q3 - mean) * rT;
                    if (MODE == TEMP) {
                        const float p0 = v0 - m, p1 = v1 - m, p2 = v2 - m;
                        const float p3 = NWG ? 0.0f : sc - m;
                        const float ev = ((w0 * p0 + w1 * p1) + w2 * p2) + w3 * p3;
                        const float rT2 = rT * rT;
                        dw0 += w0 * (ev - p0) * rT2;
                        dw1 += w1 * (ev - p1) * rT2;
                        dw2 += w2 * (ev - p2) * rT2;
                        dw3 += w3 * (ev - p3) * rT2;
                    }
                }
                // channels in the reference's accumulation order
                float binit;
                if (NWG) {
                    binit = t == term_step ? 1.0f : 0.0f;
                } else if (INIT) {
                    float lp = (a0 - S) * c;
                    lp = lp < 0.0f ? lp : 0.0f;
                    binit = fast_exp2(lp);
                } else {
                    binit = 0.0f;
                }
                const float beta = (NWG || INIT) ? ((binit + db) + lb) + ubt : (db + lb) + ubt;
                float g;
                bool live;
                if (NWG) {
                    // the terminal beta is constant: no initial tangent; the reference
                    // skips cells with beta == 0 and |g| < 1e-20
                    g = ((dg + lg) + ug);
                    live = ok && !(beta == 0.0f && fabsf(g) < 1e-20f);
                } else if (MODE == HVP) {
                    g = INIT ? ((binit * (x0 - dSb) * rT + dg) + lg) + ug : (dg + lg) + ug;
                    live = ok && beta <= 3.0e38f && beta != 0.0f;
                } else {
                    g = (dg + lg) + ug;
                    if (INIT) {
                        float init = binit * (x0 - dSb) * rT;
                        if (MODE == TEMP) init -= binit * (a0 - S) * rT * rT;
                        g = g + init;
                    }
                    live = ok && !(beta <= 1e-20f && fabsf(g) <= 1e-20f);
                }
                const float bl = live ? beta : 0.0f;
                const float gl = live ? g : 0.0f;
                // FULL HVP: gl w_k + bl dw_k = w_k (gl + bl (d_k - mean) / T), and the
                // output takes the candidates 0 and 3 (fewer instructions than the
                // weight tangents themselves; the same sums up to rounding)
                constexpr bool GROUPED = FULL && MODE == HVP && !NWG;
                float og0, og1, og2, o;
                if constexpr (GROUPED) {
                    const float bT = bl * rT;
                    const float t0 = fmaf(bT, d0 - mean_hvp, gl), t1 = fmaf(bT, d1 - mean_hvp, gl);
                    const float t2 = fmaf(bT, d2 - mean_hvp, gl), t3 = fmaf(bT, d3 - mean_hvp, gl);
                    og0 = w0 * t0;
                    og1 = w1 * t1;
                    og2 = w2 * t2;
                    o = fmaf(w3, t3, og0);
                } else {
                    o = gl * (w0 + w3) + bl * (dw0 + dw3);
                    og0 = gl * w0 + bl * dw0;
                    og1 = gl * w1 + bl * dw1;
                    og2 = gl * w2 + bl * dw2;
                }
                if (DOT) {
                    dacc += o * vd;
                } else if constexpr (QT) {
                    if ((u & 3) == 0) quad.w = o;
                    if ((u & 3) == 1) quad.z = o;
                    if ((u & 3) == 2) quad.y = o;
                    if ((u & 3) == 3) {
                        quad.x = o;
                        *reinterpret_cast<float4*>(otile + Tile::slot(lane, u >> 2)) = quad;
                    }
                } else {
                    otile[tbase + u] = o;
                }
                const float ob0 = bl * w0, ob1 = bl * w1, ob2 = bl * w2;
                pub[u] = make_float4(ob1, og1, ob0, og0);
                // successor flows for the next steps; lane 63 takes the ring
                qub = wave_shr1(qub);
                qug = wave_shr1(qug);
                lb = ob2;
                lg = og2;
                ubt = wave_shl1_or(ob1, qub);
                ug = wave_shl1_or(og1, qug);
                db = db2;
                dg = dg2;
                db2 = wave_shl1_or(ob0, qdb);
                dg2 = wave_shl1_or(og0, qdg);
                qdb = wave_shr1(qdb);
                qdg = wave_shr1(qdg);
            }
            };
            const bool full = i0 + 64 <= L1 && t_hi - (P - 1) >= 63 && t_hi <= L2 - 1;
            if (inits) {
                if (full) steps(std::true_type{}, std::true_type{});
                else steps(std::true_type{}, std::false_type{});
            } else {
                if (full) steps(std::false_type{}, std::true_type{});
                else steps(std::false_type{}, std::false_type{});
            }
            wave_lds_sync();
            if constexpr (HELP) {
                // (the helper writes the tile out once this chunk is published)
            } else if constexpr (!DOT) {
                if constexpr (QT)
                    write_quads<P, -1>(otile, obase, trash, i0, L1, L2, L1max, L2max, lane, t_hi);
                else
                    write_tile<P, -1>(otile, obase, trash, i0, L1, L2, L1max, L2max, lane, t_hi);
            }
            publish(prog, wave, q * PROG_STRIDE + k + 1);
            if (x_out) {
                // this chunk's flows to the part above, by producer step
                if (lane < P) store_sys4(flows_out + k * P + lane, ring_out[ring_index(k * P, R) + lane]);
                // HELP: the word reports the chunks up to k - XD, whose flow stores (and
                // everything before) are complete once at most XD memory operations are
                // outstanding (this wave's only other memory operations are its flag
                // stores and, when the part has one stripe, the flow loads of its x_in
                // side, all issued before this chunk's flow store).  XD = 1 reports the
                // chunks before this one: the part above learns of a chunk's flows one
                // chunk after their store (measured at C5 HVP: 3276-3280 us against
                // 3305-3310 with XD = 2 and 3346-3356 with XD = 4).
                // Plain form: at least (QT ? P/4 : P) + P/2 + 2 loads, 2 flow stores and
                // 2 NSTORE output stores follow the flow store of chunk k - 2.
                constexpr int XD = HELP ? 1 : 2;
                if (k >= XD) {
                    if constexpr (HELP) wait_vmcnt<XD>();
                    else wait_vmcnt<(QT ? NQ : P) + P / 2 + 4 + 2 * NSTORE>();
                    if (lane == 0) store_flag(flag_out, progress_word(epoch, k - XD + 1));
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
constexpr int PT = 16;   // tangent sweep chunk

// LDS of one workgroup whose stripe boundaries use rings of R columns
size_t lds_tangent_r(int mode, int R) {
    const int buf = 65 * PT * (mode == HVP ? 2 : 1) + PT * 64 + 64 + 64;
    return (size_t)NW * buf * sizeof(float) + ((size_t)NW * R + NW * (64 + PT)) * sizeof(float);
}
size_t lds_tangent(int mode, int max_L1, int max_L2) {
    return lds_tangent_r(mode, ring_len(max_L1, max_L2, 256));
}

// (help: the helper form's NW/2 extra chunk buffers)
size_t lds_dual_r(bool has_v, bool dot, int P, int R, bool help = false) {
    const int buf = 65 * P * (has_v ? 2 : 1) + 2 * P * 64 + 128 + (dot ? 0 : 65 * P) + 64;
    return (size_t)(help ? NW + NW / 2 : NW) * buf * sizeof(float) +
           ((size_t)NW * R + NW * (64 + P)) * sizeof(float4);
}

// Largest reverse-sweep chunk (8 or 4 steps) whose buffers and rings fit in LDS, for a
// workgroup that runs `rows` rows of stripes.
int dual_chunk(bool has_v, bool dot, int rows, int max_L2) {
    const int R = ring_len(rows, max_L2, 128);
    if (lds_dual_r(has_v, dot, 8, R) <= kLdsLimit) return 8;
    if (lds_dual_r(has_v, dot, 4, R) <= kLdsLimit) return 4;
    return 0;
}

// Workspace after the primal layout: tangent table + last rows, then [B] each of
// the tangent sweep's dS, the partition, dS/dgap and dS/dT, then for split elements
// the parts' partial sums and the reverse sweep's boundary flows (float4 by step).
struct Second {
    Layout prim;
    float* tan_sk;
    float* tan_brow;
    float* sdot;
    float* part;
    float* dgap;
    float* dT;
    float* spart;     // [B][stripe]
    float4* flows4;   // [B][stripe][step]
    size_t bytes;
};

Second second_layout(void* ws, int B, int L1, int L2) {
    Second w;
    w.prim = layout(ws, B, L1, L2, 1, true);
    char* p = (char*)ws + round256(w.prim.bytes);
    const size_t ns = ((size_t)L1 + 63) / 64;
    w.tan_sk = (float*)p;
    w.tan_brow = w.tan_sk + (size_t)B * ns * stored_steps(L2) * 64;
    p += round256(table_floats(B, L1, L2) * sizeof(float));
    w.sdot = (float*)p;
    w.part = w.sdot + B;
    w.dgap = w.part + B;
    w.dT = w.dgap + B;
    p += round256((size_t)4 * B * sizeof(float));
    const size_t parts = (size_t)B * (ns > 0 ? ns : 1);
    w.spart = (float*)p;
    p += round256(parts * sizeof(float));
    w.flows4 = (float4*)p;
    p += round256(parts * (size_t)stored_steps(L2) * sizeof(float4));
    w.bytes = (size_t)(p - (char*)ws);
    return w;
}

static bool helpers_enabled();

template <int MODE, bool NWG = false>
int launch_tangent(const float* scores, const float* V, const int* lengths, int B, int L1, int L2,
                   float gap, float T, const Second& w, float* sdot, hipStream_t st) {
    const int ns = (L1 + 63) / 64;
    // rings of an unsplit element that do not fit: parts of at most NW stripes
    const sw::Split sp =
        sw::choose_split(B, L1, w.prim, lds_tangent(MODE, L1, L2) <= kLdsLimit ? 0 : NW);
    const int R = ring_len(sp.G > 1 ? sp.SPW * 64 : L1, L2, 256);
    const size_t lds = lds_tangent_r(MODE, R);
    D2P_REQUIRE(lds <= kLdsLimit, "sequence too long for the LDS stripe rings");
    // helper waves for parts of at most NW/2 stripes (waves NW/2.. would idle)
    const int part_stripes = sp.G > 1 ? sp.SPW : ns;
    auto kern = part_stripes <= NW / 2 && helpers_enabled()
                    ? sw_tangent_kernel<MODE, PT, NWG, true>
                    : sw_tangent_kernel<MODE, PT, NWG, false>;
    if (sp.G > 1) D2P_TRY(launch_flag_reset(w.prim.fflag, B * sp.G, st));
    D2P_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds));
    D2P_LAUNCH(NWG ? "nw_tangent" : "sw_tangent", kern, dim3(split_grid(B, sp.G)), dim3(NW * 64), lds, st, scores, V,
               lengths, w.prim.alpha_sk, w.prim.brow, w.part, w.tan_sk, w.tan_brow, sdot,
               w.prim.status, w.prim.fflag, w.spart, B, L1, L2, ns, gap, T, R, sp.G, sp.SPW,
               next_epoch());
    if (MODE == HVP && sp.G > 1 && launch_sum_parts(w.spart, sdot, B, sp.G, st) != D2P_OK)
        return D2P_ERR_HIP;
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

// D2P_AMD_SW_HELPERS=0 turns the helper waves off (for tests: both forms must agree)
static bool helpers_enabled() {
    const char* e = std::getenv("D2P_AMD_SW_HELPERS");
    return !(e && e[0] == '0');
}

template <int MODE, bool DOT, bool NWG = false>
int launch_dual(const float* scores, const float* V, const int* lengths, int B, int L1, int L2,
                float gap, float T, const Second& w, const float* dS, float* out, float* dot,
                hipStream_t st) {
    const int ns = (L1 + 63) / 64;
    constexpr bool has_v = MODE == HVP || DOT;
    const sw::Split sp =
        sw::choose_split(B, L1, w.prim, dual_chunk(has_v, DOT, L1, L2) > 0 ? 0 : NW);
    const int rows = sp.G > 1 ? sp.SPW * 64 : L1;
    const int R = ring_len(rows, L2, 128);
    const int P = dual_chunk(has_v, DOT, rows, L2);
    D2P_REQUIRE(P > 0, "sequence too long for the LDS stripe rings");
    size_t lds = lds_dual_r(has_v, DOT, P, R);
    auto k8 = sw_dual_kernel<MODE, 8, DOT, NWG>;
    auto k4 = sw_dual_kernel<MODE, 4, DOT, NWG>;
    auto kern = P == 8 ? k8 : k4;
    // helper waves move the data when a part has at most NW/2 stripes (the others idle)
    if constexpr (!DOT) {
        if (P == 8 && (rows + 63) / 64 <= NW / 2 && helpers_enabled() &&
            lds_dual_r(has_v, DOT, P, R, true) <= kLdsLimit) {
            kern = sw_dual_kernel<MODE, 8, DOT, NWG, true>;
            lds = lds_dual_r(has_v, DOT, P, R, true);
        }
    }
    if (sp.G > 1) D2P_TRY(launch_flag_reset(w.prim.bflag, B * sp.G, st));
    D2P_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds));
    D2P_LAUNCH(NWG ? "nw_dual" : "sw_dual", kern, dim3(split_grid(B, sp.G)), dim3(NW * 64), lds, st, scores, V,
               lengths, w.prim.alpha_sk, w.prim.brow, w.tan_sk, w.tan_brow, w.part, dS, out, dot,
               w.prim.status, w.prim.trash, w.prim.bflag, w.flows4, w.spart, B, L1, L2, ns, gap,
               T, R, sp.G, sp.SPW, next_epoch());
    if (DOT && sp.G > 1 && launch_sum_parts(w.spart, dot, B, sp.G, st) != D2P_OK)
        return D2P_ERR_HIP;
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

// D2P_AMD_SW_FUSED_TANGENT=0: the forward and the HVP's tangent sweep as two launches
// (for tests: both forms must agree)
static bool fused_tangent() {
    const char* e = std::getenv("D2P_AMD_SW_FUSED_TANGENT");
    return !(e && e[0] == '0');
}

// The primal forward (alpha table, partition) and the HVP's forward tangent along V
// (tangent table, w.sdot = the value's tangent): one fused sweep, or two.
template <bool NWG>
int forward_and_tangent(const float* scores, const float* V, const int* lengths, int B, int L1,
                        int L2, float gap, float T, const Second& w, hipStream_t st) {
    if (fused_tangent())
        return sw::launch_forward_tangent(scores, V, lengths, B, L1, L2, gap, T, w.prim, w.part,
                                          w.tan_sk, w.tan_brow, w.sdot, w.spart, st, NWG);
    D2P_TRY(sw::launch_forward(scores, lengths, B, L1, L2, gap, T, w.prim, w.part, st, NWG));
    return launch_tangent<HVP, NWG>(scores, V, lengths, B, L1, L2, gap, T, w, w.sdot, st);
}

int check(int B, int L1, int L2, float T) {
    // rings that do not fit for an unsplit element force parts of at most NW stripes
    return sw::check_shape(B, L1, L2, T);
}

}  // namespace sw2
}  // namespace d2p_amd

using namespace d2p_amd;

extern "C" size_t d2p_sw_second_workspace_bytes(int B, int max_L1, int max_L2) {
    if (B <= 0 || max_L1 < 0 || max_L2 < 0) return 0;
    return sw2::second_layout(nullptr, B, max_L1, max_L2).bytes;
}

namespace {

// The linear-gap second-order paths; global selects soft Needleman-Wunsch, whose
// value is the terminal cell (its beta is the constant 1, so dS/dtheta never enters
// the reverse sweeps and no marginal backward is needed for it).
template <bool NWG>
int hvp_impl(const float* scores, const float* tangent, const int* lengths, int B, int max_L1,
             int max_L2, float gap, float temperature, float* hvp, void* workspace,
             size_t workspace_bytes, void* stream) {
    D2P_TRY(sw2::check(B, max_L1, max_L2, temperature));
    if (B == 0) return D2P_OK;
    D2P_REQUIRE(scores && tangent && hvp, "null pointer argument");
    const size_t need = d2p_sw_second_workspace_bytes(B, max_L1, max_L2);
    D2P_REQUIRE(workspace && workspace_bytes >= need, "workspace too small");
    hipStream_t st = (hipStream_t)stream;
    const sw2::Second w = sw2::second_layout(workspace, B, max_L1, max_L2);
    D2P_TRY(sw2::forward_and_tangent<NWG>(scores, tangent, lengths, B, max_L1, max_L2, gap,
                                          temperature, w, st));
    D2P_TRY(sw2::launch_dual<sw2::HVP, false, NWG>(scores, tangent, lengths, B, max_L1, max_L2,
                                                   gap, temperature, w, w.sdot, hvp, nullptr, st));
    return wf::launch_poison(w.prim.status, B, (long long)max_L1 * max_L2, hvp, nullptr, nullptr,
                             nullptr, nullptr, nullptr, st);
}

template <bool NWG>
int param_jacobian_impl(const float* scores, int param_type, const int* lengths, int B,
                        int max_L1, int max_L2, float gap, float temperature, float* jacobian,
                        void* workspace, size_t workspace_bytes, void* stream) {
    D2P_TRY(sw2::check(B, max_L1, max_L2, temperature));
    D2P_REQUIRE(param_type == 0 || param_type == 1, "param_type must be 0 or 1");
    if (B == 0) return D2P_OK;
    D2P_REQUIRE(scores && jacobian, "null pointer argument");
    const size_t need = d2p_sw_second_workspace_bytes(B, max_L1, max_L2);
    D2P_REQUIRE(workspace && workspace_bytes >= need, "workspace too small");
    hipStream_t st = (hipStream_t)stream;
    const sw2::Second w = sw2::second_layout(workspace, B, max_L1, max_L2);
    D2P_TRY(sw::launch_forward(scores, lengths, B, max_L1, max_L2, gap, temperature, w.prim,
                               w.part, st, NWG));
    // SW: dS/dtheta from the marginal backward; its marginals go to the output, which
    // the reverse sweep below overwrites completely
    if (!NWG)
        D2P_TRY(sw::launch_backward(scores, lengths, B, max_L1, max_L2, gap, temperature,
                                    w.prim, w.part, jacobian, w.dgap, w.dT, st, true));
    if (param_type == 0) {
        D2P_TRY(sw2::launch_tangent<sw2::GAP, NWG>(scores, nullptr, lengths, B, max_L1, max_L2,
                                                   gap, temperature, w, nullptr, st));
        D2P_TRY(sw2::launch_dual<sw2::GAP, false, NWG>(scores, nullptr, lengths, B, max_L1,
                                                       max_L2, gap, temperature, w, w.dgap,
                                                       jacobian, nullptr, st));
    } else {
        D2P_TRY(sw2::launch_tangent<sw2::TEMP, NWG>(scores, nullptr, lengths, B, max_L1, max_L2,
                                                    gap, temperature, w, nullptr, st));
        D2P_TRY(sw2::launch_dual<sw2::TEMP, false, NWG>(scores, nullptr, lengths, B, max_L1,
                                                        max_L2, gap, temperature, w, w.dT,
                                                        jacobian, nullptr, st));
    }
    return wf::launch_poison(w.prim.status, B, (long long)max_L1 * max_L2, jacobian, nullptr,
                             nullptr, nullptr, nullptr, nullptr, st);
}

template <bool NWG>
int backward_full_impl(const float* scores, const float* grad_alignment, const int* lengths,
                       int B, int max_L1, int max_L2, float gap, float temperature,
                       float* grad_scores, float* grad_gap, float* grad_T, void* workspace,
                       size_t workspace_bytes, void* stream) {
    D2P_TRY(sw2::check(B, max_L1, max_L2, temperature));
    if (B == 0) return D2P_OK;
    D2P_REQUIRE(scores && grad_alignment && grad_scores && grad_gap && grad_T,
                "null pointer argument");
    const size_t need = d2p_sw_second_workspace_bytes(B, max_L1, max_L2);
    D2P_REQUIRE(workspace && workspace_bytes >= need, "workspace too small");
    hipStream_t st = (hipStream_t)stream;
    const sw2::Second w = sw2::second_layout(workspace, B, max_L1, max_L2);
    const float* ga = grad_alignment;
    // the forward with the tangent along grad_alignment (for grad_scores = H ga)
    D2P_TRY(sw2::forward_and_tangent<NWG>(scores, ga, lengths, B, max_L1, max_L2, gap,
                                          temperature, w, st));
    // SW: dS/dgap and dS/dT; the marginals land in grad_scores, overwritten by the HVP
    if (!NWG)
        D2P_TRY(sw::launch_backward(scores, lengths, B, max_L1, max_L2, gap, temperature,
                                    w.prim, w.part, grad_scores, w.dgap, w.dT, st, true));
    // grad_scores = H grad_alignment
    D2P_TRY(sw2::launch_dual<sw2::HVP, false, NWG>(scores, ga, lengths, B, max_L1, max_L2, gap,
                                                   temperature, w, w.sdot, grad_scores, nullptr,
                                                   st));
    // grad_gap[b] = <grad_alignment, dP/dgap>, grad_T[b] = <grad_alignment, dP/dT>
    D2P_TRY(sw2::launch_tangent<sw2::GAP, NWG>(scores, nullptr, lengths, B, max_L1, max_L2, gap,
                                               temperature, w, nullptr, st));
    D2P_TRY(sw2::launch_dual<sw2::GAP, true, NWG>(scores, ga, lengths, B, max_L1, max_L2, gap,
                                                  temperature, w, w.dgap, nullptr, grad_gap, st));
    D2P_TRY(sw2::launch_tangent<sw2::TEMP, NWG>(scores, nullptr, lengths, B, max_L1, max_L2, gap,
                                                temperature, w, nullptr, st));
    D2P_TRY(sw2::launch_dual<sw2::TEMP, true, NWG>(scores, ga, lengths, B, max_L1, max_L2, gap,
                                                   temperature, w, w.dT, nullptr, grad_T, st));
    return wf::launch_poison(w.prim.status, B, (long long)max_L1 * max_L2, grad_scores, nullptr,
                             grad_gap, grad_T, nullptr, nullptr, st);
}

}  // namespace

extern "C" int d2p_sw_hvp(const float* scores, const float* tangent, const int* lengths, int B,
                          int max_L1, int max_L2, float gap, float temperature, float* hvp,
                          void* workspace, size_t workspace_bytes, void* stream) {
    return hvp_impl<false>(scores, tangent, lengths, B, max_L1, max_L2, gap, temperature, hvp,
                           workspace, workspace_bytes, stream);
}

extern "C" int d2p_sw_param_jacobian(const float* scores, int param_type, const int* lengths,
                                     int B, int max_L1, int max_L2, float gap, float temperature,
                                     float* jacobian, void* workspace, size_t workspace_bytes,
                                     void* stream) {
    return param_jacobian_impl<false>(scores, param_type, lengths, B, max_L1, max_L2, gap,
                                      temperature, jacobian, workspace, workspace_bytes, stream);
}

extern "C" int d2p_sw_backward_full(const float* scores, const float* grad_alignment,
                                    const int* lengths, int B, int max_L1, int max_L2, float gap,
                                    float temperature, float* grad_scores, float* grad_gap,
                                    float* grad_T, void* workspace, size_t workspace_bytes,
                                    void* stream) {
    return backward_full_impl<false>(scores, grad_alignment, lengths, B, max_L1, max_L2, gap,
                                     temperature, grad_scores, grad_gap, grad_T, workspace,
                                     workspace_bytes, stream);
}

extern "C" size_t d2p_nw_second_workspace_bytes(int B, int max_L1, int max_L2) {
    return d2p_sw_second_workspace_bytes(B, max_L1, max_L2);
}

extern "C" int d2p_nw_hvp(const float* scores, const float* tangent, const int* lengths, int B,
                          int max_L1, int max_L2, float gap, float temperature, float* hvp,
                          void* workspace, size_t workspace_bytes, void* stream) {
    return hvp_impl<true>(scores, tangent, lengths, B, max_L1, max_L2, gap, temperature, hvp,
                          workspace, workspace_bytes, stream);
}

extern "C" int d2p_nw_param_jacobian(const float* scores, int param_type, const int* lengths,
                                     int B, int max_L1, int max_L2, float gap, float temperature,
                                     float* jacobian, void* workspace, size_t workspace_bytes,
                                     void* stream) {
    return param_jacobian_impl<true>(scores, param_type, lengths, B, max_L1, max_L2, gap,
                                     temperature, jacobian, workspace, workspace_bytes, stream);
}

extern "C" int d2p_nw_backward_full(const float* scores, const float* grad_alignment,
                                    const int* lengths, int B, int max_L1, int max_L2, float gap,
                                    float temperature, float* grad_scores, float* grad_gap,
                                    float* grad_T, void* workspace, size_t workspace_bytes,
                                    void* stream) {
    return backward_full_impl<true>(scores, grad_alignment, lengths, B, max_L1, max_L2, gap,
                                    temperature, grad_scores, grad_gap, grad_T, workspace,
                                    workspace_bytes, stream);
}
