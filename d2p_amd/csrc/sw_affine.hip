// sw_affine.hip -- affine-gap soft Smith-Waterman on gfx950.
//
// Reference behaviour restated (not translated):
//   forward   /root/reference/src/sw_affine/kernels_cpu.cpp:94-195
//   backward  /root/reference/src/sw_affine/kernels_cpu.cpp:201-356
// Three states per cell (i, j >= 1):
//   M = LSE_T(M[i-1,j-1]+s, I[i-1,j-1]+s, D[i-1,j-1]+s (only i>1 && j>1), s)
//   I = LSE_T(M[i-1,j]+open, I[i-1,j]+ext)            (only i > 1)
//   D = LSE_T(M[i,j-1]+open, D[i,j-1]+ext)            (only j > 1)
// so a gap of length k costs open + (k-1)*ext; M[0,0] = 0, every other row/column 0
// value is NINF, and S = LSE_T over the three states of all cells 0..L1 x 0..L2.
// The marginal of cell (i,j) is beta_M * (sum of M's four weights).
//
// Mapping: the stripe pipeline of wavefront.hip.h.  The forward carries (M, I, D) per
// lane; lane 0 of a stripe reads (M, I, D) of the stripe above from a float4 ring.
// The three planes are stored as skewed tables table[b][stripe][plane][step][lane]
// plus each stripe's last row by step.  The backward runs three beta channels; a
// cell's successors hand it, in the reference's accumulation order,
//   beta_M = ((init + from M[i+1,j+1]) + from D[i,j+1]) + from I[i+1,j]
//   beta_I =  (init + from M[i+1,j+1]) + from I[i+1,j]
//   beta_D =  (init + from M[i+1,j+1]) + from D[i,j+1].

#include <vector>

#include <cstdlib>
#include <type_traits>

#include "wavefront.hip.h"
#include "../../include/d2p_amd.h"
#include "capi_util.hip.h"
#include "swa_internal.hip.h"

namespace d2p_amd {
namespace swa {

using namespace wf;

constexpr int PF = 16;           // steps per chunk, forward
constexpr int PB = 8;            // steps per chunk, backward (three alpha planes staged)
constexpr int DUMMY = 64 + PF;   // per-wave sink entries for the lanes that do not publish

// (the larger term's exponential is exp2(0) = 1 exactly, and the other's argument
// (min - max) c is -|a - b| c bit for bit: one exponential, the same sum; a NaN in a
// or b still makes the sum NaN)
__device__ __forceinline__ float lse2(float a, float b, float c, float tl) {
    const float m = fmaxf(a, b);
    return m + tl * fast_log2(1.0f + fast_exp2(-fabsf(a - b) * c));
}

__device__ __forceinline__ float lse3(float a, float b, float x, float c, float tl) {
    const float m = fmaxf(fmaxf(a, b), x);
    const float z = (fast_exp2((a - m) * c) + fast_exp2((b - m) * c)) + fast_exp2((x - m) * c);
    return m + tl * fast_log2(z);
}

__device__ __forceinline__ float lse4(float a, float b, float x, float y, float c, float tl) {
    const float m = fmaxf(fmaxf(a, b), fmaxf(x, y));
    const float z = ((fast_exp2((a - m) * c) + fast_exp2((b - m) * c)) + fast_exp2((x - m) * c)) +
                    fast_exp2((y - m) * c);
    return m + tl * fast_log2(z);
}

// NWA: global alignment with affine gaps (soft Needleman-Wunsch,
// /root/reference/src/nw_affine/kernels_cpu.cpp:100-187): M = s + LSE(M, I, D) of
// the diagonal, I = LSE(M + open, I + ext, D + open) of the cell above, D = LSE(M +
// open, I + open, D + ext) of the cell to the left; the boundary is M[0,0] = 0,
// I[i,0] = open + (i-1) ext, D[0,j] = open + (j-1) ext (NINF elsewhere), and the
// value is LSE(M, I, D) of the terminal cell (L1, L2).  The cells left of column 0
// hold the row's boundary in the tables; row 0 is generated in registers.
// HELP (local alignment, parts of at most NW/2 stripes): wave NW/2 + l loads stripe
// l's score chunks one chunk ahead (hprog[l] = chunks loaded) and writes the M and I
// planes of each chunk's alphas to the table once wave l has finished the chunk:
// wave l leaves them in a tile of the helper's (its own buffer for even chunks, a
// region after the rings for odd ones) and stores only the D plane itself.
template <bool NWA = false, bool HELP = false>
__global__ void __launch_bounds__(NW * 64)
swa_forward_kernel(const float* __restrict__ scores, const int* __restrict__ lengths,
                   float* __restrict__ alpha_sk, float* __restrict__ brow,
                   float* __restrict__ partition, int* __restrict__ status,
                   uint64_t* __restrict__ fflag, float2* __restrict__ fpart, int B, int L1max,
                   int L2max, int NSmax, float go, float ge, float T, int R, int G, int SPW,
                   uint32_t epoch) {
    constexpr int P = PF;
    static_assert(!HELP || !NWA, "helper waves serve the local form");
    extern __shared__ __align__(16) float smem[];
    __shared__ int prog[NW];
    __shared__ int hprog[NW];     // HELP: score chunks of stripe l loaded by its helper
    __shared__ float red_m[NW], red_z[NW];
    __shared__ float term[3];     // NWA: (M, I, D) of the terminal cell
    // part of the element as in the linear forward: the first stripe of a part > 0
    // reads the previous part's last rows (M, I, D) from brow
    int b, part;
    split_decode(blockIdx.x, G, b, part);
    if (b >= B) return;
    const int lane = threadIdx.x & 63;
    const unsigned ul4 = (unsigned)lane * 4u;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    using Tile = QuadTile<P>;                             // 16-byte score loads
    constexpr int WBUF = 2 * Tile::FLOATS + 2 * 3 * 64;
    float* tiles = smem + wave * WBUF;                    // double-buffered score chunk
    float* rbufs = tiles + 2 * Tile::FLOATS;              // [2][plane][64] rows above
    __shared__ float fslot[64];   // progress word prefetched by wave 0, the only wave whose
                                  // stripe borders another part
    const uint32_t fslot_lds = lds_address(fslot);
    float4* rings = reinterpret_cast<float4*>(smem + NW * WBUF);   // [NW][R]
    float4* sink = rings + NW * R + wave * DUMMY;
    // HELP: the M and I alpha tiles ([2][P][64]) of stripe l's chunk k
    float* xtra = reinterpret_cast<float*>(rings + NW * R + NW * DUMMY);   // [NW/2][2P][64]
    auto mi_tile = [&](int l, int k) {
        return (k & 1) ? xtra + l * 2 * P * 64 : smem + (l + NW / 2) * WBUF;
    };
    int* st = status + b;

    if (lane == 0) {
        prog[wave] = -1;
        hprog[wave] = -1;
    }
    if (G == 1 && threadIdx.x == 0) *st = 0;              // G > 1: reset before the launch
    if (NWA && threadIdx.x < 3) term[threadIdx.x] = kNINF;
    __syncthreads();

    const int L1 = lengths ? min(max(lengths[2 * b], 0), L1max) : L1max;
    const int L2 = lengths ? min(max(lengths[2 * b + 1], 0), L2max) : L2max;
    const float c = kLog2e / T;
    const float tl = T * kLn2;
    const int NS = L2 > 0 ? (L1 + 63) >> 6 : 0;
    const int nsteps = L2 + 63;
    const int nch = (nsteps + P - 1) / P;
    const size_t NT = (size_t)stored_steps(L2max);
    const size_t PLANE = NT * 64;
    const float* sbase = scores + (size_t)b * L1max * L2max;

    const int s_begin = part * SPW;
    const int NL = max(min(NS, s_begin + SPW) - s_begin, 0);   // stripes of this part
    const bool has_next = s_begin + NL < NS;
    const uint64_t* flag_in = fflag + (size_t)b * G + (part > 0 ? part - 1 : 0);
    uint64_t* flag_out = fflag + (size_t)b * G + part;

    OnlineLSE acc;
    acc.init_open();

    if constexpr (HELP) {
        if (NL > NW / 2) {   // never: the host picks HELP for parts of at most NW/2 stripes
            if (threadIdx.x == 0) atomicOr(st, 2);
            return;
        }
        const int l = wave - NW / 2;
        if (l >= 0 && l < NL) {
            const int s = s_begin + l;
            const int i0 = s * 64;
            float* out = alpha_sk + ((size_t)b * NSmax + s) * 3 * PLANE + APAD * 64;
            const uint32_t ltiles = lds_address(smem + l * WBUF);   // wave l's score tiles
            auto load = [&](int k) {
                dma_quads<P, 1>(ltiles + (k & 1) * Tile::FLOATS * 4, sbase, i0, L1max, L2max,
                                lane, k * P);
            };
            if (nch > 0) {
                load(0);
                wait_vmcnt<0>();
                publish(hprog, l, 1);
                if (nch > 1) load(1);
            }
            for (int k = 0; k < nch; ++k) {
                if (k + 1 < nch) {
                    // chunk k + 1's loads: the last issued at k = 0, else followed by the
                    // 2 P/4 alpha stores of chunk k - 1
                    if (k == 0) wait_vmcnt<0>(); else wait_vmcnt<2 * (P / 4)>();
                    publish(hprog, l, k + 2);   // also completes this wave's LDS reads
                }
                // once wave l has finished chunk k, its score tile k & 1 takes chunk
                // k + 2 and its M and I rows go to the table
                wait_for(prog, l, l * PROG_STRIDE + k + 1, st);
                if (k + 2 < nch) load(k + 2);
                const float* at = mi_tile(l, k);
                float* dst = out + (size_t)k * P * 64;
#pragma unroll
                for (int pl = 0; pl < 2; ++pl) {
#pragma unroll
                    for (int i = 0; i < P / 4; ++i) {
                        const float4 v =
                            *reinterpret_cast<const float4*>(at + pl * P * 64 + 256 * i + 4 * lane);
                        *reinterpret_cast<float4*>(dst + pl * PLANE + 256 * i + 4 * lane) = v;
                    }
                }
            }
        }
    }

    for (int l = wave; l < NL; l += NW) {
        const int s = s_begin + l;
        const int i0 = s * 64;
        const int L2eff = (i0 + lane < L1) ? L2 : 0;
        const float4* ring_in = ring_from(rings, l, R);
        float4* ring_out = ring_of(rings, l, R);
        float* out = alpha_sk + ((size_t)b * NSmax + s) * 3 * PLANE + APAD * 64;   // M, step 0
        float* brow_s = brow + ((size_t)b * NSmax + s) * 3 * NT;                    // [3][NT]
        const float* brow_up = brow + ((size_t)b * NSmax + (s > 0 ? s - 1 : 0)) * 3 * NT;
        const bool x_in = l == 0 && part > 0;        // rows above from the previous part
        const bool x_out = l == NL - 1 && has_next;  // last rows feed the next part
        int seen = -1;       // chunks of the previous part known to be complete
        // NWA: I of this lane's row (i0 + lane + 1) at column 0
        const float bndI = (NWA && i0 + lane < L1) ? go + (float)(i0 + lane) * ge : kNINF;
        // steps t < 0 hold the column-0 boundary (NINF; NWA: I = bndI), read by the
        // reverse sweep
#pragma unroll
        for (int t = -APAD; t < 0; ++t) {
            lane_store(out + t * 64, ul4, kNINF);
            lane_store(out + PLANE + t * 64, ul4, bndI);
            lane_store(out + 2 * PLANE + t * 64, ul4, kNINF);
        }
        wave_lds_sync();   // the previous stripe's tile reads are complete
        const uint32_t tile_lds = lds_address(tiles);
        const uint32_t row_lds = lds_address(rbufs);
        // the rows above of chunk k: lane j < P carries the step kP + 63 + j, per plane
        auto issue_rows = [&](int k) {
            const uint32_t off = (uint32_t)min(k * P + 63 + min(lane, P - 1), nsteps - 1) * 4u;
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) {
                uint32_t o = off;
                uint32_t dst = row_lds + (uint32_t)(((k & 1) * 3 + pl) * 64 * 4);
                lds_dma_dword_sys<0>(brow_up + pl * NT, o, dst, 0u);
            }
        };
        if (x_in) {
            seen = wait_part(flag_in, epoch, min(lead(P), nch), st);
            issue_rows(0);
        }
        if (!HELP) dma_quads<P, 1>(tile_lds, sbase, i0, L1max, L2max, lane, 0);
        float cM = kNINF, cI = bndI, cD = kNINF;       // this lane's previous step
        float pM = kNINF, pI = kNINF, pD = kNINF;      // up values of the previous step
        if (NWA && lane == 0) {
            // lane 0's first diagonal: (i0, 0), the start cell M[0,0] = 0 or I's boundary
            if (s == 0) pM = 0.0f;
            else pI = go + (float)(i0 - 1) * ge;
        }

        for (int k = 0; k < nch; ++k) {
            const int t0 = k * P;
            chunk_waits<P>(prog, l, NL, k, nch, R, st);
            // this chunk's scores: loaded one chunk ago and followed by at least the
            // 3P + 3 stores of that chunk (the first chunk's load is the last issued).
            // HELP: the helper loads the scores; this wave's own loads (the rows above
            // of a part's first stripe) are followed by at least its P + 3 stores
            if (k == 0) wait_vmcnt<0>(); else if (HELP) wait_vmcnt<P>(); else wait_vmcnt<3 * P>();
            if (HELP) wait_for(hprog, l, k + 1, st);
            if (x_in && k > 0) {
                // its progress word, loaded one chunk ago before those stores
                const int got = flag_chunks_lds(fslot, epoch);
                seen = got > seen ? got : seen;
            }
            const float* tile = tiles + (k & 1) * Tile::FLOATS;
            float sv[P], aM[P], aI[P], aD[P];
            read_quads<P, 1>(tile, lane, sv);
            // lane 0's up values: column t0+j sits in lane j (NWA, first stripe: row 0,
            // where only D[0, t0+j+1] = open + (t0+j) ext is finite)
            float rM = kNINF, rI = kNINF, rD = kNINF;
            if (NWA && s == 0 && lane < P) rD = go + (float)(t0 + lane) * ge;
            if (s > 0 && lane < P) {
                if (x_in) {
                    const float* rb = rbufs + (k & 1) * 3 * 64;
                    rM = rb[lane];
                    rI = rb[64 + lane];
                    rD = rb[128 + lane];
                } else {
                    const float4 r = ring_in[ring_index(t0 + lane + 63, R)];
                    rM = r.x;
                    rI = r.y;
                    rD = r.z;
                }
            }
            if (k + 1 < nch) {
                if (x_in) {
                    const int need = min(k + 1 + lead(P), nch);
                    if (seen < need) seen = wait_part(flag_in, epoch, need, st);
                    issue_rows(k + 1);
                }
                if (!HELP)
                    dma_quads<P, 1>(tile_lds + ((k + 1) & 1) * Tile::FLOATS * 4, sbase, i0,
                                    L1max, L2max, lane, t0 + P);
                if (x_in) flag_load_lds(flag_in, fslot_lds, lane);
            }
            float4* pub = (lane == 63) ? ring_out + ring_index(t0, R) : sink + lane;
            float* outc = out + (size_t)t0 * 64;
            // HELP: the M and I rows of this chunk in the helper's tile (written to the
            // table by the helper, which has written that tile's previous chunk before
            // publishing this chunk's scores as loaded)
            float* mit = mi_tile(l, k) + lane;
            // FULL: every cell of the chunk lies inside the element, no validity masks
            auto steps = [&](auto full) {
            constexpr bool FULL = decltype(full)::value;
#pragma unroll
            for (int u = 0; u < P; ++u) {
                const int t = t0 + u;
                const float uM = wave_shr1_or(cM, rM), uI = wave_shr1_or(cI, rI),
                            uD = wave_shr1_or(cD, rD);
                rM = wave_shl1(rM);
                rI = wave_shl1(rI);
                rD = wave_shl1(rD);
                const float dM = pM, dI = pI, dD = pD;   // diagonal = previous step's up
                pM = uM;
                pI = uI;
                pD = uD;
                const float sc = sv[u];
                // out-of-table neighbours are NINF: no i>1 / j>1 guards are needed
                float M, I, D;
                if (NWA) {
                    M = sc + lse3(dM, dI, dD, c, tl);
                    I = lse3(uM + go, uI + ge, uD + go, c, tl);
                    D = lse3(cM + go, cI + go, cD + ge, c, tl);
                } else {
                    M = lse4(dM + sc, dI + sc, dD + sc, sc, c, tl);
                    I = lse2(uM + go, uI + ge, c, tl);
                    D = lse2(cM + go, cD + ge, c, tl);
                }
                const bool ok = FULL || (unsigned)(t - lane) < (unsigned)L2eff;
                // NWA: the cells left of column 0 keep the row's boundary
                const bool left = NWA && !FULL && t < lane;
                cM = ok ? M : kNINF;
                cI = ok ? I : (left ? bndI : kNINF);
                cD = ok ? D : kNINF;
                if (NWA && ok && i0 + lane == L1 - 1 && t - lane == L2 - 1) {
                    term[0] = M;
                    term[1] = I;
                    term[2] = D;
                }
                if (HELP) {
                    mit[u * 64] = cM;
                    mit[P * 64 + u * 64] = cI;
                } else {
                    lane_store(outc + u * 64, ul4, cM);
                    lane_store(outc + PLANE + u * 64, ul4, cI);
                }
                lane_store(outc + 2 * PLANE + u * 64, ul4, cD);
                pub[u] = make_float4(cM, cI, cD, 0.0f);
                aM[u] = cM;
                aI[u] = cI;
                aD[u] = cD;
            }
            };
            if (i0 + 63 < L1 && t0 >= 63 && t0 + P <= L2) steps(std::true_type{});
            else steps(std::false_type{});
            if (!NWA) {
                acc.add_block<P>(aM, c);
                acc.add_block<P>(aI, c);
                acc.add_block<P>(aD, c);
            }
            // the stripe's last row by step, per plane: three store instructions
            wave_lds_sync();
            if (lane < P) {
                const float4 r = ring_out[t0 % R + lane];
                if (x_out) {
                    store_sys(brow_s + t0 + lane, r.x);
                    store_sys(brow_s + NT + t0 + lane, r.y);
                    store_sys(brow_s + 2 * NT + t0 + lane, r.z);
                } else {
                    const unsigned o = (unsigned)(t0 + lane) * 4u;
                    lane_store(brow_s, o, r.x);
                    lane_store(brow_s + NT, o, r.y);
                    lane_store(brow_s + 2 * NT, o, r.z);
                }
            }
            publish(prog, wave, l * PROG_STRIDE + k + 1);
            if (x_out && k >= 2) {
                // at least P/4 loads and 6P + 6 stores follow the row stores of chunk
                // k - 2 (more than the counter holds; HELP: the 2P + 6 D-plane and
                // row stores of chunks k - 1 and k): those are complete
                if constexpr (HELP) wait_vmcnt<2 * P + 6>();
                else wait_vmcnt<63>();
                if (lane == 0) store_flag(flag_out, progress_word(epoch, k - 1));
            }
        }
        if (x_out) {
            wait_vmcnt<0>();
            if (lane == 0) store_flag(flag_out, progress_word(epoch, nch));
        }
    }

    if (NWA) {
        // the value: the terminal cell, written by the part that owns the last stripe;
        // an element without cells is its boundary cell (L1, L2)
        __syncthreads();
        const bool owner = NS > 0 ? (NL > 0 && s_begin + NL == NS) : part == 0;
        if (threadIdx.x == 0 && owner) {
            float v;
            if (NS > 0) v = lse3(term[0], term[1], term[2], c, tl);
            else if (L1 > 0) v = go + (float)(L1 - 1) * ge;
            else if (L2 > 0) v = go + (float)(L2 - 1) * ge;
            else v = 0.0f;
            partition[b] = v;
        }
        return;
    }
    // partition: merge lanes, waves, and the cell M[0,0] = 0
    wave_merge_lse(acc, c);
    if (lane == 0) { red_m[wave] = acc.m; red_z[wave] = acc.z; }
    __syncthreads();
    if (threadIdx.x == 0) {
        OnlineLSE tot;
        if (G == 1) {
            tot.m = 0.0f;
            tot.z = 1.0f;
        } else {
            tot.init();
        }
        for (int w = 0; w < NW; ++w) tot.merge(red_m[w], red_z[w], c);
        if (G == 1) partition[b] = tot.m + tl * fast_log2(tot.z);
        else fpart[(size_t)b * G + part] = make_float2(tot.m, tot.z);
    }
}

// NWA: global alignment (/root/reference/src/nw_affine/kernels_cpu.cpp:193-347): beta
// starts at the terminal cell only, with the weights of its three states; every state
// has three candidates (I and D also take D above / I to the left with an open), so
// the up and left flows reach all three states; a state passes flow only when its
// beta exceeds 1e-20; the flows into column 0 (I[i,0]) and row 0 (D[0,j]) add the
// boundary's own open and (i-1) or (j-1) extends to the parameter gradients.
// The second flow ring carries (diagonal D, up D) pairs instead of the diagonal D.
// HELP (local alignment, parts of at most NW/2 stripes): wave NW/2 + q moves stripe
// order q's data.  Chunk k's buffer is wave q's own for even k and the helper's for
// odd k.  The helper loads a chunk's scores and alpha rows one chunk ahead
// (publishing hprog[q] = chunks loaded), writes the chunk's output tile out once
// wave q has finished the chunk (prog[q]), and then loads chunk k + 2 into that
// buffer.  Wave q loads only its rows above and flows.
template <bool NWA = false, bool HELP = false>
__global__ void __launch_bounds__(NW * 64)
swa_backward_kernel(const float* __restrict__ scores, const int* __restrict__ lengths,
                    const float* __restrict__ alpha_sk, const float* __restrict__ brow,
                    const float* __restrict__ partition, float* __restrict__ post,
                    float* __restrict__ grad_open, float* __restrict__ grad_ext,
                    float* __restrict__ grad_T, int* __restrict__ status,
                    float* __restrict__ trash, uint64_t* __restrict__ bflag,
                    float4* __restrict__ flows4, float* __restrict__ flows1,
                    double* __restrict__ bpart, int B, int L1max, int L2max, int NSmax, float go,
                    float ge, float T, int R, int G, int SPW, uint32_t epoch) {
    constexpr int P = PB;
    static_assert(!HELP || !NWA, "helper waves move quad tiles");
    extern __shared__ __align__(16) float smem[];
    __shared__ int prog[NW];
    __shared__ int hprog[NW];     // HELP: chunks of stripe order q loaded by its helper
    __shared__ float red_o[NW], red_e[NW], red_p[NW];
    // parts run bottom-up as in the linear backward; the last stripe of a part below
    // the first hands its flows to the part above through flows4 / flows1
    int b, dpart;
    split_decode(blockIdx.x, G, b, dpart);
    if (b >= B) return;
    const int part = G - 1 - dpart;
    const int lane = threadIdx.x & 63;
    const unsigned ul4 = (unsigned)lane * 4u;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Per wave: one in-flight input buffer (scores tile, P rows of each alpha plane,
    // the row above for each plane), read into registers at the start of each chunk
    // before the next chunk's loads are issued into it, and one output tile.  In the
    // local form (QT) the score and output tiles move as 16-byte quads (P/4
    // instructions each), and the output quad of four steps is assembled in
    // registers; the global form runs at the register limit and keeps dword tiles.
    constexpr bool QT = !NWA;
    using Tile = std::conditional_t<QT, QuadTile<P>, ChunkTile<P>>;
    constexpr int NQ = QT ? P / 4 : P;              // tile load or store instructions
    constexpr int AROWS = Tile::FLOATS;             // 3 planes x P rows x 64
    constexpr int RROW = AROWS + 3 * P * 64;        // 3 planes x 64
    constexpr int OTILE = RROW + 3 * 64;
    constexpr int FB4 = OTILE + Tile::FLOATS;       // flows from the part below: float4s
    constexpr int FB1 = FB4 + 64;                   // ... and the diagonal D flows (NWA:
    constexpr int WFLOATS = FB1 + 64;               // (diagonal D, up D) pairs)
    static_assert(4 * P + 4 <= 64, "boundary flows fit their buffer");
    using F1 = std::conditional_t<NWA, float2, float>;   // second ring entry
    float* const wbuf0 = smem + wave * WFLOATS;   // this wave's chunk buffer
    __shared__ float fslot[64];   // progress word prefetched by wave 0, the only wave whose
                                  // stripe borders another part
    const uint32_t fslot_lds = lds_address(fslot);
    // rings [NW][R]: (up M, up I, diag M, diag I) and diag D (NWA: (diag D, up D)),
    // from lane 0 upward
    float4* ring4 = reinterpret_cast<float4*>(smem + NW * WFLOATS);
    F1* ring1 = reinterpret_cast<F1*>(ring4 + NW * R);
    float4* sink4 = reinterpret_cast<float4*>(ring1 + NW * R) + wave * (64 + P);
    F1* sink1 = reinterpret_cast<F1*>(reinterpret_cast<float4*>(ring1 + NW * R) +
                                      NW * (64 + P)) + wave * (64 + P);
    F1* flowsF = reinterpret_cast<F1*>(flows1);
    int* st = status + b;
    const int tbase = ChunkTile<P>::read_base(lane);   // dword tiles

    if (lane == 0) {
        prog[wave] = -1;
        hprog[wave] = -1;
    }
    __syncthreads();

    const int L1 = lengths ? min(max(lengths[2 * b], 0), L1max) : L1max;
    const int L2 = lengths ? min(max(lengths[2 * b + 1], 0), L2max) : L2max;
    const float c = kLog2e / T;
    const float S = partition[b];
    const int NS = L2 > 0 ? (L1 + 63) >> 6 : 0;
    const int nsteps = L2 + 63;
    const int nch = (nsteps + P - 1) / P;
    const size_t NT = (size_t)stored_steps(L2max);
    const size_t PLANE = NT * 64;
    const float* sbase = scores + (size_t)b * L1max * L2max;
    float* pbase = post + (size_t)b * L1max * L2max;

    {   // each part zeroes its share of the rows' padding
        const int rows = (L1max + G - 1) / G;
        zero_padding(pbase, L1, L2, L1max, L2max, NW * 64, part * rows,
                     min(L1max, part * rows + rows));
    }

    float g_open = 0.0f, g_ext = 0.0f, p_acc = 0.0f;
    float AM[P + 2], AI[P + 2], AD[P + 2];
    const int s_begin = part * SPW;
    const int NL = max(min(NS, s_begin + SPW) - s_begin, 0);   // stripes of this part
    const bool has_next = s_begin + NL < NS;
    const uint64_t* flag_in = bflag + (size_t)b * G + (part + 1 < G ? part + 1 : part);
    uint64_t* flag_out = bflag + (size_t)b * G + part;

    if constexpr (HELP) {
        if (NL > NW / 2) {   // never: the host picks HELP for parts of at most NW/2 stripes
            if (threadIdx.x == 0) atomicOr(st, 2);
            return;
        }
        const int q = wave - NW / 2;
        if (q >= 0 && q < NL) {
            const int s = s_begin + NL - 1 - q;
            const int i0 = s * 64;
            const float* astripe = alpha_sk + ((size_t)b * NSmax + s) * 3 * PLANE;
            // chunk k's buffer: wave q's own (even k) or this wave's (odd k)
            auto cbuf = [&](int k) { return smem + (k & 1 ? wave : q) * WFLOATS; };
            auto load = [&](int k) {
                const int th = nsteps - 1 - k * P;
                const uint32_t in = lds_address(cbuf(k));
                dma_quads<P, -1>(in, sbase, i0, L1max, L2max, lane, th);
#pragma unroll
                for (int pl = 0; pl < 3; ++pl)
                    dma_rows<P, -1>(in + (AROWS + pl * P * 64) * 4, astripe + pl * PLANE, th - 2,
                                    ul4);
            };
            // whole row segments of marginals where rows start aligned (write_aligned)
            const bool aligned = (L2max & (P - 1)) == 0;
            AlignedCarry<P> carry;
            carry.clear();
            if (nch > 0) {
                load(0);
                wait_vmcnt<0>();
                publish(hprog, q, 1);
                if (nch > 1) load(1);
            }
            for (int k = 0; k < nch; ++k) {
                if (k + 1 < nch) {
                    // chunk k + 1's loads are the last issued
                    wait_vmcnt<0>();
                    publish(hprog, q, k + 2);   // also completes this wave's LDS reads
                }
                // once wave q has finished chunk k, its output tile leaves and the
                // buffer takes chunk k + 2 (the stores have read the tile: their data
                // dependence waits for the reads)
                wait_for(prog, q, q * PROG_STRIDE + k + 1, st);
                if (aligned)
                    write_aligned<P, true>(cbuf(k) + OTILE, pbase, trash, carry, i0, L1max,
                                           L2max, lane, nsteps - 1 - k * P);
                else
                    write_quads<P, -1>(cbuf(k) + OTILE, pbase, trash, i0, L1, L2, L1max, L2max,
                                       lane, nsteps - 1 - k * P);
                if (k + 2 < nch) load(k + 2);
            }
        }
    }

    for (int q = wave; q < NL; q += NW) {
        const int s = s_begin + NL - 1 - q;
        const int i0 = s * 64;
        const int L2eff = (i0 + lane < L1) ? L2 : 0;
        const float* astripe = alpha_sk + ((size_t)b * NSmax + s) * 3 * PLANE;   // M at step -APAD
        const float* bup = brow + ((size_t)b * NSmax + (s > 0 ? s - 1 : 0)) * 3 * NT;
        const float4* r4_in = ring_from(ring4, q, R);
        const F1* r1_in = ring_from(ring1, q, R);
        float4* r4_out = ring_of(ring4, q, R);
        F1* r1_out = ring_of(ring1, q, R);
        const bool x_in = q == 0 && has_next;             // flows from the part below
        const bool x_out = q == NL - 1 && part > 0;       // flows to the part above
        const bool below = q > 0 || x_in;
        // chunk k's buffer: this wave's own, or (HELP, odd k) its helper's
        auto kbuf = [&](int k) {
            return HELP && (k & 1) ? smem + (wave + NW / 2) * WFLOATS : wbuf0;
        };
        // boundary flows by producer step: written by stripe s (x_out), read from s + 1
        const size_t fo = ((size_t)b * NSmax + s) * NT;
        const size_t fi = ((size_t)b * NSmax + (x_in ? s + 1 : s)) * NT;
        const float* f4_in = reinterpret_cast<const float*>(flows4 + fi);
        const float* f1_in = reinterpret_cast<const float*>(flowsF + fi);
        int seen = -1;       // chunks of the part below known to be complete

        // Loads of chunk k (t_hi = nsteps-1-kP): the score tile, P alpha rows per plane
        // (steps t_hi-2 .. t_hi-P-1) and the stripe above's last row per plane at steps
        // t_hi - j + 63 for lane j <= P (clamped; lanes past P repeat lane P).
        // NQ + 3P/4 + 3 loads (HELP: the helper loads the tile and rows; 3 loads).
        auto issue_chunk = [&](int k) {
            const int th = nsteps - 1 - k * P;
            const uint32_t in_lds = lds_address(kbuf(k));
            if constexpr (!HELP) {
                if constexpr (QT) dma_quads<P, -1>(in_lds, sbase, i0, L1max, L2max, lane, th);
                else dma_tile<P, -1>(in_lds, sbase, i0, L1max, L2max, lane, th);
#pragma unroll
                for (int pl = 0; pl < 3; ++pl)
                    dma_rows<P, -1>(in_lds + (AROWS + pl * P * 64) * 4, astripe + pl * PLANE,
                                    th - 2, ul4);
            }
            const uint32_t roff = (uint32_t)min(th - min(lane, P) + 63, nsteps - 1) * 4u;
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) {
                uint32_t o = roff, l = in_lds + (RROW + pl * 64) * 4;
                lds_dma_dword<0>(bup + pl * NT, o, l, 0u);
            }
            if (x_in) {
                // flows of producer slots kP+62 .. kP+62+P: float f of the float4 range
                // and the D flow of slot kP+62+f in lane f, clamped to the last slot
                uint32_t o = (uint32_t)min((k * P + 62) * 4 + min(lane, 4 * P + 3),
                                           (nsteps - 1) * 4 + 3) * 4u;
                uint32_t l = in_lds + FB4 * 4;
                lds_dma_dword_sys<0>(f4_in, o, l, 0u);
                // NWA: float f of the (diag D, up D) pairs from slot kP+62 in lane f
                o = NWA ? (uint32_t)min((k * P + 62) * 2 + min(lane, 2 * P + 3),
                                        (nsteps - 1) * 2 + 1) * 4u
                        : (uint32_t)min(k * P + 62 + min(lane, P), nsteps - 1) * 4u;
                l = in_lds + FB1 * 4;
                lds_dma_dword_sys<0>(f1_in, o, l, 0u);
            }
        };

        // the first two steps of chunk 0 (later chunks carry them over)
        {
            const float* a0 = astripe + (size_t)(nsteps - 1 + APAD) * 64;
            const float* a1 = astripe + (size_t)(nsteps - 2 + APAD) * 64;
            AM[P] = lane_load(a0, ul4);
            AM[P + 1] = lane_load(a1, ul4);
            AI[P] = lane_load(a0 + PLANE, ul4);
            AI[P + 1] = lane_load(a1 + PLANE, ul4);
            AD[P] = lane_load(a0 + 2 * PLANE, ul4);
            AD[P + 1] = lane_load(a1 + 2 * PLANE, ul4);
            __asm__ volatile("" ::"v"(AM[P]), "v"(AM[P + 1]), "v"(AI[P]), "v"(AI[P + 1]),
                             "v"(AD[P]), "v"(AD[P + 1]));   // completes these loads here
        }
        wave_lds_sync();   // the previous stripe's buffer reads are complete
        if (x_in) seen = wait_part(flag_in, epoch, min(lead(P), nch), st);
        issue_chunk(0);
        // NWA: the terminal cell's step on this lane; I[i,0] of this lane's row and of
        // the row above count (i-1) and (i-2) extends; row 0 (first stripe, lane 0)
        // counts the column's
        const int term_step = (NWA && i0 + lane == L1 - 1) ? L2 - 1 + lane : -1000000;
        const float ext_left = (float)(i0 + lane), ext_diag = (float)(i0 + lane - 1);
        const bool top = NWA && s == 0 && lane == 0;
        // successor contributions waiting for this lane's next steps
        float lM = 0.0f, lI = 0.0f, lD = 0.0f;                   // from (i, j+1)
        float uM = 0.0f, uI = 0.0f, uD = 0.0f;                   // from (i+1, j)
        float dM = 0.0f, dI = 0.0f, dD = 0.0f;                   // from (i+1, j+1)
        float dM2 = 0.0f, dI2 = 0.0f, dD2 = 0.0f;                // ... one step later

        for (int k = 0; k < nch; ++k) {
            const int t_hi = nsteps - 1 - k * P;
            chunk_waits<P>(prog, q, NL, k, nch, R, st);
            // this chunk's loads, followed by at least the NQ marginal stores of the
            // previous chunk (the first chunk's loads are the last issued).  HELP: the
            // helper loads the tile and rows; this wave's own loads (rows above, flows)
            // are followed by nothing, or by the previous chunk's two flow stores (x_out)
            if constexpr (HELP) {
                if (x_out && k > 0) wait_vmcnt<2>(); else wait_vmcnt<0>();
                wait_for(hprog, q, k + 1, st);
            } else {
                if (k == 0) wait_vmcnt<0>(); else wait_vmcnt<NQ>();
            }
            if (x_in && k > 0) {
                // its progress word, loaded one chunk ago before those stores
                const int got = flag_chunks_lds(fslot, epoch);
                seen = got > seen ? got : seen;
            }
            float* const wbuf = kbuf(k);
            float* const otile = wbuf + OTILE;
            float sv[P];
            if constexpr (QT) {
                read_quads<P, -1>(wbuf, lane, sv);
            } else {
#pragma unroll
                for (int u = 0; u < P; ++u) sv[u] = wbuf[tbase + u];
            }
            AM[0] = AM[P];
            AM[1] = AM[P + 1];
            AI[0] = AI[P];
            AI[1] = AI[P + 1];
            AD[0] = AD[P];
            AD[1] = AD[P + 1];
#pragma unroll
            for (int j = 0; j < P; ++j) {
                const int r = rows_row<P, -1>(j) * 64 + lane;
                AM[j + 2] = wbuf[AROWS + r];
                AI[j + 2] = wbuf[AROWS + P * 64 + r];
                AD[j + 2] = wbuf[AROWS + 2 * P * 64 + r];
            }
            const bool row_ok = s > 0 && lane <= P && t_hi - lane + 63 <= nsteps - 1;
            float bM = row_ok ? wbuf[RROW + lane] : kNINF;
            float bI = row_ok ? wbuf[RROW + 64 + lane] : kNINF;
            float bD = row_ok ? wbuf[RROW + 128 + lane] : kNINF;
            if (NWA && s == 0 && lane <= P) {
                // row 0 at column t_hi - lane (0-based; -1 is the start cell M[0,0] = 0)
                const int c0 = t_hi - lane;
                bM = c0 == -1 ? 0.0f : kNINF;
                bD = c0 >= 0 ? go + (float)c0 * ge : kNINF;
            }
            // Contributions from the stripe below for lane 63 (see the linear kernel):
            // lane 63-j holds step j; up flows from slot kP+j+63, diagonal from kP+j+62.
            float qUM = 0.0f, qUI = 0.0f, qUD = 0.0f, qDM = 0.0f, qDI = 0.0f, qDD = 0.0f;
            if (below && lane >= 64 - P) {
                const int j = 63 - lane;
                if (x_in) {
                    qUM = wbuf[FB4 + 4 * (j + 1)];
                    qUI = wbuf[FB4 + 4 * (j + 1) + 1];
                    qDM = wbuf[FB4 + 4 * j + 2];
                    qDI = wbuf[FB4 + 4 * j + 3];
                    if (NWA) {
                        qDD = wbuf[FB1 + 2 * j];
                        qUD = wbuf[FB1 + 2 * (j + 1) + 1];
                    } else {
                        qDD = wbuf[FB1 + j];
                    }
                } else {
                    const int iu = ring_index(k * P + j + 63, R);
                    const float4 ru = r4_in[iu];
                    const int id = ring_index(k * P + j + 62, R);
                    const float4 rd = r4_in[id];
                    qUM = ru.x;
                    qUI = ru.y;
                    qDM = rd.z;
                    qDI = rd.w;
                    if constexpr (NWA) {
                        qDD = r1_in[id].x;
                        qUD = r1_in[iu].y;
                    } else {
                        qDD = r1_in[id];
                    }
                }
            }
            wave_lds_sync();   // every read of the input buffer is complete
            if (k + 1 < nch) {
                if (x_in) {
                    const int need = min(k + 1 + lead(P), nch);
                    if (seen < need) seen = wait_part(flag_in, epoch, need, st);
                }
                issue_chunk(k + 1);
                if (x_in) flag_load_lds(flag_in, fslot_lds, lane);
            }
            float4* pub4 = (lane == 0) ? r4_out + ring_index(k * P, R) : sink4 + lane;
            F1* pub1 = (lane == 0) ? r1_out + ring_index(k * P, R) : sink1 + lane;
            // lane 63 starts the chunk with the ring's values for steps 0 and 1
            {
                const float u0D = NWA ? lane_bcast(qUD, 63) : 0.0f;
                if (NWA && lane == 63) uD = u0D;
                const float u0M = lane_bcast(qUM, 63), u0I = lane_bcast(qUI, 63);
                const float d0M = lane_bcast(qDM, 63), d0I = lane_bcast(qDI, 63),
                            d0D = lane_bcast(qDD, 63);
                const float d1M = lane_bcast(qDM, 62), d1I = lane_bcast(qDI, 62),
                            d1D = lane_bcast(qDD, 62);
                if (lane == 63) {
                    uM = u0M; uI = u0I;
                    dM = d0M; dI = d0I; dD = d0D;
                    dM2 = d1M; dI2 = d1I; dD2 = d1D;
                }
            }
            // lane 63 = step 2 of the diagonal flows (then shifted on)
            qDM = wave_shr1(wave_shr1(qDM));
            qDI = wave_shr1(wave_shr1(qDI));
            qDD = wave_shr1(wave_shr1(qDD));
            // the output quad being filled, memory-column order (step 4q + 3 - e in
            // element e)
            float4 quad = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            // (local) the betas' start terms 2^min((alpha - S) c, 0) are exactly 0 below
            // 2^-150: a chunk none of whose alphas comes within 150 c^-1 of S skips
            // those exponentials (most chunks: alpha grows towards S)
            bool inits = NWA;
            if (!NWA) {
                float amax = fmaxf(fmaxf(AM[0], AI[0]), AD[0]);
#pragma unroll
                for (int u = 1; u < P; ++u) amax = fmaxf(amax, fmaxf(fmaxf(AM[u], AI[u]), AD[u]));
                inits = __builtin_amdgcn_ballot_w64((amax - S) * c >= -151.0f) != 0;
            }
            // FULL: every cell of the chunk lies inside the element, no validity masks;
            // INIT: some cell of the chunk has a nonzero start term
            auto steps = [&](auto full, auto init) {
            constexpr bool FULL = decltype(full)::value;
            constexpr bool INIT = decltype(init)::value;
#pragma unroll
            for (int u = 0; u < P; ++u) {
                const int t = t_hi - u;
                const bool ok = FULL || (unsigned)(t - lane) < (unsigned)L2eff;
                // cells outside the element hold arbitrary tensor data: neutralise them
                const float sc = ok ? sv[u] : kNINF;
                // predecessors: left = own previous step, up / diagonal = lane r-1 (lane 0:
                // the stripe above's last row)
                const float nbM = wave_shl1(bM), nbI = wave_shl1(bI),
                            nbD = wave_shl1(bD);
                const float upM = wave_shr1_or(AM[u + 1], bM), upI = wave_shr1_or(AI[u + 1], bI);
                const float upD = NWA ? wave_shr1_or(AD[u + 1], bD) : kNINF;
                const float dgM = wave_shr1_or(AM[u + 2], nbM), dgI = wave_shr1_or(AI[u + 2], nbI),
                            dgD = wave_shr1_or(AD[u + 2], nbD);
                bM = nbM;
                bI = nbI;
                bD = nbD;
                const float lfM = AM[u + 1], lfI = AI[u + 1], lfD = AD[u + 1];
                // M: diagonal + start weights (NWA: the diagonal only)
                const float v0 = NWA ? dgM : dgM + sc, v1 = NWA ? dgI : dgI + sc,
                            v2 = NWA ? dgD : dgD + sc;
                // (local FULL: the cell's own M alpha, which the forward formed from these
                // operands as m + T ln(sum) >= m, takes the max's place: every exponent
                // is at most 0, the largest term at least 1/4, and the shift cancels in
                // the normalisation)
                const float m4 = NWA ? fmaxf(fmaxf(v0, v1), v2)
                                     : FULL ? AM[u] : fmaxf(fmaxf(v0, v1), fmaxf(v2, sc));
                const float e0 = fast_exp2((v0 - m4) * c), e1 = fast_exp2((v1 - m4) * c);
                const float e2 = fast_exp2((v2 - m4) * c);
                const float e3 = NWA ? 0.0f : fast_exp2((sc - m4) * c);
                const float esum = NWA ? (e0 + e1) + e2 : ((e0 + e1) + e2) + e3;
                // I: open from M above, extend from I above (NWA: open from D above)
                // (local: two terms, the larger one's weight exactly 1 and the other's
                // exponent -|a - b| c bit for bit, as lse2 forms them: one exponential)
                const float i0v = upM + go, i1v = upI + ge, i2v = upD + go;
                float f0, f1, f2 = 0.0f;
                if constexpr (NWA) {
                    const float mi = fmaxf(fmaxf(i0v, i1v), i2v);
                    f0 = fast_exp2((i0v - mi) * c);
                    f1 = fast_exp2((i1v - mi) * c);
                    f2 = fast_exp2((i2v - mi) * c);
                } else {
                    const float di = i0v - i1v;
                    const float fs = fast_exp2(-fabsf(di) * c);
                    f0 = di >= 0.0f ? 1.0f : fs;
                    f1 = di >= 0.0f ? fs : 1.0f;
                }
                // D: open from M left, extend from D left (NWA: open from I left)
                const float d0v = lfM + go, d1v = lfD + ge, d2v = lfI + go;
                float g0, g1, g2 = 0.0f;
                if constexpr (NWA) {
                    const float md = fmaxf(fmaxf(d0v, d1v), d2v);
                    g0 = fast_exp2((d0v - md) * c);
                    g1 = fast_exp2((d1v - md) * c);
                    g2 = fast_exp2((d2v - md) * c);
                } else {
                    const float dd = d0v - d1v;
                    const float gs = fast_exp2(-fabsf(dd) * c);
                    g0 = dd >= 0.0f ? 1.0f : gs;
                    g1 = dd >= 0.0f ? gs : 1.0f;
                }
                // betas in the reference's accumulation order (NWA: the terminal cell's
                // softmax weights over its three states start the recursion)
                float initM, initI, initD;
                if (NWA) {
                    initM = initI = initD = 0.0f;
                    if (t == term_step) {
                        const float m = fmaxf(fmaxf(AM[u], AI[u]), AD[u]);
                        const float eM = fast_exp2((AM[u] - m) * c), eI = fast_exp2((AI[u] - m) * c);
                        const float eD = fast_exp2((AD[u] - m) * c);
                        const float r = fast_rcp((eM + eI) + eD);
                        initM = eM * r;
                        initI = eI * r;
                        initD = eD * r;
                    }
                } else if (INIT) {
                    float lp;
                    lp = (AM[u] - S) * c;   // subtract first: exact for nearby values
                    initM = fast_exp2(lp < 0.0f ? lp : 0.0f);
                    lp = (AI[u] - S) * c;
                    initI = fast_exp2(lp < 0.0f ? lp : 0.0f);
                    lp = (AD[u] - S) * c;
                    initD = fast_exp2(lp < 0.0f ? lp : 0.0f);
                } else {
                    initM = initI = initD = 0.0f;
                }
                const float betaM = ((initM + dM) + lM) + uM;
                const float betaI = NWA ? ((initI + dI) + uI) + lI : (initI + dI) + uI;
                const float betaD = NWA ? ((initD + dD) + lD) + uD : (initD + dD) + lD;
                // skip inf / NaN betas like the reference (a NaN fails <= too); cells
                // outside the element; NWA: betas at most 1e-20 pass nothing (the local
                // form's betas are sums of flows >= 0, so it needs no lower test)
                auto pass = [&](float beta) {
                    return ok && (!NWA || beta > 1e-20f) && beta <= 3.0e38f;
                };
                const float brM = pass(betaM) ? betaM * fast_rcp(esum) : 0.0f;
                const float brI = pass(betaI) ? betaI * fast_rcp(NWA ? (f0 + f1) + f2 : f0 + f1)
                                              : 0.0f;
                const float brD = pass(betaD) ? betaD * fast_rcp(NWA ? (g0 + g1) + g2 : g0 + g1)
                                              : 0.0f;
                const float pv = brM * esum;
                if constexpr (QT) {
                    if ((u & 3) == 0) quad.w = pv;
                    if ((u & 3) == 1) quad.z = pv;
                    if ((u & 3) == 2) quad.y = pv;
                    if ((u & 3) == 3) {
                        quad.x = pv;
                        *reinterpret_cast<float4*>(otile + Tile::slot(lane, u >> 2)) = quad;
                    }
                } else {
                    otile[tbase + u] = pv;
                }
                p_acc += pv * sc;
                const float oUM = brI * f0, oUI = brI * f1, oUD = brI * f2;   // to (i-1, j)
                const float oLM = brD * g0, oLD = brD * g1, oLI = brD * g2;   // to (i, j-1)
                const float oDM = brM * e0, oDI = brM * e1, oDD = brM * e2;   // to (i-1, j-1)
                g_open += oUM;
                g_open += oLM;
                g_ext += oUI;
                g_ext += oLD;
                if (NWA) {
                    g_open += oUD;
                    g_open += oLI;
                    // the boundary cells' own open and extends: I[i,0] (left from column
                    // 0, diagonal from column 0 into the row above; no FULL chunk has a
                    // column 0) and D[0,j] (up and diagonal flows of the first row)
                    const int col = t - lane;
                    if (!FULL && col == 0) {
                        g_open += oLI + oDI;
                        g_ext += oLI * ext_left + oDI * ext_diag;
                    }
                    if (top) {
                        g_open += oUD + oDD;
                        g_ext += oUD * (float)col + oDD * (float)(col - 1);
                    }
                }
                pub4[u] = make_float4(oUM, oUI, oDM, oDI);
                if constexpr (NWA) pub1[u] = make_float2(oDD, oUD);
                else pub1[u] = oDD;
                // successor contributions for the next steps; lane 63 takes the ring
                qUM = wave_shr1(qUM);
                qUI = wave_shr1(qUI);
                lM = oLM;
                lD = oLD;
                uM = wave_shl1_or(oUM, qUM);
                uI = wave_shl1_or(oUI, qUI);
                if (NWA) {
                    qUD = wave_shr1(qUD);
                    lI = oLI;
                    uD = wave_shl1_or(oUD, qUD);
                }
                dM = dM2;
                dI = dI2;
                dD = dD2;
                dM2 = wave_shl1_or(oDM, qDM);
                dI2 = wave_shl1_or(oDI, qDI);
                dD2 = wave_shl1_or(oDD, qDD);
                qDM = wave_shr1(qDM);
                qDI = wave_shr1(qDI);
                qDD = wave_shr1(qDD);
            }
            };
            if (i0 + 63 < L1 && t_hi - P - 62 >= (NWA ? 1 : 0) && t_hi < L2) {
                if (inits) steps(std::true_type{}, std::true_type{});
                else steps(std::true_type{}, std::false_type{});
            } else {
                if (inits) steps(std::false_type{}, std::true_type{});
                else steps(std::false_type{}, std::false_type{});
            }
            wave_lds_sync();
            if constexpr (HELP)
                ;   // the helper writes the tile out once this chunk is published
            else if constexpr (QT)
                write_quads<P, -1>(otile, pbase, trash, i0, L1, L2, L1max, L2max, lane, t_hi);
            else
                write_tile<P, -1>(otile, pbase, trash, i0, L1, L2, L1max, L2max, lane, t_hi);
            publish(prog, wave, q * PROG_STRIDE + k + 1);
            if (x_out) {
                // this chunk's flows to the part above, by producer step
                if (lane < P) {
                    const int slot = ring_index(k * P, R) + lane;
                    store_sys4(flows4 + fo + k * P + lane, r4_out[slot]);
                    if constexpr (NWA) store_sys2(flowsF + fo + k * P + lane, r1_out[slot]);
                    else store_sys(flows1 + fo + k * P + lane, r1_out[slot]);
                }
                if (HELP && !x_in && k >= 1) {
                    // HELP, a part's last stripe that is not also its first: after the
                    // flow stores of chunk k - 1 it issued only that chunk's flag store
                    // (from chunk 1 on), the 3 rows-above loads of chunk k + 1 (when
                    // there is one) and this chunk's 2 flow stores; once at most those
                    // are outstanding, every chunk before this one is complete
                    const bool more = k + 1 < nch;
                    if (k >= 2 && more) wait_vmcnt<6>();
                    else if (more) wait_vmcnt<5>();
                    else if (k >= 2) wait_vmcnt<3>();
                    else wait_vmcnt<2>();
                    if (lane == 0) store_flag(flag_out, progress_word(epoch, k));
                } else if (k >= 2) {
                    // at least NQ + 3P/4 + 3 loads, 2 NQ marginal stores and 4 flow stores
                    // (HELP: the 3 rows-above loads issued in chunk k - 1 and 4 flow
                    // stores) follow the flow stores of chunk k - 2: those are complete
                    if constexpr (HELP) wait_vmcnt<7>();
                    else wait_vmcnt<3 * NQ + 3 * P / 4 + 7>();
                    if (lane == 0) store_flag(flag_out, progress_word(epoch, k - 1));
                }
            }
        }
        if (x_out) {
            wait_vmcnt<0>();
            if (lane == 0) store_flag(flag_out, progress_word(epoch, nch));
        }
    }

    g_open = wave_sum(g_open);
    g_ext = wave_sum(g_ext);
    p_acc = wave_sum(p_acc);
    if (lane == 0) { red_o[wave] = g_open; red_e[wave] = g_ext; red_p[wave] = p_acc; }
    __syncthreads();
    if (threadIdx.x == 0) {
        float go_s = 0.0f, ge_s = 0.0f, p = 0.0f;
        for (int w = 0; w < NW; ++w) { go_s += red_o[w]; ge_s += red_e[w]; p += red_p[w]; }
        if (NWA && NS == 0 && part == 0 && L1 + L2 > 0) {
            // an element without cells is its boundary cell: one open, L - 1 extends
            go_s += 1.0f;
            ge_s += (float)(L1 + L2 - 1);
        }
        if (G == 1) {
            grad_open[b] = go_s;
            grad_ext[b] = ge_s;
            grad_T[b] = (S - (p + (go_s * go + ge_s * ge))) / T;
        } else {
            double* bp = bpart + ((size_t)b * G + part) * 4;
            bp[0] = go_s;
            bp[1] = ge_s;
            bp[2] = p;
        }
    }
}

// grad_open[b], grad_ext[b], grad_T[b] of a split element from the parts' sums.
__global__ void swa_grad_merge(const double* __restrict__ bpart, const float* __restrict__ partition,
                               float* __restrict__ grad_open, float* __restrict__ grad_ext,
                               float* __restrict__ grad_T, int B, int G, float go, float ge,
                               float T) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    float go_s = 0.0f, ge_s = 0.0f, p = 0.0f;
    for (int i = 0; i < G; ++i) {
        const double* bp = bpart + ((size_t)b * G + i) * 4;
        go_s += (float)bp[0];
        ge_s += (float)bp[1];
        p += (float)bp[2];
    }
    grad_open[b] = go_s;
    grad_ext[b] = ge_s;
    grad_T[b] = (partition[b] - (p + (go_s * go + ge_s * ge))) / T;
}

}  // namespace swa
}  // namespace d2p_amd

namespace d2p_amd {
namespace swa {

namespace {
// dynamic LDS bound: 160 KiB less the kernels' static arrays (progress words,
// reductions, the prefetched progress-word slot)
constexpr size_t kLdsLimit = 160 * 1024 - 512;

// LDS of one workgroup whose stripe boundaries use rings of R columns
size_t lds_forward_r(int R) {
    return (size_t)NW * (2 * 64 * PF + 2 * 3 * 64) * sizeof(float) +
           ((size_t)NW * R + NW * DUMMY) * sizeof(float4);
}
size_t lds_backward_r(int R, bool nwa) {
    const size_t tile = (nwa ? 65 : 64) * PB;   // dword or quad tiles
    const size_t wfloats = tile + 3 * PB * 64 + 3 * 64 + tile + 2 * 64;
    const size_t f1 = nwa ? sizeof(float2) : sizeof(float);
    return (size_t)NW * wfloats * sizeof(float) + (size_t)NW * R * (sizeof(float4) + f1) +
           (size_t)NW * (64 + PB) * (sizeof(float4) + f1);
}
int ring_forward(int rows, int max_L2) { return ring_len(rows, max_L2, 256); }
int ring_backward(int rows, int max_L2) { return ring_len(rows, max_L2, 128); }

// Stripes per part that a launch may not exceed: 0 when the rings of an unsplit
// element fit in LDS, else NW (the minimum rings of such parts always fit).
int max_stripes_forward(int max_L1, int max_L2) {
    return lds_forward_r(ring_forward(max_L1, max_L2)) <= kLdsLimit ? 0 : NW;
}
int max_stripes_backward(int max_L1, int max_L2, bool nwa) {
    return lds_backward_r(ring_backward(max_L1, max_L2), nwa) <= kLdsLimit ? 0 : NW;
}
}  // namespace

int check_shape(int B, int max_L1, int max_L2, float temperature) {
    D2P_REQUIRE(B >= 0 && max_L1 >= 0 && max_L2 >= 0, "negative dimension");
    D2P_REQUIRE(temperature > 0.0f, "temperature must be positive");
    D2P_REQUIRE(wf::table_fits_int32(max_L1, max_L2),
                "DP table too large: (max_L1 + 1) * (max_L2 + 1) exceeds 2147483647");
    D2P_REQUIRE(max_L2 <= wf::MAX_L2, "max_L2 exceeds 262080 (the stripe pipeline's limit)");
    D2P_REQUIRE(max_L1 <= wf::MAX_L1, "max_L1 exceeds 2097088 (the stripe pipeline's limit)");
    // rings that do not fit for an unsplit element force parts of at most NW
    // stripes, whose minimum rings fit whatever the row length
    return D2P_OK;
}

// The affine layout's flows area: a float4 plane, then a float plane (global
// alignment: a float2 plane), of ws.flow_slots entries each.
constexpr int kFlowBytes = sizeof(float4) + sizeof(float2);

Layout affine_layout(void* workspace, int B, int max_L1, int max_L2, bool split) {
    return layout(workspace, B, max_L1, max_L2, 3, split, kFlowBytes);
}

static bool helpers_enabled();

int launch_forward(const float* scores, const int* lengths, int B, int max_L1, int max_L2,
                   float go, float ge, float T, const Layout& ws, float* partition,
                   hipStream_t st, bool nwa) {
    const int ns = (max_L1 + 63) / 64;
    const Split sp = choose_split(B, max_L1, ws, max_stripes_forward(max_L1, max_L2));
    const int R = ring_forward(sp.G > 1 ? sp.SPW * 64 : max_L1, max_L2);
    size_t lds = lds_forward_r(R);
    D2P_REQUIRE(lds <= kLdsLimit, "sequence too long for the LDS stripe rings");
    if (sp.G > 1 && launch_split_reset(ws, B, sp.G, st) != D2P_OK) return D2P_ERR_HIP;
    // helper waves (local form, parts of at most NW/2 stripes) need the odd chunks' M
    // and I tiles after the rings: NW/2 x 2P x 64 floats
    const int part_stripes = sp.G > 1 ? sp.SPW : ns;
    const size_t lds_help = lds + (size_t)(NW / 2) * 2 * PF * 64 * sizeof(float);
    const bool help =
        !nwa && part_stripes <= NW / 2 && lds_help <= kLdsLimit && helpers_enabled();
    if (help) lds = lds_help;
    auto kern = nwa ? swa_forward_kernel<true>
                    : (help ? swa_forward_kernel<false, true> : swa_forward_kernel<false, false>);
    D2P_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds));
    D2P_LAUNCH(nwa ? "nwa_forward" : "swa_forward", kern, dim3(split_grid(B, sp.G)),
               dim3(NW * 64), lds, st, scores, lengths, ws.alpha_sk, ws.brow, partition,
               ws.status, ws.fflag, ws.fpart, B, max_L1, max_L2, ns, go, ge, T, R, sp.G, sp.SPW,
               next_epoch());
    // global alignment: the part owning the terminal cell writes the value itself
    if (!nwa && sp.G > 1 && launch_partition_merge(ws, partition, B, sp.G, T, st) != D2P_OK)
        return D2P_ERR_HIP;
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

// D2P_AMD_SW_HELPERS=0 turns the helper waves off (for tests: both forms must agree)
static bool helpers_enabled() {
    const char* e = std::getenv("D2P_AMD_SW_HELPERS");
    return !(e && e[0] == '0');
}

int launch_backward(const float* scores, const int* lengths, int B, int max_L1, int max_L2,
                    float go, float ge, float T, const Layout& ws, const float* partition,
                    float* marginals, float* grad_open, float* grad_ext, float* grad_T,
                    hipStream_t st, bool nwa) {
    const int ns = (max_L1 + 63) / 64;
    const Split sp = choose_split(B, max_L1, ws, max_stripes_backward(max_L1, max_L2, nwa));
    const int R = ring_backward(sp.G > 1 ? sp.SPW * 64 : max_L1, max_L2);
    const size_t lds = lds_backward_r(R, nwa);
    D2P_REQUIRE(lds <= kLdsLimit, "sequence too long for the LDS stripe rings");
    float4* flows4 = reinterpret_cast<float4*>(ws.flows);
    float* flows1 = sp.G > 1 ? reinterpret_cast<float*>(flows4 + ws.flow_slots) : nullptr;
    if (sp.G > 1) D2P_TRY(launch_flag_reset(ws.bflag, B * sp.G, st));
    auto kern = nwa ? swa_backward_kernel<true> : swa_backward_kernel<false>;
    // helper waves move the data when a part has at most NW/2 stripes (the others idle)
    const int part_stripes = sp.G > 1 ? sp.SPW : ns;
    if (!nwa && part_stripes <= NW / 2 && helpers_enabled()) kern = swa_backward_kernel<false, true>;
    D2P_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds));
    D2P_LAUNCH(nwa ? "nwa_backward" : "swa_backward", kern, dim3(split_grid(B, sp.G)),
               dim3(NW * 64), lds, st, scores, lengths, ws.alpha_sk, ws.brow, partition,
               marginals, grad_open, grad_ext, grad_T, ws.status, ws.trash, ws.bflag, flows4,
               flows1, ws.bpart, B, max_L1, max_L2, ns, go, ge, T, R, sp.G, sp.SPW, next_epoch());
    if (sp.G > 1)
        D2P_LAUNCH("swa_grad_merge", swa_grad_merge, dim3((B + 255) / 256), dim3(256), 0, st,
                   ws.bpart, partition, grad_open, grad_ext, grad_T, B, sp.G, go, ge, T);
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

}  // namespace swa
}  // namespace d2p_amd

using namespace d2p_amd;

extern "C" size_t d2p_swa_workspace_bytes(int B, int max_L1, int max_L2) {
    if (B <= 0 || max_L1 < 0 || max_L2 < 0) return 0;
    // status words | trash line | skewed (M, I, D) tables | last rows of every stripe |
    // split-element progress words, boundary flows and partial sums
    return swa::affine_layout(nullptr, B, max_L1, max_L2, true).bytes;
}

namespace {
int affine_forward_marginals(const float* scores, const int* lengths, int B, int max_L1,
                             int max_L2, float gap_open, float gap_ext, float temperature,
                             float* value, float* marginals, float* grad_open, float* grad_ext,
                             float* grad_T, void* workspace, size_t workspace_bytes,
                             void* stream, bool nwa) {
    const int rc = swa::check_shape(B, max_L1, max_L2, temperature);
    if (rc != D2P_OK) return rc;
    if (B == 0) return D2P_OK;
    D2P_REQUIRE(scores && value && marginals && grad_open && grad_ext && grad_T,
                "null pointer argument");
    const size_t need = d2p_swa_workspace_bytes(B, max_L1, max_L2);
    D2P_REQUIRE(workspace && workspace_bytes >= need, "workspace too small");
    hipStream_t st = (hipStream_t)stream;
    const wf::Layout ws = swa::affine_layout(workspace, B, max_L1, max_L2, true);
    D2P_TRY(swa::launch_forward(scores, lengths, B, max_L1, max_L2, gap_open, gap_ext,
                                temperature, ws, value, st, nwa));
    D2P_TRY(swa::launch_backward(scores, lengths, B, max_L1, max_L2, gap_open, gap_ext,
                                 temperature, ws, value, marginals, grad_open, grad_ext, grad_T,
                                 st, nwa));
    return wf::launch_poison(ws.status, B, (long long)max_L1 * max_L2, marginals, nullptr,
                             value, grad_open, grad_ext, grad_T, st);
}
}  // namespace

extern "C" int d2p_swa_forward_marginals(const float* scores, const int* lengths, int B,
                                         int max_L1, int max_L2, float gap_open, float gap_ext,
                                         float temperature, float* partition, float* marginals,
                                         float* grad_open, float* grad_ext, float* grad_T,
                                         void* workspace, size_t workspace_bytes, void* stream) {
    return affine_forward_marginals(scores, lengths, B, max_L1, max_L2, gap_open, gap_ext,
                                    temperature, partition, marginals, grad_open, grad_ext,
                                    grad_T, workspace, workspace_bytes, stream, false);
}

extern "C" size_t d2p_nwa_workspace_bytes(int B, int max_L1, int max_L2) {
    return d2p_swa_workspace_bytes(B, max_L1, max_L2);
}

extern "C" int d2p_nwa_forward_marginals(const float* scores, const int* lengths, int B,
                                         int max_L1, int max_L2, float gap_open, float gap_ext,
                                         float temperature, float* value, float* marginals,
                                         float* grad_open, float* grad_ext, float* grad_T,
                                         void* workspace, size_t workspace_bytes, void* stream) {
    return affine_forward_marginals(scores, lengths, B, max_L1, max_L2, gap_open, gap_ext,
                                    temperature, value, marginals, grad_open, grad_ext, grad_T,
                                    workspace, workspace_bytes, stream, true);
}
