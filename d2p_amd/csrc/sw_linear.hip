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

#include <atomic>
#include <cstdlib>
#include <mutex>
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
constexpr int PR = 16;               // steps per chunk of the reverse sweeps that recompute

// One cell of the forward recurrence from its neighbours' alphas and its score: the LSE
// of the diagonal, up and left candidates and (SW) the sky term.  The forward sweep and
// the reverse sweep's recomputation of alpha from checkpoints both call this, so they
// produce the same bits.  RAWMAX: the max without canonicalising the score (the same
// value for every non-NaN input).
template <bool NWG, bool RAWMAX>
__device__ __forceinline__ float fwd_cell_e(float diag, float up, float cur, float sc, float gap,
                                            float c, float tl, float (&e)[4], float& sum) {
    // out-of-table neighbours are NINF, so no i>1 / j>1 guards are needed
    const float vd = diag + sc;
    const float vu = up + gap;
    const float vl = cur + gap;
    // exponents (v - m) / T with the subtraction first, as the reference: an fma
    // against a rounded m*c would add the rounding of m*c to alpha itself (about an
    // ulp), which the temperature Jacobians' (alpha - S) / T^2 terms amplify
    if (NWG) {
        const float m = fmaxf(fmaxf(vd, vu), vl);
        e[0] = fast_exp2((vd - m) * c);
        e[1] = fast_exp2((vu - m) * c);
        e[2] = fast_exp2((vl - m) * c);
        e[3] = 0.0f;
        sum = (e[0] + e[1]) + e[2];
        return fmaf(tl, fast_log2(sum), m);
    } else {
        const float m = RAWMAX ? max4_raw(vd, vu, vl, sc) : fmaxf(fmaxf(vd, vu), fmaxf(vl, sc));
        e[0] = fast_exp2((vd - m) * c);
        e[1] = fast_exp2((vu - m) * c);
        e[2] = fast_exp2((vl - m) * c);
        e[3] = fast_exp2((sc - m) * c);
        sum = (e[0] + e[1]) + (e[2] + e[3]);
        return fmaf(tl, fast_log2(sum), m);
    }
}
template <bool NWG, bool RAWMAX>
__device__ __forceinline__ float fwd_cell(float diag, float up, float cur, float sc, float gap,
                                          float c, float tl) {
    float e[4], sum;
    return fwd_cell_e<NWG, RAWMAX>(diag, up, cur, sc, gap, c, tl, e, sum);
}
// fwd_cell and the cell's tangent x along a direction v (the HVP's forward tangent,
// /root/reference/src/sw/kernels_cpu.cpp:279-477): the candidates' tangents
// (x_diag + v, x_up, x_left, v) weighted by the softmax weights of the same exponentials.
template <bool NWG, bool RAWMAX>
__device__ __forceinline__ float fwd_cell_tan(float diag, float up, float cur, float sc,
                                              float gap, float c, float tl, float td, float tu,
                                              float tc, float v, float& x) {
    float e[4], sum;
    const float a = fwd_cell_e<NWG, RAWMAX>(diag, up, cur, sc, gap, c, tl, e, sum);
    // (explicit fmas: the same bits in every instantiation)
    const float n2 = fmaf(e[2], tc, fmaf(e[1], tu, e[0] * (td + v)));
    const float num = NWG ? n2 : fmaf(e[3], v, n2);
    x = num * fast_rcp(sum);
    return a;
}

// Checkpoint steps of a stripe of nsteps steps for reverse sweeps of PR-step chunks that
// recompute alpha: chunk k (its highest step t_hi = nsteps - 1 - PR*k) rebuilds steps
// t_hi - PR - 1 .. t_hi - 2 from the stored steps t_hi - PR - 2 and t_hi - PR - 3,
// i.e. the steps congruent to nsteps - 3 and nsteps - 4 modulo PR; the first chunk also
// starts from the last two steps.  A forward in checkpoint mode stores only these.
__device__ __forceinline__ bool ckpt_step(int t, int nsteps) {
    const int d = (nsteps - 3 - t) & (PR - 1);
    return d == 0 || d == PR - 1 || t >= nsteps - 2;
}

// One part (G > 1: a workgroup owns stripes [part*SPW, part*SPW + SPW) of its element;
// G == 1: all of them).  The first stripe of a part > 0 reads the last row of the
// previous part's last stripe from `brow` (device-coherent loads, one chunk ahead)
// after that part's progress word allows it; the last stripe of a part publishes its
// own word two chunks behind its stores.  G == 1 writes the partition; G > 1 writes
// the part's (max, scaled sum) for the partition merge.
//
// NWG: global alignment (soft Needleman-Wunsch, /root/reference/src/nw/kernels_cpu.cpp:
// 78-154): no sky term, row 0 and column 0 hold j*gap and i*gap (the cells left of
// column 0 carry their row's i*gap, so the left and diagonal neighbours of column 0
// come out of the same registers), and `partition` receives the terminal cell
// alpha[L1, L2] instead of the LSE over all cells.
//
// HELP (parts of at most NW/2 stripes): wave NW/2 + l moves stripe l's data, so the
// sweeping wave only sweeps.  It loads each chunk's score quads one chunk ahead
// (publishing hprog[l] = chunks loaded), and writes a chunk's alpha rows (which the
// sweeping wave leaves in the helper's own, otherwise unused, tile buffers) to the
// table as one contiguous 4 KB block once wave l has finished the chunk (prog[l]).
//
// TAN (not WIDE): the HVP's forward tangent sweep in the same pass
// (/root/reference/src/sw/kernels_cpu.cpp:279-477): each cell also takes its tangent
// along the direction V from the forward's own softmax weights (fwd_cell_tan), writes
// it to tan_sk / tan_brow as the tangent sweep does, passes it across stripes through a
// second ring, and folds it into the value's tangent dS = sum_cells p_cell x_cell with
// the partition's own weights (OnlineLSEDot: no second pass for the cell
// probabilities, which need S).  G > 1 writes the part's sum beside its (max, sum).
// The direction's quads come with the scores (a second tile per chunk), the tangent
// rows leave with the alpha rows (a second tile in the helper's buffer).
struct TanArgs {
    const float* V;
    float* tan_sk;
    float* tan_brow;
    float* sdot;      // [B]: the value's tangent (G == 1)
    float* wpart;     // [B][G]: a part's tangent sum at its (max, sum) scale (G > 1)
};
template <bool NWG = false, bool HELP = false, bool WIDE = false, bool TAN = false>
__global__ void __launch_bounds__(WIDE ? 2 * NW * 64 : NW * 64)
sw_forward_kernel(const float* __restrict__ scores, const int* __restrict__ lengths,
                  float* __restrict__ alpha_sk, float* __restrict__ brow,
                  float* __restrict__ partition, int* __restrict__ status,
                  uint64_t* __restrict__ fflag, float2* __restrict__ fpart, int B, int L1max,
                  int L2max, int NSmax, float gap, float T, int R, int G, int SPW,
                  uint32_t epoch, int ckpt, TanArgs ta) {
    constexpr int P = PF;
    static_assert(PF == PR, "checkpoint rows are chosen per forward chunk");
    static_assert(!(TAN && WIDE), "the tangent sweep has no 16-wave form");
    extern __shared__ __align__(16) float smem[];
    __shared__ int prog[NW];
    __shared__ int hprog[NW];     // HELP: chunks of stripe l loaded by its helper
    __shared__ float red_m[NW], red_z[NW], red_w[NW];
    __shared__ float terminal;   // NWG: alpha[L1, L2]
    __shared__ float tterm;      // NWG, TAN: its tangent
    int b, part;
    split_decode(blockIdx.x, G, b, part);
    if (b >= B) return;
    const int lane = threadIdx.x & 63;
    const unsigned ul4 = (unsigned)lane * 4u;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    using Tile = QuadTile<P>;
    // score tiles per sweeping wave: chunk k uses tile k % NTB (WIDE: four, so that the
    // helper can load three chunks ahead)
    constexpr int NTB = WIDE ? 4 : 2;
    constexpr int NTL = TAN ? 2 : 1;   // tiles per chunk: scores (TAN: and the direction)
    // score chunks (TAN: then the direction's), two boundary rows (TAN: then two of the
    // tangent), pad
    constexpr int WBUF = NTL * (NTB * Tile::FLOATS + 2 * 64) + P;
    float* tiles = smem + wave * WBUF;                     // the score chunks
    float* rbufs = tiles + NTL * NTB * Tile::FLOATS;       // boundary row of a chunk
    __shared__ float fslot[64];   // progress word prefetched by wave 0, the only wave whose
                                  // stripe borders another part
    const uint32_t fslot_lds = lds_address(fslot);
    float* rings = smem + NW * WBUF;                       // [NW][R] (TAN: twice)
    float* trings = rings + NW * R;                        // TAN: the tangent's
    float* sink = rings + NTL * NW * R + wave * DUMMY;     // per-wave write sink
    int* st = status + b;

    if (lane == 0 && wave < NW) {
        prog[wave] = -1;
        hprog[wave] = -1;
    }
    if (G == 1 && threadIdx.x == 0) *st = 0;               // G > 1: reset before the launch
    if (NWG && threadIdx.x == 0) {
        terminal = kNINF;
        tterm = 0.0f;
    }
    __syncthreads();

    const int L1 = lengths ? min(max(lengths[2 * b], 0), L1max) : L1max;
    const int L2 = lengths ? min(max(lengths[2 * b + 1], 0), L2max) : L2max;
    const float c = kLog2e / T;
    const float tl = T * kLn2;
    const int NS = L2 > 0 ? (L1 + 63) >> 6 : 0;
    const int nsteps = L2 + 63;
    const int nch = (nsteps + P - 1) / P;
    const size_t NT = (size_t)stored_steps(L2max);
    const float* sbase = scores + (size_t)b * L1max * L2max;
    const float* vbase = TAN ? ta.V + (size_t)b * L1max * L2max : nullptr;
    const int s_begin = part * SPW;
    const int NL = max(min(NS, s_begin + SPW) - s_begin, 0);   // stripes of this part
    const bool has_next = s_begin + NL < NS;
    const uint64_t* flag_in = fflag + (size_t)b * G + (part > 0 ? part - 1 : 0);
    uint64_t* flag_out = fflag + (size_t)b * G + part;

    // the partition (TAN: and the tangent sum at its scale)
    typename std::conditional<TAN, OnlineLSEDot, OnlineLSE>::type acc;
    acc.init_open();

    if constexpr (HELP) {
        // helpers: waves HB..HB+NL-1 (WIDE: a second set of NW waves)
        constexpr int HB = WIDE ? NW : NW / 2;
        if (NL > HB) {   // never: the host picks HELP for parts of at most HB stripes
            if (threadIdx.x == 0) atomicOr(st, 2);
            return;
        }
        const int l = wave - HB;
        if (l >= 0 && l < NL) {
            const int i0 = (s_begin + l) * 64;
            float* out = alpha_sk + (((size_t)b * NSmax + s_begin + l) * NT + APAD) * 64;
            const uint32_t ltiles = lds_address(smem + l * WBUF);   // wave l's score tiles
            // its alpha tiles: this wave's own buffers, or (WIDE: no LDS for those) its
            // score tiles, once their scores are in wave l's registers
            const float* atiles = smem + (WIDE ? l : wave) * WBUF;
            // TAN: the direction's tiles follow the score tiles, the tangent's the alpha
            // tiles
            auto load = [&](int k) {
                dma_quads<P, 1>(ltiles + (k & (NTB - 1)) * Tile::FLOATS * 4, sbase, i0, L1max,
                                L2max, lane, k * P);
                if (TAN)
                    dma_quads<P, 1>(ltiles + (NTB + (k & (NTB - 1))) * Tile::FLOATS * 4, vbase,
                                    i0, L1max, L2max, lane, k * P);
            };
            // the stripe's last row (lane 63 of wave l) by step, from its ring, for the
            // reverse sweep; a part's last stripe with a next part stores its own (its
            // progress word must follow those stores).  The ring slots of chunk k are
            // rewritten R / P chunks later; wave l cannot run that far ahead of this
            // wave, whose loads it waits for.
            const bool l_x_out = l == NL - 1 && has_next;
            float* hbrow = brow + ((size_t)b * NSmax + s_begin + l) * NT;
            const float* hring = ring_of(smem + NW * WBUF, l, R);
            float* htbrow = TAN ? ta.tan_brow + ((size_t)b * NSmax + s_begin + l) * NT : nullptr;
            const float* htring = ring_of(smem + NW * WBUF + NW * R, l, R);
            auto store_row = [&](int k) {
                if (!l_x_out && lane < P) {
                    const int t0 = k * P;
                    lane_store(hbrow, (unsigned)(t0 + lane) * 4u, hring[(t0 % R) + lane]);
                    if (TAN)
                        lane_store(htbrow, (unsigned)(t0 + lane) * 4u, htring[(t0 % R) + lane]);
                }
            };
            float* tout = TAN ? ta.tan_sk + (((size_t)b * NSmax + s_begin + l) * NT + APAD) * 64
                              : nullptr;
            // the chunk's alpha rows (alpha tile k % NTB) to the table: Tile::NQ stores
            // (TAN: and as many for the tangent rows)
            // The partition of stripe l (TAN: with the tangent sum), from the chunk's alpha
            // tile: lane r takes its own row's P alphas (column r of the tile) and runs
            // the block update the sweeping wave would run, with the same running max,
            // so the lane states are the same bit for bit; the sweeping wave's chain is
            // spared the P exponentials per chunk.
            float hbm = -1e20f;   // the running max of lane r's alphas
            auto partition_block = [&](int k) {
                if constexpr (!NWG) {
                    const float* at = atiles + (k & (NTB - 1)) * Tile::FLOATS + lane;
                    float av[P], xv[P];
#pragma unroll
                    for (int u = 0; u < P; ++u) {
                        av[u] = at[u * 64];
                        if (TAN) xv[u] = at[NTB * Tile::FLOATS + u * 64];
                    }
#pragma unroll
                    for (int u = 0; u < P; ++u) hbm = fmaxf(hbm, av[u]);
                    if constexpr (TAN) acc.template add_block_max<P>(av, xv, hbm, c);
                    else acc.template add_block_max<P>(av, hbm, c);
                }
            };
            auto store_alpha = [&](int k) {
                const float* at = atiles + (k & (NTB - 1)) * Tile::FLOATS;
                float* dst = out + (size_t)k * P * 64;
                if (TAN) {
                    const float* tt = at + NTB * Tile::FLOATS;
                    float* tdst = tout + (size_t)k * P * 64;
#pragma unroll
                    for (int i = 0; i < Tile::NQ; ++i) {
                        const float4 v =
                            *reinterpret_cast<const float4*>(tt + 256 * i + 4 * lane);
                        *reinterpret_cast<float4*>(tdst + 256 * i + 4 * lane) = v;
                    }
                }
                if (!TAN && ckpt) {
                    // checkpoint mode: only the rows a recomputing reverse sweep starts
                    // from (ckpt_step): the chunk's steps congruent to nsteps - 3 and
                    // nsteps - 4 modulo PR, and the stripe's last two steps where they
                    // lie in this chunk (else the first two again).  Tile::NQ stores,
                    // as the full write-out issues: the load waits count on it.
                    const int t0 = k * P;
                    const int u0 = (nsteps - 4 - t0) & (PR - 1);
                    const int u1 = (nsteps - 3 - t0) & (PR - 1);
                    const int u2 = (unsigned)(nsteps - 2 - t0) < (unsigned)P ? nsteps - 2 - t0 : u0;
                    const int u3 = (unsigned)(nsteps - 1 - t0) < (unsigned)P ? nsteps - 1 - t0 : u1;
                    static_assert(Tile::NQ == 4, "four checkpoint stores per chunk");
                    const float v0 = at[u0 * 64 + lane], v1 = at[u1 * 64 + lane];
                    const float v2 = at[u2 * 64 + lane], v3 = at[u3 * 64 + lane];
                    dst[u0 * 64 + lane] = v0;
                    dst[u1 * 64 + lane] = v1;
                    dst[u2 * 64 + lane] = v2;
                    dst[u3 * 64 + lane] = v3;
                } else {
#pragma unroll
                    for (int i = 0; i < Tile::NQ; ++i) {
                        const float4 v =
                            *reinterpret_cast<const float4*>(at + 256 * i + 4 * lane);
                        *reinterpret_cast<float4*>(dst + 256 * i + 4 * lane) = v;
                    }
                }
            };
            if constexpr (WIDE) {
                // Chunk k's alpha rows lie over its score tile once wave l has read the
                // scores.  Iteration k starts once wave l has finished chunk k - 1 and
                // that chunk's rows have left, so its tile takes chunk k + 3: every load
                // has about three chunks of time.  (nch >= 4: nsteps = L2 + 63.)
                load(0);
                load(1);
                load(2);
                wait_vmcnt<2 * Tile::NQ>();   // chunk 0 (at least 2 NQ loads follow)
                publish(hprog, l, 1);
                wait_vmcnt<Tile::NQ>();
                publish(hprog, l, 2);
                for (int k = 0; k < nch; ++k) {
                    const bool more = k + 3 < nch;
                    if (more) load(k + 3);
                    wait_for(prog, l, l * PROG_STRIDE + k + 1, st);
                    store_alpha(k);
                    store_row(k);
                    partition_block(k);
                    if (k + 2 < nch) {
                        // chunk k + 2's loads (issued at iteration k - 1, or before the
                        // loop) are followed by chunk k - 1's alpha stores (k >= 1),
                        // chunk k + 3's loads (more) and chunk k's alpha stores
                        if (k >= 1 && more) wait_vmcnt<3 * Tile::NQ>();
                        else if (k >= 1 || more) wait_vmcnt<2 * Tile::NQ>();
                        else wait_vmcnt<Tile::NQ>();
                        publish(hprog, l, k + 3);   // also completes this wave's LDS reads
                    }
                }
            } else if (nch > 0) {
                load(0);
                wait_vmcnt<0>();
                publish(hprog, l, 1);
                if (nch > 1) load(1);
                for (int k = 0; k < nch; ++k) {
                    if (k + 1 < nch) {
                        // chunk k + 1's loads: the last issued at k = 0, else followed by
                        // the P/4 alpha stores of chunk k - 1 (TAN: and P/4 tangent stores)
                        if (k == 0) wait_vmcnt<0>(); else wait_vmcnt<NTL * Tile::NQ>();
                        publish(hprog, l, k + 2);   // also completes this wave's LDS reads
                    }
                    // once wave l has finished chunk k, its score tile k & 1 takes chunk
                    // k + 2 and its alpha rows (alpha tile k & 1) go to the table
                    wait_for(prog, l, l * PROG_STRIDE + k + 1, st);
                    if (k + 2 < nch) load(k + 2);
                    store_alpha(k);
                    store_row(k);
                    partition_block(k);
                }
            }
        }
    }

    for (int l = wave; l < NL; l += NW) {
        const int s = s_begin + l;
        set_pipeline_priority(l % NW);
        const int i0 = s * 64;
        const int L2eff = (i0 + lane < L1) ? L2 : 0;   // rows past L1 are never valid
        const float* ring_in = ring_from(rings, l, R);
        float* ring_out = ring_of(rings, l, R);
        // wave-uniform base (step 0) + 32-bit lane offset: scalar-base stores
        float* out = alpha_sk + (((size_t)b * NSmax + s) * NT + APAD) * 64;
        float* brow_s = brow + ((size_t)b * NSmax + s) * NT;   // last row, by step
        const float* brow_up = brow + ((size_t)b * NSmax + (s > 0 ? s - 1 : 0)) * NT;
        const bool x_in = l == 0 && part > 0;      // row above from the previous part
        const bool x_out = l == NL - 1 && has_next;  // last row feeds the next part
        // the cells left of column 0: NINF, or (NWG) the row's boundary i*gap
        const float left0 = NWG ? (float)(i0 + lane + 1) * gap : kNINF;
        const bool last_row = NWG && i0 + lane == L1 - 1;
        // TAN: the tangent table, last rows and ring (the boundary's tangents are 0)
        float* tout = TAN ? ta.tan_sk + (((size_t)b * NSmax + s) * NT + APAD) * 64 : nullptr;
        float* tb_s = TAN ? ta.tan_brow + ((size_t)b * NSmax + s) * NT : nullptr;
        const float* tb_up =
            TAN ? ta.tan_brow + ((size_t)b * NSmax + (s > 0 ? s - 1 : 0)) * NT : nullptr;
        const float* tring_in = ring_from(trings, l, R);
        float* tring_out = ring_of(trings, l, R);
#pragma unroll
        for (int t = -APAD; t < 0; ++t) {
            lane_store(out + t * 64, ul4, left0);
            if (TAN) lane_store(tout + t * 64, ul4, 0.0f);
        }
        wave_lds_sync();   // the previous stripe's tile reads are complete
        const uint32_t tile_lds = lds_address(tiles);
        const uint32_t row_lds = lds_address(rbufs);
        // the boundary row of chunk k: lane j < P carries the step kP + 63 + j (TAN: its
        // tangents too, two buffers on)
        auto issue_row = [&](int k) {
            uint32_t off = (uint32_t)min(k * P + 63 + min(lane, P - 1), nsteps - 1) * 4u;
            uint32_t dst = row_lds + (uint32_t)((k & 1) * 64 * 4);
            lds_dma_dword_sys<0>(brow_up, off, dst, 0u);
            if (TAN) {
                uint32_t tdst = dst + 2 * 64 * 4;
                lds_dma_dword_sys<0>(tb_up, off, tdst, 0u);
            }
        };
        // plain form: chunk k's score (TAN: and direction) tiles, by this wave
        auto issue_tiles = [&](int k) {
            const uint32_t base = tile_lds + (uint32_t)((k & 1) * Tile::FLOATS * 4);
            dma_quads<P, 1>(base, sbase, i0, L1max, L2max, lane, k * P);
            if (TAN)
                dma_quads<P, 1>(base + NTB * Tile::FLOATS * 4, vbase, i0, L1max, L2max, lane,
                                k * P);
        };
        int seen = -1;       // chunks of the previous part known to be complete
        if (x_in) {
            seen = wait_part(flag_in, epoch, min(lead(P), nch), st);
            issue_row(0);
        }
        if (!HELP) issue_tiles(0);
        // NWG: lane r starts beside column 0 of its row, its diagonal beside column 0
        // of the row above (alpha[0,0] = 0 for lane 0 of the first stripe)
        float cur = left0, up_prev = NWG ? (float)(i0 + lane) * gap : kNINF;
        float tcur = 0.0f, tup_prev = 0.0f;   // TAN: the same for the tangents
        float bm = -1e20f;   // the running max of this lane's alphas (partition)
        int slot0 = 0;       // ring slot of step t0: t0 % R (R is a multiple of P)
        ProgAhead ahead;     // progress words read during the previous chunk
        prog_ahead_reset(ahead);

        for (int k = 0; k < nch; ++k, slot0 = slot0 + P < R ? slot0 + P : slot0 + P - R) {
            const int t0 = k * P;
            chunk_waits_ahead<P>(ahead, prog, l, NL, k, nch, R, st);
            // this chunk's loads were issued one chunk ago and followed by at least the
            // P + 1 stores of that chunk (the first chunk's loads are the last issued).
            // HELP: the helper loads the scores; this wave loads only the row above of a
            // part's first stripe (followed by the last-row store), and waits for
            // nothing else: a wait for its own stores would stall it behind the
            // helpers' memory traffic
            if constexpr (HELP) {
                if (x_in) {
                    if (k == 0) wait_vmcnt<0>(); else wait_vmcnt<1>();
                }
                wait_for_ahead(ahead.help, hprog, l, k + 1, st);
            } else {
                // (TAN: the 2P + 2 stores of that chunk)
                if (k == 0) wait_vmcnt<0>(); else wait_vmcnt<NTL * P>();
            }
            if (x_in && k > 0) {
                // its progress word, loaded one chunk ago before those stores
                const int got = flag_chunks_lds(fslot, epoch);
                seen = got > seen ? got : seen;
            }
            const float* tile = tiles + (k & (NTB - 1)) * Tile::FLOATS;
            float sv[P], av[P];
            float vv[P], xv[P];   // TAN: direction, tangents
            read_quads<P, 1>(tile, lane, sv);
            if (TAN) read_quads<P, 1>(tile + NTB * Tile::FLOATS, lane, vv);
            // lane 0's up values: lane j < P holds column t0 + j of the row above (ring
            // slot = producer step); each step shifts the next one into lane 0 (one DPP
            // move instead of staging them through LDS).  Above the first stripe, row 0:
            // NINF, or (NWG) alpha[0, t0+j+1] = (t0+j+1)*gap
            float upsh = kNINF;
            if (s > 0) {
                if (lane < P) {
                    int slot = slot0 + lane + 63;
                    slot = slot < R ? slot : slot - R;
                    upsh = x_in ? rbufs[(k & 1) * 64 + lane] : ring_in[slot];
                }
            } else if (NWG) {
                upsh = (float)(t0 + lane + 1) * gap;
            }
            // TAN: the tangents of the row above the same way (row 0: 0)
            float tupsh = 0.0f;
            if (TAN && s > 0 && lane < P) {
                int slot = slot0 + lane + 63;
                slot = slot < R ? slot : slot - R;
                tupsh = x_in ? rbufs[(2 + (k & 1)) * 64 + lane] : tring_in[slot];
            }
            if (k + 1 < nch) {
                if (x_in) {
                    const int need = min(k + 1 + lead(P), nch);
                    if (seen < need) seen = wait_part(flag_in, epoch, need, st);
                    issue_row(k + 1);
                }
                if (!HELP) issue_tiles(k + 1);
                if (x_in) flag_load_lds(flag_in, fslot_lds, lane);
            }
            // lane 63 publishes its alpha of step u into ring slot (t0+u) % R; the
            // other lanes write into the sink (R is a multiple of P: no wrap in a chunk)
            float* pub = (lane == 63) ? ring_out + slot0 : sink + lane;
            float* tpub = (lane == 63) ? tring_out + slot0 : sink + lane;
            float* outc = out + (size_t)t0 * 64;
            float* toutc = TAN ? tout + (size_t)t0 * 64 : nullptr;
            // HELP: the chunk's alphas by step in the helper's tile k & 1 (written out
            // by the helper; it has written that tile's previous chunk before
            // publishing this one as loaded); WIDE: over this chunk's score tile, whose
            // scores are in registers.  TAN: the tangents in the helper's tile NTB + k & 1
            float* atile = smem + (WIDE ? wave : wave + NW / 2) * WBUF +
                           (k & (NTB - 1)) * Tile::FLOATS + lane;
            float* ttile = atile + NTB * Tile::FLOATS;
            // FULL: every cell of the chunk lies inside the element, no validity masks
            auto steps = [&](auto full) {
                constexpr bool FULL = decltype(full)::value;
#pragma unroll
                for (int u = 0; u < P; ++u) {
                    const int t = t0 + u;
                    const float up = wave_shr1_or(cur, upsh);   // lane 0: stripe above
                    upsh = wave_shl1(upsh);
                    const float diag = up_prev;
                    up_prev = up;
                    // out-of-table neighbours are NINF, so no i>1 / j>1 guards are needed
                    // (FULL: the raw max saves the scores' canonicalisation; in the
                    // masked form it only moves instructions)
                    float a, x = 0.0f;
                    if constexpr (TAN) {
                        const float tu = wave_shr1_or(tcur, tupsh);
                        tupsh = wave_shl1(tupsh);
                        const float td = tup_prev;
                        tup_prev = tu;
                        a = fwd_cell_tan<NWG, FULL>(diag, up, cur, sv[u], gap, c, tl, td, tu,
                                                    tcur, vv[u], x);
                    } else {
                        a = fwd_cell<NWG, FULL>(diag, up, cur, sv[u], gap, c, tl);
                    }
                    if (FULL) {
                        cur = a;
                        tcur = x;
                    } else {
                        const int col = t - lane;
                        const bool ok = (unsigned)col < (unsigned)L2eff;
                        // NWG: the cells left of column 0 keep the row's boundary
                        cur = ok ? a : (NWG && col < 0 ? left0 : kNINF);
                        tcur = ok ? x : 0.0f;
                        // the terminal cell never lies in a FULL chunk (lane 63's
                        // column stays below L2 - 1 there)
                        if (NWG && ok && last_row && col == L2 - 1) {
                            terminal = a;
                            if (TAN) tterm = x;
                        }
                    }
                    if (HELP) atile[u * 64] = cur;
                    else lane_store(outc + u * 64, ul4, cur);
                    pub[u] = cur;
                    av[u] = cur;
                    if (!NWG && !HELP) bm = fmaxf(bm, cur);
                    if constexpr (TAN) {
                        if (HELP) ttile[u * 64] = tcur;
                        else lane_store(toutc + u * 64, ul4, tcur);
                        tpub[u] = tcur;
                        xv[u] = tcur;
                    }
                }
            };
            if (i0 + 63 < L1 && t0 >= 63 && t0 + P <= L2) steps(std::true_type{});
            else steps(std::false_type{});
            prog_ahead(ahead, prog, HELP ? hprog : nullptr, l, NL, l);
            if constexpr (TAN) {
                if (!NWG && !HELP) acc.template add_block_max<P>(av, xv, bm, c);
            } else {
                if (!NWG && !HELP) acc.template add_block_max<P>(av, bm, c);
            }
            // the stripe's last row (lane 63) by step, contiguous, for the reverse sweep
            // of the stripe below and the next part; one store instruction (TAN: two)
            wave_lds_sync();
            if (!HELP || x_out) {
                if (lane < P) {
                    const float v = ring_out[slot0 + lane];
                    if (x_out) store_sys(brow_s + t0 + lane, v);
                    else lane_store(brow_s, (unsigned)(t0 + lane) * 4u, v);
                    if (TAN) {
                        const float tv = tring_out[slot0 + lane];
                        if (x_out) store_sys(tb_s + t0 + lane, tv);
                        else lane_store(tb_s, (unsigned)(t0 + lane) * 4u, tv);
                    }
                }
            }
            publish(prog, wave, l * PROG_STRIDE + k + 1);
            if (TAN && HELP && x_out && !x_in && k >= 1) {
                // TAN with helpers, a part's last stripe that is not also its first:
                // this wave's only memory operations are its last-row stores (NTL per
                // chunk) and its flag stores (one per chunk from chunk 1 on), so once at
                // most the previous chunk's flag store and this chunk's row stores are
                // outstanding, every chunk before this one is complete.  (Measured at
                // C5: the tangent forward 1974 against 1994-1999 us; the plain forward
                // 1319-1324 against 1307-1314, so it keeps the report below.)
                if (k == 1) wait_vmcnt<NTL>(); else wait_vmcnt<NTL + 1>();
                if (lane == 0) store_flag(flag_out, progress_word(epoch, k));
            } else if (x_out && k >= 2) {
                // at least 2 * (P/4 + P + 1) vector-memory operations (HELP: the last
                // row stores of chunks k - 1 and k) follow the row stores of chunk
                // k - 2: those (and everything before) are complete.  TAN: at least
                // 2 * (2P + 2), beyond the counter's range of 63 (HELP: 2 * 2)
                constexpr int AFTER = TAN ? 4 * P + 4 : 2 * (Tile::NQ + P + 1) - Tile::NQ;
                if constexpr (HELP) wait_vmcnt<NTL * 2>();
                else wait_vmcnt<(AFTER < 63 ? AFTER : 63)>();
                if (lane == 0) store_flag(flag_out, progress_word(epoch, k - 1));
            }
        }
        if (x_out) {
            wait_vmcnt<0>();
            if (lane == 0) store_flag(flag_out, progress_word(epoch, nch));
        }
    }

    if (NWG) {
        // the value: the terminal cell, written by the part that owns the last stripe
        // (part 0 for an element without stripes, whose value is its boundary)
        __syncthreads();
        const bool owner = NS > 0 ? (NL > 0 && s_begin + NL == NS) : part == 0;
        if (threadIdx.x == 0 && owner) {
            partition[b] = NS > 0 ? terminal : (float)(L1 + L2) * gap;
            if (TAN) ta.sdot[b] = NS > 0 ? tterm : 0.0f;   // the terminal cell's tangent
        }
        return;
    }
    // partition: merge lanes, waves, and (once per element) the cell (0,0) whose alpha is 0
    // (TAN: and whose tangent is 0).  Slot l holds stripe l's state: from sweeping wave l,
    // or (HELP) from its helper, wave HB + l; the other slots stay at the empty state.
    wave_merge_lse(acc, c);
    constexpr int HB = WIDE ? NW : NW / 2;
    if constexpr (HELP) {
        if (lane == 0 && wave < NW) {
            red_m[wave] = -3.0e38f;
            red_z[wave] = 0.0f;
            if constexpr (TAN) red_w[wave] = 0.0f;
        }
        __syncthreads();
    }
    const int slot = HELP ? wave - HB : wave;
    if (lane == 0 && slot >= 0 && slot < NW) {
        red_m[slot] = acc.m;
        red_z[slot] = acc.z;
        if constexpr (TAN) red_w[slot] = acc.w;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        if constexpr (TAN) {
            OnlineLSEDot tot;
            tot.m = G == 1 ? 0.0f : kNINF;
            tot.z = G == 1 ? 1.0f : 0.0f;
            tot.w = 0.0f;
            for (int w = 0; w < NW; ++w) tot.merge(red_m[w], red_z[w], red_w[w], c);
            if (G == 1) {
                // the cells' weights 2^((alpha - S) c) with S rounded to fp32, as the
                // two-sweep form and the reference take them: w 2^((m - S) c), not w / z
                // (their sum differs from 1 by the rounding of S, e.g. 6e-5 at |S| = 500
                // and T = 0.5, and the reverse sweep's start relies on the same weights)
                const float S = tot.m + tl * fast_log2(tot.z);
                partition[b] = S;
                ta.sdot[b] = tot.w * fast_exp2((tot.m - S) * c);
            } else {
                fpart[(size_t)b * G + part] = make_float2(tot.m, tot.z);
                ta.wpart[(size_t)b * G + part] = tot.w;
            }
            return;
        }
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

// PRECISE: accumulate dS/dgap and dS/dT per lane in double (second-order callers,
// whose Jacobians amplify errors in these sums).
// NWG: global alignment (/root/reference/src/nw/kernels_cpu.cpp:160-265): beta starts
// at 1 in the terminal cell only, the marginal is beta * w_diag, and the flows into
// row 0 and column 0 (whose alphas encode j*gap and i*gap) add flow * gaps to dS/dgap.
// HELP (plain variant, parts of at most NW/2 stripes): wave NW/2 + q moves stripe order
// q's data, so the sweeping wave only sweeps.  It loads each chunk's score quads and
// alpha rows one chunk ahead (publishing hprog[q] = chunks loaded), and writes a
// chunk's marginals out once wave q has finished the chunk (prog[q]).  The marginals
// go to the helper's own (otherwise unused) chunk buffers, so the helper can reload
// the sweeping wave's input buffer before it writes them out.
// (one workgroup per CU: its LDS allows no second; waves_per_eu says so, so that the
// register allocator does not spill to reach an occupancy the launch cannot have)
// RECOMP (plain variant, with HELP and WIDE): the helper waves rebuild each chunk's alpha
// rows from a checkpoint-mode forward's stored steps (ckpt_step) instead of loading
// them from a full table.
template <int P, bool PRECISE = false, bool NWG = false, bool HELP = false, bool WIDE = false,
          bool RECOMP = false>
__global__ void __launch_bounds__(WIDE ? 2 * NW * 64 : NW * 64)
__attribute__((amdgpu_waves_per_eu(WIDE ? 4 : 1, WIDE ? 4 : 2)))
sw_backward_kernel(const float* __restrict__ scores, const int* __restrict__ lengths,
                   const float* __restrict__ alpha_sk, const float* __restrict__ brow,
                   const float* __restrict__ partition,
                   float* __restrict__ post, float* __restrict__ grad_gap,
                   float* __restrict__ grad_T, int* __restrict__ status, float* __restrict__ trash,
                   uint64_t* __restrict__ bflag, float2* __restrict__ flows,
                   double* __restrict__ bpart, float* __restrict__ poison_value, int B, int L1max,
                   int L2max, int NSmax, float gap, float T, int R, int G, int SPW,
                   uint32_t epoch) {
    extern __shared__ __align__(16) float smem[];
    __shared__ int prog[NW];
    using Acc = typename std::conditional<PRECISE, double, float>::type;
    __shared__ Acc red_g[NW], red_p[NW];
    // parts run bottom-up: the part below (the producer of this one's flows) is
    // dispatched first
    int b, dpart;
    split_decode(blockIdx.x, G, b, dpart);
    if (b >= B) return;
    const int part = G - 1 - dpart;
    const int lane = threadIdx.x & 63;
    const unsigned ul4 = (unsigned)lane * 4u;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Per wave, two chunk buffers, each: the score tile (then the chunk's marginals),
    // P alpha rows (steps t_hi-2 .. t_hi-P-1, 64 lanes each) and one row of values from
    // the stripe above.  All three arrive by direct-to-LDS loads one chunk ahead.
    using Tile = QuadTile<P>;
    constexpr int ABUF = Tile::FLOATS;            // alpha rows
    constexpr int RBUF = ABUF + P * 64;           // row above
    constexpr int FBUF = RBUF + 64;               // flows from the part below (2P+2 floats)
    constexpr int BUF = FBUF + 64;
    static_assert(2 * P + 2 <= 64, "boundary flows fit their buffer");
    float* bufs = smem + wave * 2 * BUF;
    __shared__ float fslot[64];   // progress word prefetched by wave 0, the only wave whose
                                  // stripe borders another part
    const uint32_t fslot_lds = lds_address(fslot);
    float2* rings = reinterpret_cast<float2*>(smem + NW * 2 * BUF);  // [NW][R] (up, diag)
    float2* sink = rings + NW * R + wave * DUMMY;
    int* st = status + b;
    // The chunk's marginals go to an output tile laid over its own score tile, whose
    // values are all in registers by then (the next chunk loads into the other
    // buffer).  QOUT: a quad tile, one 16-byte quad per lane and four steps (the
    // swizzle keeps those writes conflict-free), leaving with P/4 16-byte stores;
    // otherwise (PRECISE, NWG: those variants have no registers to spare) a dword tile,
    // one write per step, leaving with P dword stores.
    constexpr bool QOUT = !PRECISE && !NWG;
    static_assert(!HELP || QOUT, "helper waves write quad output tiles");
    __shared__ int hprog[NW];     // HELP: chunks of stripe order q loaded by its helper
    // BCAST (FULL chunks of the plain variant): lane 63's flows from the stripe below
    // come as per-step broadcast LDS reads, each read used once as the boundary
    // operand of a DPP shift, instead of registers shifted one lane per step (two DPP
    // moves per step fewer).  A stripe with no stripe below reads zero flows from
    // zpairs.
    constexpr bool BCAST = !PRECISE && !NWG;
    __shared__ __align__(16) float2 zpairs[P];
    using OutTile = ChunkTile<P>;
    static_assert(OutTile::FLOATS <= BUF, "output tile fits the chunk buffer");
    const int obase_lane = OutTile::read_base(lane);
    constexpr int NSTORE = QOUT ? Tile::NQ : P;   // stores of an inside chunk

    if (lane == 0 && wave < NW) {
        prog[wave] = -1;
        hprog[wave] = -1;
    }
    if (BCAST && threadIdx.x < P) zpairs[threadIdx.x] = make_float2(0.0f, 0.0f);
    __syncthreads();

    const int L1 = lengths ? min(max(lengths[2 * b], 0), L1max) : L1max;
    const int L2 = lengths ? min(max(lengths[2 * b + 1], 0), L2max) : L2max;
    const float c = kLog2e / T;
    const float S = partition[b];
    const int NS = L2 > 0 ? (L1 + 63) >> 6 : 0;
    const int nsteps = L2 + 63;
    const int nch = (nsteps + P - 1) / P;
    const size_t NT = (size_t)stored_steps(L2max);
    const float* sbase = scores + (size_t)b * L1max * L2max;
    float* pbase = post + (size_t)b * L1max * L2max;

    {   // each part zeroes its share of the rows' padding
        const int rows = (L1max + G - 1) / G;
        zero_padding(pbase, L1, L2, L1max, L2max, (int)blockDim.x, part * rows,
                     min(L1max, part * rows + rows));
    }

    Acc g_acc = 0, p_acc = 0;
    float A[P + 2];
    const int s_begin = part * SPW;
    const int NL = max(min(NS, s_begin + SPW) - s_begin, 0);   // stripes of this part
    const bool has_next = s_begin + NL < NS;
    const uint64_t* flag_in = bflag + (size_t)b * G + (part + 1 < G ? part + 1 : part);
    uint64_t* flag_out = bflag + (size_t)b * G + part;

    if constexpr (HELP) {
        // helpers: waves HB..HB+NL-1 (WIDE: a second set of NW waves)
        constexpr int HB = WIDE ? NW : NW / 2;
        if (NL > HB) {   // never: the host picks HELP for parts of at most HB stripes
            if (threadIdx.x == 0) atomicOr(st, 2);
            return;
        }
        const int q = wave - HB;
        if (q >= 0 && q < NL) {
            const int s = s_begin + NL - 1 - q;
            const int i0 = s * 64;
            const float* astripe = alpha_sk + ((size_t)b * NSmax + s) * NT * 64;
            float* qbufs = smem + q * 2 * BUF;   // the sweeping wave's two chunk buffers
            // its output tiles: this wave's own buffers, or (WIDE: no LDS for those) its
            // input buffers, over the score tile it has read into registers
            float* obufs = smem + (WIDE ? q : wave) * 2 * BUF;
            // the row above (the stripe above's last row): lane j <= P holds its alpha
            // at step t_hi - j + 63, clamped to the last step
            const float* hbup = brow + ((size_t)b * NSmax + (s > 0 ? s - 1 : 0)) * NT;
            auto rowup_off = [&](int th, int ln) {
                return (uint32_t)min(th - min(ln, P) + 63, nsteps - 1) * 4u;
            };
            // whole 64-byte row segments of marginals where rows start aligned
            // (write_aligned), else the chunk's own row segments (also in the 16-wave
            // recomputing form, whose registers hold the recurrence instead)
            const bool aligned = !(RECOMP && WIDE) && (L2max & (P - 1)) == 0;
            AlignedCarry<P> carry;
            carry.clear();
            auto load = [&](int k) {
                const int th = nsteps - 1 - k * P;
                const uint32_t buf = lds_address(qbufs + (k & 1) * BUF);
                dma_quads<P, -1>(buf, sbase, i0, L1max, L2max, lane, th);
                dma_rows<P, -1>(buf + ABUF * 4, astripe, th - 2, ul4);
                uint32_t roff = rowup_off(th, lane);
                uint32_t rl = buf + RBUF * 4;
                lds_dma_dword<0>(hbup, roff, rl, 0u);
            };
            if constexpr (RECOMP) {
                static_assert(HELP && P == PR && !NWG, "recomputing helpers: 16-step SW sweep");
                // Chunk k's alpha rows (steps t_lo = t_hi - P - 1 .. t_hi - 2) are rebuilt
                // by running the forward recurrence from the stored alphas of steps
                // t_lo - 1 and t_lo - 2, with the row above taken from the stripe above's
                // last row (brow) and this lane's own scores; step t_lo + m goes to row m
                // of the alpha rows, where the sweeping wave reads it as it would a loaded
                // row.  Inputs are staged in registers two chunks ahead (the output tile
                // lies over the input buffer in the 16-wave form, in this wave's own
                // buffers otherwise); the recurrence for chunk k + 2 runs while wave q
                // sweeps chunk k.
                const float tl = T * kLn2;
                const int L2eff = (i0 + lane < L1) ? L2 : 0;
                // RW: this lane's scores of steps t_hi - P - 3 .. t_hi (its own row, as
                // P/4 + 1 quads in memory-column order): the recurrence reads steps t_lo
                // .. t_lo + P - 1, and the top P steps are the chunk's quad tile for
                // the sweeping wave (quad q of the tile is quad P/4 - q here).
                constexpr int RW = P / 4 + 1;
                struct RStage {
                    f32x4 row[RW];
                    float ck0, ck1;      // alphas of steps t_lo - 1 and t_lo - 2
                    float bb;            // lane j: the row above at step t_lo + 62 + j
                    float rowup;         // the sweeping wave's row above (rowup_off)
                };
                RStage set0, set1;
                auto stage = [&](RStage& g, int k) {
                    const int th = nsteps - 1 - k * P, t0 = th - P - 1;
                    int ln = lane;
                    __asm__ volatile("" : "+v"(ln));
                    stage_row<4 * RW>(g.row, sbase, i0, L1max, L2max, ln, th - 4 * RW + 1);
                    // (steps below -APAD are column-0 boundary cells, set in recomp)
                    g.ck0 = lane_load(astripe + (size_t)(max(t0 - 1, -APAD) + APAD) * 64, ul4);
                    g.ck1 = lane_load(astripe + (size_t)(max(t0 - 2, -APAD) + APAD) * 64, ul4);
                    g.bb = lane_load(hbup, (unsigned)min(t0 + 62 + min(ln, P), nsteps - 1) * 4u);
                    g.rowup = lane_load(hbup, rowup_off(th, ln));
                };
                auto recomp = [&](const RStage& g, int k, float (&rows)[P]) {
                    const int t0 = nsteps - 1 - k * P - P - 1;
                    float sv[P];   // step t0 + u: element u + 2 of the staged row
#pragma unroll
                    for (int u = 0; u < P; ++u) sv[u] = g.row[(u + 2) / 4][(u + 2) % 4];
                    // steps before 0 lie left of column 0: NINF, as in the table
                    float cur = t0 - 1 >= 0 ? g.ck0 : kNINF;
                    float bb = s > 0 ? g.bb : kNINF;
                    // the diagonal of step t0: lane r - 1's alpha of step t0 - 2, lane 0
                    // the row above at step t0 - 1 + 63
                    float up_prev = wave_shr1_or(t0 - 2 >= 0 ? g.ck1 : kNINF, bb);
                    auto run = [&](auto full) {
                        constexpr bool FULL = decltype(full)::value;
#pragma unroll
                        for (int u = 0; u < P; ++u) {
                            bb = wave_shl1(bb);   // lane 0: the row above at step t0 + u + 63
                            const float up = wave_shr1_or(cur, bb);
                            const float diag = up_prev;
                            up_prev = up;
                            const float a = fwd_cell<false, FULL>(diag, up, cur, sv[u], gap, c, tl);
                            if (FULL) {
                                cur = a;
                            } else {
                                const int col = t0 + u - lane;
                                cur = (unsigned)col < (unsigned)L2eff ? a : kNINF;
                            }
                            rows[u] = cur;
                        }
                    };
                    if (i0 + 63 < L1 && t0 >= 63 && t0 + P <= L2) run(std::true_type{});
                    else run(std::false_type{});
                };
                auto put = [&](const RStage& g, int k, const float (&rows)[P]) {
                    float* buf = qbufs + (k & 1) * BUF;
#pragma unroll
                    for (int q2 = 0; q2 < Tile::NQ; ++q2)
                        *reinterpret_cast<f32x4*>(buf + Tile::slot(lane, q2)) = g.row[Tile::NQ - q2];
#pragma unroll
                    for (int u = 0; u < P; ++u) buf[ABUF + u * 64 + lane] = rows[u];
                    buf[RBUF + lane] = g.rowup;
                };
                // nch >= 4: nsteps = L2 + 63
                {
                    float rows[P];
                    stage(set0, 0);
                    stage(set1, 1);
                    recomp(set0, 0, rows);
                    put(set0, 0, rows);
                    publish(hprog, q, 1);
                    stage(set0, 2);
                    recomp(set1, 1, rows);
                    put(set1, 1, rows);
                    publish(hprog, q, 2);
                    stage(set1, 3);
                }
                auto half = [&](RStage& g, int k) {
                    float rows[P];
                    const bool more = k + 2 < nch;
                    if (more) recomp(g, k + 2, rows);
                    int ln = lane;
                    __asm__ volatile("" : "+v"(ln));
                    wait_for(prog, q, q * PROG_STRIDE + k + 1, st);
                    if (aligned)
                        write_aligned<P, true>(obufs + (k & 1) * BUF, pbase, trash, carry, i0,
                                               L1max, L2max, ln, nsteps - 1 - k * P);
                    else
                        write_quads<P, -1>(obufs + (k & 1) * BUF, pbase, trash, i0, L1, L2,
                                           L1max, L2max, ln, nsteps - 1 - k * P);
                    if (more) {
                        // (LDS runs this wave's reads above before these writes)
                        put(g, k + 2, rows);
                        publish(hprog, q, k + 3);
                    }
                    stage(g, min(k + 4, nch - 1));
                };
                int k = 0;
                for (; k + 1 < nch; k += 2) {
                    half(set0, k);
                    half(set1, k + 1);
                }
                if (k < nch) half(set0, k);
            } else if constexpr (WIDE) {
                // The output tile lies over the input buffer, which can take chunk k + 2
                // only once chunk k's marginals have left: too late for a load issued
                // then.  So chunks 0 and 1 go straight to LDS, and every later chunk is
                // staged in this wave's registers two chunks ahead (set k & 1 holds
                // chunk k + 2 while wave q sweeps chunk k) and written into its buffer
                // once the marginals there have left.  Every vector-memory operation
                // of the loop below is unconditional (stages past the last chunk
                // reload it, unused), so that the compiler's own waits for the staged
                // registers count exactly the operations issued since: a conditional
                // one would make them wait for the marginal stores just issued as well.
                struct Stage {
                    StagedQuads<P> sq;
                    f32x4 rows[P / 4];
                    float rowup;
                };
                Stage set0, set1;
                auto stage = [&](Stage& g, int k) {
                    const int th = nsteps - 1 - k * P;
                    int ln = lane;
                    __asm__ volatile("" : "+v"(ln));
                    stage_quads<P, -1>(g.sq, sbase, i0, L1max, L2max, ln, th);
                    stage_rows<P, -1>(g.rows, astripe, th - 2, ln);
                    g.rowup = lane_load(hbup, rowup_off(th, ln));
                };
                // nch >= 4: nsteps = L2 + 63
                load(0);
                wait_vmcnt<0>();
                publish(hprog, q, 1);
                load(1);
                stage(set0, 2);
                stage(set1, 3);
                // chunk 1's loads: followed by the (at least 2 (P/4 + P/4)) staged loads
                wait_vmcnt<2 * (Tile::NQ + P / 4)>();
                publish(hprog, q, 2);
                auto half = [&](Stage& g, int k) {
                    float* buf = qbufs + (k & 1) * BUF;
                    // an opaque copy of the lane index per chunk keeps the compiler from
                    // hoisting the per-lane offsets of boundary chunks out of the loop
                    // (registers that the two stages need)
                    int ln = lane;
                    __asm__ volatile("" : "+v"(ln));
                    wait_for(prog, q, q * PROG_STRIDE + k + 1, st);
                    if (aligned)
                        write_aligned<P, true>(buf, pbase, trash, carry, i0, L1max, L2max, ln,
                                               nsteps - 1 - k * P);
                    else
                        write_quads<P, -1>(buf, pbase, trash, i0, L1, L2, L1max, L2max, ln,
                                           nsteps - 1 - k * P);
                    if (k + 2 < nch) {
                        // (LDS runs this wave's reads above before these writes)
                        put_staged_quads<P>(buf, g.sq, lane);
                        put_staged_rows<P>(buf + ABUF, g.rows, lane);
                        buf[RBUF + lane] = g.rowup;
                        publish(hprog, q, k + 3);
                    }
                    stage(g, min(k + 4, nch - 1));
                };
                int k = 0;
                for (; k + 1 < nch; k += 2) {
                    half(set0, k);
                    half(set1, k + 1);
                }
                if (k < nch) half(set0, k);
            } else {
                if (nch > 0) {
                    load(0);
                    wait_vmcnt<0>();
                    publish(hprog, q, 1);
                    if (nch > 1) load(1);
                }
                for (int k = 0; k < nch; ++k) {
                    if (k + 1 < nch) {
                        // chunk k + 1's loads: the last issued at k = 0, else followed
                        // by the (at least P/4) marginal stores of chunk k - 1
                        if (k == 0) wait_vmcnt<0>(); else wait_vmcnt<Tile::NQ>();
                        publish(hprog, q, k + 2);   // also completes this wave's LDS reads
                    }
                    // once wave q has finished chunk k, its input buffer k & 1 takes
                    // chunk k + 2 and its marginals (in output tile k & 1) leave
                    wait_for(prog, q, q * PROG_STRIDE + k + 1, st);
                    if (k + 2 < nch) load(k + 2);
                    if (aligned)
                        write_aligned<P, true>(obufs + (k & 1) * BUF, pbase, trash, carry, i0,
                                               L1max, L2max, lane, nsteps - 1 - k * P);
                    else
                        write_quads<P, -1>(obufs + (k & 1) * BUF, pbase, trash, i0, L1, L2,
                                           L1max, L2max, lane, nsteps - 1 - k * P);
                }
            }
        }
    }

    // Stripes run bottom-up: order q = 0..NL-1 handles stripe s_begin+NL-1-q, on wave
    // q % NW.
    for (int q = wave; q < NL; q += NW) {
        set_pipeline_priority(q % NW);
        const int s = s_begin + NL - 1 - q;
        const int i0 = s * 64;
        const int L2eff = (i0 + lane < L1) ? L2 : 0;
        // NWG: the terminal cell (L1, L2) starts with beta = 1; the flows into column 0
        // count i (row i0+lane+1, left) and i - 1 (diagonal) gaps, those into row 0
        // (first stripe, lane 0) the column's index
        const int term_step = (NWG && i0 + lane == L1 - 1) ? L2 - 1 + lane : -1000000;
        const float gi = (float)(i0 + lane + 1);
        const bool top = NWG && s == 0 && lane == 0;
        // alpha tables of this stripe and of the one above, from step -APAD
        const float* astripe = alpha_sk + ((size_t)b * NSmax + s) * NT * 64;
        const float* bup = brow + ((size_t)b * NSmax + (s > 0 ? s - 1 : 0)) * NT;
        const float2* ring_in = ring_from(rings, q, R);   // from stripe s+1
        float2* ring_out = ring_of(rings, q, R);          // to stripe s-1
        const bool x_in = q == 0 && has_next;             // flows from the part below
        const bool x_out = q == NL - 1 && part > 0;       // flows to the part above
        const bool below = q > 0 || x_in;
        // boundary flows by producer step: written by stripe s (x_out), read from s + 1
        float2* flows_out = flows + ((size_t)b * NSmax + s) * NT;
        const float* flows_in =
            reinterpret_cast<const float*>(flows + ((size_t)b * NSmax + (x_in ? s + 1 : s)) * NT);
        int seen = -1;       // chunks of the part below known to be complete

        // Loads of chunk k (t_hi = nsteps-1-kP) into buffer k&1: the score quad tile, P
        // alpha rows (steps t_hi-2 .. t_hi-P-1, four per load), and the row-above values
        // (lane j <= P: the alpha of the last row of the stripe above at step
        // t_hi - j + 63, clamped to the last step; lanes past P repeat lane P's address).
        auto issue_chunk = [&](int k) {
            const int th = nsteps - 1 - k * P;
            const uint32_t buf = lds_address(bufs + (k & 1) * BUF);
            if (!HELP) {
                dma_quads<P, -1>(buf, sbase, i0, L1max, L2max, lane, th);
                dma_rows<P, -1>(buf + ABUF * 4, astripe, th - 2, ul4);
            }
            if (!HELP) {
                uint32_t roff = (uint32_t)min(th - min(lane, P) + 63, nsteps - 1) * 4u;
                uint32_t rl = buf + RBUF * 4;
                lds_dma_dword<0>(bup, roff, rl, 0u);
            }
            if (x_in) {
                // flows of producer slots kP+62 .. kP+62+P (float2 each): float f of the
                // range in lane f, clamped to the last slot
                uint32_t foff = (uint32_t)min((k * P + 62) * 2 + min(lane, 2 * P + 1),
                                              (nsteps - 1) * 2 + 1) * 4u;
                uint32_t fdst = buf + FBUF * 4;
                lds_dma_dword_sys<0>(flows_in, foff, fdst, 0u);
            }
        };

        // the first two alphas of chunk 0 (steps nsteps-1, nsteps-2); later chunks
        // carry them over from the previous chunk
        A[P] = lane_load(astripe + (size_t)(nsteps - 1 + APAD) * 64, ul4);
        A[P + 1] = lane_load(astripe + (size_t)(nsteps - 2 + APAD) * 64, ul4);
        __asm__ volatile("" ::"v"(A[P]), "v"(A[P + 1]));   // completes the two loads here
        wave_lds_sync();   // the previous stripe's buffer reads are complete
        if (x_in) seen = wait_part(flag_in, epoch, min(lead(P), nch), st);
        issue_chunk(0);
        float in_left = 0.0f, in_up = 0.0f, in_diag = 0.0f, in_diag_next = 0.0f;
        int slot0 = 0;   // ring slot of step k*P: (k*P) % R (R is a multiple of P)
        ProgAhead ahead;   // progress words read during the previous chunk
        prog_ahead_reset(ahead);

        for (int k = 0; k < nch; ++k, slot0 = slot0 + P < R ? slot0 + P : slot0 + P - R) {
            const int t_hi = nsteps - 1 - k * P;
            chunk_waits_ahead<P>(ahead, prog, q, NL, k, nch, R, st);
            // this chunk's loads were issued one chunk ago and followed by at least the
            // NSTORE marginal stores of that chunk (P in a boundary chunk; the first
            // chunk's loads are the last issued).  HELP: the helper loads the tiles and
            // the row above; this wave loads only the flows from the part below (x_in),
            // followed by nothing, or by the previous chunk's flow store (x_out)
            if constexpr (HELP) {
                if (x_in) {
                    if (x_out && k > 0) wait_vmcnt<1>(); else wait_vmcnt<0>();
                }
                wait_for_ahead(ahead.help, hprog, q, k + 1, st);
            } else {
                if (k == 0) wait_vmcnt<0>(); else wait_vmcnt<NSTORE>();
            }
            if (x_in && k > 0) {
                // its progress word, loaded one chunk ago before those stores
                const int got = flag_chunks_lds(fslot, epoch);
                seen = got > seen ? got : seen;
            }
            float* buf = bufs + (k & 1) * BUF;
            // the chunk's marginal quads: over its own score tile, or (HELP) in the
            // helper's buffer k & 1, whose previous tile the helper has written out
            // before publishing this chunk as loaded
            float* obuf = HELP && !WIDE ? smem + (wave + NW / 2) * 2 * BUF + (k & 1) * BUF : buf;
            // QOUT: the score quads are read one quad ahead of their steps (quad q of
            // the output tile lies over score quad q of this lane's row and is written
            // after that quad's last step), so only two quads are live at a time
            float sv[P];
            auto read_sq = [&](int qq) {
                const float4 x = *reinterpret_cast<const float4*>(buf + Tile::slot(lane, qq));
                sv[Tile::template step<-1>(qq, 0)] = x.x;
                sv[Tile::template step<-1>(qq, 1)] = x.y;
                sv[Tile::template step<-1>(qq, 2)] = x.z;
                sv[Tile::template step<-1>(qq, 3)] = x.w;
            };
            if constexpr (QOUT) read_sq(0);
            else read_quads<P, -1>(buf, lane, sv);
            A[0] = A[P];
            A[1] = A[P + 1];
#pragma unroll
            for (int j = 0; j < P; ++j) A[j + 2] = buf[ABUF + rows_row<P, -1>(j) * 64 + lane];
            // lane j: alpha of the row above at lane-63 step t_hi - j + 63 (column
            // t_hi - j); above the first stripe, row 0: NINF, or (NWG) (column + 1) * gap
            // FULL: every cell of the chunk lies inside the element
            const bool inside = i0 + 63 < L1 && t_hi - P - 62 >= 0 && t_hi < L2;
            const bool bcast = BCAST && inside;
            float bv = 0.0f;
            // Contributions from the stripe below for lane 63.  The producer (lane 0 of
            // stripe s+1) wrote the pair for its column c into slot (nsteps-1-c) % R;
            // lane 63 at step u needs column t_hi-u-63 (up) and t_hi-u-62 (diagonal),
            // i.e. slots kP+u+63 and kP+u+62.  Lane 63-j holds step j; the register is
            // shifted up one lane per step so lane 63 sees the step it needs next.
            // bcast: step u takes the up value of step u + 1 and the diagonal value of
            // step u + 2, both in slot kP+u+64, from a broadcast read of that pair (with
            // x_in: flow pair u + 2 of the chunk's FBUF range, which starts at slot
            // kP+62); the chunk starts from slots kP+62 and kP+63.  In a FULL chunk
            // those slots lie below nsteps - 1 (no clamped flows) and kP+64 .. kP+64+P-1
            // lie in one ring block of P slots (slot0 and R are multiples of P).  The
            // reads run BD steps ahead of their use, in a window of registers.
            float pre_u = 0.0f, pre_d = 0.0f;
            constexpr int BD = 1;
            float2 rp[P], r62 = make_float2(0.0f, 0.0f), r63 = make_float2(0.0f, 0.0f);
            const float2* pp = zpairs;
            if (bcast) {
                const int s64 = slot0 + 64 < R ? slot0 + 64 : slot0 + 64 - R;
                const int s62 = s64 >= 2 ? s64 - 2 : s64 - 2 + R;
                const float2* fb = reinterpret_cast<const float2*>(buf + FBUF);
                pp = !below ? zpairs : x_in ? fb + 2 : ring_in + s64;
                const float2* pq = !below ? zpairs : x_in ? fb : ring_in + s62;
                r62 = pq[0];
                r63 = pq[1];
#pragma unroll
                for (int u = 0; u < BD; ++u) rp[u] = pp[u];
            }
            bv = buf[RBUF + lane];
            bv = (s > 0 && lane <= P && t_hi - lane + 63 <= nsteps - 1) ? bv : kNINF;
            if (NWG && s == 0)
                bv = (lane <= P && t_hi - lane + 1 >= 0) ? (float)(t_hi - lane + 1) * gap : kNINF;
            if (!bcast && below && lane >= 64 - P) {
                const int j = 63 - lane;
                if (x_in) {
                    pre_u = buf[FBUF + 2 * (j + 1)];
                    pre_d = buf[FBUF + 2 * j + 1];
                } else {
                    // slots kP+j+63 and kP+j+62, below 2R (R >= 128 > P + 63)
                    int su = slot0 + j + 63;
                    su = su < R ? su : su - R;
                    const int sd = su > 0 ? su - 1 : R - 1;
                    pre_u = ring_in[su].x;
                    pre_d = ring_in[sd].y;
                }
            }
            if (k + 1 < nch) {
                if (x_in) {
                    const int need = min(k + 1 + lead(P), nch);
                    if (seen < need) seen = wait_part(flag_in, epoch, need, st);
                }
                issue_chunk(k + 1);
                if (x_in) flag_load_lds(flag_in, fslot_lds, lane);
            }
            // lane 0 publishes (up, diag) of step u into slot (kP+u) % R
            float2* pub = (lane == 0) ? ring_out + slot0 : sink + lane;
            // lane 63 starts the chunk with the ring's values for steps 0 and 1
            {
                const float u0 = bcast ? r63.x : lane_bcast(pre_u, 63);
                const float d0 = bcast ? r62.y : lane_bcast(pre_d, 63);
                const float d1 = bcast ? r63.y : lane_bcast(pre_d, 62);
                if (lane == 63) { in_up = u0; in_diag = d0; in_diag_next = d1; }
            }
            // PRECISE and NWG: the chunk's parameter-gradient terms are kept for balanced
            // sums; otherwise each term goes into its accumulator with one fma
            constexpr bool TERMS = PRECISE || NWG;
            Acc gs[P], ps[P];
            // the quad being filled: memory-column order, i.e. step 4q + 3 - e in
            // element e (the reverse sweep's columns fall with the step)
            float4 quad = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            float pre_d2 = 0.0f;
            if (!bcast) {
                pre_d2 = wave_shr1(pre_d);    // lane 63 = step 1 (then shifted on)
                pre_d2 = wave_shr1(pre_d2);   // lane 63 = step 2
            }
            // AHEAD: the ring's up values shifted one step ahead (lane 63 = step 1), and
            // lane 0's row-above alphas too (bv of step u + 1): each step shifts the next
            // copy out before its DPP consumes this one as the fill value, so no copy of
            // a live fill register is needed.  The up alpha of step u + 1 is the
            // diagonal of step u.  (PRECISE keeps one register each: its double
            // accumulators leave none to spare.)
            constexpr bool AHEAD = !PRECISE;
            float upa_next = 0.0f;
            if constexpr (AHEAD) {
                if (!bcast) pre_u = wave_shr1(pre_u);
                upa_next = wave_shr1_or(A[1], bv);
                bv = wave_shl1(bv);
            }
            // (SW) beta_init = 2^min((alpha - S) c, 0) is exactly 0 below 2^-150: a chunk
            // none of whose alphas comes within 150 c^-1 of S skips those exponentials
            // (most chunks: alpha grows along the anti-diagonals towards S)
            bool inits = NWG;
            if (!NWG) {
                float amax = A[0];
#pragma unroll
                for (int u = 1; u < P; ++u) amax = fmaxf(amax, A[u]);
                inits = __builtin_amdgcn_ballot_w64((amax - S) * c >= -151.0f) != 0;
            }
            // FULL: every cell of the chunk lies inside the element, no validity masks;
            // INIT: some cell of the chunk has a nonzero beta_init
            auto steps = [&](auto full, auto init) {
            constexpr bool FULL = decltype(full)::value;
            constexpr bool INIT = decltype(init)::value;
#pragma unroll
            for (int u = 0; u < P; ++u) {
                const int t = t_hi - u;
                const bool ok = FULL || (unsigned)(t - lane) < (unsigned)L2eff;
                // cells outside the element hold arbitrary tensor data: neutralise them
                const float sc = ok ? sv[u] : kNINF;
                const float a0 = A[u], a1 = A[u + 1];
                // up / diagonal alphas from lane r-1; lane 0 takes the row above
                float upa, dga;
                if constexpr (QOUT) {
                    if ((u & 3) == 0 && u + 4 < P) read_sq((u >> 2) + 1);
                }
                if constexpr (FULL && BCAST) {
                    if (u + BD < P) rp[u + BD] = pp[u + BD];
                }
                if constexpr (AHEAD) {
                    const float bv2 = wave_shl1(bv);
                    upa = upa_next;
                    dga = wave_shr1_or(A[u + 2], bv);
                    upa_next = dga;
                    bv = bv2;
                } else {
                    const float bv_next = wave_shl1(bv);
                    upa = wave_shr1_or(a1, bv);
                    dga = wave_shr1_or(A[u + 2], bv_next);
                    bv = bv_next;
                }
                const float vd = dga + sc;
                const float vu = upa + gap;
                const float vl = a1 + gap;
                // The weights e_k / sum e: an error in the common shift m*c cancels, so
                // each exponent is one fma, exact up to the rounding of m*c.  That
                // rounding is ~2^75 at the 1e30 sentinels of cells outside the element,
                // so m is floored far below any real alpha (those cells' e_k become 0
                // and their flows are selected away, not multiplied).
                // (FULL: the cell's own alpha a0 = m + T ln(sum) takes the max's place.
                // The forward formed it from these same operands, so a0 >= m, every
                // exponent is at most 0 and the largest term at least 1/4 (a sum of at
                // most four terms); the shift cancels in the normalisation as m's does.
                // PRECISE keeps the max: its registers are all in use.)
                const float m = (FULL && !PRECISE) ? a0
                                : NWG ? fmaxf(fmaxf(vd, vu), fmaxf(vl, -1e20f))
                                      : fmaxf(fmaxf(vd, vu), fmaxf(fmaxf(vl, sc), -1e20f));
                const float mc = m * c;
                const float e0 = fast_exp2(fmaf(vd, c, -mc)), e1 = fast_exp2(fmaf(vu, c, -mc));
                const float e2 = fast_exp2(fmaf(vl, c, -mc));
                const float e3 = NWG ? 0.0f : fast_exp2(fmaf(sc, c, -mc));
                const float e03 = e0 + e3, e12 = e1 + e2;
                const float rin = fast_rcp(e12 + e03);
                float binit;
                if (NWG) {
                    binit = t == term_step ? 1.0f : 0.0f;
                } else if (INIT) {
                    float lp = (a0 - S) * c;   // subtract first: exact for nearby values
                    lp = lp < 0.0f ? lp : 0.0f;
                    binit = fast_exp2(lp);
                } else {
                    binit = 0.0f;
                }
                // reference accumulation order: init, diagonal, left, up successor (the
                // flows are never -0, so without a start term 0 + in_diag is in_diag;
                // NWG: a FULL chunk never holds the terminal cell)
                const float beta = ((NWG && !FULL) || INIT || !AHEAD)
                                       ? ((binit + in_diag) + in_left) + in_up
                                       : (in_diag + in_left) + in_up;
                const bool live = ok && (beta <= 3.0e38f);    // skips inf / NaN like the reference
                const float br = live ? beta * rin : 0.0f;
                const float od = br * e0, ou = br * e1, ol = br * e2;
                const float pv = br * e03;
                if constexpr (QOUT) {
                    if ((u & 3) == 0) quad.w = pv;
                    if ((u & 3) == 1) quad.z = pv;
                    if ((u & 3) == 2) quad.y = pv;
                    if ((u & 3) == 3) {
                        quad.x = pv;
                        *reinterpret_cast<float4*>(obuf + Tile::slot(lane, u >> 2)) = quad;
                    }
                } else {
                    buf[obase_lane + u] = pv;
                }
                if (PRECISE) gs[u] = (Acc)ou + (Acc)ol;
                else if (TERMS) gs[u] = br * e12;
                else g_acc = fmaf(br, e12, g_acc);
                if (NWG) {
                    // flows into the boundary: column 0 (left: i gaps, diagonal: i - 1)
                    // and row 0 (up: column + 1 gaps, diagonal: column); FULL chunks can
                    // hold column 0 (lane 63) and row 1
                    const int col = t - lane;
                    if (col == 0) gs[u] += (Acc)(ol * gi) + (Acc)(od * (gi - 1.0f));
                    if (top) gs[u] += (Acc)(ou * (float)(col + 1)) + (Acc)(od * (float)col);
                }
                if (TERMS) ps[u] = (Acc)(pv * sc);
                else p_acc = fmaf(pv, sc, p_acc);
                pub[u] = make_float2(ou, od);
                // successor contributions for the next steps; lane 63 takes the ring
                if constexpr (FULL && BCAST) {
                    in_left = ol;
                    in_up = wave_shl1_or(ou, rp[u].x);
                    in_diag = in_diag_next;
                    in_diag_next = wave_shl1_or(od, rp[u].y);
                } else {
                    if constexpr (AHEAD) {
                        const float pre_u2 = wave_shr1(pre_u);
                        in_left = ol;
                        in_up = wave_shl1_or(ou, pre_u);
                        pre_u = pre_u2;
                    } else {
                        pre_u = wave_shr1(pre_u);
                        in_left = ol;
                        in_up = wave_shl1_or(ou, pre_u);
                    }
                    in_diag = in_diag_next;
                    in_diag_next = wave_shl1_or(od, pre_d2);
                    pre_d2 = wave_shr1(pre_d2);
                }
            }
            };
            if (inside) {
                if (inits) steps(std::true_type{}, std::true_type{});
                else steps(std::true_type{}, std::false_type{});
            } else {
                if (inits) steps(std::false_type{}, std::true_type{});
                else steps(std::false_type{}, std::false_type{});
            }
            prog_ahead(ahead, prog, HELP ? hprog : nullptr, q, NL, q);

            // the chunk's parameter-gradient terms: balanced sums, then one add each
            if (TERMS) {
                g_acc += tree_sum<P>(gs);
                p_acc += tree_sum<P>(ps);
            }
            wave_lds_sync();
            // write this chunk's marginals back over the cells the scores came from:
            // NSTORE stores (P dword stores in a boundary chunk, where cells outside the
            // element's lengths go to the trash line; inside chunks carry 0 there)
            if constexpr (HELP)
                ;   // the helper writes the tile once this chunk is published
            else if constexpr (QOUT)
                write_quads<P, -1>(buf, pbase, trash, i0, L1, L2, L1max, L2max, lane, t_hi);
            else
                write_tile<P, -1>(buf, pbase, trash, i0, L1, L2, L1max, L2max, lane, t_hi);
            publish(prog, wave, q * PROG_STRIDE + k + 1);
            if (x_out) {
                // this chunk's flows to the part above, by producer step
                if (lane < P) store_sys2(flows_out + k * P + lane, ring_out[slot0 + lane]);
                if (HELP && !x_in && k >= 1) {
                    // HELP, a part's last stripe that is not also its first: its only
                    // memory operations are its flow stores and its flag stores (one
                    // per chunk from chunk 1 on), so once at most the previous chunk's
                    // flag store and this chunk's flow store are outstanding, every
                    // chunk before this one is complete
                    if (k == 1) wait_vmcnt<1>(); else wait_vmcnt<2>();
                    if (lane == 0) store_flag(flag_out, progress_word(epoch, k));
                } else if (k >= 2) {
                    // at least (2 P/4 + 1) loads and NSTORE stores of chunk k - 1, NSTORE
                    // stores of chunk k and the two chunks' flow stores follow the flow
                    // store of chunk k - 2 (HELP: the flow loads of chunk k + 1 and the
                    // two flow stores): it is complete
                    if constexpr (HELP) wait_vmcnt<3>();
                    else wait_vmcnt<2 * Tile::NQ + 2 * NSTORE + 3>();
                    if (lane == 0) store_flag(flag_out, progress_word(epoch, k - 1));
                }
            }
        }
        if (x_out) {
            wait_vmcnt<0>();
            if (lane == 0) store_flag(flag_out, progress_word(epoch, nch));
        }
    }

    g_acc = wave_sum(g_acc);
    p_acc = wave_sum(p_acc);
    if (lane == 0 && wave < NW) { red_g[wave] = g_acc; red_p[wave] = p_acc; }
    __syncthreads();
    if (threadIdx.x == 0) {
        Acc g = 0, p = 0;
        for (int w = 0; w < NW; ++w) { g += red_g[w]; p += red_p[w]; }
        // NWG: an element without cells is its boundary, (L1 + L2) gaps (part 0 counts it)
        if (NWG && NS == 0 && part == 0) g += (Acc)(L1 + L2);
        if (G == 1) {
            grad_gap[b] = (float)g;
            grad_T[b] = (float)(((Acc)S - (p + g * (Acc)gap)) / (Acc)T);
        } else {
            bpart[((size_t)b * G + part) * 2] = (double)g;
            bpart[((size_t)b * G + part) * 2 + 1] = (double)p;
        }
    }
    // The last sweep of an unsplit call: an element whose waits gave up (in the forward
    // or in this sweep) gets NaN in all its outputs (the separate poison pass of split
    // calls).  Every wave first completes its own status atomics and stores; then one
    // thread reads the status word and every wave branches on that one value, so the
    // fill below runs in every wave or in none.
    if (G == 1 && poison_value != nullptr) {
        __shared__ int poison_flag;
        wait_vmcnt<0>();
        __syncthreads();
        if (threadIdx.x == 0) poison_flag = load_status(st);
        __syncthreads();
        if (poison_flag == 0) return;
        const float nan = __builtin_nanf("");
        for (size_t i = threadIdx.x; i < (size_t)L1max * L2max; i += blockDim.x) pbase[i] = nan;
        if (threadIdx.x == 0) {
            poison_value[b] = nan;
            grad_gap[b] = nan;
            grad_T[b] = nan;
        }
    }
}

// grad_gap[b], grad_T[b] of a split element from the parts' sums.
template <bool PRECISE>
__global__ void sw_grad_merge(const double* __restrict__ bpart, const float* __restrict__ partition,
                              float* __restrict__ grad_gap, float* __restrict__ grad_T, int B,
                              int G, float gap, float T) {
    using Acc = typename std::conditional<PRECISE, double, float>::type;
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    Acc g = 0, p = 0;
    for (int i = 0; i < G; ++i) {
        g += (Acc)bpart[((size_t)b * G + i) * 2];
        p += (Acc)bpart[((size_t)b * G + i) * 2 + 1];
    }
    grad_gap[b] = (float)g;
    grad_T[b] = (float)(((Acc)partition[b] - (p + g * (Acc)gap)) / (Acc)T);
}

}  // namespace sw
}  // namespace d2p_amd

namespace d2p_amd {
namespace sw {

namespace {
// dynamic LDS bound: 160 KiB less the kernels' static arrays (progress words,
// reductions, the prefetched progress-word slot)
constexpr size_t kLdsLimit = 160 * 1024 - 512;

// LDS of one workgroup whose stripes' boundaries use rings of R columns
// ntb: score tiles per sweeping wave (4 in the 16-wave forward)
// (tan: the fused tangent sweep's second tile per chunk, rows and ring)
size_t lds_forward_r(int R, int ntb = 2, bool tan = false) {
    const int ntl = tan ? 2 : 1;
    return (size_t)wf::NW * (ntl * (ntb * 64 * PF + 2 * 64) + PF) * sizeof(float) +
           ((size_t)ntl * wf::NW * R + wf::NW * DUMMY) * sizeof(float);
}
size_t lds_backward_r(int R, int P) {
    return (size_t)wf::NW * 2 * (64 * P + 64 * P + 64 + 64) * sizeof(float) +
           ((size_t)wf::NW * R + wf::NW * DUMMY) * sizeof(float2);
}
// rings of a workgroup that runs `rows` rows of stripes
int ring_forward(int rows, int max_L2) { return wf::ring_len(rows, max_L2, 256); }
int ring_backward(int rows, int max_L2) { return wf::ring_len(rows, max_L2, 128); }

// backward: 16-step chunks when they fit in LDS, else 8-step chunks (long rows need
// long rings)
int backward_chunk(int rows, int max_L2) {
    return lds_backward_r(ring_backward(rows, max_L2), 16) <= kLdsLimit ? 16 : 8;
}

// Stripes per part that a launch may not exceed: 0 when the rings of an unsplit
// element fit in LDS, else NW (a part of at most NW stripes needs only the minimum
// ring, which always fits).
int max_stripes_forward(int max_L1, int max_L2) {
    return lds_forward_r(ring_forward(max_L1, max_L2)) <= kLdsLimit ? 0 : wf::NW;
}
int max_stripes_backward(int max_L1, int max_L2) {
    return lds_backward_r(ring_backward(max_L1, max_L2), 8) <= kLdsLimit ? 0 : wf::NW;
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

// D2P_AMD_SW_HELPERS=0 turns the helper waves off (for tests: both forms must agree)
static bool helpers_enabled() {
    const char* e = std::getenv("D2P_AMD_SW_HELPERS");
    return !(e && e[0] == '0');
}

template <bool NWG, bool HELP, bool WIDE = false, bool TAN = false>
int launch_forward_k(const float* scores, const int* lengths, int B, int max_L1, int max_L2,
                     float gap, float T, const Layout& ws, float* partition, hipStream_t st,
                     const Split& sp, int R, size_t lds, uint32_t epoch, bool ckpt,
                     TanArgs ta = TanArgs{}) {
    const int ns = (max_L1 + 63) / 64;
    D2P_HIP(hipFuncSetAttribute((const void*)sw_forward_kernel<NWG, HELP, WIDE, TAN>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    D2P_LAUNCH(TAN ? (NWG ? "nw_forward_tangent" : "sw_forward_tangent")
                   : (NWG ? "nw_forward" : "sw_forward"),
               (sw_forward_kernel<NWG, HELP, WIDE, TAN>),
               dim3(wf::split_grid(B, sp.G)), dim3((WIDE ? 2 : 1) * wf::NW * 64), lds, st, scores,
               lengths,
               ws.alpha_sk, ws.brow, partition, ws.status, ws.fflag, ws.fpart, B, max_L1, max_L2,
               ns, gap, T, R, sp.G, sp.SPW, epoch, ckpt ? 1 : 0, ta);
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

int launch_forward(const float* scores, const int* lengths, int B, int max_L1, int max_L2,
                   float gap, float T, const Layout& ws, float* partition, hipStream_t st,
                   bool global, bool ckpt) {
    const int ns = (max_L1 + 63) / 64;
    const Split sp = choose_split(B, max_L1, ws, max_stripes_forward(max_L1, max_L2));
    const int R = ring_forward(sp.G > 1 ? sp.SPW * 64 : max_L1, max_L2);
    const size_t lds = lds_forward_r(R);
    D2P_REQUIRE(lds <= kLdsLimit, "sequence too long for the LDS stripe rings");
    const uint32_t epoch = next_epoch();
    if (sp.G > 1 && wf::launch_split_reset(ws, B, sp.G, st) != D2P_OK) return D2P_ERR_HIP;
    // helper waves move the data: the idle waves when a part has at most NW/2
    // stripes, a second set of NW waves when it has at most NW
    const int part_stripes = sp.G > 1 ? sp.SPW : ns;
    const bool help = part_stripes <= wf::NW / 2 && helpers_enabled();
    const bool wide = !help && part_stripes <= wf::NW && helpers_enabled() &&
                      lds_forward_r(R, 4) <= kLdsLimit;
#define D2P_SW_FWD(G_, H_, W_) \
    launch_forward_k<G_, H_, W_>(scores, lengths, B, max_L1, max_L2, gap, T, ws, partition, st, \
                                 sp, R, W_ ? lds_forward_r(R, 4) : lds, epoch, ckpt && !global)
    if (global)
        return help ? D2P_SW_FWD(true, true, false)
                    : wide ? D2P_SW_FWD(true, true, true) : D2P_SW_FWD(true, false, false);
    // (the owner part writes the NW value: no merge)
    D2P_TRY(help ? D2P_SW_FWD(false, true, false)
                 : wide ? D2P_SW_FWD(false, true, true) : D2P_SW_FWD(false, false, false));
#undef D2P_SW_FWD
    if (sp.G > 1 && wf::launch_partition_merge(ws, partition, B, sp.G, T, st) != D2P_OK)
        return D2P_ERR_HIP;
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

int launch_forward_tangent(const float* scores, const float* V, const int* lengths, int B,
                           int max_L1, int max_L2, float gap, float T, const Layout& ws,
                           float* partition, float* tan_sk, float* tan_brow, float* sdot,
                           float* wpart, hipStream_t st, bool global) {
    // rings of an unsplit element that do not fit: parts of at most NW stripes, whose
    // rings (256 steps) fit whatever the row length
    const int ns = (max_L1 + 63) / 64;
    const bool whole = lds_forward_r(ring_forward(max_L1, max_L2), 2, true) <= kLdsLimit;
    const Split sp = choose_split(B, max_L1, ws, whole ? 0 : wf::NW);
    const int R = ring_forward(sp.G > 1 ? sp.SPW * 64 : max_L1, max_L2);
    const size_t lds = lds_forward_r(R, 2, true);
    D2P_REQUIRE(lds <= kLdsLimit, "sequence too long for the LDS stripe rings");
    const uint32_t epoch = next_epoch();
    if (sp.G > 1 && wf::launch_split_reset(ws, B, sp.G, st) != D2P_OK) return D2P_ERR_HIP;
    const int part_stripes = sp.G > 1 ? sp.SPW : ns;
    const bool help = part_stripes <= wf::NW / 2 && helpers_enabled();
    const TanArgs ta{V, tan_sk, tan_brow, sdot, wpart};
#define D2P_SW_FWDT(G_, H_) \
    launch_forward_k<G_, H_, false, true>(scores, lengths, B, max_L1, max_L2, gap, T, ws, \
                                          partition, st, sp, R, lds, epoch, false, ta)
    if (global) return help ? D2P_SW_FWDT(true, true) : D2P_SW_FWDT(true, false);
    D2P_TRY(help ? D2P_SW_FWDT(false, true) : D2P_SW_FWDT(false, false));
#undef D2P_SW_FWDT
    if (sp.G > 1 &&
        wf::launch_partition_dot_merge(ws, wpart, partition, sdot, B, sp.G, T, st) != D2P_OK)
        return D2P_ERR_HIP;
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

template <int P, bool PRECISE, bool NWG, bool HELP = false, bool WIDE = false,
          bool RECOMP = false>
int launch_backward_p(const float* scores, const int* lengths, int B, int max_L1, int max_L2,
                      float gap, float T, const Layout& ws, const float* partition,
                      float* marginals, float* grad_gap, float* grad_T, hipStream_t st,
                      const Split& sp, int R, float* poison_value) {
    const int ns = (max_L1 + 63) / 64;
    const size_t lds = lds_backward_r(R, P);
    D2P_REQUIRE(lds <= kLdsLimit, "sequence too long for the LDS stripe rings");
    const uint32_t epoch = next_epoch();
    if (sp.G > 1) D2P_TRY(wf::launch_flag_reset(ws.bflag, B * sp.G, st));
    D2P_HIP(hipFuncSetAttribute(
        (const void*)sw_backward_kernel<P, PRECISE, NWG, HELP, WIDE, RECOMP>,
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    D2P_LAUNCH(NWG ? "nw_backward" : "sw_backward",
               (sw_backward_kernel<P, PRECISE, NWG, HELP, WIDE, RECOMP>),
               dim3(wf::split_grid(B, sp.G)),
               dim3((WIDE ? 2 : 1) * wf::NW * 64), lds, st, scores, lengths, ws.alpha_sk, ws.brow, partition,
               marginals, grad_gap, grad_T, ws.status, ws.trash, ws.bflag, ws.flows, ws.bpart,
               sp.G == 1 ? poison_value : nullptr, B, max_L1, max_L2, ns, gap, T, R, sp.G, sp.SPW,
               epoch);
    if (sp.G > 1)
        D2P_LAUNCH("sw_grad_merge", sw_grad_merge<PRECISE>, dim3((B + 255) / 256), dim3(256), 0,
                   st, ws.bpart, partition, grad_gap, grad_T, B, sp.G, gap, T);
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

namespace {
// The reverse sweep's launch shape: parts, and whether its helper waves run as half the
// workgroup (parts of at most NW/2 stripes) or as a second set of NW waves.
struct BackwardShape {
    Split sp;
    int rows, R, P;
    bool help, wide;
};
BackwardShape backward_shape(int B, int max_L1, int max_L2, const Layout& ws, bool precise) {
    BackwardShape bs;
    bs.sp = choose_split(B, max_L1, ws, max_stripes_backward(max_L1, max_L2));
    bs.rows = bs.sp.G > 1 ? bs.sp.SPW * 64 : max_L1;
    bs.R = ring_backward(bs.rows, max_L2);
    bs.P = backward_chunk(bs.rows, max_L2);
    const int part_stripes = (bs.rows + 63) / 64;
    bs.help = !precise && bs.P == 16 && part_stripes <= wf::NW / 2 && helpers_enabled();
    bs.wide = !precise && bs.P == 16 && !bs.help && part_stripes <= wf::NW && helpers_enabled();
    return bs;
}
}  // namespace

// Store or recompute: whether a first-order SW call stores only the forward's checkpoint
// rows and lets the reverse sweep rebuild alpha (only the 16-wave reverse sweep can).
// Measured at C2 ([256, 512, 512]): the checkpoint forward takes 161 us against 168,
// but the recomputing reverse sweep 307 us against 262 (its helper waves' recurrence
// competes with the sweeping waves for the same SIMDs), 0.571 ms per step against
// 0.540: the full table is the default.  D2P_AMD_SW_RECOMPUTE=1 recomputes wherever
// the 16-wave reverse sweep runs.
bool recompute_alpha(int B, int max_L1, int max_L2, const Layout& ws) {
    const char* e = std::getenv("D2P_AMD_SW_RECOMPUTE");
    if (!(e && e[0] == '1')) return false;
    const BackwardShape bs = backward_shape(B, max_L1, max_L2, ws, false);
    return bs.wide || bs.help;
}

int launch_backward(const float* scores, const int* lengths, int B, int max_L1, int max_L2,
                    float gap, float T, const Layout& ws, const float* partition,
                    float* marginals, float* grad_gap, float* grad_T, hipStream_t st,
                    bool precise, bool global, float* poison_value, bool* poisoned,
                    bool recompute) {
    const BackwardShape bs = backward_shape(B, max_L1, max_L2, ws, precise);
    const Split& sp = bs.sp;
    if (poisoned != nullptr) *poisoned = sp.G == 1 && poison_value != nullptr;
    const int R = bs.R, P = bs.P;
#define D2P_SW_BWD(P_, PR_, G_)                                                               \
    launch_backward_p<P_, PR_, G_>(scores, lengths, B, max_L1, max_L2, gap, T, ws, partition, \
                                   marginals, grad_gap, grad_T, st, sp, R, poison_value)
    if (global) {
        if (P == 16) return precise ? D2P_SW_BWD(16, true, true) : D2P_SW_BWD(16, false, true);
        return precise ? D2P_SW_BWD(8, true, true) : D2P_SW_BWD(8, false, true);
    }
    // helper waves move the data: the idle waves when a part has at most NW/2
    // stripes, a second set of NW waves when it has at most NW
    const bool help = bs.help, wide = bs.wide;
    D2P_REQUIRE(!recompute || ((wide || help) && !global),
                "recomputation needs a reverse sweep with helper waves");
    if (recompute && wide)
        return launch_backward_p<16, false, false, true, true, true>(
            scores, lengths, B, max_L1, max_L2, gap, T, ws, partition, marginals, grad_gap,
            grad_T, st, sp, R, poison_value);
    if (recompute)
        return launch_backward_p<16, false, false, true, false, true>(
            scores, lengths, B, max_L1, max_L2, gap, T, ws, partition, marginals, grad_gap,
            grad_T, st, sp, R, poison_value);
    if (help)
        return launch_backward_p<16, false, false, true>(scores, lengths, B, max_L1, max_L2, gap,
                                                         T, ws, partition, marginals, grad_gap,
                                                         grad_T, st, sp, R, poison_value);
    if (wide)
        return launch_backward_p<16, false, false, true, true>(
            scores, lengths, B, max_L1, max_L2, gap, T, ws, partition, marginals, grad_gap,
            grad_T, st, sp, R, poison_value);
    if (P == 16) return precise ? D2P_SW_BWD(16, true, false) : D2P_SW_BWD(16, false, false);
    return precise ? D2P_SW_BWD(8, true, false) : D2P_SW_BWD(8, false, false);
#undef D2P_SW_BWD
}

}  // namespace sw
}  // namespace d2p_amd

using namespace d2p_amd;

extern "C" size_t d2p_sw_workspace_bytes(int B, int max_L1, int max_L2) {
    if (B <= 0 || max_L1 < 0 || max_L2 < 0) return 0;
    // status words | trash line | skewed alpha table | last row of every stripe |
    // split-element progress words, boundary flows and partial sums
    return wf::layout(nullptr, B, max_L1, max_L2, 1, true).bytes;
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
    D2P_REQUIRE(scores && partition && marginals && grad_gap && grad_T,
                "null pointer argument");
    const size_t need = d2p_sw_workspace_bytes(B, max_L1, max_L2);
    D2P_REQUIRE(workspace && workspace_bytes >= need, "workspace too small");
    hipStream_t st = (hipStream_t)stream;
    const wf::Layout ws = wf::layout(workspace, B, max_L1, max_L2, 1, true);
    const bool recompute = sw::recompute_alpha(B, max_L1, max_L2, ws);
    D2P_TRY(sw::launch_forward(scores, lengths, B, max_L1, max_L2, gap, temperature, ws,
                               partition, st, false, recompute));
    bool poisoned = false;
    D2P_TRY(sw::launch_backward(scores, lengths, B, max_L1, max_L2, gap, temperature, ws,
                                partition, marginals, grad_gap, grad_T, st, false, false,
                                partition, &poisoned, recompute));
    if (poisoned) return D2P_OK;
    return wf::launch_poison(ws.status, B, (long long)max_L1 * max_L2, marginals, nullptr,
                             partition, grad_gap, grad_T, nullptr, st);
}

// ---------------------------------------------------------------------------
// Allocation-free variant of d2p_sw_forward_marginals: the workspace is a static
// device array of this file, one copy per GPU (held from the library's first use
// on that device to the end of the process).
// ---------------------------------------------------------------------------
namespace {
constexpr size_t kScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the current device, resolved once per device (the
// array's name is only a host-side handle: never pass it to a kernel).
int scratch_on_current_device(void** out) {
    int dev = -1;
    D2P_HIP(hipGetDevice(&dev));
    D2P_REQUIRE(dev >= 0 && dev < kMaxDevices, "device ordinal out of range");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        D2P_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        D2P_REQUIRE(p != nullptr, "hipGetSymbolAddress returned a null scratch address");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return D2P_OK;
}
}  // namespace

extern "C" size_t d2p_sw_noalloc_scratch_bytes(void) { return kScratchBytes; }

extern "C" int d2p_sw_forward_marginals_noalloc(const float* scores, const int* lengths, int B,
                                                int max_L1, int max_L2, float gap,
                                                float temperature, float* partition,
                                                float* marginals, float* grad_gap,
                                                float* grad_T, void* stream) {
    const int rc = sw::check_shape(B, max_L1, max_L2, temperature);
    if (rc != D2P_OK) return rc;
    if (B == 0) return D2P_OK;
    D2P_REQUIRE(scores && partition && marginals && grad_gap && grad_T,
                "null pointer argument");
    const size_t need = d2p_sw_workspace_bytes(B, max_L1, max_L2);
    if (need > kScratchBytes) {
        set_last_error("shape needs %zu workspace bytes, more than the %zu-byte static scratch "
                       "of d2p_sw_forward_marginals_noalloc (use d2p_sw_forward_marginals)",
                       need, kScratchBytes);
        return D2P_ERR_ARG;
    }
    void* ws_ptr = nullptr;
    D2P_TRY(scratch_on_current_device(&ws_ptr));
    // the sweeps reset every word of the workspace they rely on (status and progress
    // words) themselves, with kernels: the previous call's contents do not matter
    hipStream_t st = (hipStream_t)stream;
    const wf::Layout ws = wf::layout(ws_ptr, B, max_L1, max_L2, 1, true);
    const bool recompute = sw::recompute_alpha(B, max_L1, max_L2, ws);
    D2P_TRY(sw::launch_forward(scores, lengths, B, max_L1, max_L2, gap, temperature, ws,
                               partition, st, false, recompute));
    bool poisoned = false;
    D2P_TRY(sw::launch_backward(scores, lengths, B, max_L1, max_L2, gap, temperature, ws,
                                partition, marginals, grad_gap, grad_T, st, false, false,
                                partition, &poisoned, recompute));
    if (poisoned) return D2P_OK;
    return wf::launch_poison(ws.status, B, (long long)max_L1 * max_L2, marginals, nullptr,
                             partition, grad_gap, grad_T, nullptr, st);
}

extern "C" size_t d2p_nw_workspace_bytes(int B, int max_L1, int max_L2) {
    return d2p_sw_workspace_bytes(B, max_L1, max_L2);
}

extern "C" int d2p_nw_forward_marginals(const float* scores, const int* lengths, int B,
                                        int max_L1, int max_L2, float gap, float temperature,
                                        float* value, float* marginals, float* grad_gap,
                                        float* grad_T, void* workspace,
                                        size_t workspace_bytes, void* stream) {
    const int rc = sw::check_shape(B, max_L1, max_L2, temperature);
    if (rc != D2P_OK) return rc;
    if (B == 0) return D2P_OK;
    D2P_REQUIRE(scores && value && marginals && grad_gap && grad_T,
                "null pointer argument");
    const size_t need = d2p_nw_workspace_bytes(B, max_L1, max_L2);
    D2P_REQUIRE(workspace && workspace_bytes >= need, "workspace too small");
    hipStream_t st = (hipStream_t)stream;
    const wf::Layout ws = wf::layout(workspace, B, max_L1, max_L2, 1, true);
    D2P_TRY(sw::launch_forward(scores, lengths, B, max_L1, max_L2, gap, temperature, ws, value,
                               st, true));
    bool poisoned = false;
    D2P_TRY(sw::launch_backward(scores, lengths, B, max_L1, max_L2, gap, temperature, ws, value,
                                marginals, grad_gap, grad_T, st, false, true, value, &poisoned));
    if (poisoned) return D2P_OK;
    return wf::launch_poison(ws.status, B, (long long)max_L1 * max_L2, marginals, nullptr, value,
                             grad_gap, grad_T, nullptr, st);
}
