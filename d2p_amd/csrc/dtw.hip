// dtw.hip -- soft dynamic time warping on gfx950.
//
// Reference behaviour restated (not translated):
//   forward   /root/reference/src/dtw/kernels_cpu.cpp:58-121
//   backward  /root/reference/src/dtw/kernels_cpu.cpp:127-223
//   band      /root/reference/src/dtw/kernels_cpu.cpp:24-29 (float arithmetic)
// DP over the costs c[i,j] (i, j >= 1):
//   alpha[i,j] = c[i,j] + softmin_T(alpha[i-1,j-1], alpha[i-1,j], alpha[i,j-1])
//   softmin_T(x) = m - T*log(sum exp((m - x)/T)),  m = min(x)
// alpha[0,0] = 0, every other row/column 0 value is PINF, cells outside the
// Sakoe-Chiba band (|j - i*L2/L1| > bandwidth, bandwidth >= 0) are PINF, and the
// value is alpha[L1, L2].  The backward starts from beta[L1,L2] = 1, spreads beta
// to the predecessors through the softmin weights, and the marginal is beta; the
// temperature gradient is sum beta * (softmin - E_w[alpha_pred]) / T.
//
// Mapping: the stripe pipeline of wavefront.hip.h with the linear Smith-Waterman
// layout (one alpha plane).  The band test needs i*L2/L1 per row: each lane computes
// it once per stripe, so the per-cell test is a subtraction and a compare.

#include <algorithm>
#include <cstdlib>
#include <vector>

#include <type_traits>

#include "wavefront.hip.h"
#include "../../include/d2p_amd.h"
#include "capi_util.hip.h"
#include "dtw_internal.hip.h"

namespace d2p_amd {
namespace dtw {

using namespace wf;

constexpr int DUMMY = 64 + PF;       // per-wave LDS sink for the lanes that do not publish

// HELP (costs from memory, unbanded, at most NW/2 stripes per part): wave NW/2 + l
// loads stripe l's cost chunks one chunk ahead into wave l's tiles (cprog[l] = chunks
// loaded) and writes each chunk's alpha rows to the table from a tile in its own,
// otherwise unused, buffers once wave l has finished the chunk.
template <bool HELP = false>
__global__ void __launch_bounds__(NW * 64)
dtw_forward_kernel(const float* __restrict__ costs, const int* __restrict__ lengths,
                   float* __restrict__ alpha_sk, float* __restrict__ brow,
                   float* __restrict__ value, int* __restrict__ status,
                   uint64_t* __restrict__ fflag, int B, int L1max, int L2max, int NSmax,
                   size_t elem_steps, float T, int bandwidth, int R, int G, int SPW,
                   uint32_t epoch) {
    constexpr int P = PF;
    static_assert(!HELP || P == 16, "the helper split assumes 16-step chunks");
    extern __shared__ __align__(16) float smem[];
    __shared__ int prog[NW];
    __shared__ int cprog[NW];     // HELP: chunks of stripe l's costs formed (or loaded)
                                  // by its helper
    __shared__ float terminal;
    // part of the element as in the linear-SW forward: the first stripe of a part > 0
    // reads the previous part's last row from brow
    int b, part;
    split_decode(blockIdx.x, G, b, part);
    if (b >= B) return;
    const int lane = threadIdx.x & 63;
    const unsigned ul4 = (unsigned)lane * 4u;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    using Tile = ChunkTile<P>;
    // two cost chunks, two rows
    constexpr int NTILE = 2;
    constexpr int WBUF = NTILE * Tile::FLOATS + 2 * 64;
    float* tiles = smem + wave * WBUF;                     // double-buffered cost chunk
    float* rbufs = tiles + NTILE * Tile::FLOATS;           // boundary row of a chunk
    __shared__ float fslot[64];   // progress word prefetched by wave 0, the only wave whose
                                  // stripe borders another part
    const uint32_t fslot_lds = lds_address(fslot);
    float* rings = smem + NW * WBUF;                       // [NW][R]
    float* sink = rings + NW * R + wave * DUMMY;           // per-wave write sink
    int* st = status + b;
    const int tbase = Tile::read_base(lane);

    if (lane == 0) {
        prog[wave] = -1;
        cprog[wave] = -1;
    }
    if (threadIdx.x == 0) {
        if (G == 1) *st = 0;                               // G > 1: reset before the launch
        terminal = kPINF;
    }
    __syncthreads();

    const int L1 = lengths ? min(max(lengths[2 * b], 0), L1max) : L1max;
    const int L2 = lengths ? min(max(lengths[2 * b + 1], 0), L2max) : L2max;
    const float c = kLog2e / T;
    const float tl = T * kLn2;
    // a band test with an empty side is always true (reference: L1 == 0 || L2 == 0)
    const float bw = (bandwidth < 0 || L1 == 0 || L2 == 0) ? -1.0f : (float)bandwidth;
    const int NS = L2 > 0 ? (L1 + 63) >> 6 : 0;
    const int nsteps = L2 + 63;
    const int nch = (nsteps + P - 1) / P;
    const size_t NT = (size_t)stored_steps(L2max);
    const float* cbase = costs + (size_t)b * L1max * L2max;
    const int s_begin = part * SPW;
    const int NL = max(min(NS, s_begin + SPW) - s_begin, 0);   // stripes of this part
    const bool has_next = s_begin + NL < NS;
    const uint64_t* flag_in = fflag + (size_t)b * G + (part > 0 ? part - 1 : 0);
    uint64_t* flag_out = fflag + (size_t)b * G + part;
    const int stride = band_stride(L1, L2, bw, (int)NT);   // table steps per stripe
    if ((size_t)NS * stride > elem_steps) {   // never: the host reserves enough
        if (threadIdx.x == 0) atomicOr(st, 2);
        return;
    }

    if constexpr (HELP) {
        if (NL > NW / 2 || bandwidth >= 0) {   // never: the host picks HELP for these only
            if (threadIdx.x == 0) atomicOr(st, 2);
            return;
        }
        const int l = wave - NW / 2;
        if (l >= 0 && l < NL) {
            const int s = s_begin + l;
            const int i0 = s * 64;
            // unbanded: the window is every chunk and the table starts at step 0
            float* out = band_stripe(alpha_sk, b, elem_steps, s, stride) + APAD * 64;
            const uint32_t ltiles = lds_address(smem + l * WBUF);   // wave l's cost tiles
            const float* atiles = smem + wave * WBUF;               // its alpha tiles
            auto load = [&](int k) {
                dma_tile<P, 1>(ltiles + (k & 1) * Tile::FLOATS * 4, cbase, i0, L1max, L2max,
                               lane, k * P);
            };
            if (nch > 0) {
                load(0);
                wait_vmcnt<0>();
                publish(cprog, l, 1);
                if (nch > 1) load(1);
            }
            for (int k = 0; k < nch; ++k) {
                if (k + 1 < nch) {
                    // chunk k + 1's loads: the last issued at k = 0, else followed by the
                    // P/4 alpha stores of chunk k - 1
                    if (k == 0) wait_vmcnt<0>(); else wait_vmcnt<P / 4>();
                    publish(cprog, l, k + 2);   // also completes this wave's LDS reads
                }
                // once wave l has finished chunk k, its cost tile k & 1 takes chunk k + 2
                // and its alpha rows (alpha tile k & 1) go to the table
                wait_for(prog, l, l * PROG_STRIDE + k + 1, st);
                if (k + 2 < nch) load(k + 2);
                const float* at = atiles + (k & 1) * Tile::FLOATS;
                float* dst = out + (size_t)k * P * 64;
#pragma unroll
                for (int i = 0; i < P / 4; ++i) {
                    const float4 v = *reinterpret_cast<const float4*>(at + 256 * i + 4 * lane);
                    *reinterpret_cast<float4*>(dst + 256 * i + 4 * lane) = v;
                }
            }
        }
    }

    for (int l = wave; l < NL; l += NW) {
        const int s = s_begin + l;
        const int i0 = s * 64;
        const int L2eff = (i0 + lane < L1) ? L2 : 0;   // rows past L1 are never valid
        const float ej = band_centre(i0 + lane + 1, L1, L2);
        const bool last_row = i0 + lane == L1 - 1;
        const float* ring_in = ring_from(rings, l, R);
        float* ring_out = ring_of(rings, l, R);
        // the chunks [k_lo, k_end) of the stripe's band window (all without a band),
        // and the steps [up_lo, up_end) the stripe above computed
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
        // table step t of this stripe at out + (t - sh) * 64
        const int sh = k_lo * P;
        float* out = band_stripe(alpha_sk, b, elem_steps, s, stride) + APAD * 64;
        float* brow_s = brow + ((size_t)b * NSmax + s) * NT;   // last row, by step
        const float* brow_up = brow + ((size_t)b * NSmax + (s > 0 ? s - 1 : 0)) * NT;
        const bool x_in = l == 0 && part > 0;        // row above from the previous part
        const bool x_out = l == NL - 1 && has_next;  // last row feeds the next part
        int seen = -1;       // chunks of the previous part known to be complete
        // the APAD steps before the window hold the column-0 / off-band boundary
        // (PINF), read by the reverse sweep; so does the chunk after it
#pragma unroll
        for (int t = -APAD; t < 0; ++t) lane_store(out + t * 64, ul4, kPINF);
        if (k_end < nch) {
#pragma unroll
            for (int t = 0; t < P; ++t) lane_store(out + (k_end * P - sh + t) * 64, ul4, kPINF);
        }
        // the last row outside the window is PINF
        for (int t = lane; t < k_lo * P; t += 64) {
            if (x_out) store_sys(brow_s + t, kPINF);
            else brow_s[t] = kPINF;
        }
        for (int t = k_end * P + lane; t < nch * P; t += 64) {
            if (x_out) store_sys(brow_s + t, kPINF);
            else brow_s[t] = kPINF;
        }
        publish(prog, wave, l * PROG_STRIDE + k_lo);   // nothing to do before the window
        wave_lds_sync();   // the previous stripe's tile reads are complete
        const uint32_t tile_lds = lds_address(tiles);
        const uint32_t row_lds = lds_address(rbufs);
        // the boundary row of chunk k: lane j < P carries the step kP + 63 + j
        auto issue_row = [&](int k) {
            uint32_t off = (uint32_t)min(k * P + 63 + min(lane, P - 1), nsteps - 1) * 4u;
            uint32_t dst = row_lds + (uint32_t)((k & 1) * 64 * 4);
            lds_dma_dword_sys<0>(brow_up, off, dst, 0u);
        };
        if (k_lo < k_end) {
            if (x_in) {
                seen = wait_part(flag_in, epoch, min(k_lo + lead(P), nch), st);
                issue_row(k_lo);
            }
            if (!HELP)
                dma_tile<P, 1>(tile_lds + (k_lo & 1) * Tile::FLOATS * 4, cbase, i0, L1max, L2max,
                               lane, k_lo * P);
        }
        // lane 0 of the first stripe sees alpha[0,0] = 0 as its first diagonal (when
        // its window starts at step 0)
        float cur = kPINF, up_prev = (s == 0 && lane == 0 && k_lo == 0) ? 0.0f : kPINF;

        for (int k = k_lo; k < k_end; ++k) {
            const int t0 = k * P;
            chunk_waits<P>(prog, l, NL, k, nch, R, st, k_lo);
            // this chunk's costs: loaded one chunk ago, followed by at least the P + 1
            // stores of that chunk (the first chunk's load is the last issued).
            // HELP from memory: the helper loads the costs; this wave's own loads (the
            // row above of a part's first stripe) are followed by the last-row store
            if (k == k_lo) wait_vmcnt<0>(); else if (HELP) wait_vmcnt<1>(); else wait_vmcnt<P>();
            if (x_in && k > k_lo) {
                // its progress word, loaded one chunk ago before those stores
                const int got = flag_chunks_lds(fslot, epoch);
                seen = got > seen ? got : seen;
            }
            float* tile = tiles + (NTILE == 2 ? (k & 1) * Tile::FLOATS : 0);
            float cv[P];
            if constexpr (HELP) wait_for(cprog, l, k + 1, st);   // loaded by the helper
#pragma unroll
            for (int u = 0; u < P; ++u) cv[u] = tile[tbase + u];
            // lane 0's up values: column t0+j sits in lane j (row 0 is PINF; so are the
            // steps the stripe above did not compute, which lie off the band)
            float rreg = kPINF;
            if (s > 0 && lane < P) {
                const int tu = t0 + lane + 63;
                if (x_in) rreg = rbufs[(k & 1) * 64 + lane];
                else if (tu >= up_lo && tu < up_end) rreg = ring_in[ring_index(tu, R)];
            }
            if (k + 1 < k_end) {
                if (x_in) {
                    const int need = min(k + 1 + lead(P), nch);
                    if (seen < need) seen = wait_part(flag_in, epoch, need, st);
                    issue_row(k + 1);
                }
                if (!HELP)
                    dma_tile<P, 1>(tile_lds + ((k + 1) & 1) * Tile::FLOATS * 4, cbase, i0, L1max,
                                   L2max, lane, t0 + P);
                if (x_in) flag_load_lds(flag_in, fslot_lds, lane);
            }
            float* pub = (lane == 63) ? ring_out + ring_index(t0, R) : sink + lane;
            float* outc = out + (size_t)(t0 - sh) * 64;
            // HELP from memory: the chunk's alphas by step in the helper's alpha tile
            // k & 1 (written to the table by the helper, which has written that tile's
            // previous chunk before publishing this chunk's costs as loaded)
            float* atile = smem + (wave + NW / 2) * WBUF + (k & 1) * Tile::FLOATS + lane;
            // FULL: every cell of the chunk lies inside the element, no validity masks
            auto steps = [&](auto full) {
            constexpr bool FULL = decltype(full)::value;
#pragma unroll
            for (int u = 0; u < P; ++u) {
                const int t = t0 + u;
                const float up = wave_shr1_or(cur, rreg);   // lane 0: stripe above
                rreg = wave_shl1(rreg);
                const float diag = up_prev;
                up_prev = up;
                // out-of-table and out-of-band neighbours are PINF
                const float m = fminf(fminf(diag, up), cur);
                const float z = (fast_exp2((m - diag) * c) + fast_exp2((m - up) * c)) +
                                fast_exp2((m - cur) * c);
                const float a = cv[u] + (m - tl * fast_log2(z));
                const int col = t - lane;
                const bool ok = FULL || ((unsigned)col < (unsigned)L2eff && in_band(ej, col + 1, bw));
                cur = ok ? a : kPINF;
                if (HELP) atile[u * 64] = cur;
                else lane_store(outc + u * 64, ul4, cur);
                pub[u] = cur;
                // (the terminal cell never lies in a FULL chunk: lane 0's row is above
                // L1 - 1, and the other lanes' columns stay below L2 - 1)
                if (!FULL && ok && last_row && col == L2 - 1) terminal = cur;
            }
            };
            if (bw < 0 && i0 + 63 < L1 && t0 >= 63 && t0 + P <= L2) steps(std::true_type{});
            else steps(std::false_type{});
            // the stripe's last row (lane 63) by step, contiguous, for the reverse sweep
            // of the stripe below; one store instruction
            wave_lds_sync();
            if (lane < P) {
                const float v = ring_out[t0 % R + lane];
                if (x_out) store_sys(brow_s + t0 + lane, v);
                else lane_store(brow_s, (unsigned)(t0 + lane) * 4u, v);
            }
            publish(prog, wave, l * PROG_STRIDE + k + 1);
            if (x_out && k >= 2) {
                // at least P loads and 2P + 2 stores follow the row store of chunk k - 2
                // (HELP from memory: the last-row stores of chunks k - 1 and k): it (and
                // everything before) is complete
                if constexpr (HELP) wait_vmcnt<2>();
                else wait_vmcnt<3 * P + 2>();
                if (lane == 0) store_flag(flag_out, progress_word(epoch, k - 1));
            }
        }
        publish(prog, wave, l * PROG_STRIDE + nch);   // nothing to do after the window
        if (x_out) {
            wait_vmcnt<0>();
            if (lane == 0) store_flag(flag_out, progress_word(epoch, nch));
        }
    }

    // the value: the terminal cell, in the part that owns the last stripe (part 0 for
    // an element without stripes)
    __syncthreads();
    const bool owner = NS > 0 ? (NL > 0 && s_begin + NL == NS) : part == 0;
    if (threadIdx.x == 0 && owner)
        value[b] = NS > 0 ? terminal : ((L1 == 0 && L2 == 0) ? 0.0f : kPINF);
}

// The reverse sweep reads the forward's alpha table and nothing else: a cell's
// softmin weights over its predecessors and its softmin value (the temperature
// gradient's term) are both recomputed from the predecessors' alpha with the forward's
// own arithmetic, so the costs are never loaded and the fused squared-Euclidean path
// shares this sweep unchanged.
//
// HELP (unbanded parts of at most NW/2 stripes, e.g. 256-row elements): wave NW/2 + q
// helps the wave of stripe order q.  It loads the alpha rows one chunk ahead into that
// wave's buffers (publishing hprog[q] = chunks loaded) and writes the chunk's marginals
// out of a tile in its own, otherwise unused, buffers once wave q has finished the
// chunk; wave q keeps only the row above and the boundary flows.
template <int P, bool HELP = false>
__global__ void __launch_bounds__(NW * 64)
dtw_backward_kernel(const int* __restrict__ lengths,
                    const float* __restrict__ alpha_sk, const float* __restrict__ brow,
                    float* __restrict__ post, float* __restrict__ grad_T,
                    int* __restrict__ status, float* __restrict__ trash,
                    uint64_t* __restrict__ bflag, float2* __restrict__ flows,
                    double* __restrict__ bpart, float* __restrict__ poison_value, int B,
                    int L1max, int L2max, int NSmax, size_t elem_steps, float T, int bandwidth,
                    int R, int G, int SPW, uint32_t epoch) {
    extern __shared__ __align__(16) float smem[];
    __shared__ int prog[NW];
    __shared__ int hprog[NW];     // HELP: chunks of stripe order q loaded by its helper
    __shared__ float red_g[NW];
    // parts run bottom-up as in the linear-SW backward
    int b, dpart;
    split_decode(blockIdx.x, G, b, dpart);
    if (b >= B) return;
    const int part = G - 1 - dpart;
    const int lane = threadIdx.x & 63;
    const unsigned ul4 = (unsigned)lane * 4u;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Per wave, two chunk buffers, each: the tile that stages the chunk's marginals,
    // P alpha rows (steps t_hi-2 .. t_hi-P-1) and one row of values from the stripe
    // above; the last two arrive by direct-to-LDS loads one chunk ahead.
    using Tile = ChunkTile<P>;
    constexpr int ABUF = Tile::FLOATS;
    constexpr int RBUF = ABUF + P * 64;
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
    const int tbase = Tile::read_base(lane);

    if (lane == 0) {
        prog[wave] = -1;
        hprog[wave] = -1;
    }
    __syncthreads();

    const int L1 = lengths ? min(max(lengths[2 * b], 0), L1max) : L1max;
    const int L2 = lengths ? min(max(lengths[2 * b + 1], 0), L2max) : L2max;
    const float c = kLog2e / T;
    const float tl = T * kLn2;
    const float bw = (bandwidth < 0 || L1 == 0 || L2 == 0) ? -1.0f : (float)bandwidth;
    const int NS = L2 > 0 ? (L1 + 63) >> 6 : 0;
    const int nsteps = L2 + 63;
    const int nch = (nsteps + P - 1) / P;
    const size_t NT = (size_t)stored_steps(L2max);
    float* pbase = post + (size_t)b * L1max * L2max;

    {   // each part zeroes its share of the rows' padding
        const int rows = (L1max + G - 1) / G;
        zero_padding(pbase, L1, L2, L1max, L2max, NW * 64, part * rows,
                     min(L1max, part * rows + rows));
    }

    float g_acc = 0.0f;
    float A[P + 2];
    const int s_begin = part * SPW;
    const int NL = max(min(NS, s_begin + SPW) - s_begin, 0);   // stripes of this part
    const bool has_next = s_begin + NL < NS;
    const uint64_t* flag_in = bflag + (size_t)b * G + (part + 1 < G ? part + 1 : part);
    uint64_t* flag_out = bflag + (size_t)b * G + part;
    const int stride = band_stride(L1, L2, bw, (int)NT);   // table steps per stripe
    if ((size_t)NS * stride > elem_steps) {   // never: the host reserves enough
        if (threadIdx.x == 0) atomicOr(st, 2);
        return;
    }

    if constexpr (HELP) {
        if (NL > NW / 2 || bandwidth >= 0) {   // never: the host picks HELP for these only
            if (threadIdx.x == 0) atomicOr(st, 2);
            return;
        }
        const int q = wave - NW / 2;
        if (q >= 0 && q < NL) {
            const int s = s_begin + NL - 1 - q;
            const int i0 = s * 64;
            // unbanded: the window is every chunk and the table starts at step 0
            const float* astripe = band_stripe(alpha_sk, b, elem_steps, s, stride);
            float* qbufs = smem + q * 2 * BUF;      // the sweeping wave's two chunk buffers
            float* obufs = smem + wave * 2 * BUF;   // its output tiles: this wave's buffers
            auto load = [&](int k) {
                const int th = nsteps - 1 - k * P;
                dma_rows<P, -1>(lds_address(qbufs + (k & 1) * BUF) + ABUF * 4, astripe, th - 2,
                                ul4);
            };
            // whole row segments of marginals where rows start aligned (write_aligned):
            // P/4 stores per chunk instead of P
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
                    // chunk k + 1's loads: the last issued at k = 0, else followed by the
                    // marginal stores of chunk k - 1 (P, or P/4 aligned ones)
                    if (k == 0) wait_vmcnt<0>();
                    else if (aligned) wait_vmcnt<P / 4>();
                    else wait_vmcnt<P>();
                    publish(hprog, q, k + 2);   // also completes this wave's LDS reads
                }
                // once wave q has finished chunk k, its buffer k & 1 takes chunk k + 2
                // and its marginals (in output tile k & 1) leave
                wait_for(prog, q, q * PROG_STRIDE + k + 1, st);
                if (k + 2 < nch) load(k + 2);
                if (aligned)
                    write_aligned<P, false>(obufs + (k & 1) * BUF, pbase, trash, carry, i0,
                                            L1max, L2max, lane, nsteps - 1 - k * P);
                else
                    write_tile<P, -1>(obufs + (k & 1) * BUF, pbase, trash, i0, L1, L2, L1max,
                                      L2max, lane, nsteps - 1 - k * P);
            }
        }
    }

    // Stripes run bottom-up: order q = 0..NL-1 handles stripe s_begin+NL-1-q, on wave
    // q % NW.
    for (int q = wave; q < NL; q += NW) {
        const int s = s_begin + NL - 1 - q;
        const int i0 = s * 64;
        const int L2eff = (i0 + lane < L1) ? L2 : 0;
        const float ej = band_centre(i0 + lane + 1, L1, L2);
        // the terminal cell (L1, L2) starts with beta = 1
        const int term_step = (i0 + lane == L1 - 1) ? L2 - 1 + lane : -1000000;
        // the stripe's band window as reverse chunks [k_lo, k_end) (chunk k covers steps
        // nsteps-1-kP down to nsteps-kP-P), its table from forward chunk kf_lo, and the
        // reverse slots [dn_lo, dn_end) the stripe below computed
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
        // table step t of this stripe at astripe + (t - sh + APAD) * 64
        const int sh = kf_lo * PF;
        const float* astripe = band_stripe(alpha_sk, b, elem_steps, s, stride);
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

        auto issue_chunk = [&](int k) {
            const int th = nsteps - 1 - k * P;
            const uint32_t buf = lds_address(bufs + (k & 1) * BUF);
            if (!HELP) dma_rows<P, -1>(buf + ABUF * 4, astripe, th - 2 - sh, ul4);
            uint32_t roff = (uint32_t)min(th - min(lane, P) + 63, nsteps - 1) * 4u;
            uint32_t rl = buf + RBUF * 4;
            lds_dma_dword<0>(bup, roff, rl, 0u);
            if (x_in) {
                // flows of producer slots kP+62 .. kP+62+P (float2 each): float f of the
                // range in lane f, clamped to the last slot
                uint32_t foff = (uint32_t)min((k * P + 62) * 2 + min(lane, 2 * P + 1),
                                              (nsteps - 1) * 2 + 1) * 4u;
                uint32_t fdst = buf + FBUF * 4;
                lds_dma_dword_sys<0>(flows_in, foff, fdst, 0u);
            }
        };

        if (bw >= 0.0f) {
            // cells of the stripe's rows at steps outside the window: off the band, zero
            const int a_end = nsteps - k_end * P;   // steps below are not swept
            const int b_beg = nsteps - k_lo * P;    // nor are steps from here on
            const int rows = min(64, L1 - i0);
            for (int r = 0; r < rows; ++r) {
                float* row = pbase + (size_t)(i0 + r) * L2max;
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
            A[P] = lane_load(astripe + (size_t)(th0 - sh + APAD) * 64, ul4);
            A[P + 1] = lane_load(astripe + (size_t)(th0 - sh - 1 + APAD) * 64, ul4);
        }
        __asm__ volatile("" ::"v"(A[P]), "v"(A[P + 1]));   // completes the two loads here
        wave_lds_sync();   // the previous stripe's buffer reads are complete
        if (x_in) seen = wait_part(flag_in, epoch, min(k_lo + lead(P), nch), st);
        issue_chunk(k_lo);
        float in_left = 0.0f, in_up = 0.0f, in_diag = 0.0f, in_diag_next = 0.0f;

        for (int k = k_lo; k < k_end; ++k) {
            const int t_hi = nsteps - 1 - k * P;
            chunk_waits<P>(prog, q, NL, k, nch, R, st, k_lo);
            // this chunk's loads were issued one chunk ago and followed by at least the
            // P marginal stores of that chunk (the first chunk's are the last issued).
            // HELP: the helper loads the alpha rows; this wave's own loads (row above,
            // flows) are followed by nothing, or by the previous chunk's flow store
            if constexpr (HELP) {
                if (x_out && k > k_lo) wait_vmcnt<1>(); else wait_vmcnt<0>();
                wait_for(hprog, q, k + 1, st);
            } else {
                if (k == k_lo) wait_vmcnt<0>(); else wait_vmcnt<P>();
            }
            if (x_in && k > k_lo) {
                // its progress word, loaded one chunk ago before those stores
                const int got = flag_chunks_lds(fslot, epoch);
                seen = got > seen ? got : seen;
            }
            float* buf = bufs + (k & 1) * BUF;
            // the chunk's marginals: over its own buffer's tile, or (HELP) in the
            // helper's buffer k & 1, whose previous tile the helper has written out
            // before publishing this chunk as loaded
            float* tile = HELP ? smem + (wave + NW / 2) * 2 * BUF + (k & 1) * BUF : buf;
            A[0] = A[P];
            A[1] = A[P + 1];
#pragma unroll
            for (int j = 0; j < P; ++j) A[j + 2] = buf[ABUF + rows_row<P, -1>(j) * 64 + lane];
            // lane j: alpha of the row above at lane-63 step t_hi - j + 63 (row 0: PINF)
            float bv = buf[RBUF + lane];
            bv = (s > 0 && lane <= P && t_hi - lane + 63 <= nsteps - 1) ? bv : kPINF;
            float pre_u = 0.0f, pre_d = 0.0f;
            if (below && lane >= 64 - P) {
                // slots the stripe below did not compute carry no flow (off the band)
                const int j = 63 - lane;
                const int su = k * P + j + 63, sd = su - 1;
                const bool ou = su >= dn_lo && su < dn_end, od = sd >= dn_lo && sd < dn_end;
                if (x_in) {
                    pre_u = ou ? buf[FBUF + 2 * (j + 1)] : 0.0f;
                    pre_d = od ? buf[FBUF + 2 * j + 1] : 0.0f;
                } else {
                    pre_u = ou ? ring_in[ring_index(su, R)].x : 0.0f;
                    pre_d = od ? ring_in[ring_index(sd, R)].y : 0.0f;
                }
            }
            if (k + 1 < k_end) {
                if (x_in) {
                    const int need = min(k + 1 + lead(P), nch);
                    if (seen < need) seen = wait_part(flag_in, epoch, need, st);
                }
                issue_chunk(k + 1);
                if (x_in) flag_load_lds(flag_in, fslot_lds, lane);
            }
            float2* pub = (lane == 0) ? ring_out + ring_index(k * P, R) : sink + lane;
            {
                const float u0 = lane_bcast(pre_u, 63), d0 = lane_bcast(pre_d, 63);
                const float d1 = lane_bcast(pre_d, 62);
                if (lane == 63) { in_up = u0; in_diag = d0; in_diag_next = d1; }
            }
            float pre_d2 = wave_shr1(pre_d);
            pre_d2 = wave_shr1(pre_d2);
            // FULL: every cell of the chunk lies inside the element, no validity masks
            auto steps = [&](auto full) {
            constexpr bool FULL = decltype(full)::value;
#pragma unroll
            for (int u = 0; u < P; ++u) {
                const int t = t_hi - u;
                const int col = t - lane;
                const bool ok = FULL || ((unsigned)col < (unsigned)L2eff && in_band(ej, col + 1, bw));
                const float a1 = A[u + 1];
                const float bv_next = wave_shl1(bv);
                const float upa = wave_shr1_or(a1, bv);
                const float dga = wave_shr1_or(A[u + 2], bv_next);
                bv = bv_next;
                // softmin weights over (diagonal, up, left); none if all are PINF
                const float m = fminf(fminf(dga, upa), a1);
                const float ed = fast_exp2((m - dga) * c), eu = fast_exp2((m - upa) * c);
                const float el = fast_exp2((m - a1) * c);
                const float z = (ed + eu) + el;
                const float rin = m < kPINF ? fast_rcp(z) : 0.0f;
                // reference accumulation order: init, diagonal, left, up successor.  A
                // FULL chunk never holds the terminal cell (its lane-0 row lies above
                // L1 - 1 and every other lane's terminal step above t_hi), and the flows
                // are never -0, so there the zero start term is left out exactly
                float beta;
                if (FULL) {
                    beta = (in_diag + in_left) + in_up;
                } else {
                    const float binit = t == term_step ? 1.0f : 0.0f;
                    beta = ((binit + in_diag) + in_left) + in_up;
                }
                const float bl = ok ? beta : 0.0f;
                const float br = bl * rin;
                const float od = br * ed, ou = br * eu, ol = br * el;
                tile[tbase + u] = bl;
                // temperature gradient: beta * (softmin value - E_w[predecessor alpha]);
                // the softmin value is the forward's m - T ln2 log2(z), bit for bit
                // (PINF, hence skipped, when every predecessor is PINF)
                const float smv = m - tl * fast_log2(z);
                const float ea = (od * dga + ou * upa) + ol * a1;   // beta * E_w[alpha_pred]
                g_acc += (ok && smv < kPINF) ? bl * smv - ea : 0.0f;
                pub[u] = make_float2(ou, od);
                pre_u = wave_shr1(pre_u);
                in_left = ol;
                in_up = wave_shl1_or(ou, pre_u);
                in_diag = in_diag_next;
                in_diag_next = wave_shl1_or(od, pre_d2);
                pre_d2 = wave_shr1(pre_d2);
            }
            };
            if (bw < 0 && i0 + 63 < L1 && t_hi - P - 62 >= 0 && t_hi < L2) steps(std::true_type{});
            else steps(std::false_type{});
            wave_lds_sync();
            // (HELP: the helper writes the tile once this chunk is published)
            if constexpr (!HELP)
                write_tile<P, -1>(tile, pbase, trash, i0, L1, L2, L1max, L2max, lane, t_hi);
            publish(prog, wave, q * PROG_STRIDE + k + 1);
            if (x_out) {
                // this chunk's flows to the part above, by producer step
                if (lane < P) store_sys2(flows_out + k * P + lane, ring_out[ring_index(k * P, R) + lane]);
                if (k >= 2) {
                    // at least P/4 + 1 loads, 2P marginal stores and 2 flow stores
                    // follow the flow store of chunk k - 2 (HELP: the row-above load
                    // issued in chunk k - 1 and the two flow stores): it is complete
                    if constexpr (HELP) wait_vmcnt<3>();
                    else wait_vmcnt<2 * P + P / 4 + 3>();
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

    g_acc = wave_sum(g_acc);
    if (lane == 0) red_g[wave] = g_acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        float g = 0.0f;
        for (int w = 0; w < NW; ++w) g += red_g[w];
        if (G == 1) grad_T[b] = g / T;
        else bpart[((size_t)b * G + part) * 4] = g;
    }
    // An unsplit element whose waits gave up (in the forward or in this sweep) gets NaN
    // in all its outputs here (the separate poison pass of split calls).  Every wave
    // first completes its own status atomics and stores; then one thread reads the
    // status word and every wave branches on that one value.
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
            grad_T[b] = nan;
        }
    }
}

// grad_T[b] of a split element from the parts' sums.
__global__ void dtw_grad_merge(const double* __restrict__ bpart, float* __restrict__ grad_T,
                               int B, int G, float T) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    float g = 0.0f;
    for (int i = 0; i < G; ++i) g += (float)bpart[((size_t)b * G + i) * 4];
    grad_T[b] = g / T;
}

}  // namespace dtw
}  // namespace d2p_amd

namespace d2p_amd {
namespace dtw {

namespace {
// dynamic LDS bound: 160 KiB less the kernels' static arrays (progress words,
// reductions, the prefetched progress-word slot)
constexpr size_t kLdsLimit = 160 * 1024 - 512;

// LDS of one workgroup whose stripe boundaries use rings of R columns
size_t lds_forward_r(int R) {
    return (size_t)NW * (2 * 65 * PF + 2 * 64) * sizeof(float) +
           ((size_t)NW * R + NW * DUMMY) * sizeof(float);
}
size_t lds_backward_r(int R, int P) {
    return (size_t)NW * 2 * (65 * P + 64 * P + 64 + 64) * sizeof(float) +
           ((size_t)NW * R + NW * DUMMY) * sizeof(float2);
}
int ring_forward(int rows, int max_L2) { return ring_len(rows, max_L2, 256); }
int ring_backward(int rows, int max_L2) { return ring_len(rows, max_L2, 128); }

// 16-step backward chunks when they fit in LDS, else 8-step chunks
int backward_chunk(int rows, int max_L2) {
    return lds_backward_r(ring_backward(rows, max_L2), 16) <= kLdsLimit ? 16 : 8;
}

// Stripes per part that a launch may not exceed: 0 when the rings of an unsplit
// element fit in LDS, else NW (the minimum rings of such parts always fit).
int max_stripes_forward(int max_L1, int max_L2) {
    return lds_forward_r(ring_forward(max_L1, max_L2)) <= kLdsLimit ? 0 : NW;
}
int max_stripes_backward(int max_L1, int max_L2) {
    return lds_backward_r(ring_backward(max_L1, max_L2), 8) <= kLdsLimit ? 0 : NW;
}

// D2P_AMD_DTW_HELPERS=0 turns the reverse sweep's helper waves off (for tests: both
// forms must agree bit for bit)
bool dtw_helpers_enabled() {
    const char* e = std::getenv("D2P_AMD_DTW_HELPERS");
    return !(e && e[0] == '0');
}

template <int P>
int launch_backward_p(const int* lengths, int B, int max_L1, int max_L2,
                      float T, int bandwidth, const Layout& ws, float* marginals, float* grad_T,
                      hipStream_t st, const Split& sp, int R, float* poison_value) {
    const int ns = (max_L1 + 63) / 64;
    const size_t lds = lds_backward_r(R, P);
    D2P_REQUIRE(lds <= kLdsLimit, "sequence too long for the LDS stripe rings");
    if (sp.G > 1) D2P_TRY(launch_flag_reset(ws.bflag, B * sp.G, st));
    // helper waves for unbanded parts of at most NW/2 stripes (waves NW/2.. would idle)
    const int part_stripes = sp.G > 1 ? sp.SPW : ns;
    const bool help = bandwidth < 0 && part_stripes <= NW / 2 && dtw_helpers_enabled();
    auto kern = help ? dtw_backward_kernel<P, true> : dtw_backward_kernel<P, false>;
    D2P_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds));
    D2P_LAUNCH("dtw_backward", kern, dim3(split_grid(B, sp.G)), dim3(NW * 64),
               lds, st, lengths, ws.alpha_sk, ws.brow, marginals, grad_T, ws.status, ws.trash,
               ws.bflag, ws.flows, ws.bpart, sp.G == 1 ? poison_value : nullptr, B, max_L1,
               max_L2, ns, ws.elem_steps, T, bandwidth, R, sp.G, sp.SPW, next_epoch());
    if (sp.G > 1)
        D2P_LAUNCH("dtw_grad_merge", dtw_grad_merge, dim3((B + 255) / 256), dim3(256), 0, st,
                   ws.bpart, grad_T, B, sp.G, T);
    D2P_HIP(hipGetLastError());
    return D2P_OK;
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

int launch_forward(const float* costs, const int* lengths, int B, int max_L1, int max_L2,
                   float T, int bandwidth, const Layout& ws, float* value, hipStream_t st) {
    const int ns = (max_L1 + 63) / 64;
    const Split sp = choose_split(B, max_L1, ws, max_stripes_forward(max_L1, max_L2));
    const int R = ring_forward(sp.G > 1 ? sp.SPW * 64 : max_L1, max_L2);
    const size_t lds = lds_forward_r(R);
    D2P_REQUIRE(lds <= kLdsLimit, "sequence too long for the LDS stripe rings");
    if (sp.G > 1 && launch_split_reset(ws, B, sp.G, st) != D2P_OK) return D2P_ERR_HIP;
    // helper waves for unbanded parts of at most NW/2 stripes (waves NW/2.. would idle)
    const int part_stripes = sp.G > 1 ? sp.SPW : ns;
    const bool help = bandwidth < 0 && part_stripes <= NW / 2 && dtw_helpers_enabled();
    auto kern = help ? dtw_forward_kernel<true> : dtw_forward_kernel<false>;
    D2P_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds));
    D2P_LAUNCH("dtw_forward", kern, dim3(split_grid(B, sp.G)), dim3(NW * 64),
               lds, st, costs, lengths, ws.alpha_sk, ws.brow, value, ws.status, ws.fflag, B,
               max_L1, max_L2, ns, ws.elem_steps, T, bandwidth, R, sp.G, sp.SPW, next_epoch());
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

int launch_backward(const int* lengths, int B, int max_L1, int max_L2, float T,
                    int bandwidth, const Layout& ws, float* marginals, float* grad_T,
                    hipStream_t st, float* poison_value, bool* poisoned) {
    const Split sp = choose_split(B, max_L1, ws, max_stripes_backward(max_L1, max_L2));
    const int rows = sp.G > 1 ? sp.SPW * 64 : max_L1;
    const int R = ring_backward(rows, max_L2);
    if (poisoned != nullptr) *poisoned = sp.G == 1 && poison_value != nullptr;
    if (backward_chunk(rows, max_L2) == 16)
        return launch_backward_p<16>(lengths, B, max_L1, max_L2, T, bandwidth, ws, marginals,
                                     grad_T, st, sp, R, poison_value);
    return launch_backward_p<8>(lengths, B, max_L1, max_L2, T, bandwidth, ws, marginals, grad_T,
                                st, sp, R, poison_value);
}

}  // namespace dtw
}  // namespace d2p_amd

using namespace d2p_amd;

extern "C" size_t d2p_dtw_workspace_bytes_banded(int B, int max_L1, int max_L2, int bandwidth) {
    if (B <= 0 || max_L1 < 0 || max_L2 < 0) return 0;
    // status words | trash line | skewed alpha table (banded: each stripe's window) |
    // last row of every stripe | split-element progress words, boundary flows and
    // partial sums
    return wf::layout(nullptr, B, max_L1, max_L2, 1, true, 8,
                      dtw::band_elem_steps(max_L1, max_L2, bandwidth))
        .bytes;
}

extern "C" size_t d2p_dtw_workspace_bytes(int B, int max_L1, int max_L2) {
    return d2p_dtw_workspace_bytes_banded(B, max_L1, max_L2, -1);
}

extern "C" int d2p_dtw_forward_marginals(const float* costs, const int* lengths, int B,
                                         int max_L1, int max_L2, float temperature,
                                         int bandwidth, float* value, float* marginals,
                                         float* grad_T, void* workspace, size_t workspace_bytes,
                                         void* stream) {
    const int rc = dtw::check_shape(B, max_L1, max_L2, temperature);
    if (rc != D2P_OK) return rc;
    if (B == 0) return D2P_OK;
    D2P_REQUIRE(costs && value && marginals && grad_T, "null pointer argument");
    const size_t need = d2p_dtw_workspace_bytes_banded(B, max_L1, max_L2, bandwidth);
    D2P_REQUIRE(workspace && workspace_bytes >= need, "workspace too small");
    hipStream_t st = (hipStream_t)stream;
    const wf::Layout ws = wf::layout(workspace, B, max_L1, max_L2, 1, true, 8,
                                     dtw::band_elem_steps(max_L1, max_L2, bandwidth));
    D2P_TRY(dtw::launch_forward(costs, lengths, B, max_L1, max_L2, temperature, bandwidth, ws,
                                value, st));
    bool poisoned = false;
    D2P_TRY(dtw::launch_backward(lengths, B, max_L1, max_L2, temperature, bandwidth, ws,
                                 marginals, grad_T, st, value, &poisoned));
    if (poisoned) return D2P_OK;
    return wf::launch_poison(ws.status, B, (long long)max_L1 * max_L2, marginals, nullptr, value,
                             grad_T, nullptr, nullptr, st);
}
