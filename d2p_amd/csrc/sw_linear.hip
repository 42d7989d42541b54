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
//   * rows are cut into 64-row stripes; stripe s belongs to wave s % NW.  Lane r
//     holds DP row 64*s+r+1 and sweeps the columns with a one-column skew per lane
//     (lane r works on column t-r at step t), so a wave's 64 cells at one step lie on
//     one anti-diagonal;
//   * the up / diagonal neighbours come from lane r-1 through a DPP wave shift; the
//     boundary lane reads the stripe above through an LDS ring, staged in the DPP
//     "old" operand;
//   * waves do not meet at barriers: each wave publishes its progress (stripe, chunks
//     done) in LDS with release semantics, and a stripe waits, chunk by chunk, only
//     for the part of the stripe above it reads (and, so that the ring is not
//     overwritten, for the stripe below to have caught up);
//   * scores (and, in the backward, marginals) are staged per chunk of P steps through
//     a padded LDS tile so every HBM access is a contiguous row segment;
//   * the forward stores alpha in a skewed layout alpha_sk[b][stripe][t][lane], one
//     contiguous 256-byte vector per wave step, which the backward streams back in
//     reverse.
// The backward is the reverse sweep of the reference (scatter form, no atomics): each
// cell receives its successors' contributions from the DPP neighbour or from its own
// previous step, in the reference's accumulation order
//   beta = ((beta_init + from(i+1,j+1)) + from(i,j+1)) + from(i+1,j).
//
// Every wait is bounded: a wave that spins SPIN_LIMIT times sets bit 0 of the
// element's status word and goes on, so a logic error can never hang the GPU.

#include <vector>

#include "dp_common.hip.h"
#include "../../include/d2p_amd.h"
#include "capi_util.hip.h"

namespace d2p_amd {
namespace sw {

constexpr int NW = 8;                // waves per workgroup
constexpr int PF = 16;               // steps per chunk, forward sweep
constexpr int PB = 16;               // steps per chunk, backward sweep
constexpr int SPIN_LIMIT = 1 << 22;  // ~0.2 s of polling before giving up
constexpr int PROG_STRIDE = 1 << 16; // progress word = stripe * PROG_STRIDE + chunks done
constexpr int DUMMY = 64 + PF;       // per-wave LDS sink for the lanes that do not publish

// A stripe's chunk k reads boundary values the neighbouring stripe produces up to
// 62 + P steps later in its own sweep, i.e. in its chunk k + 1 + 62/P; so it waits
// until that stripe has completed k + lead(P) chunks.
constexpr int lead(int P) { return 2 + 62 / P; }

// Ring length (columns) of one stripe boundary.  It must exceed the pipeline window
// (LEAD chunks plus back-pressure slack); when a wave owns several stripes (more
// than NW stripes) it must also satisfy NW * R > L2 + 64 + 4P, which rules out a
// cycle of back-pressure waits across a whole round of waves.
__host__ inline int ring_len(int max_L1, int max_L2, int min_len) {
    const int ns = (max_L1 + 63) / 64;
    int r = min_len;
    if (ns > NW) {
        const int need = (max_L2 + 64 + 4 * PF + NW - 1) / NW + 1;
        r = r > need ? r : need;
    }
    return (r + PF - 1) / PF * PF;   // a multiple of both chunk lengths
}

// Steps stored per stripe in the skewed alpha table: APAD leading steps t < 0 (all
// NINF, so the reverse sweep reads the steps before the first one without guards)
// and then whole forward chunks.
constexpr int APAD = PB + 2;
__host__ __device__ inline int stored_steps(int L2max) {
    return APAD + ((L2max + 63 + PF - 1) / PF) * PF;
}

__host__ inline size_t status_bytes(int B) { return ((size_t)B * sizeof(int) + 255) / 256 * 256; }
constexpr size_t TRASH_BYTES = 256;  // one line the backward's masked lanes store into

// Progress flags live in LDS.  The writer completes its LDS writes (ring data)
// before the flag write; a reader that sees the flag issues its data reads after the
// flag read.  LDS executes each wave's operations in order, so relaxed atomics plus
// an LDS-only wait suffice.  (A C++ release/acquire, or a volatile access, would also
// drain every HBM load and store in flight, i.e. s_waitcnt vmcnt(0), every chunk.)
__device__ __forceinline__ void publish(int* prog, int wave, int value) {
    wave_lds_sync();
    __hip_atomic_store(prog + wave, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Waits until prog[w] >= need; bounded.  The loaded value is made wave-uniform.
__device__ __forceinline__ void wait_for(int* prog, int w, int need, int* status_b) {
    int spins = 0;
    while (__builtin_amdgcn_readfirstlane(__hip_atomic_load(
               prog + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) < need) {
        __builtin_amdgcn_s_sleep(2);
        if (++spins >= SPIN_LIMIT) {
            atomicOr(status_b, 1);
            break;
        }
    }
    wave_lds_sync();
}

__device__ __forceinline__ int ring_index(int slot, int R) {
    slot %= R;
    return slot < 0 ? slot + R : slot;
}

// Direct HBM -> LDS load of one dword per lane (global_load_lds_dword): lane l's value
// lands at LDS byte address lds + 4*l; the LDS address travels in M0.  Each call then
// advances `lds` by `lds_step` and `voff` by `vstep` bytes.  Written as inline
// assembly so that (a) the compiler does not make every later LDS access wait for
// the load (completion is waited for explicitly with wait_vmcnt), and (b) the running
// addresses stay in two registers instead of being hoisted out of the loop as one
// precomputed address per instruction.
// M0 is a reserved register the compiler may use itself (LDS-DMA builtins, indexed
// register moves); this file uses neither, so clobbering it here is safe, and the
// compiler's reminder about reserved clobbers is silenced.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <int LDS_STEP>
__device__ __forceinline__ void lds_dma_dword(const float* sbase, uint32_t& voff, uint32_t& lds,
                                              uint32_t vstep) {
    __asm__ volatile(
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dword %0, %2\n\t"
        "s_add_u32 %1, %1, %4\n\t"
        "v_add_u32 %0, %3, %0"
        : "+v"(voff), "+s"(lds)
        : "s"(sbase), "s"(vstep), "n"(LDS_STEP)
        : "memory", "m0", "scc");
}
#pragma clang diagnostic pop

// Waits until at most N vector-memory operations of this wave are outstanding
// (gfx9 counts loads, stores and LDS DMA on one in-order counter).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Accesses base + byte offset with a wave-uniform base and a 32-bit per-lane offset,
// the form the scalar-base global instructions take (no 64-bit address per lane).
__device__ __forceinline__ float lane_load(const float* base, unsigned off_bytes) {
    return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(base) + off_bytes);
}
__device__ __forceinline__ void lane_store(float* base, unsigned off_bytes, float v) {
    *reinterpret_cast<float*>(reinterpret_cast<char*>(base) + off_bytes) = v;
}

__device__ __forceinline__ uint32_t lds_address(const void* p) {
    return (uint32_t)(uintptr_t)p;   // low half of a flat LDS address = LDS offset
}

// A chunk covers P steps of a stripe's 64 rows; cell (row r, step u) is column
// t_first + DIR*u - r of DP row i0 + r (DIR = +1 forward, -1 reverse sweep).
//
// Score tiles are staged with P direct-to-LDS loads: instruction i, lane P*j+u
// carries row r = i+P*j, step u, and lands at float 65*i + P*j + u of the tile.  Row r,
// step u is therefore at 65*(r%P) + P*(r/P) + u, whose bank (mod 64) is r+u: the
// per-step column read of the 64 lanes is conflict-free.  The backward reuses the
// tile for the marginals it produces, and instruction i of the write-out stores
// tile floats 65*i .. 65*i+63 back to the same cells.
template <int P>
struct ChunkTile {
    static constexpr int FLOATS = 65 * P;
    __device__ static int read_base(int lane) { return 65 * (lane % P) + P * (lane / P); }
};

// True when every cell of the chunk lies inside the (max_L1 x max_L2) matrix.  Then
// cell addresses of instruction i are the lane's address of instruction 0 plus
// i*(L2max-1): one wave-uniform increment, no per-lane clamping.
template <int P, int DIR>
__device__ __forceinline__ bool chunk_inside(int i0, int L1max, int L2max, int t_first) {
    const int lo = DIR > 0 ? t_first - 63 : t_first - (P - 1) - 63;
    const int hi = DIR > 0 ? t_first + P - 1 : t_first;
    return lo >= 0 && hi < L2max && i0 + 63 < L1max;
}

template <int P, int DIR>
__device__ __forceinline__ int chunk_offset0(int i0, int L2max, int lane, int t_first) {
    const int u = lane % P, pj = lane - u;
    return (i0 + pj) * L2max + t_first + DIR * u - pj;
}

// Issues the P loads of one score chunk.  Cells outside the matrix read a clamped
// in-matrix address; the sweeps mask every cell outside the element's lengths.
template <int P, int DIR>
__device__ __forceinline__ void dma_scores(uint32_t tile_lds, const float* sbase, int i0,
                                           int L1max, int L2max, int lane, int t_first) {
    if (chunk_inside<P, DIR>(i0, L1max, L2max, t_first)) {
        uint32_t voff = (uint32_t)chunk_offset0<P, DIR>(i0, L2max, lane, t_first) * 4u;
        const uint32_t vstep = (uint32_t)(L2max - 1) * 4u;
#pragma unroll
        for (int i = 0; i < P; ++i) lds_dma_dword<260>(sbase, voff, tile_lds, vstep);
    } else {
        const int u = lane % P, pj = lane - u;
        // row/column of instruction 0; instruction i moves one row down, one column left
        int row = i0 + pj, col = t_first + DIR * u - pj;
#pragma unroll
        for (int i = 0; i < P; ++i) {
            uint32_t voff = (uint32_t)(min(row, L1max - 1) * L2max +
                                       min(max(col, 0), L2max - 1)) * 4u;
            lds_dma_dword<260>(sbase, voff, tile_lds, 0u);
            ++row;
            --col;
        }
    }
}

__global__ void __launch_bounds__(NW * 64)
sw_forward_kernel(const float* __restrict__ scores, const int* __restrict__ lengths,
                  float* __restrict__ alpha_sk, float* __restrict__ brow,
                  float* __restrict__ partition,
                  int* __restrict__ status, int L1max, int L2max, int NSmax, float gap, float T,
                  int R) {
    constexpr int P = PF;
    constexpr int LEAD = lead(P);
    extern __shared__ float smem[];
    __shared__ int prog[NW];
    __shared__ float red_m[NW], red_z[NW];
    const int b = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const unsigned ul4 = (unsigned)lane * 4u;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    using Tile = ChunkTile<P>;
    float* tiles = smem + wave * 2 * Tile::FLOATS;         // double-buffered score chunk
    float* rings = smem + NW * 2 * Tile::FLOATS;           // [2 parities][NW][R]
    float* sink = rings + 2 * NW * R + wave * DUMMY;       // per-wave write sink
    int* st = status + b;
    const int tbase = Tile::read_base(lane);

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
        const int i0 = s * 64;
        const int L2eff = (i0 + lane < L1) ? L2 : 0;   // rows past L1 are never valid
        const float* ring_in =
            rings + ((((s - 1) / NW) & 1) * NW + (s + NW - 1) % NW) * R;
        float* ring_out = rings + (((s / NW) & 1) * NW + wave) * R;
        // wave-uniform base (step 0) + 32-bit lane offset: scalar-base stores
        float* out = alpha_sk + (((size_t)b * NSmax + s) * NT + APAD) * 64;
        float* brow_s = brow + ((size_t)b * NSmax + s) * NT;   // last row, by step
#pragma unroll
        for (int t = -APAD; t < 0; ++t) lane_store(out + t * 64, ul4, kNINF);
        wave_lds_sync();   // the previous stripe's tile reads are complete
        const uint32_t tile_lds = lds_address(tiles);
        dma_scores<P, 1>(tile_lds, sbase, i0, L1max, L2max, lane, 0);
        float cur = kNINF, up_prev = kNINF;

        for (int k = 0; k < nch; ++k) {
            const int t0 = k * P;
            if (s > 0) wait_for(prog, (s - 1) % NW, (s - 1) * PROG_STRIDE + min(k + LEAD, nch), st);
            if (s + 1 < NS) {
                const int need = k - 2 - R / P;   // slots of steps < kP+P-R must be consumed
                if (need > 0) wait_for(prog, (s + 1) % NW, (s + 1) * PROG_STRIDE + need, st);
            }
            // this chunk's scores: loaded one chunk ago, followed by the P + 1 stores of
            // that chunk (the first chunk's load is the last issued)
            if (k == 0) wait_vmcnt<0>(); else wait_vmcnt<P>();
            const float* tile = tiles + (k & 1) * Tile::FLOATS;
            float sv[P];
#pragma unroll
            for (int u = 0; u < P; ++u) sv[u] = tile[tbase + u];
            // lane 0's up values: column t0+j sits in lane j (ring slot = producer step)
            float rreg = kNINF;
            if (s > 0 && lane < P) rreg = ring_in[ring_index(t0 + lane + 63, R)];
            if (k + 1 < nch)
                dma_scores<P, 1>(tile_lds + ((k + 1) & 1) * Tile::FLOATS * 4, sbase, i0, L1max,
                                 L2max, lane, t0 + P);
            // lane 63 publishes its alpha of step u into ring slot (t0+u) % R; the
            // other lanes write into the sink (R is a multiple of P: no wrap in a chunk)
            float* pub = (lane == 63) ? ring_out + ring_index(t0, R) : sink + lane;
            float* outc = out + (size_t)t0 * 64;
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
                const float sum = fast_exp2((vd - m) * c) + fast_exp2((vu - m) * c) +
                                  fast_exp2((vl - m) * c) + fast_exp2((sv[u] - m) * c);
                const float a = m + tl * fast_log2(sum);
                const bool ok = (unsigned)(t - lane) < (unsigned)L2eff;
                cur = ok ? a : kNINF;
                lane_store(outc + u * 64, ul4, cur);
                pub[u] = cur;
                acc.add(cur, c);
            }
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

__global__ void __launch_bounds__(NW * 64)
sw_backward_kernel(const float* __restrict__ scores, const int* __restrict__ lengths,
                   const float* __restrict__ alpha_sk, const float* __restrict__ brow,
                   const float* __restrict__ partition,
                   float* __restrict__ post, float* __restrict__ grad_gap,
                   float* __restrict__ grad_T, int* __restrict__ status, float* __restrict__ trash,
                   int L1max, int L2max, int NSmax, float gap, float T, int R) {
    constexpr int P = PB;
    constexpr int LEAD = lead(P);
    extern __shared__ float smem[];
    __shared__ int prog[NW];
    __shared__ float red_g[NW], red_p[NW];
    const int b = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const unsigned ul4 = (unsigned)lane * 4u;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Per wave, two chunk buffers, each: the score tile (then the chunk's marginals),
    // P alpha rows (steps t_hi-2 .. t_hi-P-1, 64 lanes each) and one row of values from
    // the stripe above.  All three arrive by direct-to-LDS loads one chunk ahead.
    using Tile = ChunkTile<P>;
    constexpr int ABUF = Tile::FLOATS;            // alpha rows
    constexpr int RBUF = ABUF + P * 64;           // row above
    constexpr int BUF = RBUF + 64;
    float* bufs = smem + wave * 2 * BUF;
    float2* rings = reinterpret_cast<float2*>(smem + NW * 2 * BUF);  // [2][NW][R] (up, diag)
    float2* sink = rings + 2 * NW * R + wave * DUMMY;
    int* st = status + b;
    const int tbase = Tile::read_base(lane);

    if (lane == 0) prog[wave] = -1;
    __syncthreads();

    const int L1 = min(max(lengths[2 * b], 0), L1max);
    const int L2 = min(max(lengths[2 * b + 1], 0), L2max);
    const float c = kLog2e / T;
    const float S = partition[b];
    const float Sc = S * c;
    const int NS = L2 > 0 ? (L1 + 63) >> 6 : 0;
    const int nsteps = L2 + 63;
    const int nch = (nsteps + P - 1) / P;
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
    float A[P + 2];

    // Stripes run bottom-up: order q = 0..NS-1 handles stripe NS-1-q, on wave q % NW.
    for (int q = wave; q < NS; q += NW) {
        const int s = NS - 1 - q;
        const int i0 = s * 64;
        const int L2eff = (i0 + lane < L1) ? L2 : 0;
        // alpha tables of this stripe and of the one above, from step -APAD
        const float* astripe = alpha_sk + ((size_t)b * NSmax + s) * NT * 64;
        const float* bup = brow + ((size_t)b * NSmax + (s > 0 ? s - 1 : 0)) * NT;
        const float2* ring_in =
            rings + ((((q - 1) / NW) & 1) * NW + (q + NW - 1) % NW) * R;   // from stripe s+1
        float2* ring_out = rings + (((q / NW) & 1) * NW + wave) * R;       // to stripe s-1
        const bool below = q > 0;
        const bool above = q + 1 < NS;

        // Loads of chunk k (t_hi = nsteps-1-kP) into buffer k&1: P score loads, P alpha
        // rows, and the row-above values (lane j <= P: the alpha of the last row of the
        // stripe above at step t_hi - j + 63, clamped to the last step; lanes past P
        // repeat lane P's address).  2P+1 loads.
        auto issue_chunk = [&](int k) {
            const int th = nsteps - 1 - k * P;
            const uint32_t buf = lds_address(bufs + (k & 1) * BUF);
            dma_scores<P, -1>(buf, sbase, i0, L1max, L2max, lane, th);
            uint32_t voff = (uint32_t)((th - 2 + APAD) * 64) * 4u + ul4;
            uint32_t lds = buf + ABUF * 4;
#pragma unroll
            for (int j = 0; j < P; ++j) lds_dma_dword<256>(astripe, voff, lds, (uint32_t)-256);
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
            if (below) wait_for(prog, (q - 1) % NW, (q - 1) * PROG_STRIDE + min(k + LEAD, nch), st);
            if (above) {
                const int need = k - 2 - R / P;   // slots of steps < kP+P-R must be consumed
                if (need > 0) wait_for(prog, (q + 1) % NW, (q + 1) * PROG_STRIDE + need, st);
            }
            // this chunk's loads were issued one chunk ago and followed by exactly the P
            // marginal stores of that chunk (the first chunk's are the last issued)
            if (k == 0) wait_vmcnt<0>(); else wait_vmcnt<P>();
            float* buf = bufs + (k & 1) * BUF;
            float* tile = buf;
            float sv[P];
#pragma unroll
            for (int u = 0; u < P; ++u) sv[u] = tile[tbase + u];
            A[0] = A[P];
            A[1] = A[P + 1];
#pragma unroll
            for (int j = 0; j < P; ++j) A[j + 2] = buf[ABUF + j * 64 + lane];
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
            float pre_d2 = wave_shr1(pre_d, 0.0f);   // lane 63 = step 1 (then shifted on)
            pre_d2 = wave_shr1(pre_d2, 0.0f);        // lane 63 = step 2
#pragma unroll
            for (int u = 0; u < P; ++u) {
                const int t = t_hi - u;
                const bool ok = (unsigned)(t - lane) < (unsigned)L2eff;
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
                float lp = a0 * c - Sc;
                lp = lp < 0.0f ? lp : 0.0f;
                const float binit = fast_exp2(lp);
                // reference accumulation order: init, diagonal, left, up successor
                const float beta = ((binit + in_diag) + in_left) + in_up;
                const bool live = ok && (beta <= 3.0e38f);    // skips inf / NaN like the reference
                const float br = live ? beta * rin : 0.0f;
                const float od = br * e0, ou = br * e1, ol = br * e2;
                const float pv = br * (e0 + e3);
                tile[tbase + u] = pv;
                g_acc += ou;
                g_acc += ol;
                p_acc += pv * sc;
                pub[u] = make_float2(ou, od);
                // successor contributions for the next steps; lane 63 takes the ring
                pre_u = wave_shr1(pre_u, 0.0f);
                in_left = ol;
                in_up = wave_shl1_or(ou, pre_u);
                in_diag = in_diag_next;
                in_diag_next = wave_shl1_or(od, pre_d2);
                pre_d2 = wave_shr1(pre_d2, 0.0f);
            }
            wave_lds_sync();
            // write this chunk's marginals back over the cells the scores came from:
            // exactly P stores (cells outside the element's lengths go to the trash
            // line in boundary chunks, and carry 0 in inside chunks)
            if (chunk_inside<P, -1>(i0, L1max, L2max, t_hi)) {
                uint32_t off4 = (uint32_t)chunk_offset0<P, -1>(i0, L2max, lane, t_hi) * 4u;
                const uint32_t step4 = (uint32_t)(L2max - 1) * 4u;
#pragma unroll
                for (int i = 0; i < P; ++i) {
                    lane_store(pbase, off4, tile[65 * i + lane]);
                    off4 += step4;
                    __asm__ volatile("" : "+v"(off4));   // keep one running offset
                }
            } else {
                const int u = lane % P, pj = lane - u;
                int row = i0 + pj, col = t_hi - u - pj;
#pragma unroll
                for (int i = 0; i < P; ++i) {
                    const bool in = row < L1 && col >= 0 && col < L2;
                    float* dst = in ? pbase + (size_t)row * L2max + col : trash + lane;
                    *dst = tile[65 * i + lane];
                    ++row;
                    --col;
                }
            }
            publish(prog, wave, q * PROG_STRIDE + k + 1);
        }
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
    // status words | trash line | skewed alpha table | last row of every stripe
    return sw::status_bytes(B) + sw::TRASH_BYTES +
           (size_t)B * ns * (size_t)sw::stored_steps(max_L2) * 65 * sizeof(float);
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
    D2P_REQUIRE(B >= 0 && max_L1 >= 0 && max_L2 >= 0, "negative dimension");
    D2P_REQUIRE(temperature > 0.0f, "temperature must be positive");
    if (B == 0) return D2P_OK;
    D2P_REQUIRE(scores && lengths && partition && marginals && grad_gap && grad_T,
                "null pointer argument");
    const size_t need = d2p_sw_workspace_bytes(B, max_L1, max_L2);
    D2P_REQUIRE(need == 0 || (workspace && workspace_bytes >= need), "workspace too small");
    D2P_REQUIRE(max_L2 + 63 < (1 << 16) * sw::PB, "max_L2 too large");
    // per-lane byte offsets within one batch element are 32-bit
    D2P_REQUIRE((size_t)max_L1 * max_L2 < ((size_t)1 << 30), "DP table too large");
    hipStream_t st = (hipStream_t)stream;
    const int ns = (max_L1 + 63) / 64;
    const int Rf = sw::ring_len(max_L1, max_L2, 256);
    const int Rb = sw::ring_len(max_L1, max_L2, 128);
    const size_t lds_f = (size_t)sw::NW * 2 * 65 * sw::PF * sizeof(float) +
                         (2 * (size_t)sw::NW * Rf + sw::NW * sw::DUMMY) * sizeof(float);
    const size_t lds_b = (size_t)sw::NW * 2 * (65 * sw::PB + 64 * sw::PB + 64) * sizeof(float) +
                         (2 * (size_t)sw::NW * Rb + sw::NW * sw::DUMMY) * sizeof(float2);
    D2P_REQUIRE(lds_f <= 160 * 1024 - 256 && lds_b <= 160 * 1024 - 256,
                "sequence too long for the LDS stripe rings (max_L2 with more than 512 rows)");
    D2P_HIP(hipFuncSetAttribute((const void*)sw::sw_forward_kernel,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_f));
    D2P_HIP(hipFuncSetAttribute((const void*)sw::sw_backward_kernel,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_b));
    int* status = (int*)workspace;
    float* trash = (float*)((char*)workspace + sw::status_bytes(B));
    float* alpha_sk = (float*)((char*)trash + sw::TRASH_BYTES);
    float* brow = alpha_sk + (size_t)B * ns * sw::stored_steps(max_L2) * 64;
    D2P_LAUNCH("sw_forward", sw::sw_forward_kernel, dim3(B), dim3(sw::NW * 64), lds_f, st,
               scores, lengths, alpha_sk, brow, partition, status, max_L1, max_L2, ns, gap,
               temperature, Rf);
    D2P_HIP(hipGetLastError());
    D2P_LAUNCH("sw_backward", sw::sw_backward_kernel, dim3(B), dim3(sw::NW * 64), lds_b, st,
               scores, lengths, alpha_sk, brow, partition, marginals, grad_gap, grad_T, status,
               trash,
               max_L1, max_L2, ns, gap, temperature, Rb);
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}
