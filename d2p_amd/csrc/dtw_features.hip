// dtw_features.hip -- soft DTW between feature sequences on gfx950: squared-Euclidean
// costs from an fp32 matrix-core product.
//
// No counterpart in the reference: its callers form the costs with
// torch.cdist(x, y) ** 2 (/root/reference/docs/algorithms/dtw.md:52) before its sweeps
// read them (/root/reference/src/dtw/kernels.cu:55-114).  Here
//   c[b, i, j] = max(|x_i|^2 + |y_j|^2 - 2 x_i . y_j, 0)
// with the dot products on v_mfma_f32_32x32x2f32 (a dense [L1, D] x [D, L2] contraction
// per element, the one GEMM-shaped piece of the path) and the norms and the epilogue
// in fp32 on the VALU.  This is the expansion torch.cdist itself uses at these sizes
// (its default compute mode, matrix products above 25 rows): the cost is exact to
// about (D + 4) u (|x_i| + |y_j|)^2 with u = 2^-24, against (D + 2) u c for a direct
// sum of D squares.  The fused op writes these costs into its marginals buffer, the
// forward sweep reads them there, and the reverse sweep, which reads only the alpha
// table, then overwrites them with the marginals: no extra [B, L1, L2] memory.

#include <algorithm>
#include <type_traits>

#include "wavefront.hip.h"
#include "../../include/d2p_amd.h"
#include "capi_util.hip.h"
#include "dtw_internal.hip.h"

namespace d2p_amd {
namespace dtw {

using wf::lane_load;

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int SQ_TILE = 64;             // rows and columns of one workgroup's cost tile
constexpr int SQ_GRID_MAX = 65535;      // grid y and z extents
constexpr int FEATURE_MAX = 128;        // largest feature dimension D

// Features padded to KP = 32, 64 or 128 (zeros add exact zeros).  MFMA step m pairs
// feature m (lanes 0..31) with feature m + KP/2 (lanes 32..63): the dot product sums
// every feature once in any pairing, and this one makes each lane's operands
// consecutive in its LDS row, so they load as 16-byte reads.  LDS rows are KP + 4
// floats (16-byte aligned).
inline int feature_chunk(int D) { return D <= 32 ? 32 : D <= 64 ? 64 : D <= 128 ? 128 : 0; }
__host__ inline size_t sqdist_lds(int KP) {
    return ((size_t)2 * SQ_TILE * (KP + 4) + 2 * SQ_TILE) * sizeof(float);
}

// One strip of 64 rows of one element's costs per workgroup iteration, in 64 x 64 tiles
// along j: the strip's x rows and norms stay in LDS, and the next tile's y rows load
// into registers during the current tile's products.  Four waves, each a 32 x 32
// quarter of a tile on the matrix cores.  Workgroups stride over strips (x) and batch
// elements (y) past the grid extents.  VEC: 16-byte global loads (D % 4 == 0, 16-byte
// aligned bases).
template <int KP, bool VEC>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(KP == 128 ? 2 : VEC ? 4 : 3)))
sqdist_mfma_kernel(const float* __restrict__ x, const float* __restrict__ y,
                   float* __restrict__ costs, int B, int L1, int L2, int D) {
    constexpr int KS = KP + 4;
    constexpr int H = KP / 2;
    constexpr int QPR = KP / 4;                  // feature quads per row
    constexpr int NV = VEC ? SQ_TILE * QPR / 256 : SQ_TILE * KP / 256;   // loads per thread
    extern __shared__ __align__(16) float sm[];
    float* xs = sm;                        // [64][KS] rows i0.. of x
    float* ys = xs + SQ_TILE * KS;         // [64][KS] rows j0.. of y
    float* nx = ys + SQ_TILE * KS;         // [64] |x_i|^2
    float* ny = nx + SQ_TILE;              // [64] |y_j|^2
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nti = (L1 + SQ_TILE - 1) / SQ_TILE, ntj = (L2 + SQ_TILE - 1) / SQ_TILE;
    // this wave's quarter; lane l's operand rows (l % 32) and half (l / 32)
    const int wi = (wave >> 1) * 32, wj = (wave & 1) * 32;
    const float* xa = xs + (wi + (lane & 31)) * KS + (lane >> 5) * H;
    const float* yb = ys + (wj + (lane & 31)) * KS + (lane >> 5) * H;
    // norms: thread t sums the half (t & 1) of row (t / 2) % 64 of y (t < 128) or x
    const int nrow = (threadIdx.x >> 1) & (SQ_TILE - 1), nh = threadIdx.x & 1;
    const bool nrow_x = threadIdx.x >= 2 * SQ_TILE;
    // thread t's staged values: n-th of VEC: quad t % QPR of row t / QPR + n 256 / QPR;
    // else: feature t % KP of row t / KP + n 256 / KP
    const int s_r = VEC ? threadIdx.x / QPR : threadIdx.x / KP;
    const int s_d = VEC ? (threadIdx.x % QPR) * 4 : threadIdx.x % KP;
    constexpr int S_DR = VEC ? 256 / QPR : 256 / KP;
    const int s_dc = VEC ? min(s_d, (D - 4) & ~3) : min(s_d, D - 1);
    typedef typename std::conditional<VEC, float4, float>::type V;
    // branch-free staging: clamped in-bounds reads; values past the element and past D
    // are zeroed when stored to LDS (a select at load time waits for each load at once)
    auto load = [&](const float* base, int rlast, V* v) {
#pragma unroll
        for (int n = 0; n < NV; ++n)
            v[n] = *reinterpret_cast<const V*>(base + (size_t)min(s_r + S_DR * n, rlast) * D +
                                               s_dc);
    };
    auto stage = [&](float* dst, int rlast, const V* v) {
#pragma unroll
        for (int n = 0; n < NV; ++n) {
            const int r = s_r + S_DR * n;
            const bool ok = r <= rlast && s_d < D;
            V w = v[n];
            // (per component: a select of whole vectors becomes a select of their
            // addresses, which sends the registers to scratch memory)
            if constexpr (VEC) {
                w.x = ok ? w.x : 0.0f;
                w.y = ok ? w.y : 0.0f;
                w.z = ok ? w.z : 0.0f;
                w.w = ok ? w.w : 0.0f;
            } else {
                w = ok ? w : 0.0f;
            }
            *reinterpret_cast<V*>(dst + r * KS + s_d) = w;
        }
    };
    auto norm = [&](const float* tile) {
        const float* row = tile + nrow * KS + nh * H;
        float s = 0.0f;
#pragma unroll
        for (int d = 0; d < H; d += 4) {
            const float4 v = *reinterpret_cast<const float4*>(row + d);
            s = fmaf(v.x, v.x, s);
            s = fmaf(v.y, v.y, s);
            s = fmaf(v.z, v.z, s);
            s = fmaf(v.w, v.w, s);
        }
        return s + __shfl_xor(s, 1, 64);   // the row's other half (lane t ^ 1)
    };
    for (int b = blockIdx.y; b < B; b += gridDim.y) {
        const float* yb0 = y + (size_t)b * L2 * D;
        for (int ti = blockIdx.x; ti < nti; ti += gridDim.x) {
            const int i0 = ti * SQ_TILE;
            const int rx = L1 - 1 - i0;   // last row of the strip
            V xv[NV], yv[NV];
            load(x + ((size_t)b * L1 + i0) * D, rx, xv);
            load(yb0, L2 - 1, yv);
            __syncthreads();   // the previous strip's reads are complete
            stage(xs, rx, xv);
            stage(ys, L2 - 1, yv);
            __syncthreads();
            if (nrow_x) {
                const float s = norm(xs);
                if (nh == 0) nx[nrow] = s;
            }
            for (int tj = 0; tj < ntj; ++tj) {
                const int j0 = tj * SQ_TILE;
                if (!nrow_x) {
                    const float s = norm(ys);
                    if (nh == 0) ny[nrow] = s;
                }
                // the next tile's rows are in flight during this tile's products (the
                // last tile reloads itself: an unconditional load lets the compiler's
                // wait before it cover only the previous loads, not this tile's stores)
                const int jn = min(j0 + SQ_TILE, (ntj - 1) * SQ_TILE);
                load(yb0 + (size_t)jn * D, L2 - 1 - jn, yv);
                f32x16 acc;
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
                // (two steps of 4 unrolled: a full unroll hoists every operand read into
                // registers and costs occupancy)
#pragma unroll 2
                for (int m = 0; m < H; m += 4) {
                    const float4 a = *reinterpret_cast<const float4*>(xa + m);
                    const float4 c = *reinterpret_cast<const float4*>(yb + m);
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, c.x, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, c.y, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, c.z, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, c.w, acc, 0, 0, 0);
                }
                __syncthreads();   // the norms are written, every wave's products are done
                // accumulator v of lane l: row 8 (v / 4) + 4 (l / 32) + v % 4 of the
                // quarter, column l % 32
                const int jj = wj + (lane & 31);
                const int j = j0 + jj;
                const float nyj = ny[jj];
                float nxi[16];
#pragma unroll
                for (int v = 0; v < 16; ++v) nxi[v] = nx[wi + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3)];
                // the next tile goes to LDS before this tile's stores, so that its wait
                // for the loads does not also wait for the stores
                stage(ys, L2 - 1 - jn, yv);
                // lane l's rows are rb + (8 (v / 4) + v % 4): a per-lane base and offsets
                // common to the wave (scalar registers)
                const int rb = wi + 4 * (lane >> 5);
                float* out = costs + ((size_t)b * L1 + i0 + rb) * L2 + j;
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int dr = 8 * (v >> 2) + (v & 3);
                    if (dr <= rx - rb && j < L2)
                        out[(size_t)dr * L2] = fmaxf(fmaf(-2.0f, acc[v], nxi[v] + nyj), 0.0f);
                }
                __syncthreads();   // the next tile is staged and this tile's norms are read
            }
        }
    }
}

template <int KP, bool VEC>
int launch_sqdist_k(const float* x, const float* y, float* costs, int B, int L1, int L2, int D,
                    hipStream_t st) {
    const size_t lds = sqdist_lds(KP);
    D2P_HIP(hipFuncSetAttribute((const void*)sqdist_mfma_kernel<KP, VEC>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    const dim3 grid(std::min((L1 + SQ_TILE - 1) / SQ_TILE, SQ_GRID_MAX), std::min(B, SQ_GRID_MAX));
    D2P_LAUNCH("pairwise_sqdist", (sqdist_mfma_kernel<KP, VEC>), grid, dim3(256), lds, st, x, y,
               costs, B, L1, L2, D);
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

template <int KP>
int launch_sqdist_v(const float* x, const float* y, float* costs, int B, int L1, int L2, int D,
                    hipStream_t st) {
    const bool vec = (D & 3) == 0 && (((uintptr_t)x | (uintptr_t)y) & 15) == 0;
    return vec ? launch_sqdist_k<KP, true>(x, y, costs, B, L1, L2, D, st)
               : launch_sqdist_k<KP, false>(x, y, costs, B, L1, L2, D, st);
}

int launch_sqdist(const float* x, const float* y, float* costs, int B, int L1, int L2, int D,
                  hipStream_t st) {
    switch (feature_chunk(D)) {
        case 32: return launch_sqdist_v<32>(x, y, costs, B, L1, L2, D, st);
        case 64: return launch_sqdist_v<64>(x, y, costs, B, L1, L2, D, st);
        default: return launch_sqdist_v<128>(x, y, costs, B, L1, L2, D, st);
    }
}

// ------------------------------------------------------------------ feature gradients

// Gradients through c_ij = |x_i - y_j|^2 into the features, from G = dL/dc [B, L1, L2]
// and a per-element factor s_b (1 when absent):
//   dL/dx_i = 2 s_b (x_i sum_j G_ij - sum_j G_ij y_j)
//   dL/dy_j = 2 s_b (y_j sum_i G_ij - sum_i G_ij x_i)
// (the chain rule of the squared distance, which the expansion's derivative equals
// away from its clamp at 0).  The two products are [L, K] x [K, D] contractions on the
// matrix cores.  Workgroup (m, b): m = 0 makes dL/dx (A = G, K = L2, B = y), m = 1
// dL/dy (A = G^T, K = L1, B = x), in passes of RB output rows, so that each element's
// features are read once per pass and G twice in all.  A pass stages K in chunks of
// FG_KC through LDS, with the next chunk's loads in registers during the current
// chunk's products.  Four waves each own RB/4 rows by all KP columns: (RB/128) x
// (KP/32) accumulator tiles of 32 x 32, every operand read feeding several of them.
//
// Memory goes through buffer resources, one per chunk or pass whose records end at
// the element's last row: rows past the element read as zero (or, for a store, are
// dropped) with no test in the code, and a lane whose column lies past K or D starts
// from an offset of 2^31, past every resource's records.  No load result passes
// through a select, so loads stay in flight until their values are stored to LDS.
// W = 4: 16-byte loads (rows of G, x and y a multiple of 4 floats, 16-byte aligned
// bases); W = 1: 4-byte loads.
constexpr int FG_KC = 32;                   // K chunk staged per step
constexpr unsigned FG_OOB = 0x80000000u;    // an offset past every resource's records

// raw buffer (stride 0) over `bytes` bytes from base (clamped to [0, 2^31 - 1]), the
// gfx9 data-format word
__device__ __forceinline__ __amdgpu_buffer_rsrc_t fg_rsrc(const float* base, long long bytes) {
    const int n = (int)(bytes < 0 ? 0 : bytes > 0x7fffffffLL ? 0x7fffffffLL : bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, n, 0x00020000);
}

template <int W>
__device__ __forceinline__ void fg_load(float* v, __amdgpu_buffer_rsrc_t r, unsigned off) {
    if constexpr (W == 4) {
        typedef unsigned u4 __attribute__((ext_vector_type(4)));
        const u4 q = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
        v[0] = __uint_as_float(q.x);
        v[1] = __uint_as_float(q.y);
        v[2] = __uint_as_float(q.z);
        v[3] = __uint_as_float(q.w);
    } else {
        v[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
    }
}

template <int KP>
struct FG {
    static constexpr int RB = KP == 128 ? 128 : 256;   // output rows per pass
    static constexpr int RTW = RB / 128;               // row tiles per wave
    static constexpr int CT = KP / 32;                 // column tiles
    // A chunk: dL/dx [RB][FG_KC + 1] (rows r, k), dL/dy [FG_KC][RB] (k, rows r)
    static constexpr int AFLOATS = RB * (FG_KC + 1);
    static constexpr size_t lds() { return ((size_t)AFLOATS + FG_KC * KP + RB) * sizeof(float); }
};

// ROWS: dL/dx (rows of G, K = L2) or dL/dy (columns of G, K = L1)
template <int KP, bool ROWS, int W>
__device__ __forceinline__ void feature_grad_block(const float* __restrict__ G,
                                                   const float* __restrict__ x,
                                                   const float* __restrict__ y,
                                                   const float* __restrict__ scale,
                                                   float* __restrict__ gx, float* __restrict__ gy,
                                                   int B, int L1, int L2, int D, float* sm) {
    using F = FG<KP>;
    constexpr int RB = F::RB, RTW = F::RTW, CT = F::CT;
    constexpr int KCS = FG_KC + 1;
    float* As = sm;                              // the A chunk
    float* Bs = As + F::AFLOATS;                 // [FG_KC][KP]: B rows of the k chunk
    float* rs = Bs + FG_KC * KP;                 // [RB]: the rows' sums of A
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int L = ROWS ? L1 : L2;                // output rows
    const int K = ROWS ? L2 : L1;                // contraction length
    const int wr = wave * (RB / 4);              // this wave's first row of the pass
    // lane l's A operand of row tile t at k pair kk: row wr + 32 t + l % 32, k kk + l / 32
    const int arow = wr + (lane & 31), ak = lane >> 5;
    // A items of W values: dL/dx: item (i, j) = row i, k j..j+W-1 of the [RB][FG_KC]
    // chunk; dL/dy: k row i, rows j..j+W-1 of the [FG_KC][RB] chunk.  Thread t holds
    // items (a_i + A_DI n, a_j).
    constexpr int A_IPR = (ROWS ? FG_KC : RB) / W;          // items per chunk row
    constexpr int A_DI = 256 / A_IPR;
    constexpr int NA = RB * FG_KC / W / 256;
    const int a_i = threadIdx.x / A_IPR, a_j = (threadIdx.x % A_IPR) * W;
    // B items: k row b_k + B_DK n, features b_d..b_d+W-1 of the [FG_KC][KP] chunk
    constexpr int B_IPR = KP / W;
    constexpr int B_DK = 256 / B_IPR;
    constexpr int NB = FG_KC * KP / W / 256;
    const int b_k = threadIdx.x / B_IPR, b_d = (threadIdx.x % B_IPR) * W;
    // row sums: from the staged registers when W = 4 (dL/dx: NA rows of W values per
    // thread, reduced over the A_IPR lanes of a row; dL/dy: W rows per thread, reduced
    // over the A_DI threads of a row through LDS); from LDS when W = 1 (RPT threads per
    // row, FG_KC / RPT values each)
    constexpr int RPT = 256 / RB;
    const int srow = threadIdx.x / RPT, spart = threadIdx.x % RPT;
    for (int b = blockIdx.y; b < B; b += gridDim.y) {
        const float* Gb = G + (size_t)b * L1 * L2;
        const float* Bsrc = (ROWS ? y : x) + (size_t)b * K * D;   // B rows: [K][D]
        const float* self = (ROWS ? x : y) + (size_t)b * L * D;
        float* out = (ROWS ? gx : gy) + (size_t)b * L * D;
        const float f = 2.0f * (scale ? scale[b] : 1.0f);
        for (int r0 = 0; r0 < L; r0 += RB) {
            float av[NA][W], bv[NB][W];
            // lane bases of the items (n = 0): past L2 (dL/dy: columns of G) or D, the
            // out-of-range offset; rows past L1 (dL/dx) and k past K fall outside the
            // chunk's records
            const unsigned a_base = (unsigned)(a_i * L2 + a_j) * 4u;
            const unsigned a_lane = ROWS || r0 + a_j < L2 ? a_base : FG_OOB;
            const unsigned b_lane = b_d < D ? (unsigned)(b_k * D + b_d) * 4u : FG_OOB;
            auto load = [&](int k0) {
                // dL/dx: rows r0.. from column k0 (k past L2 tested per chunk); dL/dy:
                // rows k0.. from column r0
                const float* pa = Gb + (ROWS ? (size_t)r0 * L2 + k0 : (size_t)k0 * L2 + r0);
                const long long a_bytes =
                    ROWS ? ((long long)(L1 - r0) * L2 - k0) * 4 : ((long long)(L1 - k0) * L2 - r0) * 4;
                const __amdgpu_buffer_rsrc_t ra = fg_rsrc(pa, a_bytes);
                const unsigned a0 = !ROWS || k0 + a_j < L2 ? a_lane : FG_OOB;
#pragma unroll
                for (int n = 0; n < NA; ++n)
                    fg_load<W>(av[n], ra, a0 + (unsigned)(A_DI * n * L2) * 4u);
                const __amdgpu_buffer_rsrc_t rb_ =
                    fg_rsrc(Bsrc + (size_t)k0 * D, (long long)(K - k0) * D * 4);
#pragma unroll
                for (int n = 0; n < NB; ++n)
                    fg_load<W>(bv[n], rb_, b_lane + (unsigned)(B_DK * n * D) * 4u);
            };
            f32x16 acc[RTW][CT];
#pragma unroll
            for (int t = 0; t < RTW; ++t)
#pragma unroll
                for (int c = 0; c < CT; ++c)
#pragma unroll
                    for (int v = 0; v < 16; ++v) acc[t][c][v] = 0.0f;
            float rsum[ROWS ? NA : W];   // W = 4: this thread's partial row sums
#pragma unroll
            for (int n = 0; n < (ROWS ? NA : W); ++n) rsum[n] = 0.0f;
            if (K > 0) load(0);
            for (int k0 = 0; k0 < K; k0 += FG_KC) {
                __syncthreads();   // the previous chunk's reads are complete
#pragma unroll
                for (int n = 0; n < NA; ++n) {
                    const int i = a_i + A_DI * n;
                    if (ROWS) {
#pragma unroll
                        for (int w = 0; w < W; ++w) As[i * KCS + a_j + w] = av[n][w];
                    } else if (W == 4) {
                        *reinterpret_cast<float4*>(As + i * RB + a_j) =
                            make_float4(av[n][0], av[n][W > 1 ? 1 : 0], av[n][W > 2 ? 2 : 0],
                                        av[n][W > 3 ? 3 : 0]);
                    } else {
                        As[i * RB + a_j] = av[n][0];
                    }
                    if (W == 4) {
                        if (ROWS) {
                            rsum[n] += (av[n][0] + av[n][W > 1 ? 1 : 0]) +
                                       (av[n][W > 2 ? 2 : 0] + av[n][W > 3 ? 3 : 0]);
                        } else {
#pragma unroll
                            for (int w = 0; w < W; ++w) rsum[w] += av[n][w];
                        }
                    }
                }
#pragma unroll
                for (int n = 0; n < NB; ++n) {
                    float* dst = Bs + (b_k + B_DK * n) * KP + b_d;
                    if (W == 4)
                        *reinterpret_cast<float4*>(dst) =
                            make_float4(bv[n][0], bv[n][W > 1 ? 1 : 0], bv[n][W > 2 ? 2 : 0],
                                        bv[n][W > 3 ? 3 : 0]);
                    else
                        dst[0] = bv[n][0];
                }
                // the next chunk's loads are in flight during this chunk's products
                // (unconditional: past K every offset is out of range and reads zero,
                // with no memory access; a conditional refill would keep the staged
                // values alive beside the new ones, in copies)
                load(k0 + FG_KC);
                __syncthreads();
                if (W == 1) {
#pragma unroll
                    for (int kk = 0; kk < FG_KC / RPT; ++kk) {
                        const int k = spart * (FG_KC / RPT) + kk;
                        rsum[0] += ROWS ? As[srow * KCS + k] : As[k * RB + srow];
                    }
                }
#pragma unroll 2
                for (int kk = 0; kk < FG_KC; kk += 2) {
                    float a[RTW], bb[CT];
#pragma unroll
                    for (int t = 0; t < RTW; ++t)
                        a[t] = ROWS ? As[(arow + 32 * t) * KCS + kk + ak]
                                    : As[(kk + ak) * RB + arow + 32 * t];
#pragma unroll
                    for (int c = 0; c < CT; ++c) bb[c] = Bs[(kk + ak) * KP + 32 * c + (lane & 31)];
#pragma unroll
                    for (int t = 0; t < RTW; ++t)
#pragma unroll
                        for (int c = 0; c < CT; ++c)
                            acc[t][c] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t], bb[c],
                                                                             acc[t][c], 0, 0, 0);
                }
            }
            if (W == 1) {
                if (RPT > 1) rsum[0] += __shfl_xor(rsum[0], 1, 64);   // the row's other half
                if (spart == 0) rs[srow] = rsum[0];
            } else if (ROWS) {
                // the A_IPR consecutive lanes of a row
#pragma unroll
                for (int n = 0; n < NA; ++n) {
#pragma unroll
                    for (int o = 1; o < A_IPR; o *= 2) rsum[n] += __shfl_xor(rsum[n], o, 64);
                    if (a_j == 0) rs[a_i + A_DI * n] = rsum[n];
                }
            } else {
                // the A_DI threads of a row (one per k row of an item set) through LDS
                __syncthreads();   // the last chunk's reads are complete
#pragma unroll
                for (int w = 0; w < W; ++w) As[a_i * RB + a_j + w] = rsum[w];
                __syncthreads();
                if (threadIdx.x < RB) {
                    float t = 0.0f;
#pragma unroll
                    for (int i = 0; i < A_DI; ++i) t += As[i * RB + threadIdx.x];
                    rs[threadIdx.x] = t;
                }
            }
            __syncthreads();
            // accumulator v of lane l in tile (t, c): row 8 (v / 4) + 4 (l / 32) + v % 4,
            // column l % 32.  Lane l's rows are rb + (32 t + 8 (v / 4) + v % 4).  Per
            // tile, the 16 feature loads go out together before any store.
            const int rb = wr + 4 * (lane >> 5);
            const long long pass_bytes = (long long)(L - r0) * D * 4;   // rows past L: out of range
            const __amdgpu_buffer_rsrc_t rself = fg_rsrc(self + (size_t)r0 * D, pass_bytes);
            const __amdgpu_buffer_rsrc_t rout = fg_rsrc(out + (size_t)r0 * D, pass_bytes);
#pragma unroll
            for (int t = 0; t < RTW; ++t) {
#pragma unroll
                for (int c = 0; c < CT; ++c) {
                    const int d = 32 * c + (lane & 31);
                    const unsigned o0 = d < D ? (unsigned)(rb * D + d) * 4u : FG_OOB;
                    float sv[16];
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int dr = 32 * t + 8 * (v >> 2) + (v & 3);
                        fg_load<1>(&sv[v], rself, o0 + (unsigned)(dr * D) * 4u);
                    }
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int dr = 32 * t + 8 * (v >> 2) + (v & 3);
                        const float g = f * fmaf(sv[v], rs[rb + dr], -acc[t][c][v]);
                        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(g), rout,
                                                              o0 + (unsigned)(dr * D) * 4u, 0, 0);
                    }
                    // one tile's loads in flight at a time (registers)
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            __syncthreads();   // rs and the chunks are rewritten by the next pass
        }
    }
}

// (two waves per SIMD for the 16-byte form, its accumulators in the architectural
// registers; the 4-byte form needs more)
template <int KP, int W>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(W == 4 ? 2 : 1)))
feature_grad_kernel(const float* __restrict__ G, const float* __restrict__ x,
                    const float* __restrict__ y, const float* __restrict__ scale,
                    float* __restrict__ gx, float* __restrict__ gy, int B, int L1, int L2,
                    int D) {
    extern __shared__ __align__(16) float sm[];
    if (blockIdx.x == 0)
        feature_grad_block<KP, true, W>(G, x, y, scale, gx, gy, B, L1, L2, D, sm);
    else
        feature_grad_block<KP, false, W>(G, x, y, scale, gx, gy, B, L1, L2, D, sm);
}

template <int KP, int W>
int launch_feature_grad_w(const float* G, const float* x, const float* y, const float* scale,
                          float* gx, float* gy, int B, int L1, int L2, int D, hipStream_t st) {
    const size_t lds = FG<KP>::lds();
    D2P_HIP(hipFuncSetAttribute((const void*)feature_grad_kernel<KP, W>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    const dim3 grid(2, std::min(B, SQ_GRID_MAX));
    D2P_LAUNCH("sqeuclid_feature_grad", (feature_grad_kernel<KP, W>), grid, dim3(256), lds, st,
               G, x, y, scale, gx, gy, B, L1, L2, D);
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

template <int KP>
int launch_feature_grad_k(const float* G, const float* x, const float* y, const float* scale,
                          float* gx, float* gy, int B, int L1, int L2, int D, hipStream_t st) {
    const bool vec = (D & 3) == 0 && (L2 & 3) == 0 &&
                     (((uintptr_t)G | (uintptr_t)x | (uintptr_t)y) & 15) == 0;
    return vec ? launch_feature_grad_w<KP, 4>(G, x, y, scale, gx, gy, B, L1, L2, D, st)
               : launch_feature_grad_w<KP, 1>(G, x, y, scale, gx, gy, B, L1, L2, D, st);
}

}  // namespace dtw
}  // namespace d2p_amd

using namespace d2p_amd;

extern "C" int d2p_dtw_sqeuclid_forward_marginals(const float* x, const float* y,
                                                  const int* lengths, int B, int max_L1,
                                                  int max_L2, int D, float temperature,
                                                  int bandwidth, float* value, float* marginals,
                                                  float* grad_T, void* workspace,
                                                  size_t workspace_bytes, void* stream) {
    D2P_TRY(dtw::check_shape(B, max_L1, max_L2, temperature));
    D2P_REQUIRE(D >= 1 && D <= dtw::FEATURE_MAX, "feature dimension D must be between 1 and 128");
    if (B == 0) return D2P_OK;
    D2P_REQUIRE(x && y && value && marginals && grad_T, "null pointer argument");
    const size_t need = d2p_dtw_workspace_bytes_banded(B, max_L1, max_L2, bandwidth);
    D2P_REQUIRE(workspace && workspace_bytes >= need, "workspace too small");
    hipStream_t st = (hipStream_t)stream;
    const wf::Layout ws = wf::layout(workspace, B, max_L1, max_L2, 1, true, 8,
                                     dtw::band_elem_steps(max_L1, max_L2, bandwidth));
    // the costs go to the marginals buffer: the forward reads them, the reverse sweep
    // (which reads only the alpha table) overwrites them
    if (max_L1 > 0 && max_L2 > 0)
        D2P_TRY(dtw::launch_sqdist(x, y, marginals, B, max_L1, max_L2, D, st));
    D2P_TRY(dtw::launch_forward(marginals, lengths, B, max_L1, max_L2, temperature, bandwidth,
                                ws, value, st));
    bool poisoned = false;
    D2P_TRY(dtw::launch_backward(lengths, B, max_L1, max_L2, temperature, bandwidth, ws,
                                 marginals, grad_T, st, value, &poisoned));
    if (poisoned) return D2P_OK;
    return wf::launch_poison(ws.status, B, (long long)max_L1 * max_L2, marginals, nullptr, value,
                             grad_T, nullptr, nullptr, st);
}

extern "C" int d2p_pairwise_sqdist(const float* x, const float* y, int B, int L1, int L2, int D,
                                   float* costs, void* stream) {
    D2P_REQUIRE(B >= 0 && L1 >= 0 && L2 >= 0, "negative dimension");
    D2P_REQUIRE(D >= 1 && D <= dtw::FEATURE_MAX, "feature dimension D must be between 1 and 128");
    if (B == 0 || L1 == 0 || L2 == 0) return D2P_OK;
    D2P_REQUIRE(x && y && costs, "null pointer argument");
    return dtw::launch_sqdist(x, y, costs, B, L1, L2, D, (hipStream_t)stream);
}

extern "C" int d2p_sqeuclid_feature_grad(const float* G, const float* x, const float* y,
                                         const float* scale, int B, int L1, int L2, int D,
                                         float* grad_x, float* grad_y, void* stream) {
    D2P_REQUIRE(B >= 0 && L1 >= 0 && L2 >= 0, "negative dimension");
    D2P_REQUIRE(D >= 1 && D <= dtw::FEATURE_MAX, "feature dimension D must be between 1 and 128");
    D2P_REQUIRE((L1 + 63) / 64 + (L2 + 63) / 64 <= 2147483647 / 2, "sequences too long");
    if (B == 0 || (L1 == 0 && L2 == 0)) return D2P_OK;
    D2P_REQUIRE(x && y && grad_x && grad_y && (G || L1 == 0 || L2 == 0), "null pointer argument");
    hipStream_t st = (hipStream_t)stream;
    switch (dtw::feature_chunk(D)) {
        case 32:
            return dtw::launch_feature_grad_k<32>(G, x, y, scale, grad_x, grad_y, B, L1, L2, D, st);
        case 64:
            return dtw::launch_feature_grad_k<64>(G, x, y, scale, grad_x, grad_y, B, L1, L2, D, st);
        default:
            return dtw::launch_feature_grad_k<128>(G, x, y, scale, grad_x, grad_y, B, L1, L2, D,
                                                   st);
    }
}
