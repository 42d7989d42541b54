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
// matrix cores; the row sums of A ride along the staging.  Workgroup (m, b): m = 0
// makes dL/dx (A = G, K = L2, B = y), m = 1 dL/dy (A = G^T, K = L1, B = x), in passes
// of RB output rows, so that each element's features are read once per pass and G
// twice in all.  A pass stages K in chunks of FG_KC through LDS, with the next chunk's
// loads in registers during the current chunk's products.  Four waves each own RB/4
// rows by all KP columns: (RB/128) x (KP/32) accumulator tiles of 32 x 32, every
// operand read feeding several of them.
constexpr int FG_KC = 32;                   // K chunk staged per step

template <int KP>
struct FG {
    static constexpr int RB = KP == 128 ? 128 : 256;   // output rows per pass
    static constexpr int RTW = RB / 128;               // row tiles per wave
    static constexpr int CT = KP / 32;                 // column tiles
    static constexpr int NA = RB * FG_KC / 256;        // A values staged per thread
    static constexpr int NB = FG_KC * KP / 256;        // B values staged per thread
    // A chunk: dL/dx [RB][FG_KC + 1] (rows r, k), dL/dy [FG_KC][RB] (k, rows r)
    static constexpr int AFLOATS = RB * (FG_KC + 1);
    static constexpr size_t lds() { return ((size_t)AFLOATS + FG_KC * KP + RB) * sizeof(float); }
};

// ROWS: dL/dx (rows of G, K = L2) or dL/dy (columns of G, K = L1)
template <int KP, bool ROWS>
__device__ __forceinline__ void feature_grad_block(const float* __restrict__ G,
                                                   const float* __restrict__ x,
                                                   const float* __restrict__ y,
                                                   const float* __restrict__ scale,
                                                   float* __restrict__ gx, float* __restrict__ gy,
                                                   int B, int L1, int L2, int D, float* sm) {
    using F = FG<KP>;
    constexpr int RB = F::RB, RTW = F::RTW, CT = F::CT, NA = F::NA, NB = F::NB;
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
    // row sums: RPT threads per row, each a k range of FG_KC / RPT
    constexpr int RPT = 256 / RB;
    const int srow = threadIdx.x / RPT, spart = threadIdx.x % RPT;
    // thread t's staged A values: dL/dx element t + 256 n of the [RB][FG_KC] chunk, dL/dy
    // of the [FG_KC][RB] chunk
    const int a_r = ROWS ? threadIdx.x / FG_KC : threadIdx.x % RB;
    const int a_k = ROWS ? threadIdx.x % FG_KC : threadIdx.x / RB;
    constexpr int A_DR = 256 / FG_KC, A_DK = 256 / RB;   // per n: rows (dL/dx), k (dL/dy)
    const int bk0 = threadIdx.x / KP, bd = threadIdx.x % KP;
    constexpr int BDK = 256 / KP;                // B rows per n (KP <= 256)
    for (int b = blockIdx.y; b < B; b += gridDim.y) {
        const float* Gb = G + (size_t)b * L1 * L2;
        const float* Bsrc = (ROWS ? y : x) + (size_t)b * K * D;   // B rows: [K][D]
        const float* self = (ROWS ? x : y) + (size_t)b * L * D;
        float* out = (ROWS ? gx : gy) + (size_t)b * L * D;
        const float f = 2.0f * (scale ? scale[b] : 1.0f);
        for (int r0 = 0; r0 < L; r0 += RB) {
            const float* gb = Gb + (ROWS ? (size_t)r0 * L2 : (size_t)r0);
            float av[NA], bv[NB];
            // branch-free: clamped in-bounds reads; the values past the element, K and D
            // are zeroed only when the chunk is stored to LDS (a select at load time
            // would wait for each load at once)
            auto a_ok = [&](int k0, int n) {
                return ROWS ? (r0 + a_r + A_DR * n < L1 && k0 + a_k < L2)
                            : (r0 + a_r < L2 && k0 + a_k + A_DK * n < L1);
            };
            auto b_ok = [&](int k0, int n) { return k0 + bk0 + BDK * n < K && bd < D; };
            auto load = [&](int k0) {
#pragma unroll
                for (int n = 0; n < NA; ++n) {
                    unsigned off;
                    if (ROWS) {
                        const int r = a_r + A_DR * n, k = k0 + a_k;
                        off = (unsigned)(min(r, L1 - 1 - r0) * L2 + min(k, L2 - 1));
                    } else {
                        const int k = k0 + a_k + A_DK * n;
                        off = (unsigned)(min(k, L1 - 1) * L2 + min(a_r, L2 - 1 - r0));
                    }
                    av[n] = lane_load(gb, off * 4u);
                }
#pragma unroll
                for (int n = 0; n < NB; ++n) {
                    const int k = k0 + bk0 + BDK * n;
                    bv[n] = lane_load(Bsrc, (unsigned)(min(k, K - 1) * D + min(bd, D - 1)) * 4u);
                }
            };
            f32x16 acc[RTW][CT];
#pragma unroll
            for (int t = 0; t < RTW; ++t)
#pragma unroll
                for (int c = 0; c < CT; ++c)
#pragma unroll
                    for (int v = 0; v < 16; ++v) acc[t][c][v] = 0.0f;
            float rsum = 0.0f;
            load(0);
            for (int k0 = 0; k0 < K; k0 += FG_KC) {
                __syncthreads();   // the previous chunk's reads are complete
#pragma unroll
                for (int n = 0; n < NA; ++n) {
                    const int idx = threadIdx.x + 256 * n;
                    const float v = a_ok(k0, n) ? av[n] : 0.0f;
                    if (ROWS) As[(idx / FG_KC) * KCS + idx % FG_KC] = v;
                    else As[idx] = v;   // [k][r]: element idx = k RB + r
                }
#pragma unroll
                for (int n = 0; n < NB; ++n) Bs[threadIdx.x + 256 * n] = b_ok(k0, n) ? bv[n] : 0.0f;
                // the next chunk's loads are in flight during this chunk's products
                if (k0 + FG_KC < K) load(k0 + FG_KC);
                __syncthreads();
#pragma unroll
                for (int kk = 0; kk < FG_KC / RPT; ++kk) {
                    const int k = spart * (FG_KC / RPT) + kk;
                    rsum += ROWS ? As[srow * KCS + k] : As[k * RB + srow];
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
            if (RPT > 1) rsum += __shfl_xor(rsum, 1, 64);   // the row's other k half
            if (spart == 0) rs[srow] = rsum;
            __syncthreads();
            // accumulator v of lane l in tile (t, c): row 8 (v / 4) + 4 (l / 32) + v % 4,
            // column l % 32.  Lane l's rows are rb + (32 t + 8 (v / 4) + v % 4): a
            // per-lane base and offsets common to the wave (scalar registers).  Per tile,
            // the 16 feature loads go out together before any store (a load inside each
            // store's bounds test would wait for memory once per output); in a pass past
            // the element's end the rows are clamped for the loads and tested for the
            // stores.
            const int rb = wr + 4 * (lane >> 5);
            auto epilogue = [&](auto full) {
                constexpr bool FULL = decltype(full)::value;
#pragma unroll
                for (int t = 0; t < RTW; ++t) {
#pragma unroll
                    for (int c = 0; c < CT; ++c) {
                        const int d = 32 * c + (lane & 31);
                        const int dc = min(d, D - 1);
                        const float* sp = self + (size_t)(r0 + rb) * D + dc;
                        float* op = out + (size_t)(r0 + rb) * D + d;
                        float sv[16];
#pragma unroll
                        for (int v = 0; v < 16; ++v) {
                            const int dr = 32 * t + 8 * (v >> 2) + (v & 3);
                            sv[v] = FULL ? sp[(size_t)dr * D]
                                         : self[(size_t)min(r0 + rb + dr, L - 1) * D + dc];
                        }
#pragma unroll
                        for (int v = 0; v < 16; ++v) {
                            const int dr = 32 * t + 8 * (v >> 2) + (v & 3);
                            if ((FULL || r0 + rb + dr < L) && d < D)
                                op[(size_t)dr * D] = f * fmaf(sv[v], rs[rb + dr], -acc[t][c][v]);
                        }
                    }
                }
            };
            if (r0 + RB <= L) epilogue(std::true_type{});
            else epilogue(std::false_type{});
            __syncthreads();   // rs and the chunks are rewritten by the next pass
        }
    }
}

template <int KP>
__global__ void __launch_bounds__(256)
feature_grad_kernel(const float* __restrict__ G, const float* __restrict__ x,
                    const float* __restrict__ y, const float* __restrict__ scale,
                    float* __restrict__ gx, float* __restrict__ gy, int B, int L1, int L2,
                    int D) {
    extern __shared__ __align__(16) float sm[];
    if (blockIdx.x == 0)
        feature_grad_block<KP, true>(G, x, y, scale, gx, gy, B, L1, L2, D, sm);
    else
        feature_grad_block<KP, false>(G, x, y, scale, gx, gy, B, L1, L2, D, sm);
}

template <int KP>
int launch_feature_grad_k(const float* G, const float* x, const float* y, const float* scale,
                          float* gx, float* gy, int B, int L1, int L2, int D, hipStream_t st) {
    const size_t lds = FG<KP>::lds();
    D2P_HIP(hipFuncSetAttribute((const void*)feature_grad_kernel<KP>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    const dim3 grid(2, std::min(B, SQ_GRID_MAX));
    D2P_LAUNCH("sqeuclid_feature_grad", feature_grad_kernel<KP>, grid, dim3(256), lds, st, G, x,
               y, scale, gx, gy, B, L1, L2, D);
    D2P_HIP(hipGetLastError());
    return D2P_OK;
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
    D2P_TRY(dtw::launch_backward(lengths, B, max_L1, max_L2, temperature, bandwidth, ws,
                                 marginals, grad_T, st));
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
