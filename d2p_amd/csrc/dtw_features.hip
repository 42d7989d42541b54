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

// One 64 x 64 tile of one element's costs per workgroup iteration: four waves, each a
// 32 x 32 quarter on the matrix cores.  Workgroups stride over column tiles (x), row
// tiles (y) and batch elements (z) past the grid extents.
template <int KP>
__global__ void __launch_bounds__(256)
sqdist_mfma_kernel(const float* __restrict__ x, const float* __restrict__ y,
                   float* __restrict__ costs, int B, int L1, int L2, int D) {
    constexpr int KS = KP + 4;
    constexpr int H = KP / 2;
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
    // norms: thread t sums the half (t & 1) of row t / 2 (rows 0..63 of x, then y)
    const int nrow = threadIdx.x >> 1, nh = threadIdx.x & 1;
    // 16-byte global loads where rows and bases allow them
    const bool vec = (D & 3) == 0 && (((uintptr_t)x | (uintptr_t)y) & 15) == 0;
    for (int b = blockIdx.z; b < B; b += gridDim.z) {
        for (int ti = blockIdx.y; ti < nti; ti += gridDim.y) {
            for (int tj = blockIdx.x; tj < ntj; tj += gridDim.x) {
                const int i0 = ti * SQ_TILE, j0 = tj * SQ_TILE;
                __syncthreads();   // the previous tile's reads are complete
                const float* xb = x + ((size_t)b * L1 + i0) * D;
                const float* yb0 = y + ((size_t)b * L2 + j0) * D;
                // branch-free staging: clamped in-bounds reads, zeros past the element
                // and past D
                const int rx = L1 - 1 - i0, ry = L2 - 1 - j0;   // last rows of the tile
                if (vec) {
                    // 16-byte loads: thread t moves feature quad t % (KP/4) of rows
                    // t / (KP/4) + 256 / (KP/4) r
                    constexpr int QPR = KP / 4;
#pragma unroll
                    for (int n = 0; n < SQ_TILE * QPR / 256; ++n) {
                        const int idx = threadIdx.x + 256 * n;
                        const int r = idx / QPR, d = (idx % QPR) * 4;
                        const int dc = min(d, (D - 4) & ~3);
                        const float4 vx = *reinterpret_cast<const float4*>(
                            xb + (size_t)min(r, rx) * D + dc);
                        const float4 vy = *reinterpret_cast<const float4*>(
                            yb0 + (size_t)min(r, ry) * D + dc);
                        const bool okd = d < D;
                        const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                        *reinterpret_cast<float4*>(xs + r * KS + d) = (r <= rx && okd) ? vx : z;
                        *reinterpret_cast<float4*>(ys + r * KS + d) = (r <= ry && okd) ? vy : z;
                    }
                } else {
#pragma unroll 4
                    for (int idx = threadIdx.x; idx < SQ_TILE * KP; idx += 256) {
                        const int r = idx / KP, d = idx % KP;
                        const int dc = min(d, D - 1);
                        const float vx = xb[(size_t)min(r, rx) * D + dc];
                        const float vy = yb0[(size_t)min(r, ry) * D + dc];
                        xs[r * KS + d] = (r <= rx && d < D) ? vx : 0.0f;
                        ys[r * KS + d] = (r <= ry && d < D) ? vy : 0.0f;
                    }
                }
                __syncthreads();
                {
                    const float* row = (nrow < SQ_TILE ? xs + nrow * KS
                                                       : ys + (nrow - SQ_TILE) * KS) + nh * H;
                    float s = 0.0f;
#pragma unroll
                    for (int d = 0; d < H; d += 4) {
                        const float4 v = *reinterpret_cast<const float4*>(row + d);
                        s = fmaf(v.x, v.x, s);
                        s = fmaf(v.y, v.y, s);
                        s = fmaf(v.z, v.z, s);
                        s = fmaf(v.w, v.w, s);
                    }
                    s += __shfl_xor(s, 1, 64);   // the row's other half (lane t ^ 1)
                    if (nh == 0) (nrow < SQ_TILE ? nx : ny)[nrow & (SQ_TILE - 1)] = s;
                }
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
                __syncthreads();   // the norms
                // accumulator v of lane l: row 8 (v / 4) + 4 (l / 32) + v % 4 of the
                // quarter, column l % 32
                const int jj = wj + (lane & 31);
                const int j = j0 + jj;
                const float nyj = ny[jj];
                float* out = costs + ((size_t)b * L1 + i0) * L2 + j;
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int ii = wi + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                    if (i0 + ii < L1 && j < L2) {
                        const float c = fmaf(-2.0f, acc[v], nx[ii] + nyj);
                        out[(size_t)ii * L2] = fmaxf(c, 0.0f);
                    }
                }
            }
        }
    }
}

template <int KP>
int launch_sqdist_k(const float* x, const float* y, float* costs, int B, int L1, int L2, int D,
                    hipStream_t st) {
    const size_t lds = sqdist_lds(KP);
    D2P_HIP(hipFuncSetAttribute((const void*)sqdist_mfma_kernel<KP>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    const dim3 grid(std::min((L2 + SQ_TILE - 1) / SQ_TILE, SQ_GRID_MAX),
                    std::min((L1 + SQ_TILE - 1) / SQ_TILE, SQ_GRID_MAX),
                    std::min(B, SQ_GRID_MAX));
    D2P_LAUNCH("pairwise_sqdist", sqdist_mfma_kernel<KP>, grid, dim3(256), lds, st, x, y, costs,
               B, L1, L2, D);
    D2P_HIP(hipGetLastError());
    return D2P_OK;
}

int launch_sqdist(const float* x, const float* y, float* costs, int B, int L1, int L2, int D,
                  hipStream_t st) {
    switch (feature_chunk(D)) {
        case 32: return launch_sqdist_k<32>(x, y, costs, B, L1, L2, D, st);
        case 64: return launch_sqdist_k<64>(x, y, costs, B, L1, L2, D, st);
        default: return launch_sqdist_k<128>(x, y, costs, B, L1, L2, D, st);
    }
}

// ------------------------------------------------------------------ feature gradients

// Gradients through c_ij = |x_i - y_j|^2 into the features, from G = dL/dc [B, L1, L2]
// and a per-element factor s_b (1 when absent):
//   dL/dx_i = 2 s_b (x_i sum_j G_ij - sum_j G_ij y_j)
//   dL/dy_j = 2 s_b (y_j sum_i G_ij - sum_i G_ij x_i)
// (the chain rule of the squared distance, which the expansion's derivative equals
// away from its clamp at 0).  The two products are [64, L] x [L, D] contractions on
// the matrix cores; the row and column sums of G ride along the staging.  Workgroup
// (bx, b): bx < nbi makes rows 64 bx.. of dL/dx (K = L2, A = G), else rows
// 64 (bx - nbi).. of dL/dy (K = L1, A = G^T); four waves, each 32 rows by KP / 2
// columns (KP = 32: waves 0 and 1, all 32 columns).  G is read twice, by its row
// blocks and by its column blocks.
constexpr int FG_KC = 32;                   // K chunk staged per step
constexpr int FG_AS = FG_KC + 1;            // LDS row stride of the A chunk

__host__ inline size_t feature_grad_lds(int KP) {
    return ((size_t)64 * FG_AS + (size_t)FG_KC * KP + 64) * sizeof(float);
}

// ROWS: dL/dx (rows of G, K = L2) or dL/dy (columns of G, K = L1), rows r0.. of it
template <int KP, bool ROWS>
__device__ __forceinline__ void feature_grad_block(const float* __restrict__ G,
                                                   const float* __restrict__ x,
                                                   const float* __restrict__ y,
                                                   const float* __restrict__ scale,
                                                   float* __restrict__ gx, float* __restrict__ gy,
                                                   int B, int L1, int L2, int D, int r0,
                                                   float* sm) {
    constexpr int NT = KP >= 64 ? KP / 64 : 1;   // 32-column accumulator tiles per wave
    constexpr int NA = 64 * FG_KC / 256;         // A values staged per thread and chunk
    constexpr int NB = FG_KC * KP / 256;         // B values staged per thread and chunk
    float* As = sm;                              // [64][FG_AS]: A rows r0.., k chunk
    float* Bs = As + 64 * FG_AS;                 // [FG_KC][KP]: B rows of the k chunk
    float* rs = Bs + FG_KC * KP;                 // [64]: the rows' sums of A
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int L = ROWS ? L1 : L2;                // output rows
    const int K = ROWS ? L2 : L1;                // contraction length
    const int wr = (wave & 1) * 32;
    const int wc = (wave >> 1) * 32 * NT;
    const bool active = wc < KP;
    const float* arow = As + (wr + (lane & 31)) * FG_AS + (lane >> 5);
    // row sums: thread t adds a quarter (t % 4) of row t / 4 of each chunk
    const int srow = threadIdx.x >> 2, sq = threadIdx.x & 3;
    // thread t's first A value: row t / FG_KC, k t % FG_KC (dL/dx), or row t % 64,
    // k t / 64 (dL/dy); its n-th lies 256 / FG_KC rows (dL/dx) or 4 k (dL/dy) further
    const int ar0 = ROWS ? threadIdx.x / FG_KC : threadIdx.x % 64;
    const int ak0 = ROWS ? threadIdx.x % FG_KC : threadIdx.x / 64;
    constexpr int ADR = 256 / FG_KC, ADK = 256 / 64;
    const int bk0 = threadIdx.x / KP, bd = threadIdx.x % KP;
    constexpr int BDK = 256 / KP;                // B rows per n (KP <= 256)
    for (int b = blockIdx.y; b < B; b += gridDim.y) {
        const float* Gb = G + (size_t)b * L1 * L2;
        const float* Bsrc = (ROWS ? y : x) + (size_t)b * K * D;   // B rows: [K][D]
        const float* self = (ROWS ? x : y) + (size_t)b * L * D;
        float* out = (ROWS ? gx : gy) + (size_t)b * L * D;
        const float* gb = Gb + (ROWS ? (size_t)r0 * L2 : (size_t)r0);
        float av[NA], bv[NB];
        // a chunk's A values (G's rows for dL/dx, its columns for dL/dy) and B values
        // (the other sequence's features), branch-free: clamped in-bounds reads, zeros
        // past the element, K and D
        auto load = [&](int k0) {
#pragma unroll
            for (int n = 0; n < NA; ++n) {
                bool ok;
                unsigned off;
                if (ROWS) {
                    const int r = ar0 + ADR * n, k = k0 + ak0;
                    ok = r0 + r < L1 && k < L2;
                    off = (unsigned)(min(r, L1 - 1 - r0) * L2 + min(k, L2 - 1));
                } else {
                    const int k = k0 + ak0 + ADK * n;
                    ok = r0 + ar0 < L2 && k < L1;
                    off = (unsigned)(min(k, L1 - 1) * L2 + min(ar0, L2 - 1 - r0));
                }
                const float v = lane_load(gb, off * 4u);
                av[n] = ok ? v : 0.0f;
            }
#pragma unroll
            for (int n = 0; n < NB; ++n) {
                const int k = k0 + bk0 + BDK * n;
                const float v =
                    lane_load(Bsrc, (unsigned)(min(k, K - 1) * D + min(bd, D - 1)) * 4u);
                bv[n] = (k < K && bd < D) ? v : 0.0f;
            }
        };
        f32x16 acc[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[t][v] = 0.0f;
        float rsum = 0.0f;                       // thread t: its quarter of row t / 4
        load(0);
        for (int k0 = 0; k0 < K; k0 += FG_KC) {
            __syncthreads();   // the previous chunk's reads are complete
#pragma unroll
            for (int n = 0; n < NA; ++n) {
                const int idx = threadIdx.x + 256 * n;
                if (ROWS) As[(idx / FG_KC) * FG_AS + idx % FG_KC] = av[n];
                else As[(idx % 64) * FG_AS + idx / 64] = av[n];
            }
#pragma unroll
            for (int n = 0; n < NB; ++n) Bs[threadIdx.x + 256 * n] = bv[n];
            // the next chunk's loads are in flight during this chunk's products
            if (k0 + FG_KC < K) load(k0 + FG_KC);
            __syncthreads();
            {
                const float* ar = As + srow * FG_AS + sq * (FG_KC / 4);
#pragma unroll
                for (int kk = 0; kk < FG_KC / 4; ++kk) rsum += ar[kk];
            }
            if (active) {
                // (partly unrolled: a full unroll hoists every operand read and leaves
                // one wave per SIMD)
#pragma unroll 2
                for (int kk = 0; kk < FG_KC; kk += 2) {
                    const float a = arow[kk];
                    const float* brow = Bs + (kk + (lane >> 5)) * KP + wc + (lane & 31);
#pragma unroll
                    for (int t = 0; t < NT; ++t)
                        acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, brow[32 * t], acc[t],
                                                                      0, 0, 0);
                }
            }
        }
        // the row's four quarters (lanes 4r .. 4r + 3)
        rsum += __shfl_xor(rsum, 1, 64);
        rsum += __shfl_xor(rsum, 2, 64);
        if (sq == 0) rs[srow] = rsum;
        __syncthreads();
        const float f = 2.0f * (scale ? scale[b] : 1.0f);
        if (active) {
            // accumulator v of lane l: row 8 (v / 4) + 4 (l / 32) + v % 4, column l % 32
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const int d = wc + 32 * t + (lane & 31);
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int r = wr + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                    if (r0 + r < L && d < D) {
                        const size_t o = (size_t)(r0 + r) * D + d;
                        out[o] = f * fmaf(self[o], rs[r], -acc[t][v]);
                    }
                }
            }
        }
        __syncthreads();   // rs is rewritten for the next element
    }
}

template <int KP>
__global__ void __launch_bounds__(256)
feature_grad_kernel(const float* __restrict__ G, const float* __restrict__ x,
                    const float* __restrict__ y, const float* __restrict__ scale,
                    float* __restrict__ gx, float* __restrict__ gy, int B, int L1, int L2,
                    int D) {
    extern __shared__ __align__(16) float sm[];
    const int nbi = (L1 + 63) / 64, nbj = (L2 + 63) / 64;
    const int bx = blockIdx.x;
    if (bx < nbi)
        feature_grad_block<KP, true>(G, x, y, scale, gx, gy, B, L1, L2, D, bx * 64, sm);
    else if (bx < nbi + nbj)
        feature_grad_block<KP, false>(G, x, y, scale, gx, gy, B, L1, L2, D, (bx - nbi) * 64, sm);
}

template <int KP>
int launch_feature_grad_k(const float* G, const float* x, const float* y, const float* scale,
                          float* gx, float* gy, int B, int L1, int L2, int D, hipStream_t st) {
    const size_t lds = feature_grad_lds(KP);
    D2P_HIP(hipFuncSetAttribute((const void*)feature_grad_kernel<KP>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    const dim3 grid((L1 + 63) / 64 + (L2 + 63) / 64, std::min(B, SQ_GRID_MAX));
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
