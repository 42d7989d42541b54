/*
 * d2p_oracle.h -- CPU restatement of the reference soft-DP kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * product path: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product (d2p_amd) never links or calls it.
 *
 * Every function restates, in plain C, the arithmetic of the matching
 * reference CPU kernel (same op order, same Kahan sums, same sentinels and
 * clamps) so that its outputs are bit-identical to a build of the reference
 * sources.  Signatures mirror the reference's extern "C" CPU entry points:
 *   /root/reference/src/sw/kernels_cpu.h:95-183
 *   /root/reference/src/sw_affine/kernels_cpu.h:80-167
 *   /root/reference/src/dtw/kernels_cpu.h:83-161
 * Batch elements are independent; the batch loop is OpenMP-parallel with one
 * element per iteration, so results do not depend on the thread count.
 */
#ifndef D2P_ORACLE_H
#define D2P_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* linear-gap soft Smith-Waterman */
void oracle_sw_forward(const float* scores, float* alpha, float* partition,
                       const int* lengths, int B, int L1, int L2, float gap, float T);
void oracle_sw_backward(const float* alpha, const float* scores, const float* partition,
                        float* beta, float* posteriors, float* grad_gap, float* grad_T,
                        const int* lengths, int B, int L1, int L2, float gap, float T);
void oracle_sw_hvp(const float* alpha, const float* scores, const float* partition,
                   const float* V, float* d_alpha, float* d_partition, float* beta,
                   float* d_beta, float* H, const int* lengths, int B, int L1, int L2,
                   float gap, float T);
void oracle_sw_param_grad(const float* alpha, const float* scores, const float* partition,
                          const float* dS_dtheta, float* U, float* beta, float* W,
                          float* dP, const int* lengths, int B, int L1, int L2,
                          float gap, float T, int param_type);

/* affine-gap (M/I/D) soft Smith-Waterman */
void oracle_swa_forward(const float* scores, float* alpha, float* partition,
                        const int* lengths, int B, int L1, int L2,
                        float gap_open, float gap_ext, float T);
void oracle_swa_backward(const float* alpha, const float* scores, const float* partition,
                         float* beta, float* posteriors, float* grad_open, float* grad_ext,
                         float* grad_T, const int* lengths, int B, int L1, int L2,
                         float gap_open, float gap_ext, float T);
void oracle_swa_hvp(const float* alpha, const float* scores, const float* partition,
                    const float* V, float* d_alpha, float* d_partition, float* d_beta,
                    float* H, const int* lengths, int B, int L1, int L2,
                    float gap_open, float gap_ext, float T);
void oracle_swa_param_grad(const float* alpha, const float* scores, const float* partition,
                           const float* dS_dtheta, float* U, float* beta, float* W,
                           float* dP, const int* lengths, int B, int L1, int L2,
                           float gap_open, float gap_ext, float T, int param_type);

/* soft DTW (softmin, optional Sakoe-Chiba band; bandwidth < 0 = none) */
void oracle_dtw_forward(const float* costs, float* alpha, float* score,
                        const int* lengths, int B, int L1, int L2, float T, int64_t bandwidth);
void oracle_dtw_backward(const float* alpha, const float* costs, const float* score,
                         float* beta, float* posteriors, float* grad_T,
                         const int* lengths, int B, int L1, int L2, float T, int64_t bandwidth);
void oracle_dtw_hvp(const float* alpha, const float* costs, const float* score,
                    const float* V, float* d_alpha, float* d_score, float* beta,
                    float* d_beta, float* H, const int* lengths, int B, int L1, int L2,
                    float T, int64_t bandwidth);
void oracle_dtw_param_grad(const float* alpha, const float* costs, const float* score,
                           float* U, float* beta, float* W, float* dP_dT,
                           const int* lengths, int B, int L1, int L2, float T,
                           int64_t bandwidth);

/* Test-only extensions (no reference counterpart): the backward sweeps again, with
 * the per-element parameter gradients also accumulated in double from the same
 * fp32 per-cell terms.  sums64: SW [B][2] (gap, T), affine [B][3] (open, ext, T),
 * DTW [B] (T). */
void oracle_nw_forward(const float* scores, float* alpha, float* score, const int* lengths,
                       int B, int maxL1, int maxL2, float gap, float T);
void oracle_nw_backward(const float* alpha, const float* scores, const float* score,
                        float* beta, float* posteriors, float* grad_gap, float* grad_T,
                        const int* lengths, int B, int maxL1, int maxL2, float gap, float T);

void oracle_nw_hvp(const float* alpha, const float* scores, const float* score, const float* V,
                   float* d_alpha, float* d_score, float* beta, float* d_beta, float* H,
                   const int* lengths, int B, int maxL1, int maxL2, float gap, float T);
void oracle_nw_param_grad(const float* alpha, const float* scores, const float* score,
                          const float* dS_dtheta, float* U, float* beta, float* W, float* dP,
                          const int* lengths, int B, int maxL1, int maxL2, float gap, float T,
                          int ptype);

void oracle_sw_backward_sums64(const float* alpha, const float* scores, const float* partition,
                               float* beta, float* posteriors, double* sums64,
                               const int* lengths, int B, int L1, int L2, float gap, float T);
void oracle_swa_backward_sums64(const float* alpha, const float* scores, const float* partition,
                                float* beta, float* posteriors, double* sums64,
                                const int* lengths, int B, int L1, int L2, float gap_open,
                                float gap_ext, float T);
void oracle_dtw_backward_sums64(const float* alpha, const float* costs, const float* score,
                                float* beta, float* posteriors, double* sums64,
                                const int* lengths, int B, int L1, int L2, float T,
                                int64_t bandwidth);

int oracle_max_threads(void);

/* affine-gap soft Needleman-Wunsch (nw_affine/kernels_cpu.cpp) */
void oracle_nwa_forward(const float* scores, float* alpha, float* score, const int* lengths,
                        int B, int maxL1, int maxL2, float go, float ge, float T);
void oracle_nwa_backward(const float* alpha, const float* scores, const float* score,
                         float* beta, float* posteriors, float* grad_open, float* grad_ext,
                         float* grad_T, const int* lengths, int B, int maxL1, int maxL2,
                         float go, float ge, float T);
void oracle_nwa_hvp(const float* alpha, const float* scores, const float* score,
                    const float* V, float* d_alpha, float* d_score, float* beta,
                    float* d_beta, float* H, const int* lengths, int B, int maxL1, int maxL2,
                    float go, float ge, float T);
void oracle_nwa_param_grad(const float* alpha, const float* scores, const float* score,
                           const float* dS_dtheta, float* U, float* beta, float* W, float* dP,
                           const int* lengths, int B, int maxL1, int maxL2, float go, float ge,
                           float T, int ptype);

#ifdef __cplusplus
}
#endif

#endif
