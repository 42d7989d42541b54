/*
 * d2p_amd.h -- C ABI of the MI355X (gfx950) soft-alignment DP kernels.
 *
 * This is the drop-in boundary for the reference's device layer (L1 in the
 * reference: extern "C" host wrappers in src/{sw,sw_affine,dtw}/kernels.cuh that
 * take plain device pointers and sizes).  Every entry point:
 *   - takes device pointers to caller-owned, contiguous buffers (float32 data,
 *     int32 lengths [B,2] with 0 <= lengths[b,0] <= max_L1, 0 <= lengths[b,1] <= max_L2;
 *     a NULL lengths pointer means every element has lengths (max_L1, max_L2)),
 *   - never allocates: scratch memory is a caller-provided workspace whose size the
 *     matching *_workspace_bytes() function returns,
 *   - enqueues its kernels on `stream` (a hipStream_t passed as void*; NULL = the
 *     default stream) and returns without synchronising,
 *   - returns 0 on success, non-zero on failure; d2p_last_error() then describes it.
 * Outputs are fully written (padded cells of the marginal matrices are zero).
 * No torch types cross this boundary; the PyTorch operator layer
 * (d2p_amd/csrc/torch_ops.cpp) is one client of it.
 */
#ifndef D2P_AMD_H
#define D2P_AMD_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Message describing the last failure on the calling thread ("" if none). */
const char* d2p_last_error(void);

/* ABI version of this library (incremented on incompatible changes). */
int d2p_abi_version(void);

/* Kernel timing (instrumentation; no counterpart in the reference, which has no
 * tracing).  While enabled, every kernel this library launches is bracketed by
 * HIP events recorded on the launch stream.  d2p_profile_report() waits for the
 * recorded events and writes one line per kernel name:
 *   "<name> <launches> <total_ms> <min_ms> <max_ms>\n"
 * d2p_profile_reset() drops the accumulated statistics. */
int d2p_profile_enable(int on);
int d2p_profile_report(char* buf, size_t len);
void d2p_profile_reset(void);

/* ---------------------------------------------------------------------------
 * Linear-gap soft Smith-Waterman
 * ------------------------------------------------------------------------- */

/* Workspace bytes needed by d2p_sw_forward_marginals for the given padded shape. */
size_t d2p_sw_workspace_bytes(int B, int max_L1, int max_L2);

/* Status of the last call of any entry point below that used `workspace` (every
 * workspace starts with the [B] per-element status words): ORs them into *status
 * (0 = clean; bit 0 = a pipeline wait of some element reached its bound and gave up).
 * The outputs of such an element are NaN: every entry point ends with a pass that
 * overwrites them, so a timed-out element can never pass for a result.  Synchronises
 * `stream`.  No counterpart in the reference (its kernels do not wait on each other). */
int d2p_sw_status(const void* workspace, int B, int* status, void* stream);

/* Bound of every pipeline wait of this library's kernels on the current device, in
 * polls (default 4194304, about 0.2 s of polling inside a workgroup; the waits
 * between workgroups of a split element poll a quarter as often, each poll about
 * 1 us).  A wait that reaches it gives up as described under d2p_sw_status, and the
 * kernel still runs to its end.  A test hook with no counterpart in the reference:
 * a small bound drives the timeout path without any kernel hanging. */
int d2p_set_spin_limit(int spins);

/* Forward value and marginals in one call.
 * Replaces the pair sw_regular_forward[_warp] + sw_regular_backward[_warp]
 * (/root/reference/src/sw/kernels.cuh:139-207) as sequenced by
 * SoftSWRegularCUDAFunction::forward (/root/reference/src/sw/torch_cuda.cpp:215-241).
 *   scores    [B, max_L1, max_L2]   input
 *   partition [B]                   out: soft alignment value S
 *   marginals [B, max_L1, max_L2]   out: dS/dscores (zero in padding)
 *   grad_gap  [B]                   out: dS/dgap
 *   grad_T    [B]                   out: dS/dtemperature                        */
int d2p_sw_forward_marginals(const float* scores, const int* lengths, int B, int max_L1,
                             int max_L2, float gap, float temperature, float* partition,
                             float* marginals, float* grad_gap, float* grad_T,
                             void* workspace, size_t workspace_bytes, void* stream);

/* d2p_sw_forward_marginals with no workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  Its scratch
 * memory is a static device array of d2p_sw_noalloc_scratch_bytes() = 64 MiB that
 * each GPU the library runs on holds until the process ends; the call allocates
 * nothing (with the opt-in launch profile off).  Shapes whose
 * d2p_sw_workspace_bytes(B, max_L1, max_L2) exceeds the array are rejected with an
 * error.  Every call on one GPU shares that GPU's array: calls that overlap in time
 * on one GPU (other streams, other host threads) race and must be serialised by
 * the caller.  Same outputs as d2p_sw_forward_marginals. */
int d2p_sw_forward_marginals_noalloc(const float* scores, const int* lengths, int B,
                                     int max_L1, int max_L2, float gap, float temperature,
                                     float* partition, float* marginals, float* grad_gap,
                                     float* grad_T, void* stream);
size_t d2p_sw_noalloc_scratch_bytes(void);

/* Workspace bytes of the second-order linear-gap entry points below (d2p_sw_hvp,
 * d2p_sw_param_jacobian, d2p_sw_backward_full). */
size_t d2p_sw_second_workspace_bytes(int B, int max_L1, int max_L2);

/* Hessian-vector product of the partition: hvp = (d^2 S / dscores^2) . tangent.
 * Replaces sw_regular_hvp (/root/reference/src/sw/kernels.cuh:209-236) as sequenced by
 * soft_sw_regular_hvp_cuda (/root/reference/src/sw/torch_cuda.cpp:507-567), which
 * runs the forward first.
 *   tangent, hvp [B, max_L1, max_L2]                                              */
int d2p_sw_hvp(const float* scores, const float* tangent, const int* lengths, int B,
               int max_L1, int max_L2, float gap, float temperature, float* hvp,
               void* workspace, size_t workspace_bytes, void* stream);

/* Jacobian of the marginals with respect to gap (param_type 0) or temperature (1).
 * Replaces sw_regular_param_grad (/root/reference/src/sw/kernels.cuh:238-281) as
 * sequenced by soft_sw_regular_param_jacobian_cuda
 * (/root/reference/src/sw/torch_cuda.cpp:573-668): forward, backward for dS/dtheta,
 * then the tangent and reverse sweeps.
 *   jacobian [B, max_L1, max_L2]                                                  */
int d2p_sw_param_jacobian(const float* scores, int param_type, const int* lengths, int B,
                          int max_L1, int max_L2, float gap, float temperature,
                          float* jacobian, void* workspace, size_t workspace_bytes,
                          void* stream);

/* Backward of the marginals output for a cotangent grad_alignment:
 *   grad_scores = H . grad_alignment,
 *   grad_gap[b] = <grad_alignment[b], dP_b/dgap>, grad_T[b] = <grad_alignment[b], dP_b/dT>
 * (per element; soft_sw_backward_full_cuda, /root/reference/src/sw/torch_cuda.cpp:670-790,
 * returns their sums over the batch).  The two dot products are accumulated inside
 * the reverse sweeps; the Jacobians are never written. */
int d2p_sw_backward_full(const float* scores, const float* grad_alignment, const int* lengths,
                         int B, int max_L1, int max_L2, float gap, float temperature,
                         float* grad_scores, float* grad_gap, float* grad_T, void* workspace,
                         size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Affine-gap soft Smith-Waterman (gap of length k costs open + (k-1)*ext)
 * ------------------------------------------------------------------------- */

/* Workspace bytes needed by d2p_swa_forward_marginals for the given padded shape.
 * Like every *_forward_marginals workspace it starts with the per-element status
 * words that d2p_sw_status reads. */
size_t d2p_swa_workspace_bytes(int B, int max_L1, int max_L2);

/* Forward value and marginals in one call.
 * Replaces the pair sw_affine_forward + sw_affine_backward
 * (/root/reference/src/sw_affine/kernels.cuh:165-223) as sequenced by
 * SoftSWAffineCUDAFunction::forward (/root/reference/src/sw_affine/torch_cuda.cpp:166-190).
 *   scores     [B, max_L1, max_L2]  input
 *   partition  [B]                  out: soft alignment value S
 *   marginals  [B, max_L1, max_L2]  out: dS/dscores (zero in padding)
 *   grad_open, grad_ext, grad_T [B] out: dS/dgap_open, dS/dgap_ext, dS/dtemperature */
int d2p_swa_forward_marginals(const float* scores, const int* lengths, int B, int max_L1,
                              int max_L2, float gap_open, float gap_ext, float temperature,
                              float* partition, float* marginals, float* grad_open,
                              float* grad_ext, float* grad_T, void* workspace,
                              size_t workspace_bytes, void* stream);

/* Workspace bytes of the second-order affine-gap entry points below (d2p_swa_hvp,
 * d2p_swa_param_jacobian, d2p_swa_backward_full). */
size_t d2p_swa_second_workspace_bytes(int B, int max_L1, int max_L2);

/* Hessian-vector product of the partition: hvp = (d^2 S / dscores^2) . tangent.
 * Replaces sw_affine_hvp (/root/reference/src/sw_affine/kernels.cuh:225-231) as
 * sequenced by soft_sw_affine_hvp_cuda (/root/reference/src/sw_affine/torch_cuda.cpp:508-578),
 * which runs the forward first.
 *   tangent, hvp [B, max_L1, max_L2]                                              */
int d2p_swa_hvp(const float* scores, const float* tangent, const int* lengths, int B,
                int max_L1, int max_L2, float gap_open, float gap_ext, float temperature,
                float* hvp, void* workspace, size_t workspace_bytes, void* stream);

/* Jacobian of the marginals with respect to gap_open (param_type 0), gap_ext (1) or
 * temperature (2).  Replaces sw_affine_param_grad
 * (/root/reference/src/sw_affine/kernels.cuh:256-265) as sequenced by
 * soft_sw_affine_param_jacobian_cuda (/root/reference/src/sw_affine/torch_cuda.cpp:580-679):
 * forward, backward for dS/dtheta, then the tangent and reverse sweeps.
 *   jacobian [B, max_L1, max_L2]                                                  */
int d2p_swa_param_jacobian(const float* scores, int param_type, const int* lengths, int B,
                           int max_L1, int max_L2, float gap_open, float gap_ext,
                           float temperature, float* jacobian, void* workspace,
                           size_t workspace_bytes, void* stream);

/* Backward of the marginals output for a cotangent grad_alignment:
 *   grad_scores = H . grad_alignment, and per element the dot products of
 *   grad_alignment[b] with dP_b/dgap_open, dP_b/dgap_ext and dP_b/dT
 * (soft_sw_affine_backward_full_cuda, /root/reference/src/sw_affine/torch_cuda.cpp:681-817,
 * returns their sums over the batch).  The dot products are accumulated inside the
 * reverse sweeps; the Jacobians are never written. */
int d2p_swa_backward_full(const float* scores, const float* grad_alignment, const int* lengths,
                          int B, int max_L1, int max_L2, float gap_open, float gap_ext,
                          float temperature, float* grad_scores, float* grad_open,
                          float* grad_ext, float* grad_T, void* workspace,
                          size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Linear-gap soft Needleman-Wunsch (global alignment)
 * ------------------------------------------------------------------------- */

/* Workspace bytes needed by d2p_nw_forward_marginals (status words first). */
size_t d2p_nw_workspace_bytes(int B, int max_L1, int max_L2);

/* Forward value and marginals in one call.
 * Replaces the pair nw_forward + nw_backward (/root/reference/src/nw/kernels.cuh:97-140)
 * as sequenced by SoftNWCUDAFunction::forward (/root/reference/src/nw/torch_cuda.cpp:
 * 115-180); the CPU kernels restated are /root/reference/src/nw/kernels_cpu.cpp:78-265.
 *   scores    [B, max_L1, max_L2]  input
 *   value     [B]                  out: alpha[L1, L2] (alpha[i,0] = i*gap, alpha[0,j] = j*gap)
 *   marginals [B, max_L1, max_L2]  out: dvalue/dscores (zero in padding)
 *   grad_gap  [B]                  out: dvalue/dgap (boundary cells included)
 *   grad_T    [B]                  out: dvalue/dtemperature */
int d2p_nw_forward_marginals(const float* scores, const int* lengths, int B, int max_L1,
                             int max_L2, float gap, float temperature, float* value,
                             float* marginals, float* grad_gap, float* grad_T, void* workspace,
                             size_t workspace_bytes, void* stream);

/* Workspace bytes of the second-order global-alignment entry points below
 * (d2p_nw_hvp, d2p_nw_param_jacobian, d2p_nw_backward_full). */
size_t d2p_nw_second_workspace_bytes(int B, int max_L1, int max_L2);

/* Hessian-vector product of the value: hvp = (d^2 value / dscores^2) . tangent.
 * Replaces nw_hvp (/root/reference/src/nw/kernels.cuh:146-171) as sequenced by
 * soft_nw_hvp_cuda (/root/reference/src/nw/torch_cuda.cpp:442-503), which runs the
 * forward first.  The boundary cells' tangents are 0; the terminal beta is 1.
 *   tangent, hvp [B, max_L1, max_L2]                                              */
int d2p_nw_hvp(const float* scores, const float* tangent, const int* lengths, int B,
               int max_L1, int max_L2, float gap, float temperature, float* hvp,
               void* workspace, size_t workspace_bytes, void* stream);

/* Jacobian of the marginals with respect to gap (param_type 0: the boundary cells'
 * tangents are i and j) or temperature (1).  Replaces nw_param_grad
 * (/root/reference/src/nw/kernels.cuh:173-200) as sequenced by
 * soft_nw_param_jacobian_cuda (/root/reference/src/nw/torch_cuda.cpp:509-598); the
 * reference's dS/dtheta input is unused by its kernel and not computed here.
 *   jacobian [B, max_L1, max_L2]                                                  */
int d2p_nw_param_jacobian(const float* scores, int param_type, const int* lengths, int B,
                          int max_L1, int max_L2, float gap, float temperature,
                          float* jacobian, void* workspace, size_t workspace_bytes,
                          void* stream);

/* Backward of the marginals output for a cotangent grad_alignment:
 *   grad_scores = H . grad_alignment,
 *   grad_gap[b] = <grad_alignment[b], dP_b/dgap>, grad_T[b] = <grad_alignment[b], dP_b/dT>
 * (per element; soft_nw_backward_full_cuda, /root/reference/src/nw/torch_cuda.cpp:602-709,
 * returns their sums over the batch). */
int d2p_nw_backward_full(const float* scores, const float* grad_alignment, const int* lengths,
                         int B, int max_L1, int max_L2, float gap, float temperature,
                         float* grad_scores, float* grad_gap, float* grad_T, void* workspace,
                         size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Affine-gap soft Needleman-Wunsch (global alignment, three states)
 * M = s + LSE(M, I, D)[i-1,j-1], I = LSE(M + open, I + ext, D + open)[i-1,j],
 * D = LSE(M + open, I + open, D + ext)[i,j-1]; M[0,0] = 0, I[i,0] = open + (i-1) ext,
 * D[0,j] = open + (j-1) ext; value = LSE(M, I, D)[L1, L2]
 * (/root/reference/src/nw_affine/kernels_cpu.cpp:100-187).
 * ------------------------------------------------------------------------- */

/* Workspace bytes needed by d2p_nwa_forward_marginals (status words first). */
size_t d2p_nwa_workspace_bytes(int B, int max_L1, int max_L2);

/* Forward value and marginals in one call.
 * Replaces the pair nw_affine_forward + nw_affine_backward
 * (/root/reference/src/nw_affine/kernels.cuh:77-130) as sequenced by
 * soft_nw_affine_cuda_with_grads (/root/reference/src/nw_affine/torch_cuda.cpp:387-432);
 * the CPU kernels restated are /root/reference/src/nw_affine/kernels_cpu.cpp:100-347.
 *   scores    [B, max_L1, max_L2]  input
 *   value     [B]                  out: LSE of the terminal cell's three states
 *   marginals [B, max_L1, max_L2]  out: dvalue/dscores (zero in padding)
 *   grad_open, grad_ext [B]        out: dvalue/dgap_open, dvalue/dgap_ext (boundary
 *                                  chains I[i,0] and D[0,j] included)
 *   grad_T    [B]                  out: dvalue/dtemperature */
int d2p_nwa_forward_marginals(const float* scores, const int* lengths, int B, int max_L1,
                              int max_L2, float gap_open, float gap_ext, float temperature,
                              float* value, float* marginals, float* grad_open, float* grad_ext,
                              float* grad_T, void* workspace, size_t workspace_bytes,
                              void* stream);

/* Workspace bytes of the second-order entry points below (d2p_nwa_hvp,
 * d2p_nwa_param_jacobian, d2p_nwa_backward_full). */
size_t d2p_nwa_second_workspace_bytes(int B, int max_L1, int max_L2);

/* Hessian-vector product of the value: hvp = (d^2 value / dscores^2) . tangent.
 * Replaces nw_affine_hvp (/root/reference/src/nw_affine/kernels.cuh:132-159) as
 * sequenced by soft_nw_affine_hvp_cuda (/root/reference/src/nw_affine/torch_cuda.cpp:
 * 435-482), which runs the forward first.
 *   tangent, hvp [B, max_L1, max_L2]                                              */
int d2p_nwa_hvp(const float* scores, const float* tangent, const int* lengths, int B,
                int max_L1, int max_L2, float gap_open, float gap_ext, float temperature,
                float* hvp, void* workspace, size_t workspace_bytes, void* stream);

/* Jacobian of the marginals with respect to gap_open (param_type 0), gap_ext (1) or
 * temperature (2).  Replaces nw_affine_param_grad
 * (/root/reference/src/nw_affine/kernels.cuh:161-190) as sequenced by
 * soft_nw_affine_param_jacobian_cuda (/root/reference/src/nw_affine/torch_cuda.cpp:
 * 484-553); the reference's dS/dtheta input is unused by its kernel and not computed
 * here.
 *   jacobian [B, max_L1, max_L2]                                                  */
int d2p_nwa_param_jacobian(const float* scores, int param_type, const int* lengths, int B,
                           int max_L1, int max_L2, float gap_open, float gap_ext,
                           float temperature, float* jacobian, void* workspace,
                           size_t workspace_bytes, void* stream);

/* Backward of the marginals output for a cotangent grad_alignment:
 *   grad_scores = H . grad_alignment, grad_X[b] = <grad_alignment[b], dP_b/dX> for
 *   X in (open, ext, T) (per element; soft_nw_affine_backward_full_cuda,
 *   /root/reference/src/nw_affine/torch_cuda.cpp:555-665, returns their sums). */
int d2p_nwa_backward_full(const float* scores, const float* grad_alignment, const int* lengths,
                          int B, int max_L1, int max_L2, float gap_open, float gap_ext,
                          float temperature, float* grad_scores, float* grad_open,
                          float* grad_ext, float* grad_T, void* workspace,
                          size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Soft dynamic time warping (optional Sakoe-Chiba band)
 * ------------------------------------------------------------------------- */

/* Workspace bytes needed by d2p_dtw_forward_marginals (status words first), enough
 * for any bandwidth. */
size_t d2p_dtw_workspace_bytes(int B, int max_L1, int max_L2);

/* Workspace bytes needed by d2p_dtw_forward_marginals for one bandwidth: with a
 * Sakoe-Chiba band (bandwidth >= 0) the skewed alpha table keeps only each stripe's
 * band window, about (max_L2 + stripes * (2 * bandwidth + 160)) * 256 bytes per
 * element instead of stripes * (max_L2 + 63) * 256.  bandwidth < 0 gives
 * d2p_dtw_workspace_bytes.  No counterpart in the reference (its bindings allocate
 * full (L1+1) x (L2+1) tables, /root/reference/src/dtw/torch_cuda.cpp:166-169). */
size_t d2p_dtw_workspace_bytes_banded(int B, int max_L1, int max_L2, int bandwidth);

/* Squared-Euclidean costs + soft DTW: the forward value and marginals of soft DTW
 * over c[b,i,j] = max(|x_i|^2 + |y_j|^2 - 2 x_i . y_j, 0) (the dot products on the
 * matrix cores), formed from the features by d2p_pairwise_sqdist's kernel into the
 * marginals buffer, read there by the forward sweep and overwritten by the reverse
 * sweep (which reads only the alpha table): no [B, L1, L2] memory beyond the outputs.
 * No counterpart in the reference: its callers build the costs with
 * torch.cdist(x, y) ** 2 (/root/reference/docs/algorithms/dtw.md:52; the same
 * expansion at these sizes) and its sweeps read them
 * (/root/reference/src/dtw/kernels.cu:55-114).  The DP, outputs, lengths and band
 * rules are those of d2p_dtw_forward_marginals (same workspace,
 * d2p_dtw_workspace_bytes_banded).
 *   x [B, max_L1, D], y [B, max_L2, D]  inputs, 1 <= D <= 128
 *   value [B], marginals [B, max_L1, max_L2] (= dvalue/dcosts), grad_T [B] */
int d2p_dtw_sqeuclid_forward_marginals(const float* x, const float* y, const int* lengths, int B,
                                       int max_L1, int max_L2, int D, float temperature,
                                       int bandwidth, float* value, float* marginals,
                                       float* grad_T, void* workspace, size_t workspace_bytes,
                                       void* stream);

/* costs[b,i,j] = max(|x_i|^2 + |y_j|^2 - 2 x_i . y_j, 0), the costs of the entry point
 * above bit for bit, for callers that need the matrix itself (the op's marginal-path
 * backward).  Within (D + 4) u (|x_i| + |y_j|)^2 (u = 2^-24) of the exact squared
 * distance.  No counterpart in the reference (see above).
 *   x [B, L1, D], y [B, L2, D], costs [B, L1, L2]; 1 <= D <= 128 (any B, L1 and L2:
 *   the kernel strides over batch elements and tiles past the grid limits) */
int d2p_pairwise_sqdist(const float* x, const float* y, int B, int L1, int L2, int D,
                        float* costs, void* stream);

/* Gradients into the features through the costs above, from G = dL/dc [B, L1, L2]:
 *   grad_x[b,i] = 2 s_b (x_i sum_j G[b,i,j] - sum_j G[b,i,j] y_j)
 *   grad_y[b,j] = 2 s_b (y_j sum_i G[b,i,j] - sum_i G[b,i,j] x_i)
 * with s_b = scale[b] (scale may be null: s_b = 1), the products on the matrix cores.
 * No counterpart in the reference, whose callers leave this to torch's autograd of
 * torch.cdist(x, y) ** 2 (/root/reference/docs/algorithms/dtw.md:52).
 *   G [B, L1, L2], x [B, L1, D], y [B, L2, D], scale [B] or null
 *   grad_x [B, L1, D], grad_y [B, L2, D]; 1 <= D <= 128 */
int d2p_sqeuclid_feature_grad(const float* G, const float* x, const float* y,
                              const float* scale, int B, int L1, int L2, int D, float* grad_x,
                              float* grad_y, void* stream);

/* Forward value and alignment marginals in one call.
 * Replaces the pair dtw_forward + dtw_backward (/root/reference/src/dtw/kernels.cuh:95-129)
 * as sequenced by SoftDTWCUDAFunction::forward (/root/reference/src/dtw/torch_cuda.cpp:141-205).
 *   costs     [B, max_L1, max_L2]  input
 *   bandwidth                      Sakoe-Chiba half-width in cells, < 0 = no band
 *   value     [B]                  out: soft-DTW value alpha[L1, L2]
 *   marginals [B, max_L1, max_L2]  out: dvalue/dcosts (zero in padding and off-band)
 *   grad_T    [B]                  out: dvalue/dtemperature */
int d2p_dtw_forward_marginals(const float* costs, const int* lengths, int B, int max_L1,
                              int max_L2, float temperature, int bandwidth, float* value,
                              float* marginals, float* grad_T, void* workspace,
                              size_t workspace_bytes, void* stream);

/* Workspace bytes of the second-order DTW entry points below, enough for any
 * bandwidth. */
size_t d2p_dtw_second_workspace_bytes(int B, int max_L1, int max_L2);

/* The same for one bandwidth: banded primal and tangent tables as in
 * d2p_dtw_workspace_bytes_banded.  No counterpart in the reference. */
size_t d2p_dtw_second_workspace_bytes_banded(int B, int max_L1, int max_L2, int bandwidth);

/* Hessian-vector product of the soft-DTW value: hvp = (d^2 value / dcosts^2) . tangent.
 * Replaces dtw_hvp (/root/reference/src/dtw/kernels.cuh:131-151) as sequenced by
 * soft_dtw_hvp_cuda (/root/reference/src/dtw/torch_cuda.cpp:420-482). */
int d2p_dtw_hvp(const float* costs, const float* tangent, const int* lengths, int B, int max_L1,
                int max_L2, float temperature, int bandwidth, float* hvp, void* workspace,
                size_t workspace_bytes, void* stream);

/* Jacobian of the alignment marginals with respect to temperature.
 * Replaces dtw_param_grad (/root/reference/src/dtw/kernels.cuh:153-174) as sequenced by
 * soft_dtw_param_jacobian_cuda (/root/reference/src/dtw/torch_cuda.cpp:484-540). */
int d2p_dtw_param_jacobian(const float* costs, const int* lengths, int B, int max_L1,
                           int max_L2, float temperature, int bandwidth, float* jacobian,
                           void* workspace, size_t workspace_bytes, void* stream);

/* Backward of the marginals output for a cotangent grad_alignment:
 * grad_costs = H . grad_alignment and grad_T[b] = <grad_alignment[b], dP_b/dT> (per element;
 * soft_dtw_backward_full_cuda, /root/reference/src/dtw/torch_cuda.cpp:542-640, returns the
 * batch sum). */
int d2p_dtw_backward_full(const float* costs, const float* grad_alignment, const int* lengths,
                          int B, int max_L1, int max_L2, float temperature, int bandwidth,
                          float* grad_costs, float* grad_T, void* workspace,
                          size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Shared helpers
 * ------------------------------------------------------------------------- */

/* dst[b, k] = g[b] * src[b, k] for k < per_batch (src and dst may alias).
 * Replaces the ATen expression `grad_score.view({B,1,1}) * posteriors` of the
 * reference autograd backward (/root/reference/src/sw/torch_cuda.cpp:314,
 * src/sw_affine/torch_cuda.cpp, src/dtw/torch_cuda.cpp). */
int d2p_scale_by_batch(const float* src, const float* g, float* dst, int B,
                       long long per_batch, void* stream);

/* The same with g[b] read at g + b * g_stride (g_stride >= 0; 0: one factor for every
 * row, as in the expanded gradient of `value.sum()`), so that a caller holding a
 * strided or broadcast gradient needs no copy of it.  Replaces the same ATen
 * expression, which broadcasts a strided grad_score
 * (/root/reference/src/sw/torch_cuda.cpp:314). */
int d2p_scale_by_batch_strided(const float* src, const float* g, long long g_stride,
                               float* dst, int B, long long per_batch, void* stream);

/* dst = g[b] * src over [B, max_L1, max_L2] tensors that are zero outside each
 * element's lengths (int32 [B, 2] on the device; null: full lengths, the strided form
 * above): cells outside (L1, L2) are written as g[b] * 0 without being read, the same
 * bits as the full product of a zero there.  For a ragged batch this reads only the
 * valid cells.  Replaces the same ATen expression of the reference's autograd backward
 * (/root/reference/src/sw_affine/torch_cuda.cpp, src/sw/torch_cuda.cpp:314), whose
 * posteriors hold zeros outside the lengths. */
int d2p_scale_by_batch_lengths(const float* src, const float* g, long long g_stride,
                               const int* lengths, float* dst, int B, int max_L1, int max_L2,
                               void* stream);

#ifdef __cplusplus
}
#endif

#endif /* D2P_AMD_H */
