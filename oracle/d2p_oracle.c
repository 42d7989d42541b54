/*
 * d2p_oracle.c -- CPU restatement of the reference soft-DP kernels (C99).
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for the HIP product path.
 * Nothing under d2p_amd/ links, loads or calls this code.
 *
 * Each function below restates the reference CPU kernel cited in its comment,
 * keeping the reference's arithmetic order (anti-diagonal traversal, Kahan
 * sums, NINF/PINF = -/+1e30 sentinels, safe_exp clamp at +-88, log-posterior
 * clamp <= 0, the skip rules of the backward sweeps).  The traversal order is
 * kept on purpose: the backward sweeps accumulate into predecessors, so the
 * float rounding of beta depends on the order in which successors are
 * visited.  Build with -ffp-contract=off (see oracle/Makefile) so no FMA
 * contraction changes the rounding.
 *
 * Pinning (no function here is unpinned): every entry point is checked
 *   - bit for bit against the reference's own CPU kernels compiled from
 *     /root/reference/src/{sw,sw_affine,dtw,nw}/kernels_cpu.cpp by oracle/Makefile
 *     (tests/test_oracle_reference.py), including low temperature, the exp clamp,
 *     large near-tied costs, ragged/empty lengths and DTW bands;
 *   - bit for bit against golden fixtures written from that build
 *     (tests/golden/, tests/test_golden.py), which travel where the reference
 *     does not;
 *   - against mathematics (tests/test_oracle_math.py): 1x1 / 1xN closed forms,
 *     path enumeration, a float64 autograd restatement of the recurrences for
 *     values, marginals, parameter gradients, HVPs and parameter Jacobians,
 *     hard-max limits, HVP symmetry and linearity, thread-count invariance.
 * The *_sums64 extensions (double sums of the reference's per-cell parameter
 * gradient terms) are pinned by the float64 restatement.
 */
#include "d2p_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

#define NINF (-1e30f)
#define PINF (1e30f)

/* ---- scalar primitives: /root/reference/src/common/numerics.h:23-105 ---- */

static inline float xexp(float x) {            /* safe_exp, numerics.h:28-32 */
    if (x < -88.0f) return 0.0f;
    if (x > 88.0f) x = 88.0f;
    return expf(x);
}

typedef struct { float s, c; } kahan;            /* KahanSum, numerics.h:39-57 */
static inline void kadd(kahan* k, float v) {
    float y = v - k->c;
    float t = k->s + y;
    k->c = (t - k->s) - y;
    k->s = t;
}

static inline float fmax2(float a, float b) { return a < b ? b : a; }
static inline float fmin2(float a, float b) { return b < a ? b : a; }
static inline float fmax4(float a, float b, float c, float d) {
    return fmax2(fmax2(fmax2(a, b), c), d);
}

static float lse2(float a, float b, float T) {   /* numerics.h:63-70 */
    float m = fmax2(a, b);
    if (m <= NINF) return NINF;
    kahan k = {0.0f, 0.0f};
    kadd(&k, xexp((a - m) / T));
    kadd(&k, xexp((b - m) / T));
    return m + T * logf(k.s);
}

static float lse3(float a, float b, float c, float T) {   /* numerics.h:72-81 */
    float m = fmax2(fmax2(a, b), c);
    if (m <= NINF) return NINF;
    kahan k = {0.0f, 0.0f};
    kadd(&k, xexp((a - m) / T));
    kadd(&k, xexp((b - m) / T));
    kadd(&k, xexp((c - m) / T));
    return m + T * logf(k.s);
}

static float lse4(float a, float b, float c, float d, float T) { /* numerics.h:83-92 */
    float m = fmax4(a, b, c, d);
    if (m <= NINF) return NINF;
    kahan k = {0.0f, 0.0f};
    kadd(&k, xexp((a - m) / T));
    kadd(&k, xexp((b - m) / T));
    kadd(&k, xexp((c - m) / T));
    kadd(&k, xexp((d - m) / T));
    return m + T * logf(k.s);
}

static float softmin3(float a, float b, float c, float T) {   /* numerics.h:98-105 */
    float m = fmin2(fmin2(a, b), c);
    if (m >= PINF) return PINF;
    kahan k = {0.0f, 0.0f};
    kadd(&k, xexp((m - a) / T));
    kadd(&k, xexp((m - b) / T));
    kadd(&k, xexp((m - c) / T));
    return m - T * logf(k.s);
}

/* Normalised softmax weights of n log-domain values; NINF entries get weight
 * 0.  Kahan-summed normaliser.  sw/kernels_cpu.cpp:43-64,
 * sw_affine/kernels_cpu.cpp:56-88. */
static void softmax_w(const float* v, float* w, int n, float T) {
    float m = v[0];
    for (int q = 1; q < n; ++q) m = fmax2(m, v[q]);
    if (m <= NINF) {
        for (int q = 0; q < n; ++q) w[q] = 0.0f;
        return;
    }
    kahan k = {0.0f, 0.0f};
    for (int q = 0; q < n; ++q) {
        if (v[q] > NINF) { w[q] = xexp((v[q] - m) / T); kadd(&k, w[q]); }
        else w[q] = 0.0f;
    }
    if (k.s > 0) for (int q = 0; q < n; ++q) w[q] /= k.s;
}

/* Plain-sum softmax of four values used by the SW parameter-gradient sweeps,
 * sw/kernels_cpu.cpp:559-575 and :649-664. */
static int softmax4_plain(const float* v, float* w, float T) {
    float m = fmax4(v[0], v[1], v[2], v[3]);
    if (m <= NINF) return 0;
    for (int q = 0; q < 4; ++q) w[q] = xexp((v[q] - m) / T);
    float sum = w[0] + w[1] + w[2] + w[3];
    float inv = (sum > 1e-20f) ? 1.0f / sum : 0.0f;
    for (int q = 0; q < 4; ++q) w[q] *= inv;
    return 1;
}

static inline float clamp_lp(float x) { return x < 0.0f ? x : 0.0f; }

/* Sakoe-Chiba band test in float, dtw/kernels_cpu.cpp:24-29. */
static inline int in_band(int i, int j, int L1, int L2, int64_t bw) {
    if (bw < 0) return 1;
    if (L1 == 0 || L2 == 0) return 1;
    float ej = (float)((int64_t)i * L2) / L1;
    return fabsf((float)j - ej) <= (float)bw;
}

/* Softmin weights with a plain sum, dtw/kernels_cpu.cpp:32-52. */
static void softmin3_w(float a, float b, float c, float T, float* wa, float* wb, float* wc) {
    float m = fmin2(fmin2(a, b), c);
    if (m >= PINF) { *wa = *wb = *wc = 0.0f; return; }
    float ea = (a < PINF) ? xexp((m - a) / T) : 0.0f;
    float eb = (b < PINF) ? xexp((m - b) / T) : 0.0f;
    float ec = (c < PINF) ? xexp((m - c) / T) : 0.0f;
    float tot = ea + eb + ec;
    if (tot > 0.0f) { *wa = ea / tot; *wb = eb / tot; *wc = ec / tot; }
    else { *wa = *wb = *wc = 0.0f; }
}

/* Anti-diagonal traversal shared by every sweep: k = i + j from 2 to L1+L2
 * (forward) or back (reverse), i ascending inside a diagonal. */
#define FOR_DIAG_FWD(L1, L2, i, j)                                         \
    for (int k_ = 2; k_ <= (L1) + (L2); ++k_)                              \
        for (int i = (k_ - (L2) > 1 ? k_ - (L2) : 1),                      \
                 e_ = ((L1) < k_ - 1 ? (L1) : k_ - 1); i <= e_; ++i)       \
            for (int j = k_ - i, once_ = 1; once_; once_ = 0)
#define FOR_DIAG_REV(L1, L2, i, j)                                         \
    for (int k_ = (L1) + (L2); k_ >= 2; --k_)                              \
        for (int i = (k_ - (L2) > 1 ? k_ - (L2) : 1),                      \
                 e_ = ((L1) < k_ - 1 ? (L1) : k_ - 1); i <= e_; ++i)       \
            for (int j = k_ - i, once_ = 1; once_; once_ = 0)

#define AIDX(i, j) ((size_t)(i) * acols + (size_t)(j))
#define SIDX(i, j) ((size_t)((i) - 1) * scols + (size_t)((j) - 1))

int oracle_max_threads(void) { return omp_get_max_threads(); }

/* =========================================================================
 * Linear-gap soft Smith-Waterman
 * ========================================================================= */

/* sw/kernels_cpu.cpp:70-148 */
void oracle_sw_forward(const float* scores, float* alpha, float* partition,
                       const int* lengths, int B, int maxL1, int maxL2, float gap, float T) {
    const size_t astride = (size_t)(maxL1 + 1) * (maxL2 + 1);
    const size_t sstride = (size_t)maxL1 * maxL2;
    const size_t acols = (size_t)maxL2 + 1, scols = (size_t)maxL2;
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < B; ++b) {
        const float* s = scores + b * sstride;
        float* a = alpha + b * astride;
        int L1 = lengths[2 * b], L2 = lengths[2 * b + 1];
        for (size_t q = 0; q < astride; ++q) a[q] = NINF;
        a[0] = 0.0f;
        FOR_DIAG_FWD(L1, L2, i, j) {
            float sc = s[SIDX(i, j)];
            float vd = (i > 1 && j > 1) ? a[AIDX(i - 1, j - 1)] + sc : NINF;
            float vu = (i > 1) ? a[AIDX(i - 1, j)] + gap : NINF;
            float vl = (j > 1) ? a[AIDX(i, j - 1)] + gap : NINF;
            a[AIDX(i, j)] = lse4(vd, vu, vl, sc, T);
        }
        float m = NINF;
        for (int i = 0; i <= L1; ++i)
            for (int j = 0; j <= L2; ++j) m = fmax2(m, a[AIDX(i, j)]);
        kahan k = {0.0f, 0.0f};
        for (int i = 0; i <= L1; ++i)
            for (int j = 0; j <= L2; ++j)
                if (a[AIDX(i, j)] > NINF) kadd(&k, xexp((a[AIDX(i, j)] - m) / T));
        partition[b] = m + T * logf(k.s);
    }
}

/* sw/kernels_cpu.cpp:154-271 */
static void sw_backward_impl(const float* alpha, const float* scores, const float* partition,
                             float* beta, float* posteriors, float* grad_gap, float* grad_T,
                             double* sums64, const int* lengths, int B, int maxL1, int maxL2,
                             float gap, float T) {
    const size_t astride = (size_t)(maxL1 + 1) * (maxL2 + 1);
    const size_t sstride = (size_t)maxL1 * maxL2;
    const size_t acols = (size_t)maxL2 + 1, scols = (size_t)maxL2;
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < B; ++b) {
        const float* a = alpha + b * astride;
        const float* s = scores + b * sstride;
        float* be = beta + b * astride;
        float* post = posteriors + b * sstride;
        float S = partition[b];
        int L1 = lengths[2 * b], L2 = lengths[2 * b + 1];
        for (size_t q = 0; q < sstride; ++q) post[q] = 0.0f;
        for (size_t q = 0; q < astride; ++q) be[q] = NINF;
        for (int i = 0; i <= L1; ++i)
            for (int j = 0; j <= L2; ++j)
                be[AIDX(i, j)] = xexp(clamp_lp((a[AIDX(i, j)] - S) / T));
        float gsum = 0.0f;
        double gsum_d = 0.0;
        FOR_DIAG_REV(L1, L2, i, j) {
            float sc = s[SIDX(i, j)];
            float bij = be[AIDX(i, j)];
            if (isinf(bij) || isnan(bij) || bij == 0.0f) continue;
            float v[4], w[4];
            v[0] = (i > 1 && j > 1) ? a[AIDX(i - 1, j - 1)] + sc : NINF;
            v[1] = (i > 1) ? a[AIDX(i - 1, j)] + gap : NINF;
            v[2] = (j > 1) ? a[AIDX(i, j - 1)] + gap : NINF;
            v[3] = sc;
            softmax_w(v, w, 4, T);
            post[SIDX(i, j)] += bij * (w[0] + w[3]);
            if (i > 1 && j > 1 && w[0] > 0.0f) be[AIDX(i - 1, j - 1)] += bij * w[0];
            if (i > 1 && w[1] > 0.0f) {
                be[AIDX(i - 1, j)] += bij * w[1];
                gsum += bij * w[1];
                gsum_d += (double)(bij * w[1]);
            }
            if (j > 1 && w[2] > 0.0f) {
                be[AIDX(i, j - 1)] += bij * w[2];
                gsum += bij * w[2];
                gsum_d += (double)(bij * w[2]);
            }
        }
        kahan k = {0.0f, 0.0f};
        for (size_t q = 0; q < sstride; ++q) kadd(&k, post[q] * s[q]);
        float expected = k.s + gsum * gap;
        grad_gap[b] = gsum;
        grad_T[b] = (S - expected) / T;
        if (sums64) {
            double e = 0.0;
            for (size_t q = 0; q < sstride; ++q) e += (double)post[q] * s[q];
            sums64[2 * b] = gsum_d;
            sums64[2 * b + 1] = ((double)S - (e + gsum_d * gap)) / T;
        }
    }
}

void oracle_sw_backward(const float* alpha, const float* scores, const float* partition,
                        float* beta, float* posteriors, float* grad_gap, float* grad_T,
                        const int* lengths, int B, int maxL1, int maxL2, float gap, float T) {
    sw_backward_impl(alpha, scores, partition, beta, posteriors, grad_gap, grad_T, NULL, lengths,
                     B, maxL1, maxL2, gap, T);
}

/* The same reverse sweep; additionally sums every per-cell term of grad_gap and
 * grad_T in double: sums64[2b] = dS/dgap, sums64[2b+1] = dS/dT.  The fp32 outputs
 * are the reference's (sequential fp32 sums, which drift from the exact sum on
 * large tables); the double sums isolate that drift for the parity tests. */
void oracle_sw_backward_sums64(const float* alpha, const float* scores, const float* partition,
                               float* beta, float* posteriors, double* sums64,
                               const int* lengths, int B, int maxL1, int maxL2, float gap,
                               float T) {
    float* gg = (float*)malloc(sizeof(float) * (B > 0 ? B : 1));
    float* gt = (float*)malloc(sizeof(float) * (B > 0 ? B : 1));
    sw_backward_impl(alpha, scores, partition, beta, posteriors, gg, gt, sums64, lengths, B,
                     maxL1, maxL2, gap, T);
    free(gg);
    free(gt);
}

/* sw/kernels_cpu.cpp:279-477 */
void oracle_sw_hvp(const float* alpha, const float* scores, const float* partition,
                   const float* V, float* d_alpha, float* d_partition, float* beta,
                   float* d_beta, float* H, const int* lengths, int B, int maxL1, int maxL2,
                   float gap, float T) {
    const size_t astride = (size_t)(maxL1 + 1) * (maxL2 + 1);
    const size_t sstride = (size_t)maxL1 * maxL2;
    const size_t acols = (size_t)maxL2 + 1, scols = (size_t)maxL2;
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < B; ++b) {
        const float* a = alpha + b * astride;
        const float* s = scores + b * sstride;
        const float* vv = V + b * sstride;
        float* da = d_alpha + b * astride;
        float* be = beta + b * astride;
        float* dbe = d_beta + b * astride;
        float* h = H + b * sstride;
        float S = partition[b];
        int L1 = lengths[2 * b], L2 = lengths[2 * b + 1];
        for (size_t q = 0; q < astride; ++q) { da[q] = 0.0f; be[q] = 0.0f; dbe[q] = 0.0f; }
        for (size_t q = 0; q < sstride; ++q) h[q] = 0.0f;
        da[0] = 0.0f;
        /* tangent forward */
        FOR_DIAG_FWD(L1, L2, i, j) {
            float sc = s[SIDX(i, j)], vij = vv[SIDX(i, j)];
            float v[4], w[4];
            v[0] = (i > 1 && j > 1) ? a[AIDX(i - 1, j - 1)] + sc : NINF;
            v[1] = (i > 1) ? a[AIDX(i - 1, j)] + gap : NINF;
            v[2] = (j > 1) ? a[AIDX(i, j - 1)] + gap : NINF;
            v[3] = sc;
            softmax_w(v, w, 4, T);
            float dvd = (i > 1 && j > 1) ? da[AIDX(i - 1, j - 1)] + vij : 0.0f;
            float dvu = (i > 1) ? da[AIDX(i - 1, j)] : 0.0f;
            float dvl = (j > 1) ? da[AIDX(i, j - 1)] : 0.0f;
            da[AIDX(i, j)] = w[0] * dvd + w[1] * dvu + w[2] * dvl + w[3] * vij;
        }
        kahan k = {0.0f, 0.0f};
        for (int i = 0; i <= L1; ++i)
            for (int j = 0; j <= L2; ++j)
                kadd(&k, xexp(clamp_lp((a[AIDX(i, j)] - S) / T)) * da[AIDX(i, j)]);
        float dS = k.s;
        d_partition[b] = dS;
        for (int i = 0; i <= L1; ++i)
            for (int j = 0; j <= L2; ++j)
                be[AIDX(i, j)] = xexp(clamp_lp((a[AIDX(i, j)] - S) / T));
        for (int i = 0; i <= L1; ++i)
            for (int j = 0; j <= L2; ++j)
                dbe[AIDX(i, j)] = be[AIDX(i, j)] * (da[AIDX(i, j)] - dS) / T;
        /* tangent reverse */
        FOR_DIAG_REV(L1, L2, i, j) {
            float sc = s[SIDX(i, j)], vij = vv[SIDX(i, j)];
            float bij = be[AIDX(i, j)], dbij = dbe[AIDX(i, j)];
            if (isinf(bij) || isnan(bij) || bij == 0.0f) continue;
            float v[4], w[4];
            v[0] = (i > 1 && j > 1) ? a[AIDX(i - 1, j - 1)] + sc : NINF;
            v[1] = (i > 1) ? a[AIDX(i - 1, j)] + gap : NINF;
            v[2] = (j > 1) ? a[AIDX(i, j - 1)] + gap : NINF;
            v[3] = sc;
            softmax_w(v, w, 4, T);
            float dvd = (i > 1 && j > 1) ? da[AIDX(i - 1, j - 1)] + vij : 0.0f;
            float dvu = (i > 1) ? da[AIDX(i - 1, j)] : 0.0f;
            float dvl = (j > 1) ? da[AIDX(i, j - 1)] : 0.0f;
            float dvs = vij;
            float mean = w[0] * dvd + w[1] * dvu + w[2] * dvl + w[3] * dvs;
            float dwd = w[0] * (dvd - mean) / T;
            float dwu = w[1] * (dvu - mean) / T;
            float dwl = w[2] * (dvl - mean) / T;
            float dws = w[3] * (dvs - mean) / T;
            h[SIDX(i, j)] += dbij * (w[0] + w[3]) + bij * (dwd + dws);
            if (i > 1 && j > 1 && w[0] > 0.0f) be[AIDX(i - 1, j - 1)] += bij * w[0];
            if (i > 1 && w[1] > 0.0f) be[AIDX(i - 1, j)] += bij * w[1];
            if (j > 1 && w[2] > 0.0f) be[AIDX(i, j - 1)] += bij * w[2];
            if (i > 1 && j > 1 && w[0] > 0.0f) dbe[AIDX(i - 1, j - 1)] += dbij * w[0] + bij * dwd;
            if (i > 1 && w[1] > 0.0f) dbe[AIDX(i - 1, j)] += dbij * w[1] + bij * dwu;
            if (j > 1 && w[2] > 0.0f) dbe[AIDX(i, j - 1)] += dbij * w[2] + bij * dwl;
        }
    }
}

/* sw/kernels_cpu.cpp:491-710  (param_type 0 = gap, 1 = temperature) */
void oracle_sw_param_grad(const float* alpha, const float* scores, const float* partition,
                          const float* dS_dtheta, float* U, float* beta, float* W,
                          float* dP, const int* lengths, int B, int maxL1, int maxL2,
                          float gap, float T, int ptype) {
    const size_t astride = (size_t)(maxL1 + 1) * (maxL2 + 1);
    const size_t sstride = (size_t)maxL1 * maxL2;
    const size_t acols = (size_t)maxL2 + 1, scols = (size_t)maxL2;
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < B; ++b) {
        const float* a = alpha + b * astride;
        const float* s = scores + b * sstride;
        float* u = U + b * astride;
        float* be = beta + b * astride;
        float* ww = W + b * astride;
        float* dp = dP + b * sstride;
        float S = partition[b], dSdt = dS_dtheta[b];
        int L1 = lengths[2 * b], L2 = lengths[2 * b + 1];
        for (size_t q = 0; q < astride; ++q) { u[q] = 0.0f; be[q] = 0.0f; ww[q] = 0.0f; }
        for (size_t q = 0; q < sstride; ++q) dp[q] = 0.0f;
        u[0] = 0.0f;
        FOR_DIAG_FWD(L1, L2, i, j) {
            float sc = s[SIDX(i, j)];
            float v[4], w[4];
            v[0] = (i > 1 && j > 1) ? a[AIDX(i - 1, j - 1)] + sc : NINF;
            v[1] = (i > 1) ? a[AIDX(i - 1, j)] + gap : NINF;
            v[2] = (j > 1) ? a[AIDX(i, j - 1)] + gap : NINF;
            v[3] = sc;
            if (!softmax4_plain(v, w, T)) { u[AIDX(i, j)] = 0.0f; continue; }
            float dud = (i > 1 && j > 1) ? u[AIDX(i - 1, j - 1)] : 0.0f;
            float duu = (i > 1) ? u[AIDX(i - 1, j)] : 0.0f;
            float dul = (j > 1) ? u[AIDX(i, j - 1)] : 0.0f;
            float dus = 0.0f;
            if (ptype == 0) { duu += 1.0f; dul += 1.0f; }
            float uv = w[0] * dud + w[1] * duu + w[2] * dul + w[3] * dus;
            if (ptype == 1) {
                float mean_v = w[0] * v[0] + w[1] * v[1] + w[2] * v[2] + w[3] * v[3];
                uv += (a[AIDX(i, j)] - mean_v) / T;
            }
            u[AIDX(i, j)] = uv;
        }
        for (int i = 0; i <= L1; ++i)
            for (int j = 0; j <= L2; ++j)
                be[AIDX(i, j)] = xexp(clamp_lp((a[AIDX(i, j)] - S) / T));
        FOR_DIAG_REV(L1, L2, i, j) {
            size_t id = AIDX(i, j);
            float bc = be[id];
            float binit = 0.0f;
            if (a[id] > NINF) binit = xexp(clamp_lp((a[id] - S) / T));
            float dwi = binit * (u[id] - dSdt) / T;
            if (ptype == 1 && a[id] > NINF) dwi -= binit * (a[id] - S) / (T * T);
            float wc = ww[id] + dwi;
            if (bc <= 1e-20f && fabsf(wc) <= 1e-20f) continue;
            float sc = s[SIDX(i, j)];
            float v[4], w[4];
            v[0] = (i > 1 && j > 1) ? a[AIDX(i - 1, j - 1)] + sc : NINF;
            v[1] = (i > 1) ? a[AIDX(i - 1, j)] + gap : NINF;
            v[2] = (j > 1) ? a[AIDX(i, j - 1)] + gap : NINF;
            v[3] = sc;
            if (!softmax4_plain(v, w, T)) continue;
            float dud = (i > 1 && j > 1) ? u[AIDX(i - 1, j - 1)] : 0.0f;
            float duu = (i > 1) ? u[AIDX(i - 1, j)] : 0.0f;
            float dul = (j > 1) ? u[AIDX(i, j - 1)] : 0.0f;
            float dus = 0.0f;
            if (ptype == 0) { duu += 1.0f; dul += 1.0f; }
            float mean_du = w[0] * dud + w[1] * duu + w[2] * dul + w[3] * dus;
            float dwd = w[0] * (dud - mean_du) / T;
            float dwu = w[1] * (duu - mean_du) / T;
            float dwl = w[2] * (dul - mean_du) / T;
            float dws = w[3] * (dus - mean_du) / T;
            if (ptype == 1) {
                float mean_v = w[0] * v[0] + w[1] * v[1] + w[2] * v[2] + w[3] * v[3];
                float it2 = 1.0f / (T * T);
                dwd += w[0] * (mean_v - v[0]) * it2;
                dwu += w[1] * (mean_v - v[1]) * it2;
                dwl += w[2] * (mean_v - v[2]) * it2;
                dws += w[3] * (mean_v - v[3]) * it2;
            }
            dp[SIDX(i, j)] += wc * (w[0] + w[3]) + bc * (dwd + dws);
            if (v[0] > NINF) { be[AIDX(i - 1, j - 1)] += bc * w[0]; ww[AIDX(i - 1, j - 1)] += wc * w[0] + bc * dwd; }
            if (v[1] > NINF) { be[AIDX(i - 1, j)] += bc * w[1]; ww[AIDX(i - 1, j)] += wc * w[1] + bc * dwu; }
            if (v[2] > NINF) { be[AIDX(i, j - 1)] += bc * w[2]; ww[AIDX(i, j - 1)] += wc * w[2] + bc * dwl; }
        }
    }
}

/* =========================================================================
 * Affine-gap soft Smith-Waterman: planes M=0, I=1, D=2 of size (L1+1)(L2+1)
 * ========================================================================= */

#define PM(idx) (0 * cstride + (idx))
#define PI(idx) (1 * cstride + (idx))
#define PD(idx) (2 * cstride + (idx))

static inline float posterior_weight(float a, float S, float T) {
    /* clamped_posterior_weight, sw_affine/kernels_cpu.cpp:47-52 */
    if (a <= NINF) return 0.0f;
    return xexp(clamp_lp((a - S) / T));
}

/* sw_affine/kernels_cpu.cpp:94-195 */
void oracle_swa_forward(const float* scores, float* alpha, float* partition,
                        const int* lengths, int B, int maxL1, int maxL2,
                        float go, float ge, float T) {
    const size_t cstride = (size_t)(maxL1 + 1) * (maxL2 + 1);
    const size_t astride = 3 * cstride;
    const size_t sstride = (size_t)maxL1 * maxL2;
    const size_t acols = (size_t)maxL2 + 1, scols = (size_t)maxL2;
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < B; ++b) {
        const float* s = scores + b * sstride;
        float* a = alpha + b * astride;
        int L1 = lengths[2 * b], L2 = lengths[2 * b + 1];
        for (size_t q = 0; q < astride; ++q) a[q] = NINF;
        a[PM(0)] = 0.0f;
        FOR_DIAG_FWD(L1, L2, i, j) {
            size_t c = AIDX(i, j), cd = AIDX(i - 1, j - 1), cu = AIDX(i - 1, j), cl = AIDX(i, j - 1);
            float sc = s[SIDX(i, j)];
            int dg = (i > 1 && j > 1);
            float mM = dg ? a[PM(cd)] + sc : NINF;
            float mI = dg ? a[PI(cd)] + sc : NINF;
            float mD = dg ? a[PD(cd)] + sc : NINF;
            a[PM(c)] = lse4(mM, mI, mD, sc, T);
            float iM = (i > 1) ? a[PM(cu)] + go : NINF;
            float iI = (i > 1) ? a[PI(cu)] + ge : NINF;
            a[PI(c)] = lse2(iM, iI, T);
            float dM = (j > 1) ? a[PM(cl)] + go : NINF;
            float dD = (j > 1) ? a[PD(cl)] + ge : NINF;
            a[PD(c)] = lse2(dM, dD, T);
        }
        float m = NINF;
        for (int i = 0; i <= L1; ++i)
            for (int j = 0; j <= L2; ++j)
                for (int st = 0; st < 3; ++st) m = fmax2(m, a[st * cstride + AIDX(i, j)]);
        kahan k = {0.0f, 0.0f};
        for (int i = 0; i <= L1; ++i)
            for (int j = 0; j <= L2; ++j)
                for (int st = 0; st < 3; ++st) {
                    float val = a[st * cstride + AIDX(i, j)];
                    if (val > NINF) kadd(&k, xexp((val - m) / T));
                }
        partition[b] = m + T * logf(k.s);
    }
}

/* sw_affine/kernels_cpu.cpp:201-356 */
static void swa_backward_impl(const float* alpha, const float* scores, const float* partition,
                              float* beta, float* posteriors, float* grad_open, float* grad_ext,
                              float* grad_T, double* sums64, const int* lengths, int B,
                              int maxL1, int maxL2, float go, float ge, float T) {
    const size_t cstride = (size_t)(maxL1 + 1) * (maxL2 + 1);
    const size_t astride = 3 * cstride;
    const size_t sstride = (size_t)maxL1 * maxL2;
    const size_t acols = (size_t)maxL2 + 1, scols = (size_t)maxL2;
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < B; ++b) {
        const float* a = alpha + b * astride;
        const float* s = scores + b * sstride;
        float* be = beta + b * astride;
        float* post = posteriors + b * sstride;
        float S = partition[b];
        int L1 = lengths[2 * b], L2 = lengths[2 * b + 1];
        for (size_t q = 0; q < sstride; ++q) post[q] = 0.0f;
        for (size_t q = 0; q < astride; ++q) be[q] = 0.0f;
        for (int i = 0; i <= L1; ++i)
            for (int j = 0; j <= L2; ++j)
                for (int st = 0; st < 3; ++st) {
                    size_t id = st * cstride + AIDX(i, j);
                    be[id] = xexp(clamp_lp((a[id] - S) / T));
                }
        float gopen = 0.0f, gext = 0.0f;
        double gopen_d = 0.0, gext_d = 0.0;
        FOR_DIAG_REV(L1, L2, i, j) {
            size_t c = AIDX(i, j), cd = AIDX(i - 1, j - 1), cu = AIDX(i - 1, j), cl = AIDX(i, j - 1);
            float sc = s[SIDX(i, j)];
            float bM = be[PM(c)];
            if (!isinf(bM) && !isnan(bM) && bM != 0.0f) {
                int dg = (i > 1 && j > 1);
                float v[4], w[4];
                v[0] = dg ? a[PM(cd)] + sc : NINF;
                v[1] = dg ? a[PI(cd)] + sc : NINF;
                v[2] = dg ? a[PD(cd)] + sc : NINF;
                v[3] = sc;
                softmax_w(v, w, 4, T);
                post[SIDX(i, j)] += bM * (w[0] + w[1] + w[2] + w[3]);
                if (dg) {
                    if (w[0] > 0.0f) be[PM(cd)] += bM * w[0];
                    if (w[1] > 0.0f) be[PI(cd)] += bM * w[1];
                    if (w[2] > 0.0f) be[PD(cd)] += bM * w[2];
                }
            }
            float bI = be[PI(c)];
            if (!isinf(bI) && !isnan(bI) && bI != 0.0f) {
                float v[2], w[2];
                v[0] = (i > 1) ? a[PM(cu)] + go : NINF;
                v[1] = (i > 1) ? a[PI(cu)] + ge : NINF;
                softmax_w(v, w, 2, T);
                if (i > 1) {
                    if (w[0] > 0.0f) {
                        be[PM(cu)] += bI * w[0];
                        gopen += bI * w[0];
                        gopen_d += (double)(bI * w[0]);
                    }
                    if (w[1] > 0.0f) {
                        be[PI(cu)] += bI * w[1];
                        gext += bI * w[1];
                        gext_d += (double)(bI * w[1]);
                    }
                }
            }
            float bD = be[PD(c)];
            if (!isinf(bD) && !isnan(bD) && bD != 0.0f) {
                float v[2], w[2];
                v[0] = (j > 1) ? a[PM(cl)] + go : NINF;
                v[1] = (j > 1) ? a[PD(cl)] + ge : NINF;
                softmax_w(v, w, 2, T);
                if (j > 1) {
                    if (w[0] > 0.0f) {
                        be[PM(cl)] += bD * w[0];
                        gopen += bD * w[0];
                        gopen_d += (double)(bD * w[0]);
                    }
                    if (w[1] > 0.0f) {
                        be[PD(cl)] += bD * w[1];
                        gext += bD * w[1];
                        gext_d += (double)(bD * w[1]);
                    }
                }
            }
        }
        kahan k = {0.0f, 0.0f};
        for (size_t q = 0; q < sstride; ++q) kadd(&k, post[q] * s[q]);
        float gapcost = gopen * go + gext * ge;
        float expected = k.s + gapcost;
        grad_open[b] = gopen;
        grad_ext[b] = gext;
        grad_T[b] = (S - expected) / T;
        if (sums64) {
            double e = 0.0;
            for (size_t q = 0; q < sstride; ++q) e += (double)post[q] * s[q];
            sums64[3 * b] = gopen_d;
            sums64[3 * b + 1] = gext_d;
            sums64[3 * b + 2] = ((double)S - (e + gopen_d * go + gext_d * ge)) / T;
        }
    }
}

void oracle_swa_backward(const float* alpha, const float* scores, const float* partition,
                         float* beta, float* posteriors, float* grad_open, float* grad_ext,
                         float* grad_T, const int* lengths, int B, int maxL1, int maxL2,
                         float go, float ge, float T) {
    swa_backward_impl(alpha, scores, partition, beta, posteriors, grad_open, grad_ext, grad_T,
                      NULL, lengths, B, maxL1, maxL2, go, ge, T);
}

/* The same reverse sweep with the parameter sums also taken in double:
 * sums64[3b..3b+2] = dS/dopen, dS/dext, dS/dT (see oracle_sw_backward_sums64). */
void oracle_swa_backward_sums64(const float* alpha, const float* scores, const float* partition,
                                float* beta, float* posteriors, double* sums64,
                                const int* lengths, int B, int maxL1, int maxL2, float go,
                                float ge, float T) {
    const size_t n = sizeof(float) * (B > 0 ? B : 1);
    float *g0 = (float*)malloc(n), *g1 = (float*)malloc(n), *g2 = (float*)malloc(n);
    swa_backward_impl(alpha, scores, partition, beta, posteriors, g0, g1, g2, sums64, lengths,
                      B, maxL1, maxL2, go, ge, T);
    free(g0);
    free(g1);
    free(g2);
}



/* sw_affine/kernels_cpu.cpp:362-631 */
void oracle_swa_hvp(const float* alpha, const float* scores, const float* partition,
                    const float* V, float* d_alpha, float* d_partition, float* d_beta,
                    float* H, const int* lengths, int B, int maxL1, int maxL2,
                    float go, float ge, float T) {
    const size_t cstride = (size_t)(maxL1 + 1) * (maxL2 + 1);
    const size_t astride = 3 * cstride;
    const size_t sstride = (size_t)maxL1 * maxL2;
    const size_t acols = (size_t)maxL2 + 1, scols = (size_t)maxL2;
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < B; ++b) {
        const float* a = alpha + b * astride;
        const float* s = scores + b * sstride;
        const float* vv = V + b * sstride;
        float* da = d_alpha + b * astride;
        float* dbe = d_beta + b * astride;
        float* h = H + b * sstride;
        float S = partition[b];
        int L1 = lengths[2 * b], L2 = lengths[2 * b + 1];
        for (size_t q = 0; q < astride; ++q) { da[q] = 0.0f; dbe[q] = 0.0f; }
        for (size_t q = 0; q < sstride; ++q) h[q] = 0.0f;
        da[PM(0)] = 0.0f;
        FOR_DIAG_FWD(L1, L2, i, j) {
            size_t c = AIDX(i, j), cd = AIDX(i - 1, j - 1), cu = AIDX(i - 1, j), cl = AIDX(i, j - 1);
            float sc = s[SIDX(i, j)], vij = vv[SIDX(i, j)];
            int dg = (i > 1 && j > 1);
            float v4[4], w4[4], v2[2], w2[2];
            v4[0] = dg ? a[PM(cd)] + sc : NINF;
            v4[1] = dg ? a[PI(cd)] + sc : NINF;
            v4[2] = dg ? a[PD(cd)] + sc : NINF;
            v4[3] = sc;
            softmax_w(v4, w4, 4, T);
            float dM = dg ? da[PM(cd)] + vij : 0.0f;
            float dI = dg ? da[PI(cd)] + vij : 0.0f;
            float dD = dg ? da[PD(cd)] + vij : 0.0f;
            da[PM(c)] = w4[0] * dM + w4[1] * dI + w4[2] * dD + w4[3] * vij;
            v2[0] = (i > 1) ? a[PM(cu)] + go : NINF;
            v2[1] = (i > 1) ? a[PI(cu)] + ge : NINF;
            softmax_w(v2, w2, 2, T);
            float diM = (i > 1) ? da[PM(cu)] : 0.0f;
            float diI = (i > 1) ? da[PI(cu)] : 0.0f;
            da[PI(c)] = w2[0] * diM + w2[1] * diI;
            v2[0] = (j > 1) ? a[PM(cl)] + go : NINF;
            v2[1] = (j > 1) ? a[PD(cl)] + ge : NINF;
            softmax_w(v2, w2, 2, T);
            float ddM = (j > 1) ? da[PM(cl)] : 0.0f;
            float ddD = (j > 1) ? da[PD(cl)] : 0.0f;
            da[PD(c)] = w2[0] * ddM + w2[1] * ddD;
        }
        kahan k = {0.0f, 0.0f};
        for (int i = 0; i <= L1; ++i)
            for (int j = 0; j <= L2; ++j)
                for (int st = 0; st < 3; ++st) {
                    size_t id = st * cstride + AIDX(i, j);
                    kadd(&k, xexp(clamp_lp((a[id] - S) / T)) * da[id]);
                }
        float dS = k.s;
        d_partition[b] = dS;
        float* be = (float*)calloc(astride, sizeof(float));
        for (int i = 0; i <= L1; ++i)
            for (int j = 0; j <= L2; ++j)
                for (int st = 0; st < 3; ++st) {
                    size_t id = st * cstride + AIDX(i, j);
                    be[id] = xexp(clamp_lp((a[id] - S) / T));
                }
        for (int i = 0; i <= L1; ++i)
            for (int j = 0; j <= L2; ++j)
                for (int st = 0; st < 3; ++st) {
                    size_t id = st * cstride + AIDX(i, j);
                    dbe[id] = be[id] * (da[id] - dS) / T;
                }
        FOR_DIAG_REV(L1, L2, i, j) {
            size_t c = AIDX(i, j), cd = AIDX(i - 1, j - 1), cu = AIDX(i - 1, j), cl = AIDX(i, j - 1);
            float sc = s[SIDX(i, j)], vij = vv[SIDX(i, j)];
            int dg = (i > 1 && j > 1);
            /* M */
            float bM = be[PM(c)], dbM = dbe[PM(c)];
            float v4[4], w4[4];
            v4[0] = dg ? a[PM(cd)] + sc : NINF;
            v4[1] = dg ? a[PI(cd)] + sc : NINF;
            v4[2] = dg ? a[PD(cd)] + sc : NINF;
            v4[3] = sc;
            softmax_w(v4, w4, 4, T);
            float dM = dg ? da[PM(cd)] + vij : 0.0f;
            float dI = dg ? da[PI(cd)] + vij : 0.0f;
            float dD = dg ? da[PD(cd)] + vij : 0.0f;
            float dS4 = vij;
            float mean = w4[0] * dM + w4[1] * dI + w4[2] * dD + w4[3] * dS4;
            float dwM = w4[0] * (dM - mean) / T;
            float dwI = w4[1] * (dI - mean) / T;
            float dwD = w4[2] * (dD - mean) / T;
            float dwS = w4[3] * (dS4 - mean) / T;
            h[SIDX(i, j)] += dbM * (w4[0] + w4[1] + w4[2] + w4[3]) + bM * (dwM + dwI + dwD + dwS);
            if (dg) {
                be[PM(cd)] += bM * w4[0];
                be[PI(cd)] += bM * w4[1];
                be[PD(cd)] += bM * w4[2];
                dbe[PM(cd)] += dbM * w4[0] + bM * dwM;
                dbe[PI(cd)] += dbM * w4[1] + bM * dwI;
                dbe[PD(cd)] += dbM * w4[2] + bM * dwD;
            }
            /* I */
            float bI = be[PI(c)], dbI = dbe[PI(c)];
            float v2[2], w2[2];
            v2[0] = (i > 1) ? a[PM(cu)] + go : NINF;
            v2[1] = (i > 1) ? a[PI(cu)] + ge : NINF;
            softmax_w(v2, w2, 2, T);
            float diM = (i > 1) ? da[PM(cu)] : 0.0f;
            float diI = (i > 1) ? da[PI(cu)] : 0.0f;
            float mi = w2[0] * diM + w2[1] * diI;
            float dwiM = w2[0] * (diM - mi) / T;
            float dwiI = w2[1] * (diI - mi) / T;
            if (i > 1) {
                be[PM(cu)] += bI * w2[0];
                be[PI(cu)] += bI * w2[1];
                dbe[PM(cu)] += dbI * w2[0] + bI * dwiM;
                dbe[PI(cu)] += dbI * w2[1] + bI * dwiI;
            }
            /* D */
            float bD = be[PD(c)], dbD = dbe[PD(c)];
            v2[0] = (j > 1) ? a[PM(cl)] + go : NINF;
            v2[1] = (j > 1) ? a[PD(cl)] + ge : NINF;
            softmax_w(v2, w2, 2, T);
            float ddM = (j > 1) ? da[PM(cl)] : 0.0f;
            float ddD = (j > 1) ? da[PD(cl)] : 0.0f;
            float md = w2[0] * ddM + w2[1] * ddD;
            float dwdM = w2[0] * (ddM - md) / T;
            float dwdD = w2[1] * (ddD - md) / T;
            if (j > 1) {
                be[PM(cl)] += bD * w2[0];
                be[PD(cl)] += bD * w2[1];
                dbe[PM(cl)] += dbD * w2[0] + bD * dwdM;
                dbe[PD(cl)] += dbD * w2[1] + bD * dwdD;
            }
        }
        free(be);
    }
}

/* sw_affine/kernels_cpu.cpp:643-921  (param_type 0 = open, 1 = ext, 2 = T) */
void oracle_swa_param_grad(const float* alpha, const float* scores, const float* partition,
                           const float* dS_dtheta, float* U, float* beta, float* W,
                           float* dP, const int* lengths, int B, int maxL1, int maxL2,
                           float go, float ge, float T, int ptype) {
    const size_t cstride = (size_t)(maxL1 + 1) * (maxL2 + 1);
    const size_t astride = 3 * cstride;
    const size_t sstride = (size_t)maxL1 * maxL2;
    const size_t acols = (size_t)maxL2 + 1, scols = (size_t)maxL2;
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < B; ++b) {
        const float* a = alpha + b * astride;
        const float* s = scores + b * sstride;
        float* u = U + b * astride;
        float* be = beta + b * astride;
        float* ww = W + b * astride;
        float* dp = dP + b * sstride;
        float S = partition[b], dSdt = dS_dtheta[b];
        int L1 = lengths[2 * b], L2 = lengths[2 * b + 1];
        for (size_t q = 0; q < astride; ++q) { u[q] = 0.0f; be[q] = 0.0f; ww[q] = 0.0f; }
        for (size_t q = 0; q < sstride; ++q) dp[q] = 0.0f;
        u[PM(0)] = 0.0f;
        FOR_DIAG_FWD(L1, L2, i, j) {
            size_t c = AIDX(i, j), cd = AIDX(i - 1, j - 1), cu = AIDX(i - 1, j), cl = AIDX(i, j - 1);
            float sc = s[SIDX(i, j)];
            int dg = (i > 1 && j > 1);
            float v4[4], w4[4], v2[2], w2[2];
            v4[0] = dg ? a[PM(cd)] + sc : NINF;
            v4[1] = dg ? a[PI(cd)] + sc : NINF;
            v4[2] = dg ? a[PD(cd)] + sc : NINF;
            v4[3] = sc;
            softmax_w(v4, w4, 4, T);
            float uMM = dg ? u[PM(cd)] : 0.0f;
            float uMI = dg ? u[PI(cd)] : 0.0f;
            float uMD = dg ? u[PD(cd)] : 0.0f;
            float dUM = w4[0] * uMM + w4[1] * uMI + w4[2] * uMD;
            if (ptype == 2) {
                float E = w4[0] * v4[0] + w4[1] * v4[1] + w4[2] * v4[2] + w4[3] * v4[3];
                dUM += (a[PM(c)] - E) / T;
            }
            u[PM(c)] = dUM;
            v2[0] = (i > 1) ? a[PM(cu)] + go : NINF;
            v2[1] = (i > 1) ? a[PI(cu)] + ge : NINF;
            softmax_w(v2, w2, 2, T);
            float uIM = (i > 1) ? u[PM(cu)] : 0.0f;
            float uII = (i > 1) ? u[PI(cu)] : 0.0f;
            if (ptype == 0) uIM += 1.0f;
            if (ptype == 1) uII += 1.0f;
            float dUI = w2[0] * uIM + w2[1] * uII;
            if (ptype == 2) {
                float E = w2[0] * v2[0] + w2[1] * v2[1];
                dUI += (a[PI(c)] - E) / T;
            }
            u[PI(c)] = dUI;
            v2[0] = (j > 1) ? a[PM(cl)] + go : NINF;
            v2[1] = (j > 1) ? a[PD(cl)] + ge : NINF;
            softmax_w(v2, w2, 2, T);
            float uDM = (j > 1) ? u[PM(cl)] : 0.0f;
            float uDD = (j > 1) ? u[PD(cl)] : 0.0f;
            if (ptype == 0) uDM += 1.0f;
            if (ptype == 1) uDD += 1.0f;
            float dUD = w2[0] * uDM + w2[1] * uDD;
            if (ptype == 2) {
                float E = w2[0] * v2[0] + w2[1] * v2[1];
                dUD += (a[PD(c)] - E) / T;
            }
            u[PD(c)] = dUD;
        }
        for (int i = 0; i <= L1; ++i)
            for (int j = 0; j <= L2; ++j)
                for (int st = 0; st < 3; ++st) {
                    size_t id = st * cstride + AIDX(i, j);
                    be[id] = posterior_weight(a[id], S, T);
                }
        FOR_DIAG_REV(L1, L2, i, j) {
            size_t c = AIDX(i, j), cd = AIDX(i - 1, j - 1), cu = AIDX(i - 1, j), cl = AIDX(i, j - 1);
            float sc = s[SIDX(i, j)];
            int dg = (i > 1 && j > 1);
            /* M */
            float bM = be[PM(c)];
            float biM = posterior_weight(a[PM(c)], S, T);
            float WM = ww[PM(c)] + biM * (u[PM(c)] - dSdt) / T;
            if (ptype == 2 && a[PM(c)] > NINF) WM -= biM * (a[PM(c)] - S) / (T * T);
            float v4[4], w4[4];
            v4[0] = dg ? a[PM(cd)] + sc : NINF;
            v4[1] = dg ? a[PI(cd)] + sc : NINF;
            v4[2] = dg ? a[PD(cd)] + sc : NINF;
            v4[3] = sc;
            softmax_w(v4, w4, 4, T);
            float uMM = dg ? u[PM(cd)] : 0.0f;
            float uMI = dg ? u[PI(cd)] : 0.0f;
            float uMD = dg ? u[PD(cd)] : 0.0f;
            float uMS = 0.0f;
            float mean = w4[0] * uMM + w4[1] * uMI + w4[2] * uMD + w4[3] * uMS;
            float dwM = w4[0] * (uMM - mean) / T;
            float dwI = w4[1] * (uMI - mean) / T;
            float dwD = w4[2] * (uMD - mean) / T;
            float dwS = w4[3] * (uMS - mean) / T;
            if (ptype == 2) {
                float E = w4[0] * v4[0] + w4[1] * v4[1] + w4[2] * v4[2] + w4[3] * v4[3];
                float it2 = 1.0f / (T * T);
                dwM += w4[0] * (E - v4[0]) * it2;
                dwI += w4[1] * (E - v4[1]) * it2;
                dwD += w4[2] * (E - v4[2]) * it2;
                dwS += w4[3] * (E - v4[3]) * it2;
            }
            (void)dwS;
            dp[SIDX(i, j)] += WM;
            if (dg) {
                be[PM(cd)] += bM * w4[0];
                be[PI(cd)] += bM * w4[1];
                be[PD(cd)] += bM * w4[2];
                ww[PM(cd)] += WM * w4[0] + bM * dwM;
                ww[PI(cd)] += WM * w4[1] + bM * dwI;
                ww[PD(cd)] += WM * w4[2] + bM * dwD;
            }
            /* I */
            float bI = be[PI(c)];
            float biI = posterior_weight(a[PI(c)], S, T);
            float WI = ww[PI(c)] + biI * (u[PI(c)] - dSdt) / T;
            if (ptype == 2 && a[PI(c)] > NINF) WI -= biI * (a[PI(c)] - S) / (T * T);
            if (i > 1) {
                float v2[2], w2[2];
                v2[0] = a[PM(cu)] + go;
                v2[1] = a[PI(cu)] + ge;
                softmax_w(v2, w2, 2, T);
                float uM = u[PM(cu)], uI = u[PI(cu)];
                if (ptype == 0) uM += 1.0f;
                if (ptype == 1) uI += 1.0f;
                float sw = w2[0] * uM + w2[1] * uI;
                float d0 = w2[0] * (uM - sw) / T;
                float d1 = w2[1] * (uI - sw) / T;
                if (ptype == 2) {
                    float E = w2[0] * v2[0] + w2[1] * v2[1];
                    float it2 = 1.0f / (T * T);
                    d0 += w2[0] * (E - v2[0]) * it2;
                    d1 += w2[1] * (E - v2[1]) * it2;
                }
                be[PM(cu)] += bI * w2[0];
                be[PI(cu)] += bI * w2[1];
                ww[PM(cu)] += WI * w2[0] + bI * d0;
                ww[PI(cu)] += WI * w2[1] + bI * d1;
            }
            /* D */
            float bD = be[PD(c)];
            float biD = posterior_weight(a[PD(c)], S, T);
            float WD = ww[PD(c)] + biD * (u[PD(c)] - dSdt) / T;
            if (ptype == 2 && a[PD(c)] > NINF) WD -= biD * (a[PD(c)] - S) / (T * T);
            if (j > 1) {
                float v2[2], w2[2];
                v2[0] = a[PM(cl)] + go;
                v2[1] = a[PD(cl)] + ge;
                softmax_w(v2, w2, 2, T);
                float uM = u[PM(cl)], uD = u[PD(cl)];
                if (ptype == 0) uM += 1.0f;
                if (ptype == 1) uD += 1.0f;
                float sw = w2[0] * uM + w2[1] * uD;
                float d0 = w2[0] * (uM - sw) / T;
                float d1 = w2[1] * (uD - sw) / T;
                if (ptype == 2) {
                    float E = w2[0] * v2[0] + w2[1] * v2[1];
                    float it2 = 1.0f / (T * T);
                    d0 += w2[0] * (E - v2[0]) * it2;
                    d1 += w2[1] * (E - v2[1]) * it2;
                }
                be[PM(cl)] += bD * w2[0];
                be[PD(cl)] += bD * w2[1];
                ww[PM(cl)] += WD * w2[0] + bD * d0;
                ww[PD(cl)] += WD * w2[1] + bD * d1;
            }
        }
    }
}

/* =========================================================================
 * Soft DTW
 * ========================================================================= */

/* dtw/kernels_cpu.cpp:58-121 */
void oracle_dtw_forward(const float* costs, float* alpha, float* score,
                        const int* lengths, int B, int maxL1, int maxL2, float T, int64_t bw) {
    const size_t astride = (size_t)(maxL1 + 1) * (maxL2 + 1);
    const size_t sstride = (size_t)maxL1 * maxL2;
    const size_t acols = (size_t)maxL2 + 1, scols = (size_t)maxL2;
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < B; ++b) {
        const float* c = costs + b * sstride;
        float* a = alpha + b * astride;
        int L1 = lengths[2 * b], L2 = lengths[2 * b + 1];
        for (size_t q = 0; q < astride; ++q) a[q] = PINF;
        a[0] = 0.0f;
        FOR_DIAG_FWD(L1, L2, i, j) {
            if (!in_band(i, j, L1, L2, bw)) continue;
            float ad = a[AIDX(i - 1, j - 1)], au = a[AIDX(i - 1, j)], al = a[AIDX(i, j - 1)];
            if (!in_band(i - 1, j - 1, L1, L2, bw)) ad = PINF;
            if (!in_band(i - 1, j, L1, L2, bw)) au = PINF;
            if (!in_band(i, j - 1, L1, L2, bw)) al = PINF;
            a[AIDX(i, j)] = c[SIDX(i, j)] + softmin3(ad, au, al, T);
        }
        score[b] = a[AIDX(L1, L2)];
    }
}

/* dtw/kernels_cpu.cpp:127-223 */
static void dtw_backward_impl(const float* alpha, const float* costs, const float* score,
                              float* beta, float* posteriors, float* grad_T, double* sums64,
                              const int* lengths, int B, int maxL1, int maxL2, float T,
                              int64_t bw) {
    (void)score;
    const size_t astride = (size_t)(maxL1 + 1) * (maxL2 + 1);
    const size_t sstride = (size_t)maxL1 * maxL2;
    const size_t acols = (size_t)maxL2 + 1, scols = (size_t)maxL2;
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < B; ++b) {
        const float* a = alpha + b * astride;
        const float* c = costs + b * sstride;
        float* be = beta + b * astride;
        float* post = posteriors + b * sstride;
        int L1 = lengths[2 * b], L2 = lengths[2 * b + 1];
        for (size_t q = 0; q < sstride; ++q) post[q] = 0.0f;
        for (size_t q = 0; q < astride; ++q) be[q] = 0.0f;
        be[AIDX(L1, L2)] = 1.0f;
        float gT = 0.0f;
        double gT_d = 0.0;
        FOR_DIAG_REV(L1, L2, i, j) {
            if (!in_band(i, j, L1, L2, bw)) continue;
            float bij = be[AIDX(i, j)];
            if (bij == 0.0f) continue;
            post[SIDX(i, j)] = bij;
            float ad = a[AIDX(i - 1, j - 1)], au = a[AIDX(i - 1, j)], al = a[AIDX(i, j - 1)];
            int bd = in_band(i - 1, j - 1, L1, L2, bw), bu = in_band(i - 1, j, L1, L2, bw),
                bl = in_band(i, j - 1, L1, L2, bw);
            if (!bd) ad = PINF;
            if (!bu) au = PINF;
            if (!bl) al = PINF;
            float wd, wu, wl;
            softmin3_w(ad, au, al, T, &wd, &wu, &wl);
            if (bd && wd > 0.0f) be[AIDX(i - 1, j - 1)] += bij * wd;
            if (bu && wu > 0.0f) be[AIDX(i - 1, j)] += bij * wu;
            if (bl && wl > 0.0f) be[AIDX(i, j - 1)] += bij * wl;
            float smv = a[AIDX(i, j)] - c[SIDX(i, j)];
            if (smv < PINF) {
                float Ea = wd * ad + wu * au + wl * al;
                gT += bij * (smv - Ea) / T;
                gT_d += (double)(bij * (smv - Ea) / T);
            }
        }
        grad_T[b] = gT;
        if (sums64) sums64[b] = gT_d;
    }
}

void oracle_dtw_backward(const float* alpha, const float* costs, const float* score,
                         float* beta, float* posteriors, float* grad_T,
                         const int* lengths, int B, int maxL1, int maxL2, float T, int64_t bw) {
    dtw_backward_impl(alpha, costs, score, beta, posteriors, grad_T, NULL, lengths, B, maxL1,
                      maxL2, T, bw);
}

/* The same reverse sweep with dS/dT also summed in double into sums64[b]. */
void oracle_dtw_backward_sums64(const float* alpha, const float* costs, const float* score,
                                float* beta, float* posteriors, double* sums64,
                                const int* lengths, int B, int maxL1, int maxL2, float T,
                                int64_t bw) {
    float* gt = (float*)malloc(sizeof(float) * (B > 0 ? B : 1));
    dtw_backward_impl(alpha, costs, score, beta, posteriors, gt, sums64, lengths, B, maxL1,
                      maxL2, T, bw);
    free(gt);
}



/* dtw/kernels_cpu.cpp:229-377 */
void oracle_dtw_hvp(const float* alpha, const float* costs, const float* score,
                    const float* V, float* d_alpha, float* d_score, float* beta,
                    float* d_beta, float* H, const int* lengths, int B, int maxL1, int maxL2,
                    float T, int64_t bw) {
    (void)costs; (void)score;
    const size_t astride = (size_t)(maxL1 + 1) * (maxL2 + 1);
    const size_t sstride = (size_t)maxL1 * maxL2;
    const size_t acols = (size_t)maxL2 + 1, scols = (size_t)maxL2;
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < B; ++b) {
        const float* a = alpha + b * astride;
        const float* vv = V + b * sstride;
        float* da = d_alpha + b * astride;
        float* be = beta + b * astride;
        float* dbe = d_beta + b * astride;
        float* h = H + b * sstride;
        int L1 = lengths[2 * b], L2 = lengths[2 * b + 1];
        for (size_t q = 0; q < astride; ++q) { da[q] = 0.0f; be[q] = 0.0f; dbe[q] = 0.0f; }
        for (size_t q = 0; q < sstride; ++q) h[q] = 0.0f;
        FOR_DIAG_FWD(L1, L2, i, j) {
            if (!in_band(i, j, L1, L2, bw)) continue;
            float ad = a[AIDX(i - 1, j - 1)], au = a[AIDX(i - 1, j)], al = a[AIDX(i, j - 1)];
            int bd = in_band(i - 1, j - 1, L1, L2, bw), bu = in_band(i - 1, j, L1, L2, bw),
                bl = in_band(i, j - 1, L1, L2, bw);
            if (!bd) ad = PINF;
            if (!bu) au = PINF;
            if (!bl) al = PINF;
            float wd, wu, wl;
            softmin3_w(ad, au, al, T, &wd, &wu, &wl);
            float dad = bd ? da[AIDX(i - 1, j - 1)] : 0.0f;
            float dau = bu ? da[AIDX(i - 1, j)] : 0.0f;
            float dal = bl ? da[AIDX(i, j - 1)] : 0.0f;
            da[AIDX(i, j)] = vv[SIDX(i, j)] + wd * dad + wu * dau + wl * dal;
        }
        size_t fin = AIDX(L1, L2);
        d_score[b] = da[fin];
        be[fin] = 1.0f;
        dbe[fin] = 0.0f;
        FOR_DIAG_REV(L1, L2, i, j) {
            if (!in_band(i, j, L1, L2, bw)) continue;
            float bij = be[AIDX(i, j)], dbij = dbe[AIDX(i, j)];
            if (bij == 0.0f) continue;
            float ad = a[AIDX(i - 1, j - 1)], au = a[AIDX(i - 1, j)], al = a[AIDX(i, j - 1)];
            int bd = in_band(i - 1, j - 1, L1, L2, bw), bu = in_band(i - 1, j, L1, L2, bw),
                bl = in_band(i, j - 1, L1, L2, bw);
            if (!bd) ad = PINF;
            if (!bu) au = PINF;
            if (!bl) al = PINF;
            float wd, wu, wl;
            softmin3_w(ad, au, al, T, &wd, &wu, &wl);
            float dad = bd ? da[AIDX(i - 1, j - 1)] : 0.0f;
            float dau = bu ? da[AIDX(i - 1, j)] : 0.0f;
            float dal = bl ? da[AIDX(i, j - 1)] : 0.0f;
            float E = wd * dad + wu * dau + wl * dal;
            float dwd = wd * (-dad + E) / T;
            float dwu = wu * (-dau + E) / T;
            float dwl = wl * (-dal + E) / T;
            h[SIDX(i, j)] = dbij;
            if (bd && wd > 0.0f) { be[AIDX(i - 1, j - 1)] += bij * wd; dbe[AIDX(i - 1, j - 1)] += dbij * wd + bij * dwd; }
            if (bu && wu > 0.0f) { be[AIDX(i - 1, j)] += bij * wu; dbe[AIDX(i - 1, j)] += dbij * wu + bij * dwu; }
            if (bl && wl > 0.0f) { be[AIDX(i, j - 1)] += bij * wl; dbe[AIDX(i, j - 1)] += dbij * wl + bij * dwl; }
        }
    }
}

/* dtw/kernels_cpu.cpp:383-534 */
void oracle_dtw_param_grad(const float* alpha, const float* costs, const float* score,
                           float* U, float* beta, float* W, float* dP_dT,
                           const int* lengths, int B, int maxL1, int maxL2, float T,
                           int64_t bw) {
    (void)score;
    const size_t astride = (size_t)(maxL1 + 1) * (maxL2 + 1);
    const size_t sstride = (size_t)maxL1 * maxL2;
    const size_t acols = (size_t)maxL2 + 1, scols = (size_t)maxL2;
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < B; ++b) {
        const float* a = alpha + b * astride;
        const float* c = costs + b * sstride;
        float* u = U + b * astride;
        float* be = beta + b * astride;
        float* ww = W + b * astride;
        float* dp = dP_dT + b * sstride;
        int L1 = lengths[2 * b], L2 = lengths[2 * b + 1];
        for (size_t q = 0; q < astride; ++q) { u[q] = 0.0f; be[q] = 0.0f; ww[q] = 0.0f; }
        for (size_t q = 0; q < sstride; ++q) dp[q] = 0.0f;
        FOR_DIAG_FWD(L1, L2, i, j) {
            if (!in_band(i, j, L1, L2, bw)) continue;
            float ad = a[AIDX(i - 1, j - 1)], au = a[AIDX(i - 1, j)], al = a[AIDX(i, j - 1)];
            int bd = in_band(i - 1, j - 1, L1, L2, bw), bu = in_band(i - 1, j, L1, L2, bw),
                bl = in_band(i, j - 1, L1, L2, bw);
            if (!bd) ad = PINF;
            if (!bu) au = PINF;
            if (!bl) al = PINF;
            float wd, wu, wl;
            softmin3_w(ad, au, al, T, &wd, &wu, &wl);
            float ud = bd ? u[AIDX(i - 1, j - 1)] : 0.0f;
            float uu = bu ? u[AIDX(i - 1, j)] : 0.0f;
            float ul = bl ? u[AIDX(i, j - 1)] : 0.0f;
            float smv = a[AIDX(i, j)] - c[SIDX(i, j)];
            float Ea = wd * ad + wu * au + wl * al;
            u[AIDX(i, j)] = (smv - Ea) / T + wd * ud + wu * uu + wl * ul;
        }
        size_t fin = AIDX(L1, L2);
        be[fin] = 1.0f;
        ww[fin] = 0.0f;
        FOR_DIAG_REV(L1, L2, i, j) {
            if (!in_band(i, j, L1, L2, bw)) continue;
            float bij = be[AIDX(i, j)], Wij = ww[AIDX(i, j)];
            if (bij == 0.0f && fabsf(Wij) < 1e-20f) continue;
            dp[SIDX(i, j)] = Wij;
            float ad = a[AIDX(i - 1, j - 1)], au = a[AIDX(i - 1, j)], al = a[AIDX(i, j - 1)];
            int bd = in_band(i - 1, j - 1, L1, L2, bw), bu = in_band(i - 1, j, L1, L2, bw),
                bl = in_band(i, j - 1, L1, L2, bw);
            if (!bd) ad = PINF;
            if (!bu) au = PINF;
            if (!bl) al = PINF;
            float wd, wu, wl;
            softmin3_w(ad, au, al, T, &wd, &wu, &wl);
            float ud = bd ? u[AIDX(i - 1, j - 1)] : 0.0f;
            float uu = bu ? u[AIDX(i - 1, j)] : 0.0f;
            float ul = bl ? u[AIDX(i, j - 1)] : 0.0f;
            float Ea = wd * ad + wu * au + wl * al;
            float Eu = wd * ud + wu * uu + wl * ul;
            float iT = 1.0f / T;
            float iT2 = iT * iT;
            float dd = wd * ((Eu - ud) * iT + (ad - Ea) * iT2);
            float du = wu * ((Eu - uu) * iT + (au - Ea) * iT2);
            float dl = wl * ((Eu - ul) * iT + (al - Ea) * iT2);
            if (bd && wd > 0.0f) { be[AIDX(i - 1, j - 1)] += bij * wd; ww[AIDX(i - 1, j - 1)] += Wij * wd + bij * dd; }
            if (bu && wu > 0.0f) { be[AIDX(i - 1, j)] += bij * wu; ww[AIDX(i - 1, j)] += Wij * wu + bij * du; }
            if (bl && wl > 0.0f) { be[AIDX(i, j - 1)] += bij * wl; ww[AIDX(i, j - 1)] += Wij * wl + bij * dl; }
        }
    }
}

/* =========================================================================
 * Linear-gap soft Needleman-Wunsch (global alignment)
 * ========================================================================= */

/* nw/kernels_cpu.cpp:78-154: alpha[0,0] = 0, alpha[i,0] = i*gap, alpha[0,j] =
 * j*gap, alpha[i,j] = LSE3(diag + s, up + gap, left + gap) with no sky term and no
 * guards; the value is alpha[L1, L2]. */
void oracle_nw_forward(const float* scores, float* alpha, float* score, const int* lengths,
                       int B, int maxL1, int maxL2, float gap, float T) {
    const size_t astride = (size_t)(maxL1 + 1) * (maxL2 + 1);
    const size_t sstride = (size_t)maxL1 * maxL2;
    const size_t acols = (size_t)maxL2 + 1, scols = (size_t)maxL2;
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < B; ++b) {
        const float* s = scores + (size_t)b * sstride;
        float* a = alpha + (size_t)b * astride;
        const int L1 = lengths[2 * b], L2 = lengths[2 * b + 1];
        for (size_t q = 0; q < astride; ++q) a[q] = NINF;
        a[0] = 0.0f;
        for (int i = 1; i <= L1; ++i) a[AIDX(i, 0)] = i * gap;
        for (int j = 1; j <= L2; ++j) a[AIDX(0, j)] = j * gap;
        FOR_DIAG_FWD(L1, L2, i, j) {
            if (j < 1 || j > L2) continue;
            const float sc = s[SIDX(i, j)];
            a[AIDX(i, j)] = lse3(a[AIDX(i - 1, j - 1)] + sc, a[AIDX(i - 1, j)] + gap,
                                 a[AIDX(i, j - 1)] + gap, T);
        }
        score[b] = a[AIDX(L1, L2)];
    }
}

/* nw/kernels_cpu.cpp:160-265: beta[L1,L2] = 1; every visited cell passes beta on
 * through its softmax weights (NINF options weigh 0) and its marginal is
 * beta * w_diag.  dS/dgap adds the beta that reaches each boundary cell times the
 * number of gaps it encodes (i for alpha[i,0], j for alpha[0,j]); dS/dT =
 * (S - sum P*s - gap * dS/dgap) / T. */
void oracle_nw_backward(const float* alpha, const float* scores, const float* score,
                        float* beta, float* posteriors, float* grad_gap, float* grad_T,
                        const int* lengths, int B, int maxL1, int maxL2, float gap, float T) {
    const size_t astride = (size_t)(maxL1 + 1) * (maxL2 + 1);
    const size_t sstride = (size_t)maxL1 * maxL2;
    const size_t acols = (size_t)maxL2 + 1, scols = (size_t)maxL2;
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < B; ++b) {
        const float* a = alpha + (size_t)b * astride;
        const float* s = scores + (size_t)b * sstride;
        float* be = beta + (size_t)b * astride;
        float* post = posteriors + (size_t)b * sstride;
        const float S = score[b];
        const int L1 = lengths[2 * b], L2 = lengths[2 * b + 1];
        memset(post, 0, sizeof(float) * sstride);
        memset(be, 0, sizeof(float) * astride);
        be[AIDX(L1, L2)] = 1.0f;
        kahan gg = {0.0f, 0.0f}, ms = {0.0f, 0.0f};
        FOR_DIAG_REV(L1, L2, i, j) {
            if (j < 1 || j > L2) continue;
            const float bij = be[AIDX(i, j)];
            if (bij == 0.0f) continue;
            const float sc = s[SIDX(i, j)];
            float v[3] = {a[AIDX(i - 1, j - 1)] + sc, a[AIDX(i - 1, j)] + gap,
                          a[AIDX(i, j - 1)] + gap};
            float w[3];
            softmax_w(v, w, 3, T);
            const float pij = bij * w[0];
            post[SIDX(i, j)] = pij;
            kadd(&ms, pij * sc);
            kadd(&gg, bij * (w[1] + w[2]));
            if (w[0] > 0.0f) be[AIDX(i - 1, j - 1)] += bij * w[0];
            if (w[1] > 0.0f) be[AIDX(i - 1, j)] += bij * w[1];
            if (w[2] > 0.0f) be[AIDX(i, j - 1)] += bij * w[2];
        }
        for (int i = 1; i <= L1; ++i) kadd(&gg, be[AIDX(i, 0)] * (float)i);
        for (int j = 1; j <= L2; ++j) kadd(&gg, be[AIDX(0, j)] * (float)j);
        const float g = gg.s;
        grad_gap[b] = g;
        grad_T[b] = (S - (ms.s + g * gap)) / T;
    }
}

/* nw/kernels_cpu.cpp:278-444: forward tangent da = sum w (da_pred + V [diag]) from
 * zero boundary tangents; reverse (beta, dbeta) from (1, 0) at the terminal cell,
 * skipping cells with beta == 0 and |dbeta| < 1e-20; H = dbeta w_diag +
 * beta dw_diag with dw_k = w_k (dv_k - E_w[dv]) / T. */
void oracle_nw_hvp(const float* alpha, const float* scores, const float* score, const float* V,
                   float* d_alpha, float* d_score, float* beta, float* d_beta, float* H,
                   const int* lengths, int B, int maxL1, int maxL2, float gap, float T) {
    const size_t astride = (size_t)(maxL1 + 1) * (maxL2 + 1);
    const size_t sstride = (size_t)maxL1 * maxL2;
    const size_t acols = (size_t)maxL2 + 1, scols = (size_t)maxL2;
    (void)score;
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < B; ++b) {
        const float* a = alpha + (size_t)b * astride;
        const float* s = scores + (size_t)b * sstride;
        const float* v = V + (size_t)b * sstride;
        float* da = d_alpha + (size_t)b * astride;
        float* be = beta + (size_t)b * astride;
        float* dbe = d_beta + (size_t)b * astride;
        float* h = H + (size_t)b * sstride;
        const int L1 = lengths[2 * b], L2 = lengths[2 * b + 1];
        memset(da, 0, sizeof(float) * astride);
        memset(be, 0, sizeof(float) * astride);
        memset(dbe, 0, sizeof(float) * astride);
        memset(h, 0, sizeof(float) * sstride);
        FOR_DIAG_FWD(L1, L2, i, j) {
            if (j < 1 || j > L2) continue;
            const float sc = s[SIDX(i, j)], vij = v[SIDX(i, j)];
            float lv[3] = {a[AIDX(i - 1, j - 1)] + sc, a[AIDX(i - 1, j)] + gap,
                           a[AIDX(i, j - 1)] + gap};
            float w[3];
            softmax_w(lv, w, 3, T);
            const float dd = da[AIDX(i - 1, j - 1)] + vij, du = da[AIDX(i - 1, j)],
                        dl = da[AIDX(i, j - 1)];
            da[AIDX(i, j)] = w[0] * dd + w[1] * du + w[2] * dl;
        }
        d_score[b] = da[AIDX(L1, L2)];
        be[AIDX(L1, L2)] = 1.0f;
        dbe[AIDX(L1, L2)] = 0.0f;
        FOR_DIAG_REV(L1, L2, i, j) {
            if (j < 1 || j > L2) continue;
            const float sc = s[SIDX(i, j)], vij = v[SIDX(i, j)];
            const float bij = be[AIDX(i, j)], dbij = dbe[AIDX(i, j)];
            if (bij == 0.0f && fabsf(dbij) < 1e-20f) continue;
            float lv[3] = {a[AIDX(i - 1, j - 1)] + sc, a[AIDX(i - 1, j)] + gap,
                           a[AIDX(i, j - 1)] + gap};
            float w[3];
            softmax_w(lv, w, 3, T);
            const float dd = da[AIDX(i - 1, j - 1)] + vij, du = da[AIDX(i - 1, j)],
                        dl = da[AIDX(i, j - 1)];
            const float E = w[0] * dd + w[1] * du + w[2] * dl;
            const float wd = w[0] * (dd - E) / T, wu = w[1] * (du - E) / T,
                        wl = w[2] * (dl - E) / T;
            h[SIDX(i, j)] = dbij * w[0] + bij * wd;
            if (w[0] > 0.0f) { be[AIDX(i - 1, j - 1)] += bij * w[0]; dbe[AIDX(i - 1, j - 1)] += dbij * w[0] + bij * wd; }
            if (w[1] > 0.0f) { be[AIDX(i - 1, j)] += bij * w[1]; dbe[AIDX(i - 1, j)] += dbij * w[1] + bij * wu; }
            if (w[2] > 0.0f) { be[AIDX(i, j - 1)] += bij * w[2]; dbe[AIDX(i, j - 1)] += dbij * w[2] + bij * wl; }
        }
    }
}

/* nw/kernels_cpu.cpp:450-642: dP/dtheta for theta = gap (param_type 0; boundary
 * tangents i and j, +1 on the up / left candidates) or T (1; + (alpha - E_w[v]) / T
 * in the tangent, + w_k (E_w[v] - v_k) / T^2 in the weight tangents).  The
 * terminal beta is constant, so dS/dtheta does not enter. */
void oracle_nw_param_grad(const float* alpha, const float* scores, const float* score,
                          const float* dS_dtheta, float* U, float* beta, float* W, float* dP,
                          const int* lengths, int B, int maxL1, int maxL2, float gap, float T,
                          int ptype) {
    const size_t astride = (size_t)(maxL1 + 1) * (maxL2 + 1);
    const size_t sstride = (size_t)maxL1 * maxL2;
    const size_t acols = (size_t)maxL2 + 1, scols = (size_t)maxL2;
    (void)score;
    (void)dS_dtheta;
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < B; ++b) {
        const float* a = alpha + (size_t)b * astride;
        const float* s = scores + (size_t)b * sstride;
        float* u = U + (size_t)b * astride;
        float* be = beta + (size_t)b * astride;
        float* w = W + (size_t)b * astride;
        float* dp = dP + (size_t)b * sstride;
        const int L1 = lengths[2 * b], L2 = lengths[2 * b + 1];
        memset(u, 0, sizeof(float) * astride);
        memset(be, 0, sizeof(float) * astride);
        memset(w, 0, sizeof(float) * astride);
        memset(dp, 0, sizeof(float) * sstride);
        if (ptype == 0) {
            for (int i = 1; i <= L1; ++i) u[AIDX(i, 0)] = (float)i;
            for (int j = 1; j <= L2; ++j) u[AIDX(0, j)] = (float)j;
        }
        FOR_DIAG_FWD(L1, L2, i, j) {
            if (j < 1 || j > L2) continue;
            const float sc = s[SIDX(i, j)];
            float lv[3] = {a[AIDX(i - 1, j - 1)] + sc, a[AIDX(i - 1, j)] + gap,
                           a[AIDX(i, j - 1)] + gap};
            float wt[3];
            softmax_w(lv, wt, 3, T);
            float ud = u[AIDX(i - 1, j - 1)], uu = u[AIDX(i - 1, j)], ul = u[AIDX(i, j - 1)];
            if (ptype == 0) { uu += 1.0f; ul += 1.0f; }
            float x = wt[0] * ud + wt[1] * uu + wt[2] * ul;
            if (ptype == 1) {
                const float Ev = wt[0] * lv[0] + wt[1] * lv[1] + wt[2] * lv[2];
                x += (a[AIDX(i, j)] - Ev) / T;
            }
            u[AIDX(i, j)] = x;
        }
        be[AIDX(L1, L2)] = 1.0f;
        w[AIDX(L1, L2)] = 0.0f;
        FOR_DIAG_REV(L1, L2, i, j) {
            if (j < 1 || j > L2) continue;
            const float sc = s[SIDX(i, j)];
            const float bij = be[AIDX(i, j)], Wij = w[AIDX(i, j)];
            if (bij == 0.0f && fabsf(Wij) < 1e-20f) continue;
            float lv[3] = {a[AIDX(i - 1, j - 1)] + sc, a[AIDX(i - 1, j)] + gap,
                           a[AIDX(i, j - 1)] + gap};
            float wt[3];
            softmax_w(lv, wt, 3, T);
            float ud = u[AIDX(i - 1, j - 1)], uu = u[AIDX(i - 1, j)], ul = u[AIDX(i, j - 1)];
            if (ptype == 0) { uu += 1.0f; ul += 1.0f; }
            const float Eu = wt[0] * ud + wt[1] * uu + wt[2] * ul;
            float dd = wt[0] * (ud - Eu) / T, du = wt[1] * (uu - Eu) / T,
                  dl = wt[2] * (ul - Eu) / T;
            if (ptype == 1) {
                const float Ev = wt[0] * lv[0] + wt[1] * lv[1] + wt[2] * lv[2];
                const float iT2 = 1.0f / (T * T);
                dd += wt[0] * (Ev - lv[0]) * iT2;
                du += wt[1] * (Ev - lv[1]) * iT2;
                dl += wt[2] * (Ev - lv[2]) * iT2;
            }
            dp[SIDX(i, j)] = Wij * wt[0] + bij * dd;
            if (wt[0] > 0.0f) { be[AIDX(i - 1, j - 1)] += bij * wt[0]; w[AIDX(i - 1, j - 1)] += Wij * wt[0] + bij * dd; }
            if (wt[1] > 0.0f) { be[AIDX(i - 1, j)] += bij * wt[1]; w[AIDX(i - 1, j)] += Wij * wt[1] + bij * du; }
            if (wt[2] > 0.0f) { be[AIDX(i, j - 1)] += bij * wt[2]; w[AIDX(i, j - 1)] += Wij * wt[2] + bij * dl; }
        }
    }
}

/* ======================= affine-gap soft Needleman-Wunsch ======================= */

/* softmax3, nw_affine/kernels_cpu.cpp:59-71: Kahan sum over the terms above NINF
 * only; a non-positive sum gives NINF. */
static float nwa_lse3(float a, float b, float c, float T) {
    float m = fmax2(fmax2(a, b), c);
    if (m <= NINF) return NINF;
    kahan k = {0.0f, 0.0f};
    if (a > NINF) kadd(&k, xexp((a - m) / T));
    if (b > NINF) kadd(&k, xexp((b - m) / T));
    if (c > NINF) kadd(&k, xexp((c - m) / T));
    if (k.s <= 0.0f) return NINF;
    return m + T * logf(k.s);
}

/* softmax3_weights, nw_affine/kernels_cpu.cpp:74-94: plain-sum normaliser. */
static void nwa_w3(float a, float b, float c, float T, float* w) {
    float m = fmax2(fmax2(a, b), c);
    if (m <= NINF) { w[0] = w[1] = w[2] = 0.0f; return; }
    float ea = (a > NINF) ? xexp((a - m) / T) : 0.0f;
    float eb = (b > NINF) ? xexp((b - m) / T) : 0.0f;
    float ec = (c > NINF) ? xexp((c - m) / T) : 0.0f;
    float total = ea + eb + ec;
    if (total > 0.0f) { w[0] = ea / total; w[1] = eb / total; w[2] = ec / total; }
    else w[0] = w[1] = w[2] = 0.0f;
}

/* nw_affine/kernels_cpu.cpp:100-187: three states over (L1+1) x (L2+1),
 * M(0,0) = 0, I(i,0) = open + (i-1) ext, D(0,j) = open + (j-1) ext, everything
 * else NINF;  M = s + LSE(M, I, D)[diag],  I = LSE(M+open, I+ext, D+open)[up],
 * D = LSE(M+open, I+open, D+ext)[left];  value LSE(M, I, D)[L1, L2]. */
void oracle_nwa_forward(const float* scores, float* alpha, float* score, const int* lengths,
                        int B, int maxL1, int maxL2, float go, float ge, float T) {
    const size_t cstride = (size_t)(maxL1 + 1) * (maxL2 + 1);
    const size_t astride = 3 * cstride;
    const size_t sstride = (size_t)maxL1 * maxL2;
    const size_t acols = (size_t)maxL2 + 1, scols = (size_t)maxL2;
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < B; ++b) {
        const float* s = scores + (size_t)b * sstride;
        float* a = alpha + (size_t)b * astride;
        const int L1 = lengths[2 * b], L2 = lengths[2 * b + 1];
        for (size_t q = 0; q < astride; ++q) a[q] = NINF;
        a[PM(0)] = 0.0f;
        for (int i = 1; i <= L1; ++i) a[PI(AIDX(i, 0))] = go + (i - 1) * ge;
        for (int j = 1; j <= L2; ++j) a[PD(AIDX(0, j))] = go + (j - 1) * ge;
        FOR_DIAG_FWD(L1, L2, i, j) {
            const size_t c = AIDX(i, j), cd = AIDX(i - 1, j - 1), cu = AIDX(i - 1, j),
                         cl = AIDX(i, j - 1);
            const float sc = s[SIDX(i, j)];
            a[PM(c)] = sc + nwa_lse3(a[PM(cd)], a[PI(cd)], a[PD(cd)], T);
            a[PI(c)] = nwa_lse3(a[PM(cu)] + go, a[PI(cu)] + ge, a[PD(cu)] + go, T);
            a[PD(c)] = nwa_lse3(a[PM(cl)] + go, a[PI(cl)] + go, a[PD(cl)] + ge, T);
        }
        const size_t f = AIDX(L1, L2);
        score[b] = nwa_lse3(a[PM(f)], a[PI(f)], a[PD(f)], T);
    }
}

/* nw_affine/kernels_cpu.cpp:193-347: beta of the three terminal states = their
 * softmax weights; reverse anti-diagonals pass each state's beta (when above 1e-20
 * and its predecessors' LSE is finite) to its predecessors by their weights; the
 * marginal of (i, j) is beta_M; open / ext counts come from the I and D
 * transitions and the boundary I(i,0), D(0,j) chains; dS/dT = (S - E[path score])
 * / T with the match part Kahan-summed. */
void oracle_nwa_backward(const float* alpha, const float* scores, const float* score,
                         float* beta, float* posteriors, float* grad_open, float* grad_ext,
                         float* grad_T, const int* lengths, int B, int maxL1, int maxL2,
                         float go, float ge, float T) {
    const size_t cstride = (size_t)(maxL1 + 1) * (maxL2 + 1);
    const size_t astride = 3 * cstride;
    const size_t sstride = (size_t)maxL1 * maxL2;
    const size_t acols = (size_t)maxL2 + 1, scols = (size_t)maxL2;
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < B; ++b) {
        const float* a = alpha + (size_t)b * astride;
        const float* s = scores + (size_t)b * sstride;
        float* be = beta + (size_t)b * astride;
        float* post = posteriors + (size_t)b * sstride;
        const float S = score[b];
        const int L1 = lengths[2 * b], L2 = lengths[2 * b + 1];
        for (size_t q = 0; q < astride; ++q) be[q] = 0.0f;
        for (size_t q = 0; q < sstride; ++q) post[q] = 0.0f;
        float w[3];
        const size_t f = AIDX(L1, L2);
        nwa_w3(a[PM(f)], a[PI(f)], a[PD(f)], T, w);
        be[PM(f)] = w[0];
        be[PI(f)] = w[1];
        be[PD(f)] = w[2];
        float so = 0.0f, se = 0.0f;
        kahan ms = {0.0f, 0.0f};
        FOR_DIAG_REV(L1, L2, i, j) {
            const size_t c = AIDX(i, j), cd = AIDX(i - 1, j - 1), cu = AIDX(i - 1, j),
                         cl = AIDX(i, j - 1);
            const float sc = s[SIDX(i, j)];
            const float bM = be[PM(c)], bI = be[PI(c)], bD = be[PD(c)];
            if (bM > 1e-20f) {
                const float m1 = a[PM(cd)], m2 = a[PI(cd)], m3 = a[PD(cd)];
                if (nwa_lse3(m1, m2, m3, T) > NINF) {
                    nwa_w3(m1, m2, m3, T, w);
                    if (m1 > NINF) be[PM(cd)] += bM * w[0];
                    if (m2 > NINF) be[PI(cd)] += bM * w[1];
                    if (m3 > NINF) be[PD(cd)] += bM * w[2];
                    post[SIDX(i, j)] += bM;
                    kadd(&ms, bM * sc);
                }
            }
            if (bI > 1e-20f) {
                const float i1 = a[PM(cu)] + go, i2 = a[PI(cu)] + ge, i3 = a[PD(cu)] + go;
                if (nwa_lse3(i1, i2, i3, T) > NINF) {
                    nwa_w3(i1, i2, i3, T, w);
                    be[PM(cu)] += bI * w[0];
                    be[PI(cu)] += bI * w[1];
                    be[PD(cu)] += bI * w[2];
                    so += bI * (w[0] + w[2]);
                    se += bI * w[1];
                }
            }
            if (bD > 1e-20f) {
                const float d1 = a[PM(cl)] + go, d2 = a[PI(cl)] + go, d3 = a[PD(cl)] + ge;
                if (nwa_lse3(d1, d2, d3, T) > NINF) {
                    nwa_w3(d1, d2, d3, T, w);
                    be[PM(cl)] += bD * w[0];
                    be[PI(cl)] += bD * w[1];
                    be[PD(cl)] += bD * w[2];
                    so += bD * (w[0] + w[1]);
                    se += bD * w[2];
                }
            }
        }
        for (int i = 1; i <= L1; ++i) {
            const float bb = be[PI(AIDX(i, 0))];
            if (bb > 1e-20f) { so += bb; se += bb * (float)(i - 1); }
        }
        for (int j = 1; j <= L2; ++j) {
            const float bb = be[PD(AIDX(0, j))];
            if (bb > 1e-20f) { so += bb; se += bb * (float)(j - 1); }
        }
        grad_open[b] = so;
        grad_ext[b] = se;
        const float expected = ms.s + so * go + se * ge;
        grad_T[b] = (S - expected) / T;
    }
}

/* nw_affine/kernels_cpu.cpp:353-613: forward tangents of the three states
 * (M: V + E_w[d_pred] over the diagonal states; I, D: E_w over their up / left
 * candidates; 0 where the predecessors' LSE is NINF), d_score = E_w[d] over the
 * terminal states; reverse sweep with beta and its tangent, the weight tangents
 * w_k (d_k - E_w[d]) / T, cells visited when beta > 1e-20 or |dbeta| > 1e-20;
 * H(i, j) = dbeta_M. */
void oracle_nwa_hvp(const float* alpha, const float* scores, const float* score,
                    const float* V, float* d_alpha, float* d_score, float* beta,
                    float* d_beta, float* H, const int* lengths, int B, int maxL1, int maxL2,
                    float go, float ge, float T) {
    const size_t cstride = (size_t)(maxL1 + 1) * (maxL2 + 1);
    const size_t astride = 3 * cstride;
    const size_t sstride = (size_t)maxL1 * maxL2;
    const size_t acols = (size_t)maxL2 + 1, scols = (size_t)maxL2;
    (void)score;
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < B; ++b) {
        const float* a = alpha + (size_t)b * astride;
        const float* v = V + (size_t)b * sstride;
        float* da = d_alpha + (size_t)b * astride;
        float* be = beta + (size_t)b * astride;
        float* db = d_beta + (size_t)b * astride;
        float* h = H + (size_t)b * sstride;
        const int L1 = lengths[2 * b], L2 = lengths[2 * b + 1];
        for (size_t q = 0; q < astride; ++q) { da[q] = 0.0f; be[q] = 0.0f; db[q] = 0.0f; }
        for (size_t q = 0; q < sstride; ++q) h[q] = 0.0f;
        float w[3];
        FOR_DIAG_FWD(L1, L2, i, j) {
            const size_t c = AIDX(i, j), cd = AIDX(i - 1, j - 1), cu = AIDX(i - 1, j),
                         cl = AIDX(i, j - 1);
            const float Vs = v[SIDX(i, j)];
            {
                const float m1 = a[PM(cd)], m2 = a[PI(cd)], m3 = a[PD(cd)];
                if (nwa_lse3(m1, m2, m3, T) > NINF) {
                    nwa_w3(m1, m2, m3, T, w);
                    da[PM(c)] = Vs + w[0] * da[PM(cd)] + w[1] * da[PI(cd)] + w[2] * da[PD(cd)];
                } else da[PM(c)] = 0.0f;
            }
            {
                const float i1 = a[PM(cu)] + go, i2 = a[PI(cu)] + ge, i3 = a[PD(cu)] + go;
                if (nwa_lse3(i1, i2, i3, T) > NINF) {
                    nwa_w3(i1, i2, i3, T, w);
                    da[PI(c)] = w[0] * da[PM(cu)] + w[1] * da[PI(cu)] + w[2] * da[PD(cu)];
                } else da[PI(c)] = 0.0f;
            }
            {
                const float d1 = a[PM(cl)] + go, d2 = a[PI(cl)] + go, d3 = a[PD(cl)] + ge;
                if (nwa_lse3(d1, d2, d3, T) > NINF) {
                    nwa_w3(d1, d2, d3, T, w);
                    da[PD(c)] = w[0] * da[PM(cl)] + w[1] * da[PI(cl)] + w[2] * da[PD(cl)];
                } else da[PD(c)] = 0.0f;
            }
        }
        const size_t f = AIDX(L1, L2);
        nwa_w3(a[PM(f)], a[PI(f)], a[PD(f)], T, w);
        d_score[b] = w[0] * da[PM(f)] + w[1] * da[PI(f)] + w[2] * da[PD(f)];
        be[PM(f)] = w[0];
        be[PI(f)] = w[1];
        be[PD(f)] = w[2];
        {
            const float dm = da[PM(f)], di = da[PI(f)], dd = da[PD(f)];
            const float E = w[0] * dm + w[1] * di + w[2] * dd;
            db[PM(f)] = w[0] * (dm - E) / T;
            db[PI(f)] = w[1] * (di - E) / T;
            db[PD(f)] = w[2] * (dd - E) / T;
        }
        FOR_DIAG_REV(L1, L2, i, j) {
            const size_t c = AIDX(i, j);
            const size_t pred[3] = {AIDX(i - 1, j - 1), AIDX(i - 1, j), AIDX(i, j - 1)};
            for (int st = 0; st < 3; ++st) {   /* M (diagonal), I (up), D (left) */
                const float bs = be[st * cstride + c], dbs = db[st * cstride + c];
                if (!(bs > 1e-20f || fabsf(dbs) > 1e-20f)) continue;
                const size_t p = pred[st];
                float x[3];
                if (st == 0) { x[0] = a[PM(p)]; x[1] = a[PI(p)]; x[2] = a[PD(p)]; }
                else if (st == 1) { x[0] = a[PM(p)] + go; x[1] = a[PI(p)] + ge; x[2] = a[PD(p)] + go; }
                else { x[0] = a[PM(p)] + go; x[1] = a[PI(p)] + go; x[2] = a[PD(p)] + ge; }
                if (!(nwa_lse3(x[0], x[1], x[2], T) > NINF)) continue;
                nwa_w3(x[0], x[1], x[2], T, w);
                const float d0 = da[PM(p)], d1 = da[PI(p)], d2 = da[PD(p)];
                const float E = w[0] * d0 + w[1] * d1 + w[2] * d2;
                const float dw[3] = {w[0] * (d0 - E) / T, w[1] * (d1 - E) / T,
                                     w[2] * (d2 - E) / T};
                for (int q = 0; q < 3; ++q) {
                    if (st == 0 && !(x[q] > NINF)) continue;   /* only M checks its inputs */
                    be[q * cstride + p] += bs * w[q];
                    db[q * cstride + p] += dbs * w[q] + bs * dw[q];
                }
                if (st == 0) h[SIDX(i, j)] += dbs;
            }
        }
    }
}

/* nw_affine/kernels_cpu.cpp:619-1002: dP/dtheta for theta = open (0), ext (1) or
 * T (2).  Forward tangents U: boundary chains I(i,0), D(0,j) start at 1 (open) or
 * i-1 / j-1 (ext); each state's candidates carry their direct derivative (open:
 * M->I, D->I, M->D, I->D; ext: I->I, D->D), and for T the state adds
 * (alpha - E_w[v]) / T (M: v includes the score).  Reverse sweep as the HVP's with
 * weight tangents w_k (u_k - E_w[u]) / T (+ w_k (E_w[v] - v_k) / T^2 for T);
 * dP(i, j) = W_M.  dS/dtheta is unused: the terminal betas carry their own
 * tangents. */
void oracle_nwa_param_grad(const float* alpha, const float* scores, const float* score,
                           const float* dS_dtheta, float* U, float* beta, float* W, float* dP,
                           const int* lengths, int B, int maxL1, int maxL2, float go, float ge,
                           float T, int ptype) {
    const size_t cstride = (size_t)(maxL1 + 1) * (maxL2 + 1);
    const size_t astride = 3 * cstride;
    const size_t sstride = (size_t)maxL1 * maxL2;
    const size_t acols = (size_t)maxL2 + 1, scols = (size_t)maxL2;
    (void)score;
    (void)dS_dtheta;
    /* direct derivatives of the candidates (M, I, D predecessors) of I and of D */
    const float dI[3] = {ptype == 0 ? 1.0f : 0.0f, ptype == 1 ? 1.0f : 0.0f,
                         ptype == 0 ? 1.0f : 0.0f};
    const float dD[3] = {ptype == 0 ? 1.0f : 0.0f, ptype == 0 ? 1.0f : 0.0f,
                         ptype == 1 ? 1.0f : 0.0f};
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < B; ++b) {
        const float* a = alpha + (size_t)b * astride;
        const float* s = scores + (size_t)b * sstride;
        float* u = U + (size_t)b * astride;
        float* be = beta + (size_t)b * astride;
        float* wt = W + (size_t)b * astride;
        float* dp = dP + (size_t)b * sstride;
        const int L1 = lengths[2 * b], L2 = lengths[2 * b + 1];
        for (size_t q = 0; q < astride; ++q) { u[q] = 0.0f; be[q] = 0.0f; wt[q] = 0.0f; }
        for (size_t q = 0; q < sstride; ++q) dp[q] = 0.0f;
        if (ptype == 0 || ptype == 1) {
            for (int i = 1; i <= L1; ++i) u[PI(AIDX(i, 0))] = ptype == 0 ? 1.0f : (float)(i - 1);
            for (int j = 1; j <= L2; ++j) u[PD(AIDX(0, j))] = ptype == 0 ? 1.0f : (float)(j - 1);
        }
        float w[3];
        FOR_DIAG_FWD(L1, L2, i, j) {
            const size_t c = AIDX(i, j), cd = AIDX(i - 1, j - 1), cu = AIDX(i - 1, j),
                         cl = AIDX(i, j - 1);
            {
                const float m1 = a[PM(cd)], m2 = a[PI(cd)], m3 = a[PD(cd)];
                if (nwa_lse3(m1, m2, m3, T) > NINF) {
                    nwa_w3(m1, m2, m3, T, w);
                    float x = w[0] * u[PM(cd)] + w[1] * u[PI(cd)] + w[2] * u[PD(cd)];
                    if (ptype == 2) {
                        const float Ev = w[0] * m1 + w[1] * m2 + w[2] * m3;
                        x += (a[PM(c)] - (Ev + s[SIDX(i, j)])) / T;
                    }
                    u[PM(c)] = x;
                }
            }
            {
                const float i1 = a[PM(cu)] + go, i2 = a[PI(cu)] + ge, i3 = a[PD(cu)] + go;
                if (nwa_lse3(i1, i2, i3, T) > NINF) {
                    nwa_w3(i1, i2, i3, T, w);
                    float x = w[0] * (u[PM(cu)] + dI[0]) + w[1] * (u[PI(cu)] + dI[1]) +
                              w[2] * (u[PD(cu)] + dI[2]);
                    if (ptype == 2) {
                        const float Ev = w[0] * i1 + w[1] * i2 + w[2] * i3;
                        x += (a[PI(c)] - Ev) / T;
                    }
                    u[PI(c)] = x;
                }
            }
            {
                const float d1 = a[PM(cl)] + go, d2 = a[PI(cl)] + go, d3 = a[PD(cl)] + ge;
                if (nwa_lse3(d1, d2, d3, T) > NINF) {
                    nwa_w3(d1, d2, d3, T, w);
                    float x = w[0] * (u[PM(cl)] + dD[0]) + w[1] * (u[PI(cl)] + dD[1]) +
                              w[2] * (u[PD(cl)] + dD[2]);
                    if (ptype == 2) {
                        const float Ev = w[0] * d1 + w[1] * d2 + w[2] * d3;
                        x += (a[PD(c)] - Ev) / T;
                    }
                    u[PD(c)] = x;
                }
            }
        }
        const size_t f = AIDX(L1, L2);
        nwa_w3(a[PM(f)], a[PI(f)], a[PD(f)], T, w);
        for (int q = 0; q < 3; ++q) be[q * cstride + f] = w[q];
        {
            const float uk[3] = {u[PM(f)], u[PI(f)], u[PD(f)]};
            const float Eu = w[0] * uk[0] + w[1] * uk[1] + w[2] * uk[2];
            float dw[3];
            for (int q = 0; q < 3; ++q) dw[q] = w[q] * (uk[q] - Eu) / T;
            if (ptype == 2) {
                const float Ev = w[0] * a[PM(f)] + w[1] * a[PI(f)] + w[2] * a[PD(f)];
                const float iT2 = 1.0f / (T * T);
                for (int q = 0; q < 3; ++q) dw[q] += w[q] * (Ev - a[q * cstride + f]) * iT2;
            }
            for (int q = 0; q < 3; ++q) wt[q * cstride + f] = dw[q];
        }
        FOR_DIAG_REV(L1, L2, i, j) {
            const size_t c = AIDX(i, j);
            const size_t pred[3] = {AIDX(i - 1, j - 1), AIDX(i - 1, j), AIDX(i, j - 1)};
            for (int st = 0; st < 3; ++st) {   /* M (diagonal), I (up), D (left) */
                const float bs = be[st * cstride + c], ws = wt[st * cstride + c];
                if (!(bs > 1e-20f || fabsf(ws) > 1e-20f)) continue;
                const size_t p = pred[st];
                float x[3];
                if (st == 0) { x[0] = a[PM(p)]; x[1] = a[PI(p)]; x[2] = a[PD(p)]; }
                else if (st == 1) { x[0] = a[PM(p)] + go; x[1] = a[PI(p)] + ge; x[2] = a[PD(p)] + go; }
                else { x[0] = a[PM(p)] + go; x[1] = a[PI(p)] + go; x[2] = a[PD(p)] + ge; }
                if (!(nwa_lse3(x[0], x[1], x[2], T) > NINF)) continue;
                nwa_w3(x[0], x[1], x[2], T, w);
                float uk[3] = {u[PM(p)], u[PI(p)], u[PD(p)]};
                if (st > 0) {
                    const float* dd = st == 1 ? dI : dD;
                    for (int q = 0; q < 3; ++q) if (dd[q] != 0.0f) uk[q] += 1.0f;
                }
                const float Eu = w[0] * uk[0] + w[1] * uk[1] + w[2] * uk[2];
                float dw[3];
                for (int q = 0; q < 3; ++q) dw[q] = w[q] * (uk[q] - Eu) / T;
                if (ptype == 2) {
                    const float Ev = w[0] * x[0] + w[1] * x[1] + w[2] * x[2];
                    const float iT2 = 1.0f / (T * T);
                    for (int q = 0; q < 3; ++q) dw[q] += w[q] * (Ev - x[q]) * iT2;
                }
                for (int q = 0; q < 3; ++q) {
                    if (st == 0 && !(x[q] > NINF)) continue;   /* only M checks its inputs */
                    be[q * cstride + p] += bs * w[q];
                    wt[q * cstride + p] += ws * w[q] + bs * dw[q];
                }
                if (st == 0) dp[SIDX(i, j)] += ws;
            }
        }
    }
}
