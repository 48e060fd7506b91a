/*
 * oracle.c — CPU restatement of the reference's padded-CSR kernels.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the GPU path is
 * compared against (tests/, __graft_entry__.smoke(), bench.py's
 * cpu_baseline leg). Nothing in the sparsecore_amd product imports, links
 * or calls it.
 *
 * Each function restates one reference kernel's arithmetic, in the same
 * order, so that results are bit-identical to the reference built with
 * g++ -O3 -march=x86-64-v3 -fopenmp (its setup.py flags):
 *
 *   orc_spmm          csrc/kernels/spmm_avx2.cpp:123-262 (and spmm.cpp:84-104):
 *                     Y zeroed, then for i, for live slot s in order,
 *                     y[i,j] = fma(v_s, X[c_s,j], y[i,j]) for all j.
 *   orc_sddmm_simd    csrc/kernels/spmm_grad_avx2.cpp:108-258: per slot,
 *                     two 8-lane accumulators over 16-wide steps, their
 *                     lane-wise sum, one 8-wide step if 8..15 remain, the
 *                     128/64/32-bit horizontal add tree, then the scalar
 *                     tail (fold_tail below).
 *   orc_sddmm_scalar  csrc/kernels/spmm_grad.cpp:85-108: one running sum.
 *   orc_dense_grad    csrc/kernels/dense_grad.cpp:57-83: G = dY·X^T, one
 *                     running sum per element.
 *   orc_fmaf          out[i] = fmaf(a[i], b[i], c[i]) from libm (correctly
 *                     rounded): the reference's per-slot fma, elementwise,
 *                     for tests of the device's fma-equivalent instructions.
 *
 * Scalar running sums `acc += a[j] * b[j]` (the AVX2 kernel's 0..7-element
 * tail and the whole scalar kernels) are not one fma chain in the reference
 * build: g++ vectorizes the products of each 8- and then 4-element block and
 * adds them to acc one by one in order (product rounded, then sum rounded),
 * and contracts only the last n mod 4 terms into scalar fmas. fold_tail()
 * restates exactly that: unfused in-order adds for the first 4*floor(n/4)
 * terms, fmas for the rest. (Read off the x86 code g++ 11 emits for
 * csrc/kernels/spmm_grad{,_avx2}.cpp and dense_grad.cpp at the reference's
 * flags; checked bit-for-bit against that build in tests.)
 *
 * Threading follows csrc/kernels/parallel.hpp:35-49: OpenMP static schedule
 * over rows, serial below 32 rows. `nthreads` <= 0 keeps the OpenMP default.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <omp.h>

#define ORC_ROW_THRESHOLD 32

static int orc_threads(int nthreads) {
    return nthreads > 0 ? nthreads : omp_get_max_threads();
}

void orc_spmm(int64_t M, const int32_t* row_start, const int32_t* row_nnz,
              const int32_t* col, const float* val, const float* X, int64_t K,
              int64_t N, float* Y, int nthreads) {
    (void)K;
    memset(Y, 0, (size_t)M * (size_t)N * sizeof(float));
    if (M == 0 || N == 0 || K == 0) return;
#pragma omp parallel for schedule(static) if (M >= ORC_ROW_THRESHOLD) \
    num_threads(orc_threads(nthreads))
    for (int64_t i = 0; i < M; ++i) {
        float* y = Y + i * N;
        const int32_t base = row_start[i];
        for (int32_t s = 0; s < row_nnz[i]; ++s) {
            const float v = val[base + s];
            const float* x = X + (int64_t)col[base + s] * N;
            for (int64_t j = 0; j < N; ++j) y[j] = fmaf(v, x[j], y[j]);
        }
    }
}

/* acc += a[j] * b[j] for j < n, as the reference build evaluates it. */
static float fold_tail(const float* a, const float* b, int64_t n, float acc) {
    const int64_t n4 = n & ~(int64_t)3;
    int64_t j = 0;
    for (; j < n4; ++j) {
        const float p = a[j] * b[j];
        acc = acc + p;
    }
    for (; j < n; ++j) acc = fmaf(a[j], b[j], acc);
    return acc;
}

static float dot_avx2_order(const float* dy, const float* x, int64_t N) {
    /* lane[l] for l < 8 is acc_a lane l, lane[8 + l] is acc_b lane l. */
    float lane[16];
    for (int l = 0; l < 16; ++l) lane[l] = 0.0f;
    int64_t j = 0;
    for (; j + 16 <= N; j += 16)
        for (int l = 0; l < 16; ++l) lane[l] = fmaf(dy[j + l], x[j + l], lane[l]);
    float acc[8];
    for (int l = 0; l < 8; ++l) acc[l] = lane[l] + lane[8 + l];
    if (j + 8 <= N) {
        for (int l = 0; l < 8; ++l) acc[l] = fmaf(dy[j + l], x[j + l], acc[l]);
        j += 8;
    }
    float s4[4];
    for (int k = 0; k < 4; ++k) s4[k] = acc[k] + acc[k + 4];
    const float s2_0 = s4[0] + s4[2];
    const float s2_1 = s4[1] + s4[3];
    return fold_tail(dy + j, x + j, N - j, s2_0 + s2_1);
}

static float dot_sequential(const float* dy, const float* x, int64_t N) {
    return fold_tail(dy, x, N, 0.0f);
}

static void sddmm_impl(int64_t M, const int32_t* row_start, const int32_t* row_nnz,
                       const int32_t* col, int64_t cap_total, const float* dY,
                       const float* X, int64_t K, int64_t N, float* dW, int nthreads,
                       int simd) {
    memset(dW, 0, (size_t)cap_total * sizeof(float));
    if (M == 0 || N == 0 || K == 0 || cap_total == 0) return;
#pragma omp parallel for schedule(static) if (M >= ORC_ROW_THRESHOLD) \
    num_threads(orc_threads(nthreads))
    for (int64_t i = 0; i < M; ++i) {
        const float* dy = dY + i * N;
        const int32_t base = row_start[i];
        for (int32_t s = 0; s < row_nnz[i]; ++s) {
            const float* x = X + (int64_t)col[base + s] * N;
            dW[base + s] = simd ? dot_avx2_order(dy, x, N) : dot_sequential(dy, x, N);
        }
    }
}

void orc_sddmm_simd(int64_t M, const int32_t* row_start, const int32_t* row_nnz,
                    const int32_t* col, int64_t cap_total, const float* dY,
                    const float* X, int64_t K, int64_t N, float* dW, int nthreads) {
    sddmm_impl(M, row_start, row_nnz, col, cap_total, dY, X, K, N, dW, nthreads, 1);
}

void orc_sddmm_scalar(int64_t M, const int32_t* row_start, const int32_t* row_nnz,
                      const int32_t* col, int64_t cap_total, const float* dY,
                      const float* X, int64_t K, int64_t N, float* dW, int nthreads) {
    sddmm_impl(M, row_start, row_nnz, col, cap_total, dY, X, K, N, dW, nthreads, 0);
}

void orc_dense_grad(int64_t M, int64_t K, int64_t N, const float* dY, const float* X,
                    float* G, int nthreads) {
    memset(G, 0, (size_t)M * (size_t)K * sizeof(float));
    if (M == 0 || K == 0 || N == 0) return;
#pragma omp parallel for schedule(static) if (M >= ORC_ROW_THRESHOLD) \
    num_threads(orc_threads(nthreads))
    for (int64_t i = 0; i < M; ++i)
        for (int64_t k = 0; k < K; ++k) G[i * K + k] = dot_sequential(dY + i * N, X + k * N, N);
}

void orc_fmaf(int64_t n, const float* a, const float* b, const float* c, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = fmaf(a[i], b[i], c[i]);
}
