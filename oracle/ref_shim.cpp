// ref_shim.cpp — extern "C" entry points over the reference's own CPU kernels.
//
// TEST INFRASTRUCTURE ONLY. Compiled by oracle/Makefile together with the
// reference sources where they lie (csrc/kernels/*.cpp under the reference
// checkout), into oracle/_ref/libslref.so. It lets tests and bench.py's
// cpu_baseline leg run the reference's AVX2/OpenMP kernels unchanged on the
// host. This file holds no kernel code: it only builds a
// sparselab::PaddedCSR from raw arrays (csrc/kernels/padded_csr.hpp:47-99)
// and forwards to the reference functions.
#include <cstdint>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

#include "dense_grad.hpp"
#include "padded_csr.hpp"
#include "spmm.hpp"
#include "spmm_avx2.hpp"
#include "spmm_grad.hpp"
#include "spmm_grad_avx2.hpp"

#define REF_API extern "C" __attribute__((visibility("default")))

namespace {
thread_local std::string g_err;

template <typename F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 1;
    }
}
}  // namespace

REF_API const char* ref_last_error() { return g_err.c_str(); }

// Builds a PaddedCSR by copying the arrays (no validation: call
// ref_check_invariants for that). Returns NULL and sets the error on failure.
REF_API void* ref_csr_new(int64_t nrows, int64_t ncols, int64_t cap, const float* values,
                          const int32_t* col, const int32_t* row_start, const int32_t* row_nnz,
                          const int32_t* row_capacity) {
    sparselab::PaddedCSR* p = nullptr;
    const int rc = guarded([&] {
        p = new sparselab::PaddedCSR(
            nrows, ncols, std::vector<float>(values, values + cap),
            std::vector<int32_t>(col, col + cap),
            std::vector<int32_t>(row_start, row_start + nrows),
            std::vector<int32_t>(row_nnz, row_nnz + nrows),
            std::vector<int32_t>(row_capacity, row_capacity + nrows));
    });
    return rc == 0 ? p : nullptr;
}

REF_API void ref_csr_free(void* p) { delete static_cast<sparselab::PaddedCSR*>(p); }

// Reference invariant checker (csrc/kernels/padded_csr.cpp:79-196). Copies
// the message (empty if valid) into buf.
REF_API void ref_check_invariants(void* p, char* buf, int64_t buflen) {
    const std::string s = sparselab::check_invariants_str(*static_cast<sparselab::PaddedCSR*>(p));
    if (buflen > 0) {
        std::strncpy(buf, s.c_str(), static_cast<size_t>(buflen - 1));
        buf[buflen - 1] = '\0';
    }
}

REF_API int ref_spmm_simd(void* p, const float* X, int64_t K, int64_t N, float* Y) {
    return guarded([&] {
        sparselab::spmm_simd_avx2(*static_cast<sparselab::PaddedCSR*>(p), X, K, N, Y);
    });
}

REF_API int ref_spmm_scalar(void* p, const float* X, int64_t K, int64_t N, float* Y) {
    return guarded(
        [&] { sparselab::spmm_scalar(*static_cast<sparselab::PaddedCSR*>(p), X, K, N, Y); });
}

REF_API int ref_spmm_grad_w_simd(void* p, const float* dY, int64_t N, const float* X, int64_t K,
                                 float* dW) {
    return guarded([&] {
        sparselab::spmm_grad_w_simd(*static_cast<sparselab::PaddedCSR*>(p), dY, N, X, K, dW);
    });
}

REF_API int ref_spmm_grad_w(void* p, const float* dY, int64_t N, const float* X, int64_t K,
                            float* dW) {
    return guarded([&] {
        sparselab::spmm_grad_w(*static_cast<sparselab::PaddedCSR*>(p), dY, N, X, K, dW);
    });
}

REF_API int ref_dense_grad(int64_t M, int64_t K, int64_t N, const float* dY, const float* X,
                           float* G) {
    return guarded([&] { sparselab::dense_grad(M, K, N, dY, X, G); });
}

REF_API int ref_rewrite_row(void* p, int64_t row, int64_t n, const int32_t* cols,
                            const float* vals) {
    return guarded([&] {
        static_cast<sparselab::PaddedCSR*>(p)->rewrite_row(
            row, std::vector<int32_t>(cols, cols + n), std::vector<float>(vals, vals + n));
    });
}

// Address of p's own values buffer (what the reference exposes as the
// writable zero-copy `values` view, csrc/bindings.cpp:663-666).
REF_API float* ref_csr_values_ptr(void* p) {
    return static_cast<sparselab::PaddedCSR*>(p)->values.data();
}

// Copies the current arrays of p out (after rewrite_row).
REF_API void ref_csr_arrays(void* p, float* values, int32_t* col, int32_t* row_nnz,
                            int64_t* topology_version) {
    const auto& c = *static_cast<sparselab::PaddedCSR*>(p);
    std::memcpy(values, c.values.data(), c.values.size() * sizeof(float));
    std::memcpy(col, c.col_indices.data(), c.col_indices.size() * sizeof(int32_t));
    std::memcpy(row_nnz, c.row_nnz.data(), c.row_nnz.size() * sizeof(int32_t));
    *topology_version = c.topology_version;
}
