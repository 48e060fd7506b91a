// Dense rows of a padded-CSR product on the matrix cores (dense_rows.hip).
#pragma once

#include "common.hpp"

namespace slk {

// Bytes of slk_csr.dense_ws for T dense rows of a K-column matrix.
int64_t dense_rows_workspace_bytes(int64_t T, int64_t K);

// Whether T dense rows of a K-column matrix times a K x N X fit the dense
// kernel's 32-bit lane offsets.
bool dense_rows_apply(int64_t T, int64_t K, int64_t N);

// Y rows order[0 .. W->n_dense_rows) of Y = W·X (+ bias) on the matrix cores,
// bit-equal to the slot-order chain; three launches on st, no host sync.
int spmm_dense_rows(const slk_csr* W, const float* X, int64_t K, int64_t N, const float* bias,
                    float* Y, hipStream_t st);

// Whether slk_sddmm's dense-row kernel takes T dense rows of an M x K matrix
// at this N (SIMD order): N a multiple of 64 (whole staged column blocks).
bool dense_dw_apply(int64_t T, int64_t M, int64_t K, int64_t N);

// dW on the live slots of rows order[0 .. W->n_dense_rows) in the reference's
// SIMD order, on the matrix cores (two launches on st; padding slots and
// dbias are left to the caller's other launch).
int sddmm_dense_rows(const slk_csr* W, const float* dY, const float* X, int64_t N, float* dW,
                     hipStream_t st);

}  // namespace slk
