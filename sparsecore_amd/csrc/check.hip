// Device-side PaddedCSR invariant scan (the checks of the reference's
// check_invariants_str, csrc/kernels/padded_csr.cpp:79-196, invariants 3-7).
//
// One thread per row evaluates:
//   invariant 3  row_start[0] == 0, row_start[i] == row_start[i-1] + row_capacity[i-1]
//   invariant 4  0 <= row_nnz[i] <= row_capacity[i]
//   invariant 6  live columns in [0, ncols) and strictly ascending
//   invariant 5+7 padding columns == -1
// and folds the first violation of each kind into one int64 word with an
// atomic minimum (keys: row, or row << 32 | slot-in-row). Slot checks run
// only for rows whose slot range lies inside the arrays, so a malformed
// matrix is reported, never read out of bounds. The host turns the words into
// the reference's error message in the reference's check order.
#include "common.hpp"

namespace slk {
namespace {

constexpr unsigned long long kNone = 0x7fffffffffffffffULL;

__global__ void check_init_kernel(unsigned long long* res) {
    const int t = threadIdx.x;
    if (t < SLK_CHECK_WORDS) res[t] = (t == 0) ? 0ULL : kNone;
}

__global__ __launch_bounds__(256) void check_rows_kernel(
    int64_t M, int64_t ncols, int64_t col_len, const int32_t* __restrict__ row_start,
    const int32_t* __restrict__ row_nnz, const int32_t* __restrict__ row_capacity,
    const int32_t* __restrict__ col, unsigned long long* __restrict__ res) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= M) return;
    const int64_t start = row_start[i];
    const int64_t cap = row_capacity[i];
    const int64_t nnz = row_nnz[i];
    atomicAdd(&res[0], static_cast<unsigned long long>(cap));  // two's complement sum
    // Invariant 3 uses the reference's int32 arithmetic.
    const int32_t expected =
        (i == 0) ? 0 : static_cast<int32_t>(row_start[i - 1] + row_capacity[i - 1]);
    if (static_cast<int32_t>(start) != expected) atomicMin(&res[1], static_cast<unsigned long long>(i));
    if (nnz < 0 || nnz > cap) atomicMin(&res[2], static_cast<unsigned long long>(i));
    if (start < 0 || cap < 0 || nnz < 0 || nnz > cap || start + cap > col_len) return;
    const unsigned long long key = static_cast<unsigned long long>(i) << 32;
    int64_t prev = -1;
    for (int64_t k = 0; k < nnz; ++k) {
        const int64_t c = col[start + k];
        if (c < 0 || c >= ncols || c <= prev) {
            atomicMin(&res[3], key | static_cast<unsigned long long>(k));
            break;
        }
        prev = c;
    }
    for (int64_t k = nnz; k < cap; ++k) {
        if (col[start + k] != -1) {
            atomicMin(&res[4], key | static_cast<unsigned long long>(k));
            break;
        }
    }
}

}  // namespace
}  // namespace slk

extern "C" int slk_check_invariants(const slk_csr* W, int64_t col_indices_len, int64_t* result_dev,
                                    void* stream) {
    using namespace slk;
    clear_error();
    if (W == nullptr || result_dev == nullptr) return fail(SLK_EINVAL, "check: NULL argument");
    if (W->nrows < 0 || W->ncols < 0 || col_indices_len < 0) {
        return fail(SLK_EINVAL, "check: negative size");
    }
    if (W->nrows > 0 && (W->row_start == nullptr || W->row_nnz == nullptr ||
                         W->row_capacity == nullptr)) {
        return fail(SLK_EINVAL, "check: NULL row array");
    }
    if (W->nrows >= (int64_t{1} << 31)) return fail(SLK_EINVAL, "check: too many rows");
    hipStream_t st = as_stream(stream);
    auto* res = reinterpret_cast<unsigned long long*>(result_dev);
    hipLaunchKernelGGL(check_init_kernel, dim3(1), dim3(64), 0, st, res);
    if (int rc = check_launch("check/init")) return rc;
    if (W->nrows == 0) return SLK_OK;
    hipLaunchKernelGGL(check_rows_kernel, dim3(static_cast<unsigned>(ceil_div(W->nrows, 256))),
                       dim3(256), 0, st, W->nrows, W->ncols, col_indices_len, W->row_start,
                       W->row_nnz, W->row_capacity, W->col_indices, res);
    return check_launch("check/rows");
}
