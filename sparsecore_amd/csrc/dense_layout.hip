// Dense layout change used around the padded-CSR kernels: a float32 matrix
// transpose. SparseLinear takes activations token-major (N x K) while the
// kernels read them feature-major (K x N) — the `x.t().contiguous()` of
// sparselab/nn.py:235 and the `dY.contiguous()` of sparselab/ops.py:174.
//
// 32 x 32 tiles through LDS (one padding column, so the transposed read is
// free of bank conflicts); loads and stores are both row-contiguous. The
// result is a bitwise copy.
#include "common.hpp"

namespace slk {
namespace {

constexpr int kTile = 32;
constexpr int kTileRowsPerPass = 8;  // 256 threads = 32 x 8

__global__ __launch_bounds__(kTile * kTileRowsPerPass) void transpose_f32_kernel(
    const float* __restrict__ src, int64_t rows, int64_t cols, int64_t ld_src,
    float* __restrict__ dst, int64_t col_tiles) {
    __shared__ float tile[kTile][kTile + 1];
    const int64_t bt = blockIdx.x;
    const int64_t r0 = (bt / col_tiles) * kTile;
    const int64_t c0 = (bt % col_tiles) * kTile;
    const int tx = threadIdx.x & (kTile - 1);
    const int ty = threadIdx.x / kTile;
    // all loads unconditional at clamped (in-bounds) indices so they are in
    // flight together; guarded loads were each waited on before the next
    float v[kTile / kTileRowsPerPass];
#pragma unroll
    for (int i = 0; i < kTile; i += kTileRowsPerPass) {
        const int64_t r = r0 + ty + i, c = c0 + tx;
        const int64_t rc = r < rows ? r : rows - 1, cc = c < cols ? c : cols - 1;
        v[i / kTileRowsPerPass] = src[rc * ld_src + cc];
    }
#pragma unroll
    for (int i = 0; i < kTile; i += kTileRowsPerPass) {
        const int64_t r = r0 + ty + i, c = c0 + tx;
        if (r < rows && c < cols) tile[ty + i][tx] = v[i / kTileRowsPerPass];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kTile; i += kTileRowsPerPass) {
        const int64_t c = c0 + ty + i, r = r0 + tx;  // dst row c, column r
        if (c < cols && r < rows) dst[c * rows + r] = tile[tx][ty + i];
    }
}

}  // namespace
}  // namespace slk

extern "C" int slk_transpose_dense(const float* src, int64_t rows, int64_t cols, int64_t ld_src,
                                   float* dst, void* stream) {
    using namespace slk;
    clear_error();
    if (rows < 0 || cols < 0) return fail(SLK_EINVAL, "transpose_dense: negative shape");
    if (rows == 0 || cols == 0) return SLK_OK;
    if (ld_src < cols) {
        return fail(SLK_EINVAL, "transpose_dense: ld_src=" + std::to_string(ld_src) +
                                    " is smaller than cols=" + std::to_string(cols));
    }
    if (src == nullptr || dst == nullptr) return fail(SLK_EINVAL, "transpose_dense: NULL pointer");
    const int64_t col_tiles = ceil_div(cols, kTile);
    const int64_t blocks = ceil_div(rows, kTile) * col_tiles;
    if (blocks > INT32_MAX) return fail(SLK_EINVAL, "transpose_dense: matrix too large");
    hipLaunchKernelGGL(transpose_f32_kernel, dim3(static_cast<unsigned>(blocks)),
                       dim3(kTile * kTileRowsPerPass), 0, as_stream(stream), src, rows, cols,
                       ld_src, dst, col_tiles);
    return check_launch("transpose_dense");
}
