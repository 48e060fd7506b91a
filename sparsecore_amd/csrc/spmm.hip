// Forward SpMM  Y = W·X  for a padded-CSR W (gfx950).
//
// Reference semantics (csrc/kernels/spmm_avx2.cpp:123-262, spmm.cpp:84-104):
// Y is zeroed, then for every row i and live slot s (in slot order) the
// write-through update  y[i,j] = fma(v_s, X[c_s, j], y[i,j])  is applied to
// all j. Every output element is therefore an ordered fused multiply-add
// chain starting at +0.0. This kernel evaluates exactly that chain per
// element, so results are bit-identical to the reference CPU kernels.
//
// Work decomposition: one "item" is (row, column tile). A tile is L lanes
// of VEC consecutive columns; a 64-wide wave holds 64/L items. Items are
// ordered tile-major (item = tile * M + row) so that waves resident at the
// same time gather from the same K x (L*VEC) slab of X, which stays in L2.
// With L = 64 the item is wave-uniform, the row metadata and the (col, value)
// stream are read through the scalar cache, and each slot costs one
// coalesced VEC*64-float gather of an X row segment.
#include "common.hpp"

#include <cstdlib>

namespace slk {
namespace {

constexpr int kSpmmBlock = 256;  // 4 waves per workgroup
constexpr int kUnroll = 8;       // slots whose X gathers are in flight together

template <int VEC>
struct VecIO;

template <>
struct VecIO<4> {
    typedef f32x4 T;
    static __device__ __forceinline__ T load(const float* p) {
        return *reinterpret_cast<const f32x4*>(p);
    }
    static __device__ __forceinline__ void store(float* p, const float* a) {
        f32x4 v = {a[0], a[1], a[2], a[3]};
        *reinterpret_cast<f32x4*>(p) = v;
    }
    static __device__ __forceinline__ float get(const T& v, int k) { return v[k]; }
};

template <>
struct VecIO<1> {
    typedef float T;
    static __device__ __forceinline__ T load(const float* p) { return *p; }
    static __device__ __forceinline__ void store(float* p, const float* a) { *p = a[0]; }
    static __device__ __forceinline__ float get(const T& v, int) { return v; }
};

template <int L, int VEC>
__global__ __launch_bounds__(kSpmmBlock) void spmm_kernel(
    int64_t M, int64_t N, int64_t nitems,
    const int32_t* __restrict__ row_start, const int32_t* __restrict__ row_nnz,
    const int32_t* __restrict__ col, const float* __restrict__ val,
    const float* __restrict__ X, float* __restrict__ Y) {
    typedef VecIO<VEC> IO;
    constexpr int kItemsPerWave = kWave / L;
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t item = wave_id() * kItemsPerWave + lane / L;
    if (item >= nitems) return;  // no barriers below: early exit is safe
    const int64_t tile = item / M;
    const int64_t row = item - tile * M;
    const int64_t n0 = (tile * L + (lane % L)) * VEC;
    const bool active = n0 < N;  // N % VEC == 0 when VEC > 1, so n0 + VEC <= N

    const int32_t start = row_start[row];
    const int32_t nnz = row_nnz[row];
    const int32_t* c_ptr = col + start;
    const float* v_ptr = val + start;
    const float* xb = X + n0;

    float acc[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) acc[k] = 0.0f;

    int32_t s = 0;
    for (; s + kUnroll <= nnz; s += kUnroll) {
        int32_t c[kUnroll];
        float v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            c[u] = c_ptr[s + u];
            v[u] = v_ptr[s + u];
        }
        typename IO::T x[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            if (active) x[u] = IO::load(xb + static_cast<int64_t>(c[u]) * N);
        }
        if (active) {
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
                for (int k = 0; k < VEC; ++k) acc[k] = __builtin_fmaf(v[u], IO::get(x[u], k), acc[k]);
            }
        }
    }
    for (; s < nnz; ++s) {
        const int32_t c = c_ptr[s];
        const float v = v_ptr[s];
        if (active) {
            const typename IO::T x = IO::load(xb + static_cast<int64_t>(c) * N);
#pragma unroll
            for (int k = 0; k < VEC; ++k) acc[k] = __builtin_fmaf(v, IO::get(x, k), acc[k]);
        }
    }
    if (active) IO::store(Y + row * N + n0, acc);
}

template <int L, int VEC>
int launch(const slk_csr* W, const float* X, int64_t N, float* Y, hipStream_t st) {
    const int64_t M = W->nrows;
    const int64_t tiles = ceil_div(N, static_cast<int64_t>(L) * VEC);
    const int64_t nitems = M * tiles;
    const int64_t waves = ceil_div(nitems, kWave / L);
    const int64_t blocks = ceil_div(waves, kSpmmBlock / kWave);
    if (blocks > INT32_MAX) return fail(SLK_EINVAL, "spmm: problem too large for one launch");
    hipLaunchKernelGGL((spmm_kernel<L, VEC>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kSpmmBlock), 0, st, M, N, nitems, W->row_start, W->row_nnz,
                       W->col_indices, W->values, X, Y);
    return check_launch("spmm");
}

template <int VEC>
int dispatch_L(int L, const slk_csr* W, const float* X, int64_t N, float* Y, hipStream_t st) {
    switch (L) {
        case 1: return launch<1, VEC>(W, X, N, Y, st);
        case 2: return launch<2, VEC>(W, X, N, Y, st);
        case 4: return launch<4, VEC>(W, X, N, Y, st);
        case 8: return launch<8, VEC>(W, X, N, Y, st);
        case 16: return launch<16, VEC>(W, X, N, Y, st);
        case 32: return launch<32, VEC>(W, X, N, Y, st);
        default: return launch<64, VEC>(W, X, N, Y, st);
    }
}

// Lanes per item: the smallest power of two whose tile covers the row
// (capped at a full wave), unless SLK_SPMM_LANES overrides it.
int pick_lanes(int64_t N, int vec) {
    if (const char* e = std::getenv("SLK_SPMM_LANES")) {
        const int v = std::atoi(e);
        if (v == 1 || v == 2 || v == 4 || v == 8 || v == 16 || v == 32 || v == 64) return v;
    }
    const int64_t need = ceil_div(N, vec);
    int L = 1;
    while (L < kWave && L < need) L <<= 1;
    return L;
}

}  // namespace
}  // namespace slk

extern "C" int slk_spmm(const slk_csr* W, const float* X, int64_t K, int64_t N, float* Y,
                        void* stream) {
    using namespace slk;
    clear_error();
    if (int rc = validate_csr(W, "spmm")) return rc;
    if (N < 0 || K < 0) return fail(SLK_EINVAL, "spmm: negative X shape");
    if (W->ncols != K) {
        return fail(SLK_EINVAL, "spmm: shape mismatch. W has ncols=" + std::to_string(W->ncols) +
                                    " but X has shape[0]=" + std::to_string(K) +
                                    ". Inner dimensions must match for matmul.");
    }
    if (W->nrows == 0 || N == 0) return SLK_OK;
    if (Y == nullptr || (K > 0 && X == nullptr)) return fail(SLK_EINVAL, "spmm: NULL X or Y");
    const bool v4 = (N % 4 == 0) && (reinterpret_cast<uintptr_t>(X) % 16 == 0) &&
                    (reinterpret_cast<uintptr_t>(Y) % 16 == 0);
    hipStream_t st = as_stream(stream);
    if (v4) return dispatch_L<4>(pick_lanes(N, 4), W, X, N, Y, st);
    return dispatch_L<1>(pick_lanes(N, 1), W, X, N, Y, st);
}
