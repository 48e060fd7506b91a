// Weight gradient on live slots (SDDMM):  dW[s] = dot(dY[i,:], X[c_s,:]),
// dW[padding] = 0, for a padded-CSR W (gfx950).
//
// Two summation orders, each reproducing one reference kernel bit for bit:
//
//  * SIMD order — csrc/kernels/spmm_grad_avx2.cpp:112-258. The AVX2 kernel
//    keeps 16 running partial sums ("virtual lanes") v[0..15]: v[l] is the
//    fma chain over j = 16t + l for the full 16-wide steps t. It then forms
//    a[l] = v[l] + v[l+8] (l < 8), applies one 8-wide fma step when 8..15
//    elements remain, reduces a[0..7] as ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)),
//    and finishes the last 0..7 elements with a scalar running sum.
//    Here four lanes own one slot; lane q holds virtual lanes 4q..4q+3 and
//    reads them with one 16-byte load per step, so a wave works on 16 slots
//    at once. The combine steps are cross-lane exchanges (xor 2, then xor 1).
//
//  * scalar order — csrc/kernels/spmm_grad.cpp:89-108: one running sum over
//    j = 0..N-1. One lane per slot; used only for kernel="scalar".
//
// Scalar running sums `acc += a[j] * b[j]` are evaluated the way the
// reference's x86 build (g++ -O3 -march=x86-64-v3) evaluates them: products
// of whole 4-element groups are rounded and added one at a time in order,
// and only the final n mod 4 terms are fused multiply-adds (running_sum()).
//
// Work decomposition: slots are addressed in the flat capacity space
// [0, total_capacity), which the padded rows tile contiguously, so every
// wave owns the same number of slots no matter how skewed row lengths are.
// A slot finds its row by binary search over row_start; padding slots
// (slot-in-row >= row_nnz) are written as 0 by the lane that owns them, so
// dW needs no separate memset.
#include "common.hpp"

namespace slk {
namespace {

constexpr int kBlock = 256;
constexpr int kSlotsPerWave = 16;  // SIMD order: 4 lanes per slot

// Largest r in [0, M) with row_start[r] <= slot (rows tile [0, cap)).
__device__ __forceinline__ int64_t row_of_slot(const int32_t* __restrict__ row_start, int64_t M,
                                               int64_t slot) {
    int64_t lo = 0, hi = M;  // invariant: row_start[lo] <= slot < row_start[hi] (hi == M: +inf)
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (row_start[mid] <= slot) lo = mid; else hi = mid;
    }
    return lo;
}

// acc += a[j] * b[j] for j < n: unfused in-order adds for the first
// 4*floor(n/4) terms, fused multiply-adds for the rest.
__device__ __forceinline__ float running_sum(const float* __restrict__ a,
                                             const float* __restrict__ b, int64_t n, float acc) {
    const int64_t n4 = n & ~int64_t{3};
    int64_t j = 0;
    for (; j < n4; ++j) {
        const float p = a[j] * b[j];
        acc = acc + p;
    }
    for (; j < n; ++j) acc = __builtin_fmaf(a[j], b[j], acc);
    return acc;
}

template <bool V4>
__device__ __forceinline__ void load4(const float* p, float& a, float& b, float& c, float& d) {
    if constexpr (V4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(p);
        a = v[0]; b = v[1]; c = v[2]; d = v[3];
    } else {
        a = p[0]; b = p[1]; c = p[2]; d = p[3];
    }
}

template <bool V4>
__global__ __launch_bounds__(kBlock) void sddmm_simd_kernel(
    int64_t M, int64_t N, int64_t cap_total,
    const int32_t* __restrict__ row_start, const int32_t* __restrict__ row_nnz,
    const int32_t* __restrict__ col, const float* __restrict__ dY,
    const float* __restrict__ X, float* __restrict__ dW) {
    const int lane = threadIdx.x & (kWave - 1);
    const int g = lane >> 2;  // slot within the wave
    const int q = lane & 3;   // owns virtual lanes 4q..4q+3
    const int64_t slot = wave_id() * kSlotsPerWave + g;
    const bool in_range = slot < cap_total;

    int64_t row = 0;
    bool live = false;
    int32_t c = 0;
    if (in_range) {
        row = row_of_slot(row_start, M, slot);
        live = (slot - row_start[row]) < row_nnz[row];
        if (live) c = col[slot];
    }
    // Every lane reaches the cross-lane exchanges below; only lanes of live
    // slots touch X and dY, so padding / out-of-range lanes never load.
    const float* dyr = dY + (live ? row * N : 0);
    const float* xr = X + (live ? static_cast<int64_t>(c) * N : 0);
    const int64_t n16 = (N / 16) * 16;

    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    if (live) {
        int64_t j = 4 * q;
#pragma unroll 4
        for (; j < n16; j += 16) {
            float d0, d1, d2, d3, x0, x1, x2, x3;
            load4<V4>(dyr + j, d0, d1, d2, d3);
            load4<V4>(xr + j, x0, x1, x2, x3);
            a0 = __builtin_fmaf(d0, x0, a0);
            a1 = __builtin_fmaf(d1, x1, a1);
            a2 = __builtin_fmaf(d2, x2, a2);
            a3 = __builtin_fmaf(d3, x3, a3);
        }
    }
    // a[l] = v[l] + v[l+8]: lanes q=0,1 take the partner q^2 (v[8..15]).
    {
        const float p0 = __shfl_xor(a0, 2), p1 = __shfl_xor(a1, 2);
        const float p2 = __shfl_xor(a2, 2), p3 = __shfl_xor(a3, 2);
        a0 = a0 + p0; a1 = a1 + p1; a2 = a2 + p2; a3 = a3 + p3;
    }
    int64_t jt = n16;
    if (N - n16 >= 8) {
        if (live && q < 2) {
            float d0, d1, d2, d3, x0, x1, x2, x3;
            const int64_t j = n16 + 4 * q;
            load4<V4>(dyr + j, d0, d1, d2, d3);
            load4<V4>(xr + j, x0, x1, x2, x3);
            a0 = __builtin_fmaf(d0, x0, a0);
            a1 = __builtin_fmaf(d1, x1, a1);
            a2 = __builtin_fmaf(d2, x2, a2);
            a3 = __builtin_fmaf(d3, x3, a3);
        }
        jt += 8;
    }
    // s4[k] = a[k] + a[k+4]: lane q=0 holds a[0..3], lane q=1 holds a[4..7].
    {
        const float p0 = __shfl_xor(a0, 1), p1 = __shfl_xor(a1, 1);
        const float p2 = __shfl_xor(a2, 1), p3 = __shfl_xor(a3, 1);
        a0 = a0 + p0; a1 = a1 + p1; a2 = a2 + p2; a3 = a3 + p3;
    }
    if (in_range && q == 0) {
        float r = (a0 + a2) + (a1 + a3);
        if (live) {
            dW[slot] = running_sum(dyr + jt, xr + jt, N - jt, r);
        } else {
            dW[slot] = 0.0f;
        }
    }
}

__global__ __launch_bounds__(kBlock) void sddmm_scalar_kernel(
    int64_t M, int64_t N, int64_t cap_total,
    const int32_t* __restrict__ row_start, const int32_t* __restrict__ row_nnz,
    const int32_t* __restrict__ col, const float* __restrict__ dY,
    const float* __restrict__ X, float* __restrict__ dW) {
    const int64_t slot = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (slot >= cap_total) return;
    const int64_t row = row_of_slot(row_start, M, slot);
    if (slot - row_start[row] >= row_nnz[row]) {
        dW[slot] = 0.0f;
        return;
    }
    const float* dyr = dY + row * N;
    const float* xr = X + static_cast<int64_t>(col[slot]) * N;
    dW[slot] = running_sum(dyr, xr, N, 0.0f);
}

}  // namespace
}  // namespace slk

extern "C" int slk_sddmm(const slk_csr* W, const float* dY, int64_t dY_rows, const float* X,
                         int64_t X_rows, int64_t N, float* dW, int order, void* stream) {
    using namespace slk;
    clear_error();
    const char* who = order == SLK_DW_SCALAR ? "spmm_grad_w" : "spmm_grad_w_simd";
    if (int rc = validate_csr(W, who)) return rc;
    if (order != SLK_DW_SIMD && order != SLK_DW_SCALAR) {
        return fail(SLK_EINVAL, std::string(who) + ": unknown order " + std::to_string(order));
    }
    if (dY_rows != W->nrows) {
        return fail(SLK_EINVAL, std::string(who) + ": dY.shape[0]=" + std::to_string(dY_rows) +
                                    " but W.nrows=" + std::to_string(W->nrows) +
                                    ". dY must have the same row count as W.");
    }
    if (X_rows != W->ncols) {
        return fail(SLK_EINVAL, std::string(who) + ": X.shape[0]=" + std::to_string(X_rows) +
                                    " but W.ncols=" + std::to_string(W->ncols) +
                                    ". X must have the same row count as W has columns.");
    }
    if (N < 0) return fail(SLK_EINVAL, std::string(who) + ": negative N");
    const int64_t cap = W->total_capacity;
    if (cap == 0) return SLK_OK;
    if (dW == nullptr) return fail(SLK_EINVAL, std::string(who) + ": NULL dW");
    hipStream_t st = as_stream(stream);
    if (order == SLK_DW_SCALAR) {
        const int64_t blocks = ceil_div(cap, kBlock);
        hipLaunchKernelGGL(sddmm_scalar_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kBlock),
                           0, st, W->nrows, N, cap, W->row_start, W->row_nnz, W->col_indices, dY,
                           X, dW);
        return check_launch(who);
    }
    const int64_t waves = ceil_div(cap, kSlotsPerWave);
    const int64_t blocks = ceil_div(waves, kBlock / kWave);
    const bool v4 = (N % 4 == 0) && (reinterpret_cast<uintptr_t>(X) % 16 == 0) &&
                    (reinterpret_cast<uintptr_t>(dY) % 16 == 0);
    if (v4) {
        hipLaunchKernelGGL(sddmm_simd_kernel<true>, dim3(static_cast<unsigned>(blocks)),
                           dim3(kBlock), 0, st, W->nrows, N, cap, W->row_start, W->row_nnz,
                           W->col_indices, dY, X, dW);
    } else {
        hipLaunchKernelGGL(sddmm_simd_kernel<false>, dim3(static_cast<unsigned>(blocks)),
                           dim3(kBlock), 0, st, W->nrows, N, cap, W->row_start, W->row_nnz,
                           W->col_indices, dY, X, dW);
    }
    return check_launch(who);
}
