// Backward of a narrow SparseLinear layer — W with at most 64 rows, such as
// a classifier head — in one launch, from the output gradient in the layout
// torch's autograd hands back for y = x·Wᵀ: token-major dYt (N x M,
// dY[i, n] = dYt[n·M + i]). It computes dW on the live slots, the bias
// gradient and dX = Wᵀ·dY, each bit-identical to the general path
// (slk_sddmm_bias, and slk_spmm on the transpose slk_transpose_fill builds),
// without that path's layout copy of dY, transpose-cache refresh and second
// launch — on a layer this small each of those costs more than its work.
//
// Three kinds of waves share the grid; a role is uniform per workgroup (dX)
// or per wave (dW, bias), so no barrier is divergent:
//  * dX workgroups come first. Each stages W's slots (column, value) and row
//    bounds in LDS, then every wave takes items (column c, n tile of 64·VEC):
//    lane m binary-searches row m of the staged W for column c, a ballot
//    lists the rows that hold c in ascending order, and each lane runs the
//    chain dX[c, n] = fma(W[m, c], dY[m, n], ...) over those rows from +0.0.
//    Row c of Wᵀ lists exactly those rows in that order (a stable transpose),
//    so the chain is the reference's spmm(WT, dY) element for element.
//  * dW waves: slk_sddmm's SIMD order (16 slots per wave, 4 lanes per slot)
//    or scalar order (one lane per slot), with dY read at stride M.
//  * bias waves: one per row, slk_sddmm_bias's lane-strided sum.
#include "dw_common.hpp"

namespace slk {
namespace {

constexpr int kNarrowBlock = 256;  // 4 waves
constexpr int kNarrowWaves = kNarrowBlock / kWave;
constexpr int kDxItemsPerWave = 2;
constexpr int kDxBatch = 8;  // rows whose dY loads are in flight together

__device__ __forceinline__ float lane_f(float v, int32_t lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

template <int VEC>
__device__ void dx_run(int64_t M, int64_t N, int64_t items, int64_t ntiles,
                         const int32_t* __restrict__ s_col, const float* __restrict__ s_val,
                         const int32_t* __restrict__ s_rs, const int32_t* __restrict__ s_rn,
                         const float* __restrict__ dYt, float* __restrict__ dX,
                         int64_t first, int64_t stride) {
    const int lane = threadIdx.x & (kWave - 1);
    for (int64_t it = first; it < items; it += stride) {
        const int64_t c = it / ntiles;
        const int64_t n0 = ((it - c * ntiles) * kWave + lane) * VEC;
        const bool active = n0 < N;  // N % VEC == 0
        // lane m: is column c live in row m, and with which value
        bool found = false;
        float v = 0.0f;
        if (lane < M) {
            const int32_t lo = s_rs[lane];
            int32_t a = 0, e = s_rn[lane];
            while (a < e) {
                const int32_t mid = (a + e) >> 1;
                if (s_col[lo + mid] < c) a = mid + 1; else e = mid;
            }
            if (a < s_rn[lane] && s_col[lo + a] == c) {
                found = true;
                v = s_val[lo + a];
            }
        }
        uint64_t rows = __ballot(found);
        float acc[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] = 0.0f;
        while (rows != 0) {
            float d[kDxBatch][VEC];
            float w[kDxBatch];
            int cnt = 0;
#pragma unroll
            for (int u = 0; u < kDxBatch; ++u) {
                if (rows != 0) {
                    const int m = __builtin_ctzll(rows);
                    rows &= rows - 1;
                    w[u] = lane_f(v, m);
#pragma unroll
                    for (int e = 0; e < VEC; ++e) d[u][e] = active ? dYt[(n0 + e) * M + m] : 0.0f;
                    cnt = u + 1;
                }
            }
#pragma unroll
            for (int u = 0; u < kDxBatch; ++u) {
                if (u < cnt) {
#pragma unroll
                    for (int e = 0; e < VEC; ++e) acc[e] = __builtin_fmaf(w[u], d[u][e], acc[e]);
                }
            }
        }
        if (active) {
            float* out = dX + c * N + n0;
            if constexpr (VEC == 4) {
                *reinterpret_cast<f32x4*>(out) = f32x4{acc[0], acc[1], acc[2], acc[3]};
            } else {
                out[0] = acc[0];
            }
        }
    }
}

// dW in SIMD order for the 16 slots of wave `wid` (sddmm.hip's
// sddmm_simd_kernel with dY[i, j] = dYt[j·M + i]).
template <bool V4X>
__device__ void dw_simd_wave(int64_t M, int64_t N, int64_t cap, int64_t wid,
                             const int32_t* __restrict__ row_start,
                             const int32_t* __restrict__ row_nnz, const int32_t* __restrict__ col,
                             const float* __restrict__ dYt, const float* __restrict__ X,
                             float* __restrict__ dW) {
    constexpr int kSlots = 16;
    const int lane = threadIdx.x & (kWave - 1);
    const int g = lane >> 2;  // slot within the wave
    const int q = lane & 3;   // owns virtual lanes 4q..4q+3
    const int64_t wslot = wid * kSlots;
    const int64_t slot = wslot + g;
    const bool in_range = slot < cap;
    const WaveRows rows(row_start, M, wslot, min(wslot + kSlots - 1, cap - 1));
    int64_t row = 0;
    bool live = false;
    int32_t c = 0;
    if (in_range) {
        row = rows.of(row_start, rows.first_row, slot);
        live = (slot - row_start[row]) < row_nnz[row];
        if (live) c = col[slot];
    }
    const float* dyr = dYt + (live ? row : 0);  // element j at dyr[j·M]
    const float* xr = X + (live ? static_cast<int64_t>(c) * N : 0);
    const int64_t n16 = (N / 16) * 16;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    if (live) {
#pragma unroll 4
        for (int64_t j = 4 * q; j < n16; j += 16) {
            float x0, x1, x2, x3;
            if constexpr (V4X) {
                const f32x4 xv = *reinterpret_cast<const f32x4*>(xr + j);
                x0 = xv[0]; x1 = xv[1]; x2 = xv[2]; x3 = xv[3];
            } else {
                x0 = xr[j]; x1 = xr[j + 1]; x2 = xr[j + 2]; x3 = xr[j + 3];
            }
            a0 = __builtin_fmaf(dyr[j * M], x0, a0);
            a1 = __builtin_fmaf(dyr[(j + 1) * M], x1, a1);
            a2 = __builtin_fmaf(dyr[(j + 2) * M], x2, a2);
            a3 = __builtin_fmaf(dyr[(j + 3) * M], x3, a3);
        }
    }
    {  // a[l] = v[l] + v[l+8]
        const float p0 = __shfl_xor(a0, 2), p1 = __shfl_xor(a1, 2);
        const float p2 = __shfl_xor(a2, 2), p3 = __shfl_xor(a3, 2);
        a0 = a0 + p0; a1 = a1 + p1; a2 = a2 + p2; a3 = a3 + p3;
    }
    int64_t jt = n16;
    if (N - n16 >= 8) {  // one 8-wide step
        if (live && q < 2) {
            const int64_t j = n16 + 4 * q;
            a0 = __builtin_fmaf(dyr[j * M], xr[j], a0);
            a1 = __builtin_fmaf(dyr[(j + 1) * M], xr[j + 1], a1);
            a2 = __builtin_fmaf(dyr[(j + 2) * M], xr[j + 2], a2);
            a3 = __builtin_fmaf(dyr[(j + 3) * M], xr[j + 3], a3);
        }
        jt += 8;
    }
    {  // s4[k] = a[k] + a[k+4]
        const float p0 = __shfl_xor(a0, 1), p1 = __shfl_xor(a1, 1);
        const float p2 = __shfl_xor(a2, 1), p3 = __shfl_xor(a3, 1);
        a0 = a0 + p0; a1 = a1 + p1; a2 = a2 + p2; a3 = a3 + p3;
    }
    if (in_range && q == 0) {
        const float r = (a0 + a2) + (a1 + a3);
        dW[slot] = live ? running_sum(dyr + jt * M, xr + jt, N - jt, r, M) : 0.0f;
    }
}

// dW in scalar order for the 64 slots of wave `wid` (sddmm_scalar_kernel).
__device__ void dw_scalar_wave(int64_t M, int64_t N, int64_t cap, int64_t wid,
                               const int32_t* __restrict__ row_start,
                               const int32_t* __restrict__ row_nnz,
                               const int32_t* __restrict__ col, const float* __restrict__ dYt,
                               const float* __restrict__ X, float* __restrict__ dW) {
    const int64_t wslot = wid * kWave;
    const WaveRows rows(row_start, M, wslot, min(wslot + kWave - 1, cap - 1));
    const int64_t slot = wslot + (threadIdx.x & (kWave - 1));
    if (slot >= cap) return;
    const int64_t row = rows.of(row_start, rows.first_row, slot);
    if (slot - row_start[row] >= row_nnz[row]) {
        dW[slot] = 0.0f;
        return;
    }
    dW[slot] = running_sum(dYt + row, X + static_cast<int64_t>(col[slot]) * N, N, 0.0f, M);
}

template <int VEC, bool V4X, bool SIMD>
__global__ __launch_bounds__(kNarrowBlock) void narrow_backward_kernel(
    int64_t M, int64_t N, int64_t cap, const int32_t* __restrict__ row_start,
    const int32_t* __restrict__ row_nnz, const int32_t* __restrict__ col,
    const float* __restrict__ val, const float* __restrict__ dYt, const float* __restrict__ X,
    float* __restrict__ dW, float* __restrict__ dbias, float* __restrict__ dX,
    int64_t dx_blocks, int64_t dx_items, int64_t ntiles, int64_t dw_waves) {
    const int wib = threadIdx.x >> 6;  // wave in block
    if (static_cast<int64_t>(blockIdx.x) < dx_blocks) {  // block-uniform: a dX workgroup
        extern __shared__ __align__(16) char smem[];
        int32_t* s_col = reinterpret_cast<int32_t*>(smem);
        float* s_val = reinterpret_cast<float*>(s_col + cap);
        int32_t* s_rs = reinterpret_cast<int32_t*>(s_val + cap);
        int32_t* s_rn = s_rs + M;
        for (int64_t t = threadIdx.x; t < cap; t += kNarrowBlock) {
            s_col[t] = col[t];
            s_val[t] = val[t];
        }
        for (int64_t t = threadIdx.x; t < M; t += kNarrowBlock) {
            s_rs[t] = row_start[t];
            s_rn[t] = row_nnz[t];
        }
        __syncthreads();
        dx_run<VEC>(M, N, dx_items, ntiles, s_col, s_val, s_rs, s_rn, dYt, dX,
                    static_cast<int64_t>(blockIdx.x) * kNarrowWaves + wib,
                    dx_blocks * kNarrowWaves);
        return;
    }
    const int64_t w = (static_cast<int64_t>(blockIdx.x) - dx_blocks) * kNarrowWaves + wib;
    if (w < dw_waves) {
        if constexpr (SIMD) {
            dw_simd_wave<V4X>(M, N, cap, w, row_start, row_nnz, col, dYt, X, dW);
        } else {
            dw_scalar_wave(M, N, cap, w, row_start, row_nnz, col, dYt, X, dW);
        }
    } else if (dbias != nullptr) {
        bias_row_sum(dYt, M, N, w - dw_waves, dbias, 1, M);
    }
}

template <int VEC, bool V4X, bool SIMD>
void launch_narrow(const slk_csr* W, const float* dYt, int64_t N, const float* X, float* dW,
                   float* dbias, float* dX, int64_t dx_blocks, int64_t dx_items, int64_t ntiles,
                   int64_t dw_waves, int64_t blocks, size_t lds, hipStream_t st) {
    hipLaunchKernelGGL((narrow_backward_kernel<VEC, V4X, SIMD>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kNarrowBlock), lds, st, W->nrows, N, W->total_capacity, W->row_start,
                       W->row_nnz, W->col_indices, W->values, dYt, X, dW, dbias, dX, dx_blocks,
                       dx_items, ntiles, dw_waves);
}

}  // namespace
}  // namespace slk

extern "C" int slk_backward_narrow(const slk_csr* W, const float* dYt, int64_t N, const float* X,
                                   int64_t X_rows, float* dW, float* dbias, float* dX, int order,
                                   void* stream) {
    using namespace slk;
    clear_error();
    const char* who = "backward_narrow";
    if (int rc = validate_csr(W, who)) return rc;
    if (order != SLK_DW_SIMD && order != SLK_DW_SCALAR) {
        return fail(SLK_EINVAL, std::string(who) + ": unknown order " + std::to_string(order));
    }
    const int64_t M = W->nrows, K = W->ncols, cap = W->total_capacity;
    if (M > SLK_NARROW_MAX_ROWS || cap > SLK_NARROW_MAX_CAPACITY) {
        return fail(SLK_EINVAL, std::string(who) + ": W is " + std::to_string(M) + " rows with " +
                                    std::to_string(cap) + " slots; at most " +
                                    std::to_string(SLK_NARROW_MAX_ROWS) + " rows and " +
                                    std::to_string(SLK_NARROW_MAX_CAPACITY) + " slots");
    }
    if (N < 0) return fail(SLK_EINVAL, std::string(who) + ": N must be >= 0");
    if (X_rows != K) {
        return fail(SLK_EINVAL, std::string(who) + ": X.shape[0]=" + std::to_string(X_rows) +
                                    " must equal W.ncols=" + std::to_string(K));
    }
    if (N > 0 && M > 0 && dYt == nullptr) return fail(SLK_EINVAL, std::string(who) + ": NULL dYt");
    if (dW == nullptr && dbias == nullptr && dX == nullptr) return SLK_OK;
    if (dW != nullptr && N > 0 && K > 0 && X == nullptr) {
        return fail(SLK_EINVAL, std::string(who) + ": NULL X");
    }
    hipStream_t st = as_stream(stream);
    // N == 0 or M == 0 needs no special case: every chain is empty, so the
    // kernel writes dW = 0, dbias = 0 and dX = 0 without reading dY.
    const bool simd = order == SLK_DW_SIMD;
    const bool v4x = X != nullptr && N % 4 == 0 && reinterpret_cast<uintptr_t>(X) % 16 == 0;
    const int vec = (N % 4 == 0 && reinterpret_cast<uintptr_t>(dX) % 16 == 0) ? 4 : 1;
    const int64_t ntiles = ceil_div(N, int64_t{kWave} * vec);
    const int64_t dx_items = dX != nullptr ? K * ntiles : 0;
    const int64_t dx_blocks = ceil_div(dx_items, int64_t{kNarrowWaves} * kDxItemsPerWave);
    const int64_t dw_waves = dW != nullptr ? ceil_div(cap, simd ? 16 : kWave) : 0;
    const int64_t tail_waves = dw_waves + (dbias != nullptr ? M : 0);
    const int64_t blocks = dx_blocks + ceil_div(tail_waves, int64_t{kNarrowWaves});
    if (blocks == 0) return SLK_OK;
    if (blocks > INT32_MAX) return fail(SLK_EINVAL, std::string(who) + ": problem too large");
    const size_t lds = dx_blocks > 0 ? static_cast<size_t>(8 * cap + 8 * M) : 0;
#define SLK_NARROW_ARGS W, dYt, N, X, dW, dbias, dX, dx_blocks, dx_items, ntiles, dw_waves, blocks, lds, st
    if (vec == 4) {
        if (v4x) simd ? launch_narrow<4, true, true>(SLK_NARROW_ARGS) : launch_narrow<4, true, false>(SLK_NARROW_ARGS);
        else simd ? launch_narrow<4, false, true>(SLK_NARROW_ARGS) : launch_narrow<4, false, false>(SLK_NARROW_ARGS);
    } else {
        if (v4x) simd ? launch_narrow<1, true, true>(SLK_NARROW_ARGS) : launch_narrow<1, true, false>(SLK_NARROW_ARGS);
        else simd ? launch_narrow<1, false, true>(SLK_NARROW_ARGS) : launch_narrow<1, false, false>(SLK_NARROW_ARGS);
    }
#undef SLK_NARROW_ARGS
    return check_launch(who);
}
