// Dense rows of the forward product Y = W·X on the matrix cores (gfx950).
//
// Why it is exact. gfx950's fp32 K=1 MFMA outer products
// (v_mfma_f32_32x32x1_2b_f32) add each product a·b to its accumulator with a
// single rounding: bit for bit the IEEE fma(a, b, c), including subnormals,
// signed zeros, infinities and NaN (checked on the device against the host's
// fmaf by tests/test_gpu_dense_rows.py). The reference evaluates every Y
// element as the chain y = fma(v_s, X[c_s, n], y) over the row's live slots
// in slot order — ascending column order — from +0.0
// (csrc/kernels/spmm_avx2.cpp:123-262). A row spread densely over all K
// columns (W_d[i, k] = the value of the slot at column k, 0 where the row has
// none) and multiplied in ascending k order, one outer product per column,
// therefore runs the same chain with extra steps fma(0, x, y) at the absent
// columns. For finite x such a step adds ±0 and leaves y unchanged (a zero y
// may flip sign; ±0 compare equal), so every element equals the reference's
// under ==. For x = ±inf or NaN it would give NaN where the reference skips
// the column; then every dense output of that column is non-finite, so the
// MFMA kernel raises a status word whenever one of its outputs is not finite
// and a third launch recomputes the dense rows slot by slot (as the reference
// does) when the word is set. A chain that overflows on its own sets it too
// and is recomputed to the same value.
//
// Layout. dense_ws = [status word, 256 B][W_d: Tp rows x Ks floats], Tp = the
// dense-row count rounded up to a workgroup's 128 rows, Ks = K rounded up to
// whole loop trips plus the groups the last trip prefetches (all zero past
// K). Rows are positions of W's row_order (longest first), so the dense rows
// are its head.
//
// Kernels.
//   dense_fill_kernel     one workgroup per dense row: zero the row, then
//                         scatter its live slots (every call: values change).
//   dense_mfma_kernel     4 waves x 32 rows, 64 columns per workgroup; each
//                         wave one 32 x 64 accumulator tile (32 AGPRs) and
//                         one v_mfma_f32_32x32x1_2b_f32 per column k (A: the
//                         32 rows' W_d[., k], duplicated over both lane
//                         halves; B: X[k, 64 columns]). Operands come through
//                         buffer loads with wave-uniform bases and 32-bit lane
//                         offsets, kDenseDG groups of 4 columns in flight,
//                         each load issued under one MFMA (sched_barrier keeps
//                         that order); X rows past K read as 0 through the
//                         buffer range check.
//   dense_fallback_kernel exits unless the status word is set; then the
//                         reference chain per (row, column), grid-strided.
#include "common.hpp"
#include "dense_rows.hpp"

namespace slk {
namespace {

constexpr int kDenseDG = 8;                        // groups of 4 columns in flight
constexpr int kDenseWaveRows = 32;                 // rows of one wave's tile
constexpr int kDenseBlockRows = 4 * kDenseWaveRows;  // rows of a workgroup
constexpr int kDenseCols = 64;                     // columns of a workgroup
constexpr int64_t kDenseHeader = 256;              // status word, padded
constexpr uint32_t kBufWord3 = 0x00020000;         // gfx9 buffer resource dword 3

typedef float f32x32 __attribute__((ext_vector_type(32)));

// Loop trips run 2·kDenseDG groups of 4 columns; the prefetch reads kDenseDG
// groups past the last trip, which the row stride keeps inside the zeroed row.
__host__ __device__ inline int64_t dense_groups(int64_t K) {
    return ceil_div(ceil_div(K, 4), 2 * kDenseDG) * (2 * kDenseDG);
}
__host__ __device__ inline int64_t dense_stride(int64_t K) { return 4 * (dense_groups(K) + kDenseDG); }
__host__ __device__ inline int64_t dense_pad_rows(int64_t T) {
    return ceil_div(T, kDenseBlockRows) * kDenseBlockRows;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), kBufWord3);
}

// Row p of W_d (p < Tp): zeros, then row order[p]'s live slots (p < T).
__global__ __launch_bounds__(256) void dense_fill_kernel(
    const int32_t* __restrict__ order, int64_t T, const int32_t* __restrict__ row_start,
    const int32_t* __restrict__ row_nnz, const int32_t* __restrict__ col,
    const float* __restrict__ val, int64_t Ks, float* __restrict__ Wd, int* __restrict__ status) {
    const int64_t p = blockIdx.x;
    float* dst = Wd + p * Ks;
    const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int64_t i = 4 * static_cast<int64_t>(threadIdx.x); i < Ks; i += 4 * 256)
        *reinterpret_cast<f32x4*>(dst + i) = z;
    __syncthreads();  // the zeros land before the slots that overwrite them
    if (p < T) {
        const int32_t row = order[p];
        const int32_t s0 = row_start[row], n = row_nnz[row];
        for (int32_t i = threadIdx.x; i < n; i += 256) dst[col[s0 + i]] = val[s0 + i];
    }
    if (p == 0 && threadIdx.x == 0) *status = 0;
}

__global__ __launch_bounds__(256) void dense_mfma_kernel(
    const int32_t* __restrict__ order, int64_t T, const float* __restrict__ Wd, int64_t Ks,
    int32_t ng, const float* __restrict__ X, int32_t K, int64_t N, const float* __restrict__ bias,
    float* __restrict__ Y, int* __restrict__ status) {
    const int lane = threadIdx.x & (kWave - 1);
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t nrg = ceil_div(T, kDenseBlockRows);
    const int64_t lb = xcd_logical_block(blockIdx.x, gridDim.x);
    const int64_t ct = lb / nrg, rg = lb - ct * nrg;  // a column tile's row groups share an XCD
    const int64_t r0 = rg * kDenseBlockRows + w * kDenseWaveRows;
    const int64_t c0 = ct * kDenseCols;
    // A: lane l holds row r0 + l % 32 (both halves the same rows); B: lane l
    // holds column c0 + l (clamped to N - 1: those lanes' outputs are dropped)
    const uint32_t aoff = static_cast<uint32_t>((lane & (kDenseWaveRows - 1)) * Ks * 4);
    const __amdgpu_buffer_rsrc_t rsA =
        buf_rsrc(Wd + r0 * Ks, static_cast<uint32_t>(kDenseWaveRows * Ks * 4));
    const int64_t cl = c0 + lane < N ? c0 + lane : N - 1;
    const uint32_t rowb = static_cast<uint32_t>(N * 4);
    uint32_t boff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) boff[j] = static_cast<uint32_t>(cl * 4) + j * rowb;
    // X rows 4g .. 4g+3 through a resource based at row 4g whose range ends
    // at row K, so rows past K read as 0 (32-bit row arithmetic keeps the
    // resource on the scalar unit)
    auto rsB = [&](int32_t g) {
        const int32_t k0 = 4 * g;
        const int32_t kb = k0 < K ? k0 : K;
        const int32_t left = K - kb;
        const uint32_t rows = left < 4 ? static_cast<uint32_t>(left) : 4u;
        return buf_rsrc(reinterpret_cast<const char*>(X) + static_cast<uint64_t>(static_cast<uint32_t>(kb)) * rowb,
                        rows * rowb);
    };
    auto ldA = [&](int32_t g) -> f32x4 {
        return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsA, aoff, 16 * g, 0));
    };
    auto ldB = [&](const __amdgpu_buffer_rsrc_t& r, int j) -> float {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, boff[j], 0, 0));
    };

    f32x32 acc;
#pragma unroll
    for (int r = 0; r < 32; ++r) acc[r] = 0.0f;
    f32x4 ar[kDenseDG];
    float br[kDenseDG][4];
    static_for<kDenseDG>([&](auto S) {
        constexpr int s = decltype(S)::value;
        ar[s] = ldA(s);
        const auto rb = rsB(s);
#pragma unroll
        for (int j = 0; j < 4; ++j) br[s][j] = ldB(rb, j);
        __builtin_amdgcn_sched_barrier(0);  // groups issue in order (the waits count on it)
    });
    // Two passes over the ring per trip, so that half of a trip's loads are
    // consumed inside it (the compiler then keeps the loop's waits partial).
    for (int32_t g0 = 0; g0 < ng; g0 += 2 * kDenseDG) {
        static_for<2 * kDenseDG>([&](auto S) {
            constexpr int t = decltype(S)::value;
            constexpr int s = t % kDenseDG;
            const int32_t gn = g0 + t + kDenseDG;
            const auto rn = rsB(gn);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc = __builtin_amdgcn_mfma_f32_32x32x1f32(ar[s][j], br[s][j], acc, 0, 0, 0);
                br[s][j] = ldB(rn, j);
                if (j == 3) ar[s] = ldA(gn);
                __builtin_amdgcn_sched_barrier(0);
            }
        });
    }
    // accumulator r: block r / 16 (columns +32 in the second), row
    // 8 (r mod 16) / 4 + 4 (lane / 32) + r mod 4, column lane mod 32
    bool bad = false;
#pragma unroll
    for (int r = 0; r < 32; ++r) bad |= !__builtin_isfinite(acc[r]);
    if (bad) *status = 1;
#pragma unroll
    for (int r = 0; r < 32; ++r) {
        const int rr = r & 15;
        const int64_t p = r0 + 8 * (rr >> 2) + 4 * (lane >> 5) + (rr & 3);
        const int64_t n = c0 + 32 * (r >> 4) + (lane & 31);
        if (p < T && n < N) {
            const int64_t row = order[p];
            float y = acc[r];
            if (bias != nullptr) y = y + bias[row];
            Y[row * N + n] = y;
        }
    }
}

// The reference chain for the dense rows, run only when the status word is
// set: each wave takes (row, 256-column tile) items, lane l columns
// tile·256 + l + 64 e.
__global__ __launch_bounds__(256) void dense_fallback_kernel(
    const int* __restrict__ status, const int32_t* __restrict__ order, int64_t T,
    const int32_t* __restrict__ row_start, const int32_t* __restrict__ row_nnz,
    const int32_t* __restrict__ col, const float* __restrict__ val, const float* __restrict__ X,
    int64_t N, const float* __restrict__ bias, float* __restrict__ Y) {
    if (*status == 0) return;
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t tiles = ceil_div(N, 256);
    const int64_t nw = static_cast<int64_t>(gridDim.x) * 4;
    for (int64_t it = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); it < T * tiles; it += nw) {
        const int64_t p = it / tiles, tile = it - p * tiles;
        const int32_t row = order[p];
        const int32_t s0 = row_start[row], n = row_nnz[row];
        float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int32_t i = 0; i < n; ++i) {
            const float v = val[s0 + i];
            const float* xr = X + static_cast<int64_t>(col[s0 + i]) * N;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int64_t c = tile * 256 + lane + 64 * e;
                if (c < N) y[e] = __builtin_fmaf(v, xr[c], y[e]);
            }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t c = tile * 256 + lane + 64 * e;
            if (c < N) Y[static_cast<int64_t>(row) * N + c] = bias != nullptr ? y[e] + bias[row] : y[e];
        }
    }
}

// ─────────────────────────── weight gradient ───────────────────────────────
//
// dW on the live slots of the dense rows, in the reference's SIMD order
// (csrc/kernels/spmm_grad_avx2.cpp:108-258) for N a multiple of 16: per
// (row i, column c), 16 running fma chains v[l] over n = 16t + l, then
// a[l] = v[l] + v[l + 8], s4[k] = a[k] + a[k + 4], (s4[0] + s4[2]) +
// (s4[1] + s4[3]). On the matrix cores: a wave owns a 32-row x 32-column tile
// of (i, c) pairs and eight accumulator sets; instruction l of step t is one
// v_mfma_f32_32x32x1_2b_f32 whose block 0 adds dY[i, 16t + l]·X[c, 16t + l]
// (chain l) and whose block 1 adds chain l + 8's term, each one fma. Blocks 0
// and 1 put the same (i, c) in the same lane and register (r and r + 16), so
// the combine runs lane by lane in the vector unit, in the reference's order.
// Results go to a dense T x K buffer (dense_ws), and one workgroup per dense
// row copies its live slots out of it; padding slots are left to the
// segment kernel, which zeroes every row's padding.

// Operands through LDS: a workgroup (4 waves, 2 x 2 tiles) owns 64 dense rows
// x 64 columns and stages, per stage of 64 columns of N, the 64 dY rows and
// 64 X rows it needs, one 256-byte row segment per direct-to-LDS dword load
// (whole cache lines; a lane per float), in rows padded to 68 floats so a
// wave's reads of 32 rows hit every bank once; two stages double-buffered.
// Each wave then reads its operands from LDS: per step of 16 columns, 32
// bytes of its A row and of its B row per lane (lanes 0-31 columns 0-7 of
// the step, lanes 32-63 columns 8-15).
constexpr int kDwStageN = 64;                   // columns of N per stage
constexpr int kDwRow = kDwStageN + 4;           // padded LDS row (floats)
constexpr int kDwStageFloats = 2 * 64 * kDwRow;  // dY rows, then X rows
// s_waitcnt operand: at most 32 vector-memory operations outstanding, no LDS
// or scalar ones (gfx9: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
constexpr int kVmcntLe32 = (32 & 15) | ((32 >> 4) << 14) | (7 << 4);
constexpr int kVmcntLe0 = 7 << 4;

__global__ __launch_bounds__(256) void dense_dw_kernel(
    const int32_t* __restrict__ order, int64_t T, const float* __restrict__ dY,
    const float* __restrict__ X, int64_t K, int32_t N, float* __restrict__ dWd, int64_t Ks) {
    __shared__ float st[2][kDwStageFloats];  // 68 KiB
    const int lane = threadIdx.x & (kWave - 1);
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t nrg = ceil_div(T, 64);
    const int64_t lb = xcd_logical_block(blockIdx.x, gridDim.x);
    const int64_t cg = lb / nrg, rg = lb - cg * nrg;  // a column group's row groups share an XCD
    const int64_t ib = rg * 64, cb = cg * 64;         // the workgroup's rows and columns
    // staging: wave w copies rows w, w + 4, .. of each operand (uniform row
    // bases; rows past T or K copy a real row whose results are dropped)
    const float* src[32];
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        int64_t p = ib + w + 4 * q;
        p = p < T ? p : T - 1;
        src[q] = dY + static_cast<int64_t>(order[p]) * N;
        int64_t c = cb + w + 4 * q;
        c = c < K ? c : K - 1;
        src[16 + q] = X + c * N;
    }
    auto stage = [&](int buf, int32_t s) {
#pragma unroll
        for (int q = 0; q < 32; ++q) {
            const int r = (q < 16 ? 0 : 64) + w + 4 * (q & 15);
            __builtin_amdgcn_global_load_lds(src[q] + s * kDwStageN + lane, &st[buf][r * kDwRow], 4, 0, 0);
        }
    };
    f32x32 acc[8];
#pragma unroll
    for (int l = 0; l < 8; ++l)
#pragma unroll
        for (int r = 0; r < 32; ++r) acc[l][r] = 0.0f;
    // the wave's tile: A rows (w & 1)·32 + lane mod 32, B rows (w >> 1)·32 + ..
    const int h = lane >> 5;
    const int arow = (w & 1) * 32 + (lane & 31), brow = 64 + (w >> 1) * 32 + (lane & 31);
    const int32_t ns = N / kDwStageN;
    stage(0, 0);
    for (int32_t s = 0; s < ns; ++s) {
        const int b = s & 1;
        // Each wave waits for its own copies of stage s, then the barrier
        // makes all four waves' copies visible. A bare s_barrier: a
        // workgroup fence there would also wait for stage s + 1's copies.
        if (s + 1 < ns) {
            stage(b ^ 1, s + 1);  // its last readers passed the previous barrier
            __builtin_amdgcn_s_waitcnt(kVmcntLe32);
        } else {
            __builtin_amdgcn_s_waitcnt(kVmcntLe0);
        }
        __builtin_amdgcn_s_barrier();
        const float* A = &st[b][arow * kDwRow + 8 * h];
        const float* B = &st[b][brow * kDwRow + 8 * h];
        f32x4 op[2][4];  // this step's and the next step's a0, a1, b0, b1
        auto rd = [&](f32x4 (&o)[4], int t) {
            o[0] = *reinterpret_cast<const f32x4*>(A + 16 * t);
            o[1] = *reinterpret_cast<const f32x4*>(A + 16 * t + 4);
            o[2] = *reinterpret_cast<const f32x4*>(B + 16 * t);
            o[3] = *reinterpret_cast<const f32x4*>(B + 16 * t + 4);
        };
        rd(op[0], 0);
        // the next step's reads issue before this step's MFMAs (sched_barrier
        // keeps them there), so their latency hides under eight MFMAs
        static_for<kDwStageN / 16>([&](auto T) {
            constexpr int t = decltype(T)::value;
            if constexpr (t + 1 < kDwStageN / 16) rd(op[(t + 1) & 1], t + 1);
            __builtin_amdgcn_sched_barrier(0);
            const f32x4(&o)[4] = op[t & 1];
#pragma unroll
            for (int l = 0; l < 8; ++l)
                acc[l] = __builtin_amdgcn_mfma_f32_32x32x1f32(o[l >> 2][l & 3], o[2 + (l >> 2)][l & 3],
                                                              acc[l], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        });
        __builtin_amdgcn_s_waitcnt(kVmcntLe32 | (0 << 8));  // (reads consumed)
        __builtin_amdgcn_s_barrier();  // stage s read by every wave before it is refilled
    }
    const int64_t i0 = ib + (w & 1) * 32, c0 = cb + (w >> 1) * 32;
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
        float a[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) a[l] = acc[l][rr] + acc[l][rr + 16];
        float s4[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) s4[k] = a[k] + a[k + 4];
        const float sum = (s4[0] + s4[2]) + (s4[1] + s4[3]);
        const int64_t row = i0 + 8 * (rr >> 2) + 4 * (lane >> 5) + (rr & 3);
        const int64_t col = c0 + (lane & 31);
        if (row < T && col < K) dWd[row * Ks + col] = sum;
    }
}

// dW[s] for the live slots of dense row order[p] out of the dense buffer.
__global__ __launch_bounds__(256) void dense_dw_scatter_kernel(
    const int32_t* __restrict__ order, const int32_t* __restrict__ row_start,
    const int32_t* __restrict__ row_nnz, const int32_t* __restrict__ col,
    const float* __restrict__ dWd, int64_t Ks, float* __restrict__ dW) {
    const int64_t p = blockIdx.x;
    const int32_t row = order[p];
    const int32_t s0 = row_start[row], n = row_nnz[row];
    const float* src = dWd + p * Ks;
    for (int32_t i = threadIdx.x; i < n; i += 256) dW[s0 + i] = src[col[s0 + i]];
}

// One v_mfma_f32_32x32x1_2b_f32 per case t on the given lane operands and
// accumulator registers (slk_dense_mfma_probe).
__global__ __launch_bounds__(64) void dense_mfma_probe_kernel(const float* __restrict__ A,
                                                              const float* __restrict__ B,
                                                              const float* __restrict__ C,
                                                              float* __restrict__ D, int64_t n) {
    const int64_t t = blockIdx.x;
    if (t >= n) return;
    const int64_t l = t * kWave + threadIdx.x;
    f32x32 acc;
#pragma unroll
    for (int r = 0; r < 32; ++r) acc[r] = C[l * 32 + r];
    acc = __builtin_amdgcn_mfma_f32_32x32x1f32(A[l], B[l], acc, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 32; ++r) D[l * 32 + r] = acc[r];
}

}  // namespace

int64_t dense_rows_workspace_bytes(int64_t T, int64_t K) {
    if (T <= 0 || K <= 0) return 0;
    return kDenseHeader + dense_pad_rows(T) * dense_stride(K) * 4;
}

bool dense_rows_apply(int64_t T, int64_t K, int64_t N) {
    // 32-bit lane offsets: a wave's 32 rows of W_d and 4 X rows in one resource
    return T > 0 && K > 0 && N > 0 && kDenseWaveRows * dense_stride(K) * 4 < (int64_t{1} << 31) &&
           N * 16 < (int64_t{1} << 31) && K < (int64_t{1} << 30);
}

bool dense_dw_apply(int64_t T, int64_t M, int64_t K, int64_t N) {
    (void)M;
    (void)K;
    return T > 0 && N >= kDwStageN && N % kDwStageN == 0 && N <= INT32_MAX;  // whole stages
}

int sddmm_dense_rows(const slk_csr* W, const float* dY, const float* X, int64_t N, float* dW,
                     hipStream_t st) {
    const int64_t T = W->n_dense_rows, K = W->ncols;
    const int64_t Ks = dense_stride(K);
    float* dWd = reinterpret_cast<float*>(static_cast<char*>(W->dense_ws) + kDenseHeader);
    const int64_t nb = ceil_div(T, 64) * ceil_div(K, 64);
    if (nb > INT32_MAX) return fail(SLK_EINVAL, "spmm_grad_w_simd: dense rows: too large");
    hipLaunchKernelGGL(dense_dw_kernel, dim3(static_cast<unsigned>(nb)), dim3(256), 0, st,
                       W->row_order, T, dY, X, K, static_cast<int32_t>(N), dWd, Ks);
    if (int rc = check_launch("spmm_grad_w_simd: dense rows")) return rc;
    hipLaunchKernelGGL(dense_dw_scatter_kernel, dim3(static_cast<unsigned>(T)), dim3(256), 0, st,
                       W->row_order, W->row_start, W->row_nnz, W->col_indices, dWd, Ks, dW);
    return check_launch("spmm_grad_w_simd: dense rows scatter");
}

int spmm_dense_rows(const slk_csr* W, const float* X, int64_t K, int64_t N, const float* bias,
                    float* Y, hipStream_t st) {
    const int64_t T = W->n_dense_rows;
    const int64_t Tp = dense_pad_rows(T), Ks = dense_stride(K);
    char* ws = static_cast<char*>(W->dense_ws);
    int* status = reinterpret_cast<int*>(ws);
    float* Wd = reinterpret_cast<float*>(ws + kDenseHeader);
    hipLaunchKernelGGL(dense_fill_kernel, dim3(static_cast<unsigned>(Tp)), dim3(256), 0, st,
                       W->row_order, T, W->row_start, W->row_nnz, W->col_indices, W->values, Ks,
                       Wd, status);
    if (int rc = check_launch("spmm dense rows: fill")) return rc;
    const int64_t nb = (Tp / kDenseBlockRows) * ceil_div(N, kDenseCols);
    hipLaunchKernelGGL(dense_mfma_kernel, dim3(static_cast<unsigned>(nb)), dim3(256), 0, st,
                       W->row_order, T, Wd, Ks, static_cast<int32_t>(dense_groups(K)), X,
                       static_cast<int32_t>(K), N, bias, Y, status);
    if (int rc = check_launch("spmm dense rows: mfma")) return rc;
    const int64_t items = T * ceil_div(N, 256);
    const int64_t fb = items < 1024 ? ceil_div(items, 4) : 256;
    hipLaunchKernelGGL(dense_fallback_kernel, dim3(static_cast<unsigned>(fb)), dim3(256), 0, st,
                       status, W->row_order, T, W->row_start, W->row_nnz, W->col_indices,
                       W->values, X, N, bias, Y);
    return check_launch("spmm dense rows: fallback");
}

}  // namespace slk

extern "C" int64_t slk_dense_rows_workspace_bytes(int64_t n_dense_rows, int64_t ncols) {
    return slk::dense_rows_workspace_bytes(n_dense_rows, ncols);
}

extern "C" int slk_dense_mfma_probe(const float* A, const float* B, const float* C, float* D,
                                    int64_t n, void* stream) {
    slk::clear_error();
    if (n < 0) return slk::fail(SLK_EINVAL, "dense_mfma_probe: negative case count");
    if (n == 0) return SLK_OK;
    if (A == nullptr || B == nullptr || C == nullptr || D == nullptr)
        return slk::fail(SLK_EINVAL, "dense_mfma_probe: NULL operand");
    if (n > INT32_MAX) return slk::fail(SLK_EINVAL, "dense_mfma_probe: too many cases");
    hipLaunchKernelGGL(slk::dense_mfma_probe_kernel, dim3(static_cast<unsigned>(n)), dim3(64), 0,
                       slk::as_stream(stream), A, B, C, D, n);
    return slk::check_launch("dense_mfma_probe");
}
