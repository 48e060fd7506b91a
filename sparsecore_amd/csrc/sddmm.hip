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
// A wave finds the rows of its slots with a 64-way search over row_start;
// padding slots (slot-in-row >= row_nnz) are written as 0 by the lane that
// owns them, so dW needs no separate memset.
//
// Kernels: sddmm_simd_kernel (one 16-slot group per wave, whole rows at a
// time; small or unaligned N), sddmm_simd_win_kernel<G> (G groups per wave
// swept through N window by window with dY staged in LDS; large N) and
// sddmm_scalar_kernel. slk_sddmm_bias appends one wave per row that sums the
// row of dY (the bias gradient) to the same launch.
#include "dense_rows.hpp"
#include "dw_common.hpp"

#include <cstdlib>

namespace slk {
namespace {

constexpr int kBlock = 256;
constexpr int kSlotsPerWave = 16;  // SIMD order: 4 lanes per slot group
constexpr int64_t kWinMinN = 1024;
constexpr int64_t kWinMinSlots = 2048 * kSlotsPerWave;  // 2048 waves

template <bool V4>
__device__ __forceinline__ void load4(const float* p, float& a, float& b, float& c, float& d) {
    if constexpr (V4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(p);
        a = v[0]; b = v[1]; c = v[2]; d = v[3];
    } else {
        a = p[0]; b = p[1]; c = p[2]; d = p[3];
    }
}

// One wave of sddmm_simd_kernel: the 16-slot group wid (wid >= slot_waves: a
// bias-gradient wave).
template <bool V4>
__device__ __forceinline__ void sddmm_simd_wave(
    int64_t wid, int64_t M, int64_t N, int64_t cap_total,
    const int32_t* __restrict__ row_start, const int32_t* __restrict__ row_nnz,
    const int32_t* __restrict__ col, const float* __restrict__ dY,
    const float* __restrict__ X, float* __restrict__ dW, float* __restrict__ dbias,
    int64_t slot_waves) {
    const int lane = threadIdx.x & (kWave - 1);
    const int g = lane >> 2;  // slot within the wave
    const int q = lane & 3;   // owns virtual lanes 4q..4q+3
    if (wid >= slot_waves) {  // wave-uniform: a bias-gradient wave
        if (dbias != nullptr) bias_row_sum(dY, M, N, wid - slot_waves, dbias, N, 1);
        return;
    }
    const int64_t wslot = wid * kSlotsPerWave;
    const int64_t slot = wslot + g;
    const bool in_range = slot < cap_total;
    const WaveRows rows(row_start, M, wslot, min(wslot + kSlotsPerWave - 1, cap_total - 1));

    int64_t row = 0;
    bool live = false;
    int32_t c = 0;
    if (in_range) {
        row = rows.of(row_start, rows.first_row, slot);
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

template <bool V4>
__global__ __launch_bounds__(kBlock) void sddmm_simd_kernel(
    int64_t M, int64_t N, int64_t cap_total,
    const int32_t* __restrict__ row_start, const int32_t* __restrict__ row_nnz,
    const int32_t* __restrict__ col, const float* __restrict__ dY,
    const float* __restrict__ X, float* __restrict__ dW, float* __restrict__ dbias,
    int64_t slot_waves) {
    sddmm_simd_wave<V4>(wave_id(), M, N, cap_total, row_start, row_nnz, col, dY, X, dW, dbias,
                        slot_waves);
}

// Small layers: the whole backward in one launch (slk_backward_fused). The
// first dx_items waves compute dX = WT·dY, one (WT row, 64-column tile) per
// wave and one column per lane: the fma chain over the row's slots in slot
// order from +0.0 — the bits of spmm on WT — with WT's values read as W's
// through perm, so no refresh launch comes first. A 32-slot piece of the row
// at a time: its columns and perm entries, then all its gathers of dY before
// the values through perm, then the fmas. The gathers take no branch (lanes
// past the piece repeat its last slot, columns past N load column N - 1 and
// are not stored): a branch per gather makes the compiler wait for each
// gather before the next. The remaining waves are sddmm_simd_kernel's (dW in
// the SIMD order, and the bias-gradient waves). No barriers: a workgroup may
// hold waves of both.
constexpr int kPermPiece = 32;  // slots per piece: x[] within 64 VGPRs for the whole kernel
__device__ __forceinline__ void spmm_perm_wave(int64_t item, int64_t R, int64_t N,
                                               const int32_t* __restrict__ rs,
                                               const int32_t* __restrict__ nz,
                                               const int32_t* __restrict__ colT,
                                               const int64_t* __restrict__ perm,
                                               const float* __restrict__ vals,
                                               const float* __restrict__ B,
                                               float* __restrict__ out) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t tile = item / R;
    const int64_t r = item - tile * R;
    const int64_t n = tile * kWave + lane;
    const int64_t nc = n < N ? n : N - 1;  // in bounds; not stored past N
    const int32_t start = rs[r], nnz = nz[r];
    float acc = 0.0f;
    for (int32_t k = 0; k < nnz; k += kPermPiece) {
        const int32_t m = nnz - k < kPermPiece ? nnz - k : kPermPiece;  // wave-uniform, >= 1
        const int64_t sl = start + k + (lane < m ? lane : m - 1);
        const int32_t c = colT[sl];
        const int64_t ps = perm[sl];
        float x[kPermPiece];
#pragma unroll
        for (int u = 0; u < kPermPiece; ++u)
            x[u] = B[static_cast<int64_t>(__builtin_amdgcn_readlane(c, u)) * N + nc];
        const float v = vals[ps];
#pragma unroll
        for (int u = 0; u < kPermPiece; ++u)
            if (u < m)
                acc = __builtin_fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), u)),
                                     x[u], acc);
    }
    if (n < N) out[r * N + n] = acc;
}

template <bool V4>
__global__ __launch_bounds__(kBlock) void backward_fused_kernel(
    int64_t dx_items, int64_t KT, const int32_t* __restrict__ rsT,
    const int32_t* __restrict__ nzT, const int32_t* __restrict__ colT,
    const int64_t* __restrict__ perm, float* __restrict__ dX, int64_t M, int64_t N,
    int64_t cap_total, const int32_t* __restrict__ row_start,
    const int32_t* __restrict__ row_nnz, const int32_t* __restrict__ col,
    const float* __restrict__ vals, const float* __restrict__ dY, const float* __restrict__ X,
    float* __restrict__ dW, float* __restrict__ dbias, int64_t slot_waves) {
    const int64_t wid = wave_id();
    if (wid < dx_items) {
        spmm_perm_wave(wid, KT, N, rsT, nzT, colT, perm, vals, dY, dX);
    } else {
        sddmm_simd_wave<V4>(wid - dx_items, M, N, cap_total, row_start, row_nnz, col, dY, X, dW,
                            dbias, slot_waves);
    }
}

// SIMD order, N swept window by window, dY staged in LDS (16-byte path).
//
// Same arithmetic as sddmm_simd_kernel, slot by slot. Two things bound that
// kernel at large N, and this one removes both (measured with rocprofv3 on
// a 2304x768 layer at N=8192):
//  * Locality. Streaming each slot's whole X and dY rows makes the resident
//    waves touch every X row at scattered offsets: L2 hit rate 26%. Here a
//    wave owns G groups of 16 slots and advances all of them through N one
//    256-float window at a time; waves start together and do the same work
//    per window, so at any moment they read one narrow band of X and dY
//    columns, which stays in L2 (87% hits) — the locality tile-major order
//    gives the forward.
//  * Load issue. With locality fixed, the kernel runs at the rate of 16-byte
//    wave loads, and loading dY per lane doubles their count although all 16
//    slots of a group usually share one dY row. Each group instead stages the
//    dY windows of the first and the last row of its slots in LDS, one 1 KB
//    load per row per window, prefetched a window ahead in registers; lanes
//    read their pieces from LDS, so X is the only per-lane stream. A lane
//    whose slot lies in a third row of its group (rows shorter than 16 slots)
//    loads its dY pieces directly.
// The 16 partial sums of every slot stay in registers across windows. The LDS
// region is private to the wave: wave-level fences order its stores and loads.
constexpr int64_t kWin = 256;  // floats per window: 16 steps of 16

__device__ __forceinline__ void fma4x(f32x4 d, f32x4 x, float& a0, float& a1, float& a2,
                                      float& a3) {
    a0 = __builtin_fmaf(d[0], x[0], a0);
    a1 = __builtin_fmaf(d[1], x[1], a1);
    a2 = __builtin_fmaf(d[2], x[2], a2);
    a3 = __builtin_fmaf(d[3], x[3], a3);
}

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Zeroes the padding slots of one row of dW (one wave): used where the slots
// are walked through a schedule that lists live slots only.
__device__ __forceinline__ void zero_row_padding(const int32_t* __restrict__ row_start,
                                                 const int32_t* __restrict__ row_nnz,
                                                 const int32_t* __restrict__ row_cap, int64_t M,
                                                 int64_t row, float* __restrict__ dW) {
    if (row >= M) return;
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t s0 = row_start[row];
    const int64_t e = s0 + row_cap[row];
    for (int64_t s = s0 + row_nnz[row] + lane; s < e; s += kWave) dW[s] = 0.0f;
}

template <int G>
__global__ __launch_bounds__(kBlock) void sddmm_simd_win_kernel(
    int64_t M, int64_t N, int64_t cap_total,
    const int32_t* __restrict__ row_start, const int32_t* __restrict__ row_nnz,
    const int32_t* __restrict__ col, const float* __restrict__ dY,
    const float* __restrict__ X, float* __restrict__ dW, float* __restrict__ dbias,
    int64_t slot_waves) {
    constexpr int kWavesPerBlock = kBlock / kWave;
    constexpr int NS = 2;  // staged dY rows per group: its first and its last
    __shared__ f32x4 dys[kWavesPerBlock][G][NS][kWave];  // 2 KiB per group
    const int lane = threadIdx.x & (kWave - 1);
    const int wv = threadIdx.x >> 6;
    const int g = lane >> 2;
    const int q = lane & 3;
    const int64_t wid = wave_id();
    if (wid >= slot_waves) {  // wave-uniform: a per-row bias wave
        if (dbias != nullptr) bias_row_sum(dY, M, N, wid - slot_waves, dbias, N, 1);
        return;
    }
    // The wave's 16·G slots of the flat capacity space.
    const int64_t space = cap_total;
    const int64_t base = wid * (kSlotsPerWave * G);

    bool in[G], live[G], direct[G];
    int sel[G];
    int32_t rs[G][NS];  // rows whose dY windows group k stages
    int64_t slot_of[G];
    const float* dyr[G];
    const float* xr[G];
    WaveRows rows(row_start, M, base, min(base + kSlotsPerWave * G - 1, cap_total - 1));
    int64_t r = rows.first_row;
    bool any_direct = false;
#pragma unroll
    for (int k = 0; k < G; ++k) {
        const int64_t gbase = base + kSlotsPerWave * k;
        const int64_t e = gbase + g;
        in[k] = e < space;
        live[k] = false;
        slot_of[k] = e;
        if (in[k]) {
            r = rows.of(row_start, r, e);
            live[k] = (e - row_start[r]) < row_nnz[r];
        }
        // first and last row of group k (lane 0 holds its first entry)
        const int last = gbase < space
                             ? 4 * static_cast<int>(min<int64_t>(kSlotsPerWave - 1, space - 1 - gbase))
                             : 0;
        // staged rows: those of the group's first and last entries
        const int32_t ri = static_cast<int32_t>(r);
        rs[k][0] = __builtin_amdgcn_readfirstlane(ri);
        rs[k][NS - 1] = __builtin_amdgcn_readlane(ri, last);
        sel[k] = NS - 1;
        direct[k] = live[k];
#pragma unroll
        for (int b = NS - 1; b >= 0; --b) {  // the first staged copy of this row
            if (ri == rs[k][b]) {
                sel[k] = b;
                direct[k] = false;
            }
        }
        any_direct |= __ballot(direct[k]) != 0;
        dyr[k] = dY + (live[k] ? r * N : 0);
        xr[k] = X + (live[k] ? static_cast<int64_t>(col[slot_of[k]]) * N : 0);
    }
    const int64_t n16 = (N / 16) * 16;
    const int64_t nwin = ceil_div(n16, kWin);
    float acc[G][4];
    f32x4 pst[G][NS];
#pragma unroll
    for (int k = 0; k < G; ++k) {
        acc[k][0] = acc[k][1] = acc[k][2] = acc[k][3] = 0.f;
#pragma unroll
        for (int b = 0; b < NS; ++b) pst[k][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // buffer b is staged only when its row differs from buffer b-1's
    auto fetch = [&](int64_t w) {
        const int64_t j = w * kWin + 4 * lane;
        if (j < n16) {
#pragma unroll
            for (int k = 0; k < G; ++k) {
#pragma unroll
                for (int b = 0; b < NS; ++b) {
                    if (b == 0 || rs[k][b] != rs[k][b - 1])
                        pst[k][b] = *reinterpret_cast<const f32x4*>(
                            dY + static_cast<int64_t>(rs[k][b]) * N + j);
                }
            }
        }
    };
    if (nwin > 0) fetch(0);
    for (int64_t w = 0; w < nwin; ++w) {
#pragma unroll
        for (int k = 0; k < G; ++k) {
#pragma unroll
            for (int b = 0; b < NS; ++b)
                if (b == 0 || rs[k][b] != rs[k][b - 1]) dys[wv][k][b][lane] = pst[k][b];
        }
        wave_sync();
        if (w + 1 < nwin) fetch(w + 1);
        const int64_t j0 = w * kWin;
        const int tn = static_cast<int>(min<int64_t>(16, n16 / 16 - w * 16));
#pragma unroll
        for (int k = 0; k < G; ++k) {
            if (!live[k]) continue;
            const int sk = sel[k];
            const float* xw = xr[k] + j0 + 4 * q;
            if (!any_direct) {
                int t = 0;
                for (; t + 4 <= tn; t += 4) {
                    const f32x4 x0 = *reinterpret_cast<const f32x4*>(xw + 16 * t);
                    const f32x4 x1 = *reinterpret_cast<const f32x4*>(xw + 16 * t + 16);
                    const f32x4 x2 = *reinterpret_cast<const f32x4*>(xw + 16 * t + 32);
                    const f32x4 x3 = *reinterpret_cast<const f32x4*>(xw + 16 * t + 48);
                    fma4x(dys[wv][k][sk][q + 4 * t], x0, acc[k][0], acc[k][1], acc[k][2], acc[k][3]);
                    fma4x(dys[wv][k][sk][q + 4 * t + 4], x1, acc[k][0], acc[k][1], acc[k][2], acc[k][3]);
                    fma4x(dys[wv][k][sk][q + 4 * t + 8], x2, acc[k][0], acc[k][1], acc[k][2], acc[k][3]);
                    fma4x(dys[wv][k][sk][q + 4 * t + 12], x3, acc[k][0], acc[k][1], acc[k][2], acc[k][3]);
                }
                for (; t < tn; ++t)
                    fma4x(dys[wv][k][sk][q + 4 * t], *reinterpret_cast<const f32x4*>(xw + 16 * t),
                          acc[k][0], acc[k][1], acc[k][2], acc[k][3]);
            } else {
                const float* dw = dyr[k] + j0 + 4 * q;
                for (int t = 0; t < tn; ++t) {
                    // the LDS piece is read unconditionally: a branch between an LDS and
                    // a global load gets merged into a load through a select of the two
                    // addresses, which this compiler cannot lower
                    f32x4 d = dys[wv][k][sk][q + 4 * t];
                    if (direct[k]) d = *reinterpret_cast<const f32x4*>(dw + 16 * t);
                    fma4x(d, *reinterpret_cast<const f32x4*>(xw + 16 * t),
                          acc[k][0], acc[k][1], acc[k][2], acc[k][3]);
                }
            }
        }
        wave_sync();  // every lane has read this window before it is overwritten
    }
    // a[l] = v[l] + v[l+8]: lanes q=0,1 take the partner q^2 (v[8..15]).
#pragma unroll
    for (int k = 0; k < G; ++k) {
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[k][e] = acc[k][e] + __shfl_xor(acc[k][e], 2);
    }
    int64_t jt = n16;
    if (N - n16 >= 8) {
        if (q < 2) {
            const int64_t j = n16 + 4 * q;
#pragma unroll
            for (int k = 0; k < G; ++k) {
                if (live[k]) {
                    fma4x(*reinterpret_cast<const f32x4*>(dyr[k] + j),
                          *reinterpret_cast<const f32x4*>(xr[k] + j),
                          acc[k][0], acc[k][1], acc[k][2], acc[k][3]);
                }
            }
        }
        jt += 8;
    }
    // s4[k] = a[k] + a[k+4]: lane q=0 holds a[0..3], lane q=1 holds a[4..7].
#pragma unroll
    for (int k = 0; k < G; ++k) {
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[k][e] = acc[k][e] + __shfl_xor(acc[k][e], 1);
    }
    if (q == 0) {
#pragma unroll
        for (int k = 0; k < G; ++k) {
            if (!in[k]) continue;
            const float rsum = (acc[k][0] + acc[k][2]) + (acc[k][1] + acc[k][3]);
            dW[slot_of[k]] = live[k] ? running_sum(dyr[k] + jt, xr[k] + jt, N - jt, rsum) : 0.0f;
        }
    }
}

// Scalar order (csrc/kernels/spmm_grad.cpp:89-108): one lane per slot, one
// running chain over j.
__global__ __launch_bounds__(kBlock) void sddmm_scalar_kernel(
    int64_t M, int64_t N, int64_t cap_total,
    const int32_t* __restrict__ row_start, const int32_t* __restrict__ row_nnz,
    const int32_t* __restrict__ col, const float* __restrict__ dY,
    const float* __restrict__ X, float* __restrict__ dW, float* __restrict__ dbias,
    int64_t slot_waves) {
    const int64_t wid = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
    if (wid >= slot_waves) {  // wave-uniform: a bias-gradient wave
        if (dbias != nullptr) bias_row_sum(dY, M, N, wid - slot_waves, dbias, N, 1);
        return;
    }
    const int64_t wslot = wid * kWave;
    const WaveRows rows(row_start, M, wslot, min(wslot + kWave - 1, cap_total - 1));
    const int64_t slot = wslot + (threadIdx.x & (kWave - 1));
    if (slot >= cap_total) return;
    const int64_t row = rows.of(row_start, rows.first_row, slot);
    if (slot - row_start[row] >= row_nnz[row]) {
        dW[slot] = 0.0f;
        return;
    }
    const float* dyr = dY + row * N;
    const float* xr = X + static_cast<int64_t>(col[slot]) * N;
    dW[slot] = running_sum(dyr, xr, N, 0.0f);
}



// SIMD order over a segment list: X from LDS, dY in registers (16-byte path).
//
// On gfx950 a 64-lane 16-byte LDS read costs the same whether its lanes read
// one row (a broadcast) or sixteen: about 4.6 cycles per CU measured, so a
// kernel that read both operands of every fma from LDS (two reads per 16
// fmas) would be LDS-bound. Here a quad of lanes owns a segment, up to S
// consecutive live slots of one row inside one column block
// (slk_seg_list_build): the quad loads the row's dY pieces once per step from
// global memory, one window ahead, and applies them to all S slots, whose X
// pieces it reads from LDS. That is S LDS reads and one 64-byte global load
// per S slot-steps. A workgroup of GS quads takes one group of GS segments,
// all in one column block (the list pads each block to a multiple of
// SLK_SEG_GROUP, itself a multiple of GS); for every 64-float window it
// stages the block's C rows of X in LDS
// (rows padded by four 16-byte pieces, so a row starts 16 banks after the
// previous one, the width of one slot's four lanes), prefetched a window
// ahead in registers. Per slot the arithmetic is sddmm_simd_kernel's: the 16
// running sums advance in step order across the windows, then the same
// combine and scalar tail. Empty segments (padding, or slots past a short
// segment's count) compute on a clamped address and store nothing.
// Workgroups past the groups in use (*groups, read on the device) exit at
// once, and so does a group of padding only (a 64-segment half of a block's
// last 128); the workgroups after max_groups are one wave per row that
// zeroes the row's padding slots and, with dbias, sums its dY row. More
// segments per workgroup stage each X window for more slots: 128 on the
// 16384^2 layers (95%: 7.79 -> 6.89 ms, 99%: 2.39 -> 2.22; 256 was slower).
// Visiting each segment's slots in an order that keeps the four rows of an
// LDS pass on different banks (below) took the bank-conflict share of the
// 95% layer's cycles from 35% to 14% and its time 6.91 -> 6.46 ms. Wider
// blocks (256 columns, 8 or 16 slots per segment) measured 8.2-8.4 ms: each
// staged X window then serves fewer slots per byte staged.
constexpr int kSegWin = 64;                  // floats per window (4 steps)
constexpr int kSegPieces = kSegWin / 4;      // 16-byte pieces per row
constexpr int kSegStride = kSegPieces + 4;   // pieces per LDS row (padded)
static_assert(SLK_SEG_GROUP % 128 == 0, "the list padding holds whole groups of 64 and 128");
constexpr int64_t kSegGroupMinGroups = 2048;  // 128-segment groups from this many

// (lean kernels are held to 128 VGPRs, 4 waves per SIMD: at 130 a workgroup
// of 8 waves no longer fits twice per CU; the 128-column, 64-segment one
// would spill there)
template <int C, int S, bool LEAN, int GS>
__global__ __launch_bounds__(GS * 4)
__attribute__((amdgpu_waves_per_eu((LEAN && !(C == 128 && GS == 64)) ? 4 : 1))) void sddmm_seg_kernel(
    int64_t M, int64_t K, int64_t N, const int32_t* __restrict__ row_start,
    const int32_t* __restrict__ row_nnz, const int32_t* __restrict__ row_cap,
    const int32_t* __restrict__ col, const float* __restrict__ dY, const float* __restrict__ X,
    float* __restrict__ dW, float* __restrict__ dbias, const int32_t* __restrict__ seg_start,
    const int32_t* __restrict__ seg_row, const int32_t* __restrict__ seg_count,
    const int32_t* __restrict__ groups, int64_t max_groups) {
    constexpr int kSegThreads = GS * 4;                        // one quad per segment
    constexpr int kSegRowsPerPass = kSegThreads / kSegPieces;  // staged rows per pass
    constexpr int kLoads = C * kSegPieces / kSegThreads;       // staged pieces per thread
    static_assert(kLoads * kSegThreads == C * kSegPieces, "whole rows per pass");
    __shared__ f32x4 xs[C * kSegStride];
    const int wv = threadIdx.x >> 6;
    const int q = threadIdx.x & 3;
    const int64_t grp = blockIdx.x;
    if (grp >= max_groups) {  // block-uniform: per-row waves
        const int64_t row = (grp - max_groups) * (kSegThreads / kWave) + wv;
        zero_row_padding(row_start, row_nnz, row_cap, M, row, dW);
        if (dbias != nullptr) bias_row_sum(dY, M, N, row, dbias, N, 1);
        return;
    }
    // Groups in use G: workgroups [0, G) take them in XCD-contiguous order
    // (a bijection on [0, G)), so the groups an XCD runs together mostly lie
    // in one column block and share its X band in that XCD's L2 (C4 768x3072
    // layer 281 -> 232 us). Ordering the list by row panels to share dY rows
    // instead was slower: the concurrent groups then span many X bands.
    const int64_t G = static_cast<int64_t>(groups[0]) * (SLK_SEG_GROUP / GS);
    if (grp >= G) return;  // block-uniform
    const int64_t e0 = xcd_logical_block(grp, G) * GS;
    if (seg_count[e0] == 0) return;  // padding only: segments precede their block's padding
    const int32_t c_lo = col[seg_start[e0]] / C * C;
    const int64_t e = e0 + (threadIdx.x >> 2);  // this quad's segment
    const int32_t s0 = seg_start[e];
    const int32_t cnt = seg_count[e];
    const int64_t row = seg_row[e];
    // Visiting order of the segment's slots. A 16-lane LDS pass serves four
    // quads, each reading 16 consecutive floats of its slot's X row; a row
    // starts 16·(c mod 4) banks into the 64 (stride kSegStride pieces), so the
    // pass is conflict-free when the four rows differ in c mod 4. Quad j of
    // the pass takes, at step k, a slot with c ≡ k + j (mod 4) where it has
    // one (the slots' results are independent: the order changes no bits),
    // and a step without a slot reads the block row of that residue.
    const int jq = (threadIdx.x >> 2) & 3;
    uint32_t byres[4] = {0u, 0u, 0u, 0u};
    int32_t xo0[S];
#pragma unroll
    for (int k = 0; k < S; ++k) {
        const int32_t c = k < cnt ? col[s0 + k] - c_lo : 0;
        xo0[k] = c * kSegStride + q;
#pragma unroll
        for (int r = 0; r < 4; ++r) byres[r] |= (k < cnt && (c & 3) == r) ? (1u << k) : 0u;
    }
    static_assert(S <= 8, "slot of each step packed in 4 bits");
    // Steps at or past every quad's count are empty in the whole wave: the
    // list sorts each group's segments by count, so a wave's counts are close
    // and it skips those steps two at a time.
    int kmax = cnt;
#pragma unroll
    for (int o = 32; o >= 4; o >>= 1) kmax = max(kmax, __shfl_xor(kmax, o));
    kmax = __builtin_amdgcn_readfirstlane(kmax);
    uint32_t avail = (1u << cnt) - 1u;  // cnt <= S
    int32_t xo[S];
    uint32_t slots = 0xFFFFFFFFu;  // 4 bits per step: its slot, 15 = none
#pragma unroll
    for (int k = 0; k < S; ++k) {
        const int want = (k + jq) & 3;
        const uint32_t bw =
            (want == 0 ? byres[0] : want == 1 ? byres[1] : want == 2 ? byres[2] : byres[3]) & avail;
        const uint32_t m = bw != 0u ? bw : avail;
        const int pick = m != 0u ? __builtin_ctz(m) : -1;
        avail &= ~(m & (0u - m));
        if (pick >= 0)
            slots = (slots & ~(15u << (4 * k))) | (static_cast<uint32_t>(pick) << (4 * k));
        int32_t v = want * kSegStride + q;
#pragma unroll
        for (int i = 0; i < S; ++i) v = pick == i ? xo0[i] : v;
        xo[k] = v;
    }
    // X row of step k (the epilogue's tail), from xo
    auto xrow = [&](int k) { return X + static_cast<int64_t>(c_lo + (xo[k] - q) / kSegStride) * N; };
    const int32_t nC = static_cast<int32_t>(min<int64_t>(C, K - c_lo));

    // staging: thread t copies piece (t mod 16) of block rows t/16 + 16i. Rows
    // past the matrix (a last block narrower than C) and pieces past n16 (a
    // last window shorter than 64 floats) load a clamped, in-bounds address
    // instead: those LDS rows and steps are never read, and the loads stay
    // branch-free.
    const int pc = threadIdx.x % kSegPieces;
    const int rr0 = threadIdx.x / kSegPieces;
    const float* xband = X + static_cast<int64_t>(c_lo) * N;
    uint32_t xoff[kLoads];  // byte offsets in the band: C*N*4 < 2^32 (launcher check)
#pragma unroll
    for (int i = 0; i < kLoads; ++i)
        xoff[i] = static_cast<uint32_t>(min(rr0 + i * kSegRowsPerPass, nC - 1)) *
                  static_cast<uint32_t>(N) * 4u;
    const float* dyr = dY + row * N + 4 * q;
    const int64_t n16 = (N / 16) * 16;  // >= 16 (the launcher's bar)
    const int64_t nwin = ceil_div(n16, kSegWin);
    float acc[S][4];
#pragma unroll
    for (int k = 0; k < S; ++k) acc[k][0] = acc[k][1] = acc[k][2] = acc[k][3] = 0.f;
    f32x4 pre[kLoads];
    f32x4 dcur[kSegWin / 16], dnext[kSegWin / 16];
    auto fetch_x = [&](int64_t w) {
        const uint32_t jx = static_cast<uint32_t>(min<int64_t>(w * kSegWin + 4 * pc, n16 - 4)) * 4u;
#pragma unroll
        for (int i = 0; i < kLoads; ++i)
            pre[i] = *reinterpret_cast<const f32x4*>(reinterpret_cast<const char*>(xband) + xoff[i] + jx);
    };
    auto fetch_dy = [&](int64_t w, f32x4 (&d)[kSegWin / 16]) {
#pragma unroll
        for (int t = 0; t < kSegWin / 16; ++t)
            d[t] = *reinterpret_cast<const f32x4*>(dyr + min<int64_t>(w * kSegWin + 16 * t, n16 - 16));
    };
    // LEAN: dY loaded at the start of its own window (its latency overlaps the
    // LDS store and the barrier) and S/2 X reads in flight, for fewer registers
    constexpr int SH = LEAN ? S / 2 : S;
    fetch_x(0);
    if constexpr (!LEAN) fetch_dy(0, dnext);
    for (int64_t w = 0; w < nwin; ++w) {
        if constexpr (LEAN) fetch_dy(w, dcur);
#pragma unroll
        for (int i = 0; i < kLoads; ++i) xs[(rr0 + i * kSegRowsPerPass) * kSegStride + pc] = pre[i];
        if constexpr (!LEAN) {
#pragma unroll
            for (int t = 0; t < kSegWin / 16; ++t) dcur[t] = dnext[t];
        }
        __syncthreads();
        // the last window refetches itself (unused)
        fetch_x(min(w + 1, nwin - 1));
        if constexpr (!LEAN) fetch_dy(min(w + 1, nwin - 1), dnext);
        const int tn = static_cast<int>(min<int64_t>(kSegWin / 16, n16 / 16 - w * (kSegWin / 16)));
#pragma unroll
        for (int t = 0; t < kSegWin / 16; ++t) {
#pragma unroll
            for (int k0 = 0; k0 < S; k0 += SH) {
                if (t < tn && k0 < kmax) {  // block-uniform, wave-uniform
                    f32x4 x[SH];
#pragma unroll
                    for (int k = 0; k < SH; k += 2) {
                        if (k == 0 || k0 + k < kmax) {
                            x[k] = xs[xo[k0 + k] + 4 * t];
                            x[k + 1] = xs[xo[k0 + k + 1] + 4 * t];
                        }
                    }
#pragma unroll
                    for (int k = 0; k < SH; k += 2) {
                        if (k == 0 || k0 + k < kmax) {
                            fma4x(dcur[t], x[k], acc[k0 + k][0], acc[k0 + k][1],
                                  acc[k0 + k][2], acc[k0 + k][3]);
                            fma4x(dcur[t], x[k + 1], acc[k0 + k + 1][0], acc[k0 + k + 1][1],
                                  acc[k0 + k + 1][2], acc[k0 + k + 1][3]);
                        }
                    }
                }
                // SH reads in flight at a time: hoisting the next reads ahead
                // of these fmas would take 16 registers per read
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __syncthreads();  // every lane has read this window before it is overwritten
    }
    // a[l] = v[l] + v[l+8]: lanes q=0,1 take the partner q^2 (v[8..15]).
#pragma unroll
    for (int k = 0; k < S; ++k) {
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[k][c] = acc[k][c] + __shfl_xor(acc[k][c], 2);
    }
    int64_t jt = n16;
    if (N - n16 >= 8) {
        if (q < 2) {
            const int64_t j = n16 + 4 * q;
            const f32x4 d = *reinterpret_cast<const f32x4*>(dY + row * N + j);
#pragma unroll
            for (int k = 0; k < S; ++k) {
                if (((slots >> (4 * k)) & 15u) != 15u) {
                    fma4x(d, *reinterpret_cast<const f32x4*>(xrow(k) + j), acc[k][0], acc[k][1],
                          acc[k][2], acc[k][3]);
                }
            }
        }
        jt += 8;
    }
    // s4[k] = a[k] + a[k+4]: lane q=0 holds a[0..3], lane q=1 holds a[4..7].
#pragma unroll
    for (int k = 0; k < S; ++k) {
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[k][c] = acc[k][c] + __shfl_xor(acc[k][c], 1);
    }
    if (q == 0) {
#pragma unroll
        for (int k = 0; k < S; ++k) {
            const uint32_t sk = (slots >> (4 * k)) & 15u;
            if (sk == 15u) continue;
            const float rsum = (acc[k][0] + acc[k][2]) + (acc[k][1] + acc[k][3]);
            dW[s0 + sk] = running_sum(dY + row * N + jt, xrow(k) + jt, N - jt, rsum);
        }
    }
}

int sddmm_impl(const slk_csr* W, const float* dY, int64_t dY_rows, const float* X,
               int64_t X_rows, int64_t N, float* dW, float* dbias, int order, void* stream) {
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
    const int64_t bias_waves = dbias != nullptr ? W->nrows : 0;
    if (cap == 0 && bias_waves == 0) return SLK_OK;
    if (dW == nullptr && cap > 0) return fail(SLK_EINVAL, std::string(who) + ": NULL dW");
    hipStream_t st = as_stream(stream);
    if (order == SLK_DW_SCALAR) {
        const int64_t slot_waves = ceil_div(cap, kWave);
        const int64_t blocks = ceil_div(slot_waves + bias_waves, kBlock / kWave);
        if (blocks > INT32_MAX) return fail(SLK_EINVAL, std::string(who) + ": problem too large");
        hipLaunchKernelGGL(sddmm_scalar_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kBlock),
                           0, st, W->nrows, N, cap, W->row_start, W->row_nnz, W->col_indices, dY,
                           X, dW, dbias, slot_waves);
        return check_launch(who);
    }
    const bool v4 = (N % 4 == 0) && (reinterpret_cast<uintptr_t>(X) % 16 == 0) &&
                    (reinterpret_cast<uintptr_t>(dY) % 16 == 0);
    // Windowed sweep (G groups per wave) for the 16-byte path at large N:
    // G = 4 from 2048 waves of 4 groups, G = 2 from 1024 waves of 2 (measured
    // on the C3/C4 layer shapes: the 10M-GPT attention-out layer, 53 k slots,
    // runs 133 -> 105 us with G = 2); SLK_TUNE_SDDMM_G = 1|2|4 overrides G
    // (1 = one group per wave, whole rows).
    int G = 1;
    if (v4 && N >= kWinMinN) G = cap >= 4 * kWinMinSlots ? 4 : cap >= kWinMinSlots ? 2 : 1;
    if (const int64_t t = tuning(SLK_TUNE_SDDMM_G); t >= 0) G = static_cast<int>(t);
    if (!v4 || (G != 2 && G != 4)) G = 1;
    const int64_t slot_waves = ceil_div(cap, kSlotsPerWave * G);
    const int64_t blocks = ceil_div(slot_waves + bias_waves, kBlock / kWave);
    if (blocks > INT32_MAX) return fail(SLK_EINVAL, std::string(who) + ": problem too large");
    const dim3 grid(static_cast<unsigned>(blocks));
#define SLK_SDDMM_ARGS \
    W->nrows, N, cap, W->row_start, W->row_nnz, W->col_indices, dY, X, dW, dbias, slot_waves
    // A segment list: X through LDS, dY rows in registers.
    // (C·N floats of a band addressed with 32-bit byte offsets)
    if (v4 && W->seg_start != nullptr && N >= 16 && W->seg_block * N * 4 < (int64_t{1} << 32)) {
        // A list without the dense rows: those on the matrix cores first
        // (the segment kernel's per-row waves still zero their padding and
        // sum their dbias).
        if (W->seg_dense_rows > 0) {
            if (W->seg_dense_rows != W->n_dense_rows || W->dense_ws == nullptr ||
                !dense_dw_apply(W->n_dense_rows, W->nrows, W->ncols, N)) {
                return fail(SLK_EINVAL, std::string(who) +
                                            ": a segment list without the dense rows needs "
                                            "seg_dense_rows == n_dense_rows, dense_ws and N a "
                                            "multiple of 64");
            }
            if (int rc = sddmm_dense_rows(W, dY, X, N, dW, st)) return rc;
        }
        // 128 segments per workgroup on large lists (below, 64: measured on
        // the 60M-GPT layers); SLK_TUNE_SEG_GROUP = 64|128 overrides
        int gs = W->n_seg >= int64_t{128} * kSegGroupMinGroups ? 128 : 64;
        if (const int64_t t = tuning(SLK_TUNE_SEG_GROUP); t == 64 || t == 128) gs = static_cast<int>(t);
        const int64_t max_groups = W->n_seg / gs;
        const int64_t sblocks = max_groups + ceil_div(W->nrows, int64_t{gs * 4 / kWave});
        if (sblocks > INT32_MAX) return fail(SLK_EINVAL, std::string(who) + ": problem too large");
#define SLK_SEG_ARGS                                                                         \
    W->nrows, W->ncols, N, W->row_start, W->row_nnz, W->row_capacity, W->col_indices, dY, X, \
        dW, dbias, W->seg_start, W->seg_row, W->seg_count, W->seg_groups, max_groups
        const dim3 sgrid(static_cast<unsigned>(sblocks));
        // 8-slot segments: the lean variant (4 waves per SIMD at 64 columns,
        // 3 at 128; 2-15% faster on the 60M-GPT and 16384^2 layers). 4-slot
        // segments, used where rows hold few slots per block, keep dY loaded a
        // window ahead: their quads touch many different dY rows (16384^2 at
        // 99%: 2.6 ms against 3.6 lean). SLK_TUNE_SEG_LEAN = 0|1 overrides.
        bool lean = W->seg_slots == 8;
        if (const int64_t t = tuning(SLK_TUNE_SEG_LEAN); t >= 0) lean = t == 1;
#define SLK_SEG_LAUNCH_GS(CB, SS, GS)                                                        \
    do {                                                                                     \
        if (lean) {                                                                          \
            hipLaunchKernelGGL((sddmm_seg_kernel<CB, SS, true, GS>), sgrid, dim3(GS * 4), 0, \
                               st, SLK_SEG_ARGS);                                            \
        } else {                                                                             \
            hipLaunchKernelGGL((sddmm_seg_kernel<CB, SS, false, GS>), sgrid, dim3(GS * 4), 0, \
                               st, SLK_SEG_ARGS);                                            \
        }                                                                                    \
    } while (0)
#define SLK_SEG_LAUNCH(CB, SS)                            \
    do {                                                  \
        if (gs == 128) SLK_SEG_LAUNCH_GS(CB, SS, 128);    \
        else SLK_SEG_LAUNCH_GS(CB, SS, 64);               \
    } while (0)
        if (W->seg_block == 64 && W->seg_slots == 4) SLK_SEG_LAUNCH(64, 4);
        else if (W->seg_block == 64) SLK_SEG_LAUNCH(64, 8);
        else if (W->seg_slots == 4) SLK_SEG_LAUNCH(128, 4);
        else SLK_SEG_LAUNCH(128, 8);
#undef SLK_SEG_LAUNCH
#undef SLK_SEG_LAUNCH_GS
#undef SLK_SEG_ARGS
        return check_launch(who);
    }
    if (G == 2) {
        hipLaunchKernelGGL(sddmm_simd_win_kernel<2>, grid, dim3(kBlock), 0, st, SLK_SDDMM_ARGS);
    } else if (G == 4) {
        hipLaunchKernelGGL(sddmm_simd_win_kernel<4>, grid, dim3(kBlock), 0, st, SLK_SDDMM_ARGS);
    } else if (v4) {
        hipLaunchKernelGGL(sddmm_simd_kernel<true>, grid, dim3(kBlock), 0, st, SLK_SDDMM_ARGS);
    } else {
        hipLaunchKernelGGL(sddmm_simd_kernel<false>, grid, dim3(kBlock), 0, st, SLK_SDDMM_ARGS);
    }
#undef SLK_SDDMM_ARGS
    return check_launch(who);
}

}  // namespace
}  // namespace slk

extern "C" int slk_sddmm(const slk_csr* W, const float* dY, int64_t dY_rows, const float* X,
                         int64_t X_rows, int64_t N, float* dW, int order, void* stream) {
    return slk::sddmm_impl(W, dY, dY_rows, X, X_rows, N, dW, nullptr, order, stream);
}

extern "C" int slk_sddmm_bias(const slk_csr* W, const float* dY, int64_t dY_rows, const float* X,
                              int64_t X_rows, int64_t N, float* dW, float* dbias, int order,
                              void* stream) {
    if (dbias == nullptr && W != nullptr && W->nrows > 0) {
        slk::clear_error();
        return slk::fail(SLK_EINVAL, "spmm_grad_w: NULL dbias");
    }
    return slk::sddmm_impl(W, dY, dY_rows, X, X_rows, N, dW, dbias, order, stream);
}

extern "C" int slk_backward_fused(const slk_csr* W, const slk_csr* WT, const int64_t* perm,
                                  const float* dY, const float* X, int64_t N, float* dW,
                                  float* dbias, float* dX, void* stream) {
    using namespace slk;
    clear_error();
    const char* who = "backward_fused";
    if (int rc = validate_csr(W, who)) return rc;
    if (WT == nullptr) return fail(SLK_EINVAL, "backward_fused: NULL WT");
    if (WT->nrows != W->ncols || WT->ncols != W->nrows || WT->row_start == nullptr ||
        WT->row_nnz == nullptr || (WT->total_capacity > 0 && WT->col_indices == nullptr))
        return fail(SLK_EINVAL, "backward_fused: WT is not W's transpose (shape or arrays)");
    if (N < 0) return fail(SLK_EINVAL, "backward_fused: negative N");
    const int64_t M = W->nrows, K = W->ncols, cap = W->total_capacity;
    if (cap > 0 && (dW == nullptr || W->values == nullptr))
        return fail(SLK_EINVAL, "backward_fused: NULL dW or W values");
    if (WT->total_capacity > 0 && perm == nullptr)
        return fail(SLK_EINVAL, "backward_fused: NULL perm");
    if (N > 0 && ((M > 0 && dY == nullptr) || (K > 0 && (X == nullptr || dX == nullptr))))
        return fail(SLK_EINVAL, "backward_fused: NULL dY, X or dX");
    const int64_t dx_items = N > 0 ? K * ceil_div(N, int64_t{kWave}) : 0;
    const int64_t slot_waves = ceil_div(cap, int64_t{kSlotsPerWave});
    const int64_t bias_waves = dbias != nullptr ? M : 0;
    const int64_t waves = dx_items + slot_waves + bias_waves;
    if (waves == 0) return SLK_OK;
    const int64_t blocks = ceil_div(waves, int64_t{kBlock / kWave});
    if (blocks > INT32_MAX) return fail(SLK_EINVAL, "backward_fused: problem too large");
    hipStream_t st = as_stream(stream);
    const bool v4 = (N % 4 == 0) && (reinterpret_cast<uintptr_t>(X) % 16 == 0) &&
                    (reinterpret_cast<uintptr_t>(dY) % 16 == 0);
#define SLK_FUSED_ARGS                                                                         \
    dx_items, K, WT->row_start, WT->row_nnz, WT->col_indices, perm, dX, M, N, cap, W->row_start, \
        W->row_nnz, W->col_indices, W->values, dY, X, dW, dbias, slot_waves
    if (v4) {
        hipLaunchKernelGGL(backward_fused_kernel<true>, dim3(static_cast<unsigned>(blocks)),
                           dim3(kBlock), 0, st, SLK_FUSED_ARGS);
    } else {
        hipLaunchKernelGGL(backward_fused_kernel<false>, dim3(static_cast<unsigned>(blocks)),
                           dim3(kBlock), 0, st, SLK_FUSED_ARGS);
    }
#undef SLK_FUSED_ARGS
    return check_launch(who);
}
