// Device helpers shared by the weight-gradient launches (sddmm.hip,
// narrow.hip): the row of a slot, the reference's scalar running sum and the
// bias-gradient row sum.
#pragma once

#include "common.hpp"

namespace slk {

// Largest r in [lo, hi) with row_start[r] <= slot, given row_start[lo] <= slot
// (rows tile [0, cap) in order, so this is the row holding the slot).
__device__ __forceinline__ int64_t row_in_range(const int32_t* __restrict__ row_start,
                                                int64_t lo, int64_t hi, int64_t slot) {
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (row_start[mid] <= slot) lo = mid; else hi = mid;
    }
    return lo;
}

// The same for a wave-uniform slot, searched by the whole wave: each round
// the 64 lanes probe 64 evenly spaced rows and a ballot keeps the interval
// between the last probe <= slot and the next one. A 16384-row matrix takes
// 3 dependent loads instead of a binary search's 14. Every lane must call it.
__device__ __forceinline__ int64_t wave_row_of_slot(const int32_t* __restrict__ row_start,
                                                    int64_t M, int64_t slot) {
    const int lane = threadIdx.x & (kWave - 1);
    int64_t lo = 0, hi = M;  // row_start[lo] <= slot; hi == M or row_start[hi] > slot
    while (hi - lo > 1) {
        const int64_t step = ceil_div(hi - lo, kWave);
        const int64_t p = lo + static_cast<int64_t>(lane + 1) * step;
        const bool le = p < hi && row_start[p] <= slot;  // a prefix of the lanes
        lo += static_cast<int64_t>(__popcll(__ballot(le))) * step;
        hi = min(hi, lo + step);
    }
    return lo;
}

// Rows of the slots [first, last] of a wave (wave-uniform bounds, every lane
// calls it): the two ends by wave search, then each lane narrows its own slot
// inside that range (usually zero or one step).
struct WaveRows {
    int64_t first_row = 0, last_row = 0;
    WaveRows() = default;
    __device__ __forceinline__ WaveRows(const int32_t* __restrict__ row_start, int64_t M,
                                        int64_t first, int64_t last)
        : first_row(wave_row_of_slot(row_start, M, first)),
          last_row(wave_row_of_slot(row_start, M, last)) {}
    __device__ __forceinline__ int64_t of(const int32_t* __restrict__ row_start, int64_t from,
                                          int64_t slot) const {
        return row_in_range(row_start, from, last_row + 1, slot);
    }
};

// acc += a[j·sa] * b[j] for j < n: unfused in-order adds for the first
// 4*floor(n/4) terms, fused multiply-adds for the rest (sa: a's stride).
__device__ __forceinline__ float running_sum(const float* __restrict__ a,
                                             const float* __restrict__ b, int64_t n, float acc,
                                             int64_t sa = 1) {
    const int64_t n4 = n & ~int64_t{3};
    int64_t j = 0;
    for (; j < n4; ++j) {
        const float p = a[j * sa] * b[j];
        acc = acc + p;
    }
    for (; j < n; ++j) acc = __builtin_fmaf(a[j * sa], b[j], acc);
    return acc;
}

// dbias[row] = sum_j dY[row, j], one wave per row: lane-strided partial sums
// combined by a butterfly, so the order is fixed and the result repeatable.
// This is the gradient of SparseLinear's bias add (sparselab/nn.py:237-241),
// which torch's autograd forms as a separate reduction; here it rides in the
// weight-gradient launch as extra waves. dY[row, j] sits at
// dY[row·rs + j·js] (row-major: rs = N, js = 1; token-major: rs = 1, js = M).
__device__ __forceinline__ void bias_row_sum(const float* __restrict__ dY, int64_t M, int64_t N,
                                             int64_t row, float* __restrict__ dbias,
                                             int64_t rs, int64_t js) {
    if (row >= M) return;
    const int lane = threadIdx.x & (kWave - 1);
    const float* p = dY + row * rs;
    float acc = 0.0f;
    for (int64_t j = lane; j < N; j += kWave) acc = acc + p[j * js];
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) acc = acc + __shfl_xor(acc, off);
    if (lane == 0) dbias[row] = acc;
}

}  // namespace slk
