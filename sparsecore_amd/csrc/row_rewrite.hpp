// Per-row pieces of the SET / RigL topology update, shared by the drop/grow
// kernels (topology.hip: exact keys; rigl.hip: keys certified from an
// approximate gradient). One 256-thread workgroup owns one row; survivors and
// grown columns are bitmaps over the row's columns in LDS.
//
// Reference rule (sparselab/router.py:429-478 SET, :676-732 RigL): keep the
// live slots with |v| > threshold; if none survives, keep the first slot of
// largest |v|; grow columns outside the kept set with value 0; rewrite the row
// sorted by column (PaddedCSR.rewrite_row, csrc/kernels/padded_csr.cpp:219-296).
#pragma once

#include "common.hpp"

namespace slk {
namespace {

constexpr int kRowThreads = 256;

// Inclusive scan of one int64 per thread over a workgroup of kRowThreads
// threads: a shuffle scan inside each wave, then the wave totals. tmp holds
// kRowThreads entries and keeps the scan on return (tmp[kRowThreads - 1] is
// the total).
__device__ int64_t block_inclusive_scan(int64_t v, int64_t* tmp) {
    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int w = t / kWave;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const int64_t up = __shfl_up(v, off);
        if (lane >= off) v += up;
    }
    __shared__ int64_t wsum[kRowThreads / kWave];
    if (lane == kWave - 1) wsum[w] = v;
    __syncthreads();
    for (int q = 0; q < w; ++q) v += wsum[q];
    tmp[t] = v;
    __syncthreads();
    return v;
}

__device__ __forceinline__ bool bit_of(const uint32_t* bm, int64_t c) {
    return (bm[c >> 5] >> (c & 31)) & 1u;
}

// Marks the row's survivors in `keep` (zeroed by the caller, followed by a
// barrier) and returns their count: live slots with |v| > thr, or, if none,
// the first slot of largest |v| (np.argmax over |v|, NaN above everything).
__device__ int64_t mark_survivors(const float* __restrict__ values,
                                  const int32_t* __restrict__ cols, int32_t start,
                                  int32_t n_live, float thr, uint32_t* keep, int64_t* tmp,
                                  unsigned long long* s_best) {
    const int t = threadIdx.x;
    if (t == 0) *s_best = 0;
    __syncthreads();
    int64_t kept = 0;
    unsigned long long best = 0;
    // four slots per thread per pass, their loads issued before any use (a
    // long row then costs one memory latency per 1024 slots, not per 256)
    constexpr int kU = 4;
    for (int32_t s0 = t; s0 < n_live; s0 += kU * kRowThreads) {
        uint32_t u[kU];
        int32_t c[kU];
#pragma unroll
        for (int q = 0; q < kU; ++q) {
            const int32_t s = s0 + q * kRowThreads;
            const int32_t sc = s < n_live ? s : n_live - 1;  // in the row, unused past it
            u[q] = __float_as_uint(fabsf(values[start + sc]));
            c[q] = cols[start + sc];
        }
#pragma unroll
        for (int q = 0; q < kU; ++q) {
            const int32_t s = s0 + q * kRowThreads;
            if (s >= n_live) continue;
            if (__uint_as_float(u[q]) > thr) {
                ++kept;
                atomicOr(&keep[c[q] >> 5], 1u << (c[q] & 31));
            }
            const unsigned long long key = (static_cast<unsigned long long>(u[q]) << 32) |
                                           (0xFFFFFFFFull - static_cast<uint32_t>(s));
            if (key > best) best = key;
        }
    }
    block_inclusive_scan(kept, tmp);
    int64_t n_keep = tmp[kRowThreads - 1];
    __syncthreads();
    if (n_keep == 0) {
        atomicMax(s_best, best);
        __syncthreads();
        if (t == 0) {
            const int32_t s = static_cast<int32_t>(0xFFFFFFFFull - (*s_best & 0xFFFFFFFFull));
            const int32_t c = cols[start + s];
            keep[c >> 5] |= 1u << (c & 31);
        }
        n_keep = 1;
        __syncthreads();
    }
    return n_keep;
}

// Writes the new row: the survivors (keep) with their values and the grown
// columns (grow) with 0.0, sorted by column, through the row's staging area;
// slots past n_keep + n_grow become padding (-1, 0) and lower row_nnz[i],
// adding the removed slots to *removed. wpre holds Kw words of LDS scratch.
__device__ void write_back_row(const uint32_t* keep, const uint32_t* grow, uint32_t* wpre,
                               int64_t Kw, int64_t i, int32_t start, int32_t n_live,
                               int64_t n_keep, int64_t n_grow, float* __restrict__ values,
                               int32_t* __restrict__ cols, int32_t* __restrict__ row_nnz,
                               int32_t* __restrict__ stage_col, float* __restrict__ stage_val,
                               unsigned long long* __restrict__ removed, int64_t* tmp) {
    const int t = threadIdx.x;
    // Slot of column c in the new row = number of marked columns below c.
    const int64_t per = ceil_div(Kw, kRowThreads);
    const int64_t w0 = t * per;
    const int64_t w1 = w0 + per < Kw ? w0 + per : Kw;
    int64_t cnt = 0;
    for (int64_t w = w0; w < w1; ++w) cnt += __popc(keep[w] | grow[w]);
    const int64_t incl = block_inclusive_scan(cnt, tmp);
    int64_t run = incl - cnt;
    for (int64_t w = w0; w < w1; ++w) {
        wpre[w] = static_cast<uint32_t>(run);
        run += __popc(keep[w] | grow[w]);
    }
    __syncthreads();

    auto rank_of = [&](int64_t c) -> int64_t {
        const uint32_t word = keep[c >> 5] | grow[c >> 5];
        const uint32_t below_mask = (c & 31) ? (0xFFFFFFFFu >> (32 - (c & 31))) : 0u;
        return static_cast<int64_t>(wpre[c >> 5]) + __popc(word & below_mask);
    };
    // (keep and grow hold n_keep + n_grow <= n_live columns, so every rank
    // is below n_live; the guards keep any miscount inside the row)
    for (int32_t s = t; s < n_live; s += kRowThreads) {
        const int32_t c = cols[start + s];
        if (bit_of(keep, c)) {
            const int64_t r = rank_of(c);
            if (r < n_live) {
                stage_col[start + r] = c;
                stage_val[start + r] = values[start + s];
            }
        }
    }
    for (int64_t w = t; w < Kw; w += kRowThreads) {
        uint32_t bits = grow[w];
        while (bits) {
            const int b = __builtin_ctz(bits);
            bits &= bits - 1;
            const int64_t c = w * 32 + b;
            const int64_t r = rank_of(c);
            if (r < n_live) {
                stage_col[start + r] = static_cast<int32_t>(c);
                stage_val[start + r] = 0.0f;
            }
        }
    }
    __syncthreads();
    // The new row is n_keep + n_grow slots; a RigL row short of growable
    // columns pads the rest (col -1, value 0) and records its new length.
    const int64_t n_new = n_keep + n_grow;
    for (int32_t s = t; s < n_live; s += kRowThreads) {
        const bool live_s = s < n_new;
        cols[start + s] = live_s ? stage_col[start + s] : -1;
        values[start + s] = live_s ? stage_val[start + s] : 0.0f;
    }
    if (t == 0 && n_new < n_live) {
        row_nnz[i] = static_cast<int32_t>(n_new);
        atomicAdd(removed, static_cast<unsigned long long>(n_live - n_new));
    }
}

// hist[bin] += 1 for every lane with `valid`, the wave's lanes sharing a bin
// folded into one atomic (radix digits of float magnitudes are often one
// value across a whole row: one atomic per lane would serialize on it). Two
// folding rounds, then one atomic per remaining lane. Every lane of the wave
// must call it.
__device__ __forceinline__ void hist_add(uint32_t* hist, uint32_t bin, bool valid) {
    const int lane = threadIdx.x & (kWave - 1);
    uint64_t pend = __ballot(valid);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        if (pend == 0) break;
        const int leader = __ffsll(static_cast<unsigned long long>(pend)) - 1;
        // (a lane read into a scalar register: no LDS round trip, unlike a shuffle)
        const uint32_t b = __builtin_amdgcn_readlane(bin, leader);
        const uint64_t same = __ballot(valid && bin == b) & pend;
        if (lane == leader) atomicAdd(&hist[b], static_cast<uint32_t>(__popcll(same)));
        pend &= ~same;
    }
    if ((pend >> lane) & 1ull) atomicAdd(&hist[bin], 1u);
}

// Selects, among `n` candidates given by cand(e) -> (column, key, ok), the
// `need` with the smallest 32-bit keys, ties to the lower column, and sets
// their columns in `grow`. Candidates must be enumerated in ascending column
// order by index e (0 <= e < n). Radix select with 8-bit digits, then one
// ordered take pass. hist: 256 words; s_digit, s_below: shared scalars.
template <class Cand>
__device__ void select_smallest_keys(Cand cand, int64_t n, int64_t need, uint32_t* grow,
                                     uint32_t* hist, uint32_t* s_digit, int64_t* s_below,
                                     int64_t* tmp) {
    const int t = threadIdx.x;
    if (need <= 0) return;
    uint32_t prefix = 0;
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        hist[t] = 0;
        __syncthreads();
        const int64_t n_pad = ceil_div(n, kRowThreads) * kRowThreads;  // uniform trip count
        for (int64_t e = t; e < n_pad; e += kRowThreads) {
            int64_t c = 0;
            uint32_t u = 0;
            const bool ok = e < n && cand(e, c, u) &&
                            (pass == 0 || (u >> (shift + 8)) == prefix);
            hist_add(hist, (u >> shift) & 255u, ok);
        }
        __syncthreads();
        const int64_t h = hist[t];
        const int64_t incl = block_inclusive_scan(h, tmp);
        if (incl - h < need && need <= incl) {
            *s_digit = static_cast<uint32_t>(t);
            *s_below = incl - h;
        }
        __syncthreads();
        prefix = (prefix << 8) | *s_digit;
        need -= *s_below;
        __syncthreads();
    }
    // every key below the selected one, and the first `need` (by column)
    // whose key equals it
    const uint32_t T = prefix;
    int64_t taken_eq = 0;
    for (int64_t e0 = 0; e0 < n; e0 += kRowThreads) {
        const int64_t e = e0 + t;
        bool lt = false, eq = false;
        int64_t c = 0;
        if (e < n) {
            uint32_t u;
            if (cand(e, c, u)) {
                lt = u < T;
                eq = u == T;
            }
        }
        const int64_t incl = block_inclusive_scan(eq ? 1 : 0, tmp);
        const int64_t chunk_eq = tmp[kRowThreads - 1];
        if (lt || (eq && taken_eq + incl - 1 < need)) atomicOr(&grow[c >> 5], 1u << (c & 31));
        taken_eq += chunk_eq;
        __syncthreads();
    }
    __syncthreads();
}

}  // namespace
}  // namespace slk
