// On-device transpose of a padded-CSR matrix, plus the cache-hit refresh.
//
// Reference: sparselab/layout.py:460-536 (transpose_with_perm) builds WT
// (ncols x nrows) with padding ratio pr and perm[t] = W slot feeding WT slot t
// (-1 on padding). Each WT row lists its source rows in ascending order (a
// stable argsort of the column stream), which — together with the capacity
// rule max(1, ceil(nnz * (1 + pr))) in float64 (layout.py:46-68) — fixes
// every output array uniquely. This file computes the same arrays as a
// counting sort keyed by column:
//
//   T1 hist    one workgroup per block of B consecutive W rows counts the
//              block's columns in LDS and writes bh[b][c].
//   T2 colscan turns bh[.][c] into the exclusive prefix over blocks (the
//              block's starting rank inside WT row c), 16 waves per 64
//              columns, and writes WT row_nnz / row_capacity.
//   T3 scan    exclusive scan of the WT capacities -> WT row_start, capT.
//   (host)     reads capT, allocates the WT slot arrays.
//   T4 pad     writes padding slots (col -1, value 0, perm -1), one wave
//              per WT row.
//   T5 scatter places every live slot at WT row_start[c] + rank. With at
//              most 32 rows per block (every shape up to 2^29 entries of
//              M x K), one workgroup per block marks, per column, which of
//              its rows hold it (bit r - r0 of an LDS word; a row's columns
//              are distinct), and the rank of slot (r, c) is the block's
//              start in WT row c plus the number of earlier rows of the
//              block marked at c: every slot is placed in parallel, and the
//              order (rows ascending within a WT row) is the stable one.
//              Larger blocks use one wave that walks the rows in order with
//              a running rank per column in LDS.
//
// Integer atomics appear only in T1's LDS histogram (counts are
// order-independent). Columns are processed in chunks of kColChunk so the LDS
// footprint stays bounded for any ncols.
//
// For ncols <= 65535 and 2^20+ slots the same arrays come from a stable
// radix sort by column instead (the radix path, further below), which needs
// no searches.
#include "common.hpp"

namespace slk {
namespace {

constexpr int kColChunk = 16384;          // LDS counters per pass (64 KiB)
constexpr int64_t kHistBudget = 1 << 24;  // max bh entries (64 MiB)

struct BlockPlan {
    int64_t rows_per_block;
    int64_t nblk;
};

BlockPlan plan_blocks(int64_t M, int64_t K) {
    BlockPlan p{1, 0};
    if (M <= 0) return p;
    int64_t target = ceil_div(M, 4);
    const int64_t cap_by_budget = K > 0 ? kHistBudget / K : target;
    if (cap_by_budget < target) target = cap_by_budget;
    if (target < 1) target = 1;
    p.rows_per_block = ceil_div(M, target);
    p.nblk = ceil_div(M, p.rows_per_block);
    return p;
}

__global__ __launch_bounds__(256) void tr_hist_kernel(
    int64_t M, int64_t K, int64_t B, const int32_t* __restrict__ row_start,
    const int32_t* __restrict__ row_capacity, const int32_t* __restrict__ col,
    int32_t* __restrict__ bh) {
    extern __shared__ int32_t hist[];
    const int64_t b = blockIdx.x;
    const int64_t r0 = b * B;
    const int64_t r1 = (r0 + B < M) ? r0 + B : M;
    const int64_t lo = row_start[r0];
    const int64_t hi = static_cast<int64_t>(row_start[r1 - 1]) + row_capacity[r1 - 1];
    for (int64_t c0 = 0; c0 < K; c0 += kColChunk) {
        const int64_t kc = (K - c0 < kColChunk) ? K - c0 : kColChunk;
        for (int64_t t = threadIdx.x; t < kc; t += blockDim.x) hist[t] = 0;
        __syncthreads();
        // Padding slots carry col = -1 (PaddedCSR invariant 5+7), live slots
        // carry their column, so the flat slot range of the block suffices.
        for (int64_t s = lo + threadIdx.x; s < hi; s += blockDim.x) {
            const int64_t c = col[s] - c0;
            if (c >= 0 && c < kc) atomicAdd(&hist[c], 1);
        }
        __syncthreads();
        for (int64_t t = threadIdx.x; t < kc; t += blockDim.x) bh[b * K + c0 + t] = hist[t];
        __syncthreads();
    }
}

// T2: 16 waves per workgroup, one lane per column: wave w sums its share of
// the blocks for the workgroup's 64 columns (coalesced rows of bh), the
// partial sums are combined in LDS, and each wave rewrites its share as the
// exclusive prefix.
constexpr int kColScanWaves = 16;

__global__ __launch_bounds__(kColScanWaves * kWave) void tr_colscan_kernel(
    int64_t K, int64_t nblk, double one_plus_pr, int32_t* __restrict__ bh,
    int32_t* __restrict__ nnz_t, int32_t* __restrict__ cap_t, bool write_prefix) {
    __shared__ int32_t part[kColScanWaves][kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int w = threadIdx.x >> 6;
    const int64_t c = static_cast<int64_t>(blockIdx.x) * kWave + lane;
    const bool ok = c < K;
    const int64_t per = ceil_div(nblk, kColScanWaves);
    const int64_t b0 = min(nblk, w * per);
    const int64_t b1 = min(nblk, b0 + per);
    int32_t sum = 0;
    if (ok) {
        constexpr int G = 8;  // blocks per group: the group's loads go out first
        for (int64_t g = b0; g < b1; g += G) {
            int32_t x[G];
#pragma unroll
            for (int q = 0; q < G; ++q) x[q] = g + q < b1 ? bh[(g + q) * K + c] : 0;
#pragma unroll
            for (int q = 0; q < G; ++q) sum += x[q];
        }
    }
    part[w][lane] = sum;
    __syncthreads();
    int32_t run = 0;
    for (int v = 0; v < w; ++v) run += part[v][lane];
    if (ok && write_prefix) {
        for (int64_t b = b0; b < b1; ++b) {
            const int32_t t = bh[b * K + c];
            bh[b * K + c] = run;
            run += t;
        }
    } else if (ok) {
        run += sum;
    }
    if (ok && w == kColScanWaves - 1) {  // the last share ends at the column total
        nnz_t[c] = run;
        // layout.py:66-67: np.maximum(1, np.ceil(nnz.astype(float64) * (1 + pr))).astype(int32)
        const double scaled = ceil(static_cast<double>(run) * one_plus_pr);
        cap_t[c] = scaled < 1.0 ? 1 : static_cast<int32_t>(scaled);
    }
}

constexpr int kScanThreads = 1024;

// T3 (and R3): one workgroup of 16 waves; wave w owns a contiguous range of
// columns, read 64 at a time (coalesced). start_t = exclusive scan of cap_t,
// *cap_total its sum; where nnz_t is given, also off[c] = start_t[c] -
// (exclusive scan of nnz_t)[c] (the padding before column c's run in WT) and
// *nlive the sum of nnz_t. Pass 1 sums each wave's range, the wave totals
// are scanned in LDS, pass 2 scans each 64-column step by shuffles.
__global__ __launch_bounds__(kScanThreads) void tr_scan_kernel(
    int64_t K, const int32_t* __restrict__ cap_t, int32_t* __restrict__ start_t,
    int64_t* __restrict__ cap_total, const int32_t* __restrict__ nnz_t,
    int32_t* __restrict__ off, int64_t* __restrict__ nlive) {
    constexpr int kWaves = kScanThreads / kWave;
    __shared__ int64_t wc[kWaves], wn[kWaves];
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x >> 6;
    const bool two = nnz_t != nullptr;
    const int64_t per = ceil_div(ceil_div(K, kWaves), kWave) * kWave;
    const int64_t lo = w * per < K ? w * per : K;
    const int64_t hi = lo + per < K ? lo + per : K;
    constexpr int G = 8;  // steps per group: the group's loads go out first
    int64_t sc = 0, sn = 0;
    for (int64_t g0 = lo; g0 < hi; g0 += G * kWave) {
        int32_t xc[G], xn[G];
#pragma unroll
        for (int q = 0; q < G; ++q) {
            const int64_t c = g0 + q * kWave + lane;
            xc[q] = c < hi ? cap_t[c] : 0;
            xn[q] = (two && c < hi) ? nnz_t[c] : 0;
        }
#pragma unroll
        for (int q = 0; q < G; ++q) {
            sc += xc[q];
            sn += xn[q];
        }
    }
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) {
        sc += __shfl_xor(sc, o);
        sn += __shfl_xor(sn, o);
    }
    if (lane == 0) {
        wc[w] = sc;
        wn[w] = sn;
    }
    __syncthreads();
    if (threadIdx.x == 0) {  // the wave totals become exclusive prefixes
        int64_t ac = 0, an = 0;
        for (int q = 0; q < kWaves; ++q) {
            const int64_t xc = wc[q], xn = wn[q];
            wc[q] = ac;
            wn[q] = an;
            ac += xc;
            an += xn;
        }
        *cap_total = ac;
        if (two) *nlive = an;
    }
    __syncthreads();
    int64_t rc = wc[w], rn = wn[w];
    // Pass 2: the G steps of a group are scanned together, one shuffle round
    // for all of them at a time, so their LDS round trips overlap. Within a
    // step the sums are int32: they stay below the WT capacity, which the
    // caller checks against the int32 slot range before any fill uses them.
    for (int64_t g0 = lo; g0 < hi; g0 += G * kWave) {
        int32_t yc[G], yn[G], ic[G], in[G];
#pragma unroll
        for (int q = 0; q < G; ++q) {
            const int64_t c = g0 + q * kWave + lane;
            yc[q] = c < hi ? cap_t[c] : 0;
            yn[q] = (two && c < hi) ? nnz_t[c] : 0;
            ic[q] = yc[q];
            in[q] = yn[q];
        }
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) {
            int32_t uc[G], un[G];
#pragma unroll
            for (int q = 0; q < G; ++q) {
                uc[q] = __shfl_up(ic[q], o);
                un[q] = two ? __shfl_up(in[q], o) : 0;
            }
#pragma unroll
            for (int q = 0; q < G; ++q) {
                if (lane >= o) {
                    ic[q] += uc[q];
                    in[q] += un[q];
                }
            }
        }
#pragma unroll
        for (int q = 0; q < G; ++q) {
            const int64_t c = g0 + q * kWave + lane;
            if (c < hi) {
                start_t[c] = static_cast<int32_t>(rc + ic[q] - yc[q]);
                if (two) off[c] = static_cast<int32_t>((rc + ic[q] - yc[q]) - (rn + in[q] - yn[q]));
            }
            rc += static_cast<uint32_t>(__shfl(ic[q], kWave - 1));
            if (two) rn += static_cast<uint32_t>(__shfl(in[q], kWave - 1));
        }
    }
}

// T3 / R3 for ncols <= kScanLdsMax: the same outputs as tr_scan_kernel from
// one round of coalesced loads into LDS; thread t then scans its 16
// consecutive columns there, the per-thread sums go through one workgroup
// scan (wave shuffles, then the 16 wave totals), and the results leave LDS
// by coalesced stores.
constexpr int kScanLdsMax = 16384;

__global__ __launch_bounds__(kScanThreads) void tr_scan_lds_kernel(
    int64_t K, const int32_t* __restrict__ cap_t, int32_t* __restrict__ start_t,
    int64_t* __restrict__ cap_total, const int32_t* __restrict__ nnz_t,
    int32_t* __restrict__ off, int64_t* __restrict__ nlive) {
    constexpr int kWaves = kScanThreads / kWave;
    constexpr int kPer = kScanLdsMax / kScanThreads;
    __shared__ int32_t sc[kScanLdsMax], sn[kScanLdsMax];
    __shared__ int64_t wc[kWaves], wn[kWaves];
    const int t = threadIdx.x, lane = t & (kWave - 1), w = t >> 6;
    const bool two = nnz_t != nullptr;
#pragma unroll
    for (int h = 0; h < kPer; h += kPer / 2) {  // two halves of loads, each issued at once
        int32_t a[kPer / 2], b[kPer / 2];
#pragma unroll
        for (int q = 0; q < kPer / 2; ++q) {
            const int64_t c = (h + q) * kScanThreads + t;
            a[q] = c < K ? cap_t[c] : 0;
            b[q] = (two && c < K) ? nnz_t[c] : 0;
        }
#pragma unroll
        for (int q = 0; q < kPer / 2; ++q) {
            sc[(h + q) * kScanThreads + t] = a[q];
            sn[(h + q) * kScanThreads + t] = b[q];
        }
    }
    __syncthreads();
    int64_t s1 = 0, s2 = 0;
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
        s1 += sc[t * kPer + q];
        s2 += sn[t * kPer + q];
    }
    int64_t x1 = s1, x2 = s2;  // inclusive scans over the wave
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const int64_t u1 = __shfl_up(x1, o), u2 = __shfl_up(x2, o);
        if (lane >= o) {
            x1 += u1;
            x2 += u2;
        }
    }
    if (lane == kWave - 1) {
        wc[w] = x1;
        wn[w] = x2;
    }
    __syncthreads();
    if (t == 0) {  // the wave totals become exclusive prefixes
        int64_t a1 = 0, a2 = 0;
        for (int q = 0; q < kWaves; ++q) {
            const int64_t y1 = wc[q], y2 = wn[q];
            wc[q] = a1;
            wn[q] = a2;
            a1 += y1;
            a2 += y2;
        }
        *cap_total = a1;
        if (two) *nlive = a2;
    }
    __syncthreads();
    int64_t r1 = wc[w] + x1 - s1, r2 = wn[w] + x2 - s2;
    // each thread's columns become their start and padding offset, in place
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
        const int i = t * kPer + q;
        const int32_t c1 = sc[i], c2 = sn[i];
        sc[i] = static_cast<int32_t>(r1);
        sn[i] = static_cast<int32_t>(r1 - r2);
        r1 += c1;
        r2 += c2;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
        const int64_t c = q * kScanThreads + t;
        if (c < K) {
            start_t[c] = sc[c];
            if (two) off[c] = sn[c];
        }
    }
}

// The capacity scan: the LDS kernel where the columns fit, else the
// two-pass one.
void launch_scan(int64_t K, const int32_t* cap_t, int32_t* start_t, int64_t* cap_total,
                 const int32_t* nnz_t, int32_t* off, int64_t* nlive, hipStream_t st) {
    if (K <= kScanLdsMax) {
        hipLaunchKernelGGL(tr_scan_lds_kernel, dim3(1), dim3(kScanThreads), 0, st, K, cap_t,
                           start_t, cap_total, nnz_t, off, nlive);
    } else {
        hipLaunchKernelGGL(tr_scan_kernel, dim3(1), dim3(kScanThreads), 0, st, K, cap_t, start_t,
                           cap_total, nnz_t, off, nlive);
    }
}

// T4: one wave per WT row; lanes write consecutive padding slots.
__global__ __launch_bounds__(256) void tr_pad_kernel(int64_t K, const int32_t* __restrict__ start_t,
                                                     const int32_t* __restrict__ nnz_t,
                                                     const int32_t* __restrict__ cap_t,
                                                     float* __restrict__ val_t,
                                                     int32_t* __restrict__ col_t,
                                                     int64_t* __restrict__ perm) {
    const int64_t c = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
    if (c >= K) return;
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t rs = start_t[c];
    const int64_t end = rs + cap_t[c];
    for (int64_t p = rs + nnz_t[c] + lane; p < end; p += kWave) {
        col_t[p] = -1;
        val_t[p] = 0.0f;
        perm[p] = -1;
    }
}

__global__ __launch_bounds__(kWave) void tr_scatter_kernel(
    int64_t M, int64_t K, int64_t B, const int32_t* __restrict__ row_start,
    const int32_t* __restrict__ row_nnz, const int32_t* __restrict__ col,
    const float* __restrict__ val, const int32_t* __restrict__ bh,
    const int32_t* __restrict__ start_t, float* __restrict__ val_t,
    int32_t* __restrict__ col_t, int64_t* __restrict__ perm) {
    extern __shared__ int32_t cur[];
    const int lane = threadIdx.x;
    const int64_t b = blockIdx.x;
    const int64_t r0 = b * B;
    const int64_t r1 = (r0 + B < M) ? r0 + B : M;
    for (int64_t c0 = 0; c0 < K; c0 += kColChunk) {
        const int64_t kc = (K - c0 < kColChunk) ? K - c0 : kColChunk;
        for (int64_t t = lane; t < kc; t += kWave) cur[t] = start_t[c0 + t] + bh[b * K + c0 + t];
        __syncthreads();
        for (int64_t r = r0; r < r1; ++r) {
            const int64_t start = row_start[r];
            const int32_t nnz = row_nnz[r];
            for (int32_t k0 = 0; k0 < nnz; k0 += kWave) {
                const int32_t k = k0 + lane;
                if (k < nnz) {
                    const int64_t s = start + k;
                    const int64_t c = col[s] - c0;
                    if (c >= 0 && c < kc) {
                        const int32_t pos = cur[c];
                        cur[c] = pos + 1;
                        perm[pos] = s;
                        col_t[pos] = static_cast<int32_t>(r);
                        val_t[pos] = val[s];
                    }
                }
                // Orders this batch's counter updates before the next batch
                // (a later row may share a column with this one).
                __syncthreads();
            }
        }
        __syncthreads();
    }
}

// T5 for blocks of at most 32 rows (see above): one 256-thread workgroup per
// block, LDS holds one mask word per column of the current column chunk.
constexpr int kParScatterThreads = 1024;
constexpr int64_t kParScatterMaxRows = 32;

__global__ __launch_bounds__(kParScatterThreads) void tr_scatter_par_kernel(
    int64_t M, int64_t K, int64_t B, const int32_t* __restrict__ row_start,
    const int32_t* __restrict__ row_nnz, const int32_t* __restrict__ col,
    const float* __restrict__ val, const int32_t* __restrict__ bh,
    const int32_t* __restrict__ start_t, float* __restrict__ val_t,
    int32_t* __restrict__ col_t, int64_t* __restrict__ perm) {
    extern __shared__ uint32_t mask[];
    const int t = threadIdx.x;
    const int64_t b = blockIdx.x;
    const int64_t r0 = b * B;
    const int64_t r1 = (r0 + B < M) ? r0 + B : M;
    for (int64_t c0 = 0; c0 < K; c0 += kColChunk) {
        const int64_t kc = (K - c0 < kColChunk) ? K - c0 : kColChunk;
        for (int64_t u = t; u < kc; u += kParScatterThreads) mask[u] = 0;
        __syncthreads();
        for (int64_t r = r0; r < r1; ++r) {
            const int64_t s0 = row_start[r];
            const int32_t n = row_nnz[r];
            const uint32_t bit = 1u << (r - r0);
            for (int32_t k = t; k < n; k += kParScatterThreads) {
                const int64_t c = col[s0 + k] - c0;
                if (c >= 0 && c < kc) atomicOr(&mask[c], bit);
            }
        }
        __syncthreads();
        for (int64_t r = r0; r < r1; ++r) {
            const int64_t s0 = row_start[r];
            const int32_t n = row_nnz[r];
            const uint32_t below = (1u << (r - r0)) - 1u;
            for (int32_t k = t; k < n; k += kParScatterThreads) {
                const int64_t s = s0 + k;
                const int32_t c = col[s];
                const int64_t cc = c - c0;
                if (cc >= 0 && cc < kc) {
                    const int64_t pos = static_cast<int64_t>(start_t[c]) + bh[b * K + c] +
                                        __popc(mask[cc] & below);
                    perm[pos] = s;
                    col_t[pos] = static_cast<int32_t>(r);
                    val_t[pos] = val[s];
                }
            }
        }
        __syncthreads();  // every read of this chunk's masks is done
    }
}

// T5 by tiles of kTileSub blocks (of B <= 32 rows) x kTileCols columns, one
// 1024-thread workgroup each: the same positions as tr_scatter_par_kernel
// (start of WT row c + the block's start in it + the earlier rows of the
// block marked at c), but a workgroup's writes now fall into kTileCols WT
// rows, a run of about B·kTileSub·density consecutive slots in each, which
// the L2 merges into whole lines before they reach HBM. (A workgroup per
// block over all columns writes one or two slots per WT row: every write a
// partial line.) Each row's slots of the tile are found by binary search on
// its columns; the tile's slots are then visited flat, a slot's row found by
// binary search over the rows' run offsets in LDS.
constexpr int kTileSub = 32;
constexpr int kTileCols = 512;
constexpr int kTileThreads = 1024;
static_assert(kTileSub * kParScatterMaxRows <= kTileThreads, "one boundary per thread and row");

__global__ __launch_bounds__(kTileThreads) void tr_scatter_tile_kernel(
    int64_t M, int64_t K, int64_t B, int64_t nblk, int64_t ntc,
    const int32_t* __restrict__ row_start, const int32_t* __restrict__ row_nnz,
    const int32_t* __restrict__ col, const float* __restrict__ val,
    const int32_t* __restrict__ bh, const int32_t* __restrict__ start_t,
    float* __restrict__ val_t, int32_t* __restrict__ col_t, int64_t* __restrict__ perm) {
    __shared__ uint32_t mask[kTileSub][kTileCols];  // 64 KiB
    __shared__ int32_t lo[kTileThreads], hi[kTileThreads];
    __shared__ int32_t pre[kTileThreads];  // exclusive offsets of the rows' runs
    __shared__ int32_t wsum[kTileThreads / kWave];
    __shared__ int32_t s_total;
    const int t = threadIdx.x;
    const int64_t tr = blockIdx.x / ntc, tc = blockIdx.x % ntc;
    const int64_t b0 = tr * kTileSub;
    const int64_t nsub = nblk - b0 < kTileSub ? nblk - b0 : kTileSub;
    const int64_t r0 = b0 * B;
    const int64_t r1 = (b0 + nsub) * B < M ? (b0 + nsub) * B : M;
    const int R = static_cast<int>(r1 - r0);  // <= kTileSub * B <= 1024
    const int32_t c0 = static_cast<int32_t>(tc * kTileCols);
    const int32_t c1 = static_cast<int32_t>(c0 + kTileCols < K ? c0 + kTileCols : K);
    for (int u = t; u < kTileSub * kTileCols; u += kTileThreads) (&mask[0][0])[u] = 0;
    // each row's run of columns in [c0, c1): lo = first slot with col >= c0,
    // hi = first with col >= c1 (live columns ascend within a row)
    for (int i = t; i < 2 * R; i += kTileThreads) {
        const int rl = i < R ? i : i - R;
        const int32_t bound = i < R ? c0 : c1;
        const int64_t s0 = row_start[r0 + rl];
        int32_t a = 0, e = row_nnz[r0 + rl];
        while (a < e) {
            const int32_t m = (a + e) >> 1;
            if (col[s0 + m] < bound) a = m + 1;
            else e = m;
        }
        if (i < R) lo[rl] = a;
        else hi[rl] = a;
    }
    __syncthreads();
    {  // exclusive scan of the run lengths (rows past R: 0)
        const int len = t < R ? hi[t] - lo[t] : 0;
        const int lane = t & (kWave - 1), w = t / kWave;
        int v = len;
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
            const int up = __shfl_up(v, off);
            if (lane >= off) v += up;
        }
        if (lane == kWave - 1) wsum[w] = v;
        __syncthreads();
        int base = 0;
        for (int q = 0; q < w; ++q) base += wsum[q];
        pre[t] = base + v - len;
        if (t == kTileThreads - 1) s_total = base + v;
        __syncthreads();
    }
    const int total = s_total;
    auto row_of = [&](int e) -> int {  // the last row whose run starts at or before e
        int a = 0, b = R - 1;
        while (a < b) {
            const int m = (a + b + 1) >> 1;
            if (pre[m] <= e) a = m;
            else b = m - 1;
        }
        return a;
    };
    // The flat passes take kFlatU slots per thread at a time, every load of
    // the group issued before the first use (elements past the total repeat
    // the last one and change nothing), so a thread's slots cost one memory
    // latency per group instead of one each.
    constexpr int kFlatU = 4;
    auto locate = [&](int e, int& rl, int64_t& s) {
        const int ec = e < total ? e : total - 1;
        rl = row_of(ec);
        s = row_start[r0 + rl] + lo[rl] + (ec - pre[rl]);
    };
    for (int e0 = t; e0 < total; e0 += kFlatU * kTileThreads) {
        int rl[kFlatU];
        int64_t s[kFlatU];
        int32_t c[kFlatU];
#pragma unroll
        for (int q = 0; q < kFlatU; ++q) locate(e0 + q * kTileThreads, rl[q], s[q]);
#pragma unroll
        for (int q = 0; q < kFlatU; ++q) c[q] = col[s[q]];
#pragma unroll
        for (int q = 0; q < kFlatU; ++q)
            if (e0 + q * kTileThreads < total) atomicOr(&mask[rl[q] / B][c[q] - c0], 1u << (rl[q] % B));
    }
    __syncthreads();
    for (int e0 = t; e0 < total; e0 += kFlatU * kTileThreads) {
        int rl[kFlatU];
        int64_t s[kFlatU];
        int32_t c[kFlatU];
        float v[kFlatU];
        int32_t st[kFlatU], bb[kFlatU];
#pragma unroll
        for (int q = 0; q < kFlatU; ++q) locate(e0 + q * kTileThreads, rl[q], s[q]);
#pragma unroll
        for (int q = 0; q < kFlatU; ++q) {
            c[q] = col[s[q]];
            v[q] = val[s[q]];
        }
#pragma unroll
        for (int q = 0; q < kFlatU; ++q) {
            st[q] = start_t[c[q]];
            bb[q] = bh[(b0 + rl[q] / B) * K + c[q]];
        }
#pragma unroll
        for (int q = 0; q < kFlatU; ++q) {
            if (e0 + q * kTileThreads >= total) continue;
            const int64_t sb = rl[q] / B;
            const uint32_t below = (1u << (rl[q] % B)) - 1u;
            const int64_t pos = static_cast<int64_t>(st[q]) + bb[q] +
                                __popc(mask[sb][c[q] - c0] & below);
            perm[pos] = s[q];
            col_t[pos] = static_cast<int32_t>(r0 + rl[q]);
            val_t[pos] = v[q];
        }
    }
}

// ─────────────── radix path: a stable two-pass LSD sort by column ───────────
//
// For ncols <= 65535 the counting sort above is replaced by a least-
// significant-digit radix sort of the live slots keyed by column: pass 1 by
// the low 8 bits, pass 2 by the high 8 (one pass when ncols <= 256). Each
// pass is stable, and the slots enter pass 1 in W's slot order (rows
// ascending, then columns), so the result lists each column's slots by
// ascending row: the order of every WT row, hence the same arrays. No pass
// searches anything; loads are contiguous and each tile's writes go out as
// runs (one per digit) through an LDS staging buffer.
//
//   R1 count   one workgroup per 8 tiles of 4096 slots: the column counts
//              of its slots (LDS, written as a partial table) and, per tile,
//              the count of each low digit (hist1[d][tile]).
//   R2 colscan sums the partial tables per column (T2's kernel): WT row_nnz,
//              row_capacity.
//   R3 scan    WT row_start and capT, and off[c] = row_start[c] - (live
//              slots of columns < c): the padding before column c's run.
//   R0 rowid   each live slot's row.
//   R4 scan    per digit, the exclusive prefix of its counts over tiles.
//   R5 scatter pass 1: per tile, each live slot's rank among the tile's slots
//              of its digit (wave ballots; earlier waves' and iterations'
//              counts in LDS), staged by digit in LDS, written as (column,
//              slot, row, value) at digit base + tile prefix + rank.
//   R6 hist    pass 2's per-tile digit counts over pass 1's output.
//   R7 scan    as R4.
//   R8 scatter pass 2, writing perm, col_indices and values of WT at sorted
//              position + off[column].
constexpr int kRxThreads = 256;          // one thread per digit value
constexpr int kRxIpt = 16;               // items per thread and tile
constexpr int kRxTile = kRxThreads * kRxIpt;
constexpr int kRxSbTiles = 8;            // tiles per R1 workgroup
constexpr int64_t kRxMaxCols = 65535;    // two 8-bit passes, keys as uint16
constexpr int64_t kRxMinCapacity = 1 << 20;  // below: the counting sort (fewer launches)

struct RxPlan {
    int64_t nt;    // tiles of kRxTile slots over [0, total_capacity)
    int64_t nsb;   // R1 workgroups
    int passes;    // 1 (ncols <= 256) or 2
    // workspace offsets (bytes, 256-aligned)
    int64_t o_colpart, o_hist1, o_hist2, o_tot1, o_tot2, o_nlive, o_off, o_rowid, o_key, o_s,
        o_r, o_v, bytes;
};

int64_t align256(int64_t x) { return (x + 255) & ~int64_t{255}; }

bool rx_eligible(const slk_csr* W) {
    return W->ncols >= 1 && W->ncols <= kRxMaxCols && W->nrows >= 1 && W->nrows <= INT32_MAX &&
           W->total_capacity >= 1 && W->total_capacity <= INT32_MAX;
}

bool rx_chosen(const slk_csr* W) {
    const int64_t t = tuning(SLK_TUNE_TRANSPOSE_RADIX);
    if (t == 0 || !rx_eligible(W)) return false;
    return t > 0 || W->total_capacity >= kRxMinCapacity;
}

RxPlan rx_plan(const slk_csr* W) {
    RxPlan p{};
    const int64_t cap = W->total_capacity, K = W->ncols;
    p.nt = ceil_div(cap, kRxTile);
    p.nsb = ceil_div(p.nt, kRxSbTiles);
    p.passes = K <= 256 ? 1 : 2;
    int64_t o = 0;
    auto take = [&](int64_t n) {
        const int64_t at = o;
        o = align256(o + n);
        return at;
    };
    p.o_colpart = take(p.nsb * K * 4);
    p.o_hist1 = take(256 * p.nt * 4);
    p.o_hist2 = take(256 * p.nt * 4);
    p.o_tot1 = take(256 * 4);
    p.o_tot2 = take(256 * 4);
    p.o_nlive = take(8);
    p.o_off = take(K * 4);
    p.o_rowid = take(cap * 4);
    p.o_key = take(cap * 2);
    p.o_s = take(cap * 4);
    p.o_r = take(cap * 4);
    p.o_v = take(cap * 4);
    p.bytes = o;
    return p;
}

// Exclusive prefix of v over the 256 threads of a workgroup (4 waves); total
// gets the sum. `part` holds 4 ints of LDS. Ends with a barrier.
__device__ __forceinline__ int rx_block_scan(int v, int* part, int& total) {
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const int up = __shfl_up(x, off);
        if (lane >= off) x += up;
    }
    if (lane == kWave - 1) part[w] = x;
    __syncthreads();
    int base = 0;
#pragma unroll
    for (int q = 0; q < kRxThreads / kWave; ++q) base += q < w ? part[q] : 0;
    total = part[0] + part[1] + part[2] + part[3];
    __syncthreads();
    return base + x - v;
}

// R1: per workgroup, tiles [8 sb, 8 sb + 8): column counts into colpart[sb]
// (column chunks of kColChunk), low-digit counts per tile into hist1.
__global__ __launch_bounds__(kRxThreads) void tr_rx_count_kernel(
    int64_t cap, int64_t K, int64_t nt, const int32_t* __restrict__ col,
    int32_t* __restrict__ colpart, int32_t* __restrict__ hist1) {
    extern __shared__ int32_t ccnt[];
    __shared__ int32_t dig[256];
    const int tid = threadIdx.x;
    const int64_t sb = blockIdx.x;
    const int64_t t0 = sb * kRxSbTiles;
    const int64_t t1 = t0 + kRxSbTiles < nt ? t0 + kRxSbTiles : nt;
    for (int64_t c0 = 0; c0 < K; c0 += kColChunk) {
        const int64_t kc = K - c0 < kColChunk ? K - c0 : kColChunk;
        const bool first = c0 == 0;
        for (int64_t i = tid; i < kc; i += kRxThreads) ccnt[i] = 0;
        dig[tid] = 0;
        __syncthreads();
        // each tile's columns are requested while the previous tile is counted
        auto load = [&](int32_t (&c)[kRxIpt], int64_t t) {
#pragma unroll
            for (int k = 0; k < kRxIpt; ++k) {
                const int64_t s = t * kRxTile + k * kRxThreads + tid;
                c[k] = (t < t1 && s < cap) ? col[s] : -1;
            }
        };
        int32_t c[kRxIpt], nc[kRxIpt];
        load(c, t0);
        for (int64_t t = t0; t < t1; ++t) {
            load(nc, t + 1);
#pragma unroll
            for (int k = 0; k < kRxIpt; ++k) {
                if (c[k] < 0) continue;
                const int64_t cc = c[k] - c0;
                if (cc >= 0 && cc < kc) atomicAdd(&ccnt[cc], 1);
                if (first) atomicAdd(&dig[c[k] & 255], 1);
            }
            if (first) {
                __syncthreads();
                hist1[tid * nt + t] = dig[tid];
                dig[tid] = 0;
                __syncthreads();
            }
#pragma unroll
            for (int k = 0; k < kRxIpt; ++k) c[k] = nc[k];
        }
        __syncthreads();
        for (int64_t i = tid; i < kc; i += kRxThreads) colpart[sb * K + c0 + i] = ccnt[i];
        __syncthreads();
    }
}

// R0: rowid[s] = r for the live slots of row r; one workgroup of 4 waves
// per row.
__global__ __launch_bounds__(256) void tr_rx_rowid_kernel(int64_t M,
                                                          const int32_t* __restrict__ row_start,
                                                          const int32_t* __restrict__ row_nnz,
                                                          int32_t* __restrict__ rowid) {
    const int64_t r = blockIdx.x;
    const int64_t s0 = row_start[r];
    const int64_t n = row_nnz[r];
    for (int64_t k = threadIdx.x; k < n; k += blockDim.x) rowid[s0 + k] = static_cast<int32_t>(r);
}

// R4 / R7: one workgroup per digit d: hist[d][0, nt) becomes its exclusive
// prefix, tot[d] its sum.
__global__ __launch_bounds__(kRxThreads) void tr_rx_digit_scan_kernel(int64_t nt,
                                                                      int32_t* __restrict__ hist,
                                                                      int32_t* __restrict__ tot) {
    __shared__ int part[kRxThreads / kWave];
    int32_t* h = hist + static_cast<int64_t>(blockIdx.x) * nt;
    const int64_t per = ceil_div(nt, kRxThreads);
    const int64_t a = threadIdx.x * per;
    const int64_t e = a + per < nt ? a + per : nt;
    constexpr int G = 8;  // entries per group: the group's loads go out first
    int s = 0;
    for (int64_t g = a; g < e; g += G) {
        int x[G];
#pragma unroll
        for (int q = 0; q < G; ++q) x[q] = g + q < e ? h[g + q] : 0;
#pragma unroll
        for (int q = 0; q < G; ++q) s += x[q];
    }
    int total;
    int run = rx_block_scan(s, part, total);
    for (int64_t g = a; g < e; g += G) {
        int x[G];
#pragma unroll
        for (int q = 0; q < G; ++q) x[q] = g + q < e ? h[g + q] : 0;
#pragma unroll
        for (int q = 0; q < G; ++q) {
            if (g + q < e) h[g + q] = run;
            run += x[q];
        }
    }
    if (threadIdx.x == 0) tot[blockIdx.x] = total;
}

// R6: per tile of pass 1's output, the count of each high digit.
__global__ __launch_bounds__(kRxThreads) void tr_rx_hist_kernel(
    int64_t nt, int shift, const int64_t* __restrict__ nlive, const uint16_t* __restrict__ key,
    int32_t* __restrict__ hist) {
    __shared__ int32_t dig[256];
    const int tid = threadIdx.x;
    const int64_t t = blockIdx.x;
    const int64_t n = *nlive;
    dig[tid] = 0;
    __syncthreads();
    const int64_t base = t * kRxTile;
    if (base < n) {
        int32_t c[kRxIpt];
#pragma unroll
        for (int k = 0; k < kRxIpt; ++k) {
            const int64_t i = base + k * kRxThreads + tid;
            c[k] = i < n ? static_cast<int32_t>(key[i]) : -1;
        }
#pragma unroll
        for (int k = 0; k < kRxIpt; ++k)
            if (c[k] >= 0) atomicAdd(&dig[(c[k] >> shift) & 255], 1);
    }
    __syncthreads();
    hist[tid * nt + t] = dig[tid];
}

struct RxScatterArgs {
    int64_t cap;  // pass 1: items are W's slots [0, cap)
    int64_t nt;
    int shift;
    const int32_t* hist;  // scanned: hist[d][t] = items of digit d in tiles < t
    const int32_t* tot;   // items of each digit
    const int64_t* nlive;  // pass 2: items [0, *nlive)
    // pass 1 input (W)
    const int32_t* col;
    const float* val;
    const int32_t* rowid;
    // pass 2 input (pass 1's output)
    const uint16_t* key_in;
    const int32_t* s_in;
    const int32_t* r_in;
    const float* v_in;
    // pass 1 output
    uint16_t* key_out;
    int32_t* s_out;
    int32_t* r_out;
    float* v_out;
    // final output
    const int32_t* off;
    int64_t* perm;
    int32_t* col_t;
    float* val_t;
};

// R5 / R8: one workgroup per tile of kRxTile items, consecutive tiles on one
// XCD (neighbouring tiles write neighbouring parts of each digit's run).
// Wave w of the tile owns items [w·1024, (w+1)·1024) of it, 64 per step, so
// the order (wave, step, lane) is the items' order. The rank of an item
// among the tile's items of its digit d is the count of d in earlier waves
// plus, inside its wave, the count in earlier steps (a per-wave counter in
// LDS, read and advanced by the lowest lane of each digit and broadcast)
// plus the earlier lanes of its step with the same 8 digit bits (8 ballots).
// No barrier until every item of the wave is ranked.
template <bool FROM_W, bool FINAL>
__global__ __launch_bounds__(kRxThreads) void tr_rx_scatter_kernel(RxScatterArgs a) {
    constexpr int kWaves = kRxThreads / kWave;
    constexpr int kPerWave = kRxTile / kWaves;
    __shared__ int32_t cnt[kWaves][256];
    __shared__ int32_t loff[256], gbase[256], dbase[256];
    __shared__ int part[kWaves];
    __shared__ int32_t st_key[kRxTile], st_s[kRxTile], st_r[kRxTile];
    __shared__ float st_v[kRxTile];
    const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid >> 6;
    const int64_t n = FROM_W ? a.cap : *a.nlive;
    // one tile per workgroup; consecutive tiles on one XCD, so the partial
    // lines that tiles in flight write to each digit's run meet in one L2
    // (a persistent grid that loads the next tile during this one was
    // slower: fewer workgroups per CU, for the registers of two tiles)
    const int64_t t = xcd_logical_block(blockIdx.x, gridDim.x);
    if (t * kRxTile >= n) return;  // workgroup-uniform, before any barrier

    int total;
    dbase[tid] = rx_block_scan(a.tot[tid], part, total);

    struct Items {
        int32_t c[kRxIpt], s[kRxIpt], r[kRxIpt];
        float v[kRxIpt];
    };
    auto load = [&](Items& x) {
        const int64_t wbase = t * kRxTile + static_cast<int64_t>(w) * kPerWave + lane;
#pragma unroll
        for (int k = 0; k < kRxIpt; ++k) {
            const int64_t i = wbase + k * kWave;
            const bool in = i < n;
            if constexpr (FROM_W) {
                x.c[k] = in ? a.col[i] : -1;
                x.s[k] = static_cast<int32_t>(i);
            } else {
                x.c[k] = in ? static_cast<int32_t>(a.key_in[i]) : -1;
                x.s[k] = in ? a.s_in[i] : 0;
            }
        }
#pragma unroll
        for (int k = 0; k < kRxIpt; ++k) {
            const int64_t i = wbase + k * kWave;
            if constexpr (FROM_W) {
                x.r[k] = x.c[k] >= 0 ? a.rowid[i] : 0;
                x.v[k] = x.c[k] >= 0 ? a.val[i] : 0.0f;
            } else {
                x.r[k] = x.c[k] >= 0 ? a.r_in[i] : 0;
                x.v[k] = x.c[k] >= 0 ? a.v_in[i] : 0.0f;
            }
        }
    };
    const uint64_t below = (uint64_t{1} << lane) - 1u;
    Items cur;
    load(cur);
    {
        // each wave clears its own counters (its lanes, in order, before use)
#pragma unroll
        for (int q = 0; q < 256 / kWave; ++q) cnt[w][q * kWave + lane] = 0;
        int32_t rk[kRxIpt];
#pragma unroll
        for (int k = 0; k < kRxIpt; ++k) {
            const bool ok = cur.c[k] >= 0;
            const int d = ok ? (cur.c[k] >> a.shift) & 255 : 0;
            uint64_t peers = __ballot(ok);
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                const bool bit = (d >> b) & 1;
                const uint64_t m = __ballot(bit);
                peers &= bit ? m : ~m;
            }
            const int wr = __popcll(peers & below);
            const int leader = ok ? __ffsll(static_cast<unsigned long long>(peers)) - 1 : lane;
            int old = 0;
            if (ok && wr == 0) {
                old = cnt[w][d];
                cnt[w][d] = old + __popcll(peers);
            }
            old = __shfl(old, leader);
            rk[k] = old + wr;
        }
        __syncthreads();
        // per digit (thread = digit): the tile's count, earlier waves' counts
        int tile_d = 0;
#pragma unroll
        for (int q = 0; q < kWaves; ++q) {
            const int x = cnt[q][tid];
            cnt[q][tid] = tile_d;
            tile_d += x;
        }
        gbase[tid] = dbase[tid] + a.hist[static_cast<int64_t>(tid) * a.nt + t];
        int live;
        loff[tid] = rx_block_scan(tile_d, part, live);
        __syncthreads();
#pragma unroll
        for (int k = 0; k < kRxIpt; ++k) {
            if (cur.c[k] < 0) continue;
            const int d = (cur.c[k] >> a.shift) & 255;
            const int lp = loff[d] + cnt[w][d] + rk[k];
            st_key[lp] = cur.c[k];
            st_s[lp] = cur.s[k];
            st_r[lp] = cur.r[k];
            st_v[lp] = cur.v[k];
        }
        __syncthreads();
        for (int j = tid; j < live; j += kRxThreads) {
            const int32_t cc = st_key[j];
            const int d = (cc >> a.shift) & 255;
            const int64_t p = static_cast<int64_t>(gbase[d]) + (j - loff[d]);
            if constexpr (FINAL) {
                const int64_t pos = p + a.off[cc];
                a.perm[pos] = st_s[j];
                a.col_t[pos] = st_r[j];
                a.val_t[pos] = st_v[j];
            } else {
                a.key_out[p] = static_cast<uint16_t>(cc);
                a.s_out[p] = st_s[j];
                a.r_out[p] = st_r[j];
                a.v_out[p] = st_v[j];
            }
        }
    }
}

// slk_row_hints: one workgroup counts the entries of row_nnz above
// heavy_bar and at or above dense_bar (float64 compares).
constexpr int kHintThreads = 1024;

__global__ __launch_bounds__(kHintThreads) void row_hints_kernel(
    const int32_t* __restrict__ row_nnz, int64_t n, double heavy_bar, double dense_bar,
    int64_t dense_min_rows, int64_t* __restrict__ out) {
    constexpr int kWaves = kHintThreads / kWave;
    __shared__ int64_t ph[kWaves], pd[kWaves];
    const int t = threadIdx.x, lane = t & (kWave - 1), w = t >> 6;
    int64_t h = 0, d = 0;
    for (int64_t i0 = 0; i0 < n; i0 += 8 * kHintThreads) {
        int32_t v[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int64_t i = i0 + q * kHintThreads + t;
            v[q] = i < n ? row_nnz[i] : -1;
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            if (v[q] < 0) continue;
            const double x = static_cast<double>(v[q]);
            h += x > heavy_bar;
            d += x >= dense_bar;
        }
    }
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) {
        h += __shfl_xor(h, o);
        d += __shfl_xor(d, o);
    }
    if (lane == 0) {
        ph[w] = h;
        pd[w] = d;
    }
    __syncthreads();
    if (t == 0) {
        int64_t th = 0, td = 0;
        for (int q = 0; q < kWaves; ++q) {
            th += ph[q];
            td += pd[q];
        }
        out[0] = th;
        out[1] = td >= dense_min_rows ? td : 0;
    }
}

__global__ __launch_bounds__(256) void tr_refresh_kernel(const float* __restrict__ w_val,
                                                         int64_t w_cap,
                                                         const int64_t* __restrict__ perm,
                                                         int64_t cap_t, float* __restrict__ val_t) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < cap_t;
         t += stride) {
        const int64_t p = perm[t];
        if (p >= 0 && p < w_cap) val_t[t] = w_val[p];
    }
}

}  // namespace
}  // namespace slk

namespace slk {
namespace {

// The radix path's count (R1-R3). Returns SLK_OK or an error code.
int rx_count(const slk_csr* W, double padding_ratio, void* workspace, int64_t workspace_bytes,
             int32_t* WT_row_start, int32_t* WT_row_nnz, int32_t* WT_row_capacity,
             int64_t* capT_dev, hipStream_t st) {
    const RxPlan x = rx_plan(W);
    if (workspace_bytes < x.bytes || workspace == nullptr) {
        return fail(SLK_EINVAL, "transpose: workspace of " + std::to_string(workspace_bytes) +
                                    " bytes is smaller than the required " +
                                    std::to_string(x.bytes));
    }
    char* ws = static_cast<char*>(workspace);
    const int64_t K = W->ncols;
    int32_t* colpart = reinterpret_cast<int32_t*>(ws + x.o_colpart);
    const size_t lds = static_cast<size_t>(K < kColChunk ? K : kColChunk) * sizeof(int32_t);
    hipLaunchKernelGGL(tr_rx_count_kernel, dim3(static_cast<unsigned>(x.nsb)), dim3(kRxThreads),
                       lds, st, W->total_capacity, K, x.nt, W->col_indices, colpart,
                       reinterpret_cast<int32_t*>(ws + x.o_hist1));
    if (int rc = check_launch("transpose_count/rx_count")) return rc;
    hipLaunchKernelGGL(tr_colscan_kernel, dim3(static_cast<unsigned>(ceil_div(K, kWave))),
                       dim3(kColScanWaves * kWave), 0, st, K, x.nsb, 1.0 + padding_ratio, colpart,
                       WT_row_nnz, WT_row_capacity, false);
    if (int rc = check_launch("transpose_count/colscan")) return rc;
    launch_scan(K, WT_row_capacity, WT_row_start, capT_dev, WT_row_nnz,
                reinterpret_cast<int32_t*>(ws + x.o_off),
                reinterpret_cast<int64_t*>(ws + x.o_nlive), st);
    return check_launch("transpose_count/rx_scan");
}

// The radix path's fill (R0, R4-R8 and the padding). The workspace holds
// what rx_count wrote.
int rx_fill(const slk_csr* W, const void* workspace, int64_t workspace_bytes,
            const int32_t* WT_row_start, const int32_t* WT_row_nnz,
            const int32_t* WT_row_capacity, float* WT_values, int32_t* WT_col_indices,
            int64_t* perm, hipStream_t st) {
    const RxPlan x = rx_plan(W);
    if (workspace_bytes < x.bytes || workspace == nullptr) {
        return fail(SLK_EINVAL, "transpose: workspace too small");
    }
    char* ws = const_cast<char*>(static_cast<const char*>(workspace));
    const int64_t M = W->nrows, K = W->ncols;
    hipLaunchKernelGGL(tr_pad_kernel, dim3(static_cast<unsigned>(ceil_div(K, 256 / kWave))),
                       dim3(256), 0, st, K, WT_row_start, WT_row_nnz, WT_row_capacity, WT_values,
                       WT_col_indices, perm);
    if (int rc = check_launch("transpose_fill/pad")) return rc;
    int32_t* rowid = reinterpret_cast<int32_t*>(ws + x.o_rowid);
    hipLaunchKernelGGL(tr_rx_rowid_kernel, dim3(static_cast<unsigned>(M)), dim3(256), 0, st, M,
                       W->row_start, W->row_nnz, rowid);
    if (int rc = check_launch("transpose_fill/rowid")) return rc;
    int32_t* hist1 = reinterpret_cast<int32_t*>(ws + x.o_hist1);
    int32_t* hist2 = reinterpret_cast<int32_t*>(ws + x.o_hist2);
    int32_t* tot1 = reinterpret_cast<int32_t*>(ws + x.o_tot1);
    int32_t* tot2 = reinterpret_cast<int32_t*>(ws + x.o_tot2);
    const int64_t* nlive = reinterpret_cast<const int64_t*>(ws + x.o_nlive);
    hipLaunchKernelGGL(tr_rx_digit_scan_kernel, dim3(256), dim3(kRxThreads), 0, st, x.nt, hist1,
                       tot1);
    if (int rc = check_launch("transpose_fill/rx_scan1")) return rc;

    RxScatterArgs a{};
    a.cap = W->total_capacity;
    a.nt = x.nt;
    a.shift = 0;
    a.hist = hist1;
    a.tot = tot1;
    a.nlive = nlive;
    a.col = W->col_indices;
    a.val = W->values;
    a.rowid = rowid;
    a.off = reinterpret_cast<const int32_t*>(ws + x.o_off);
    a.perm = perm;
    a.col_t = WT_col_indices;
    a.val_t = WT_values;
    const dim3 grid(static_cast<unsigned>(x.nt));
    if (x.passes == 1) {
        hipLaunchKernelGGL((tr_rx_scatter_kernel<true, true>), grid, dim3(kRxThreads), 0, st, a);
        return check_launch("transpose_fill/rx_scatter");
    }
    uint16_t* key = reinterpret_cast<uint16_t*>(ws + x.o_key);
    int32_t* s1 = reinterpret_cast<int32_t*>(ws + x.o_s);
    int32_t* r1 = reinterpret_cast<int32_t*>(ws + x.o_r);
    float* v1 = reinterpret_cast<float*>(ws + x.o_v);
    a.key_out = key;
    a.s_out = s1;
    a.r_out = r1;
    a.v_out = v1;
    hipLaunchKernelGGL((tr_rx_scatter_kernel<true, false>), grid, dim3(kRxThreads), 0, st, a);
    if (int rc = check_launch("transpose_fill/rx_scatter1")) return rc;
    hipLaunchKernelGGL(tr_rx_hist_kernel, grid, dim3(kRxThreads), 0, st, x.nt, 8, nlive, key,
                       hist2);
    if (int rc = check_launch("transpose_fill/rx_hist2")) return rc;
    hipLaunchKernelGGL(tr_rx_digit_scan_kernel, dim3(256), dim3(kRxThreads), 0, st, x.nt, hist2,
                       tot2);
    if (int rc = check_launch("transpose_fill/rx_scan2")) return rc;
    a.shift = 8;
    a.hist = hist2;
    a.tot = tot2;
    a.key_in = key;
    a.s_in = s1;
    a.r_in = r1;
    a.v_in = v1;
    hipLaunchKernelGGL((tr_rx_scatter_kernel<false, true>), grid, dim3(kRxThreads), 0, st, a);
    return check_launch("transpose_fill/rx_scatter2");
}

}  // namespace
}  // namespace slk

extern "C" int64_t slk_transpose_workspace_bytes(const slk_csr* W) {
    if (W == nullptr || W->nrows <= 0 || W->ncols <= 0) return 0;
    const slk::BlockPlan p = slk::plan_blocks(W->nrows, W->ncols);
    const int64_t counting = p.nblk * W->ncols * static_cast<int64_t>(sizeof(int32_t));
    // Whichever path count and fill take (the radix path where eligible,
    // unless slk_set_tuning turns it off) finds enough room.
    if (!slk::rx_eligible(W)) return counting;
    const int64_t radix = slk::rx_plan(W).bytes;
    return radix > counting ? radix : counting;
}

extern "C" int slk_transpose_count(const slk_csr* W, double padding_ratio, void* workspace,
                                   int64_t workspace_bytes, int32_t* WT_row_start,
                                   int32_t* WT_row_nnz, int32_t* WT_row_capacity,
                                   int64_t* capT_dev, void* stream) {
    using namespace slk;
    clear_error();
    if (int rc = validate_csr(W, "transpose")) return rc;
    if (!(padding_ratio >= 0.0)) {
        return fail(SLK_EINVAL,
                    "padding_ratio must be >= 0, got " + std::to_string(padding_ratio));
    }
    const int64_t M = W->nrows, K = W->ncols;
    if (capT_dev == nullptr) return fail(SLK_EINVAL, "transpose: NULL capT");
    hipStream_t st = as_stream(stream);
    if (K == 0) {
        // WT has no rows: capT = 0. Written by a kernel (graph-capture safe).
        hipLaunchKernelGGL(tr_scan_kernel, dim3(1), dim3(kScanThreads), 0, st, int64_t{0},
                           WT_row_capacity, WT_row_start, capT_dev, nullptr, nullptr, nullptr);
        return check_launch("transpose_count");
    }
    if (WT_row_start == nullptr || WT_row_nnz == nullptr || WT_row_capacity == nullptr) {
        return fail(SLK_EINVAL, "transpose: NULL WT row arrays");
    }
    if (rx_chosen(W)) {
        return rx_count(W, padding_ratio, workspace, workspace_bytes, WT_row_start, WT_row_nnz,
                        WT_row_capacity, capT_dev, st);
    }
    const BlockPlan p = plan_blocks(M, K);
    const int64_t need = p.nblk * K * static_cast<int64_t>(sizeof(int32_t));
    if (workspace_bytes < need || (need > 0 && workspace == nullptr)) {
        return fail(SLK_EINVAL, "transpose: workspace of " + std::to_string(workspace_bytes) +
                                    " bytes is smaller than the required " +
                                    std::to_string(need));
    }
    int32_t* bh = static_cast<int32_t*>(workspace);
    const size_t lds = static_cast<size_t>(K < kColChunk ? K : kColChunk) * sizeof(int32_t);
    if (p.nblk > 0) {
        hipLaunchKernelGGL(tr_hist_kernel, dim3(static_cast<unsigned>(p.nblk)), dim3(256), lds, st,
                           M, K, p.rows_per_block, W->row_start, W->row_capacity, W->col_indices,
                           bh);
        if (int rc = check_launch("transpose_count/hist")) return rc;
    }
    hipLaunchKernelGGL(tr_colscan_kernel, dim3(static_cast<unsigned>(ceil_div(K, kWave))),
                       dim3(kColScanWaves * kWave), 0, st, K, p.nblk, 1.0 + padding_ratio, bh,
                       WT_row_nnz, WT_row_capacity, true);
    if (int rc = check_launch("transpose_count/colscan")) return rc;
    launch_scan(K, WT_row_capacity, WT_row_start, capT_dev, nullptr, nullptr, nullptr, st);
    return check_launch("transpose_count/scan");
}

extern "C" int slk_transpose_fill(const slk_csr* W, const void* workspace, int64_t workspace_bytes,
                                  const int32_t* WT_row_start, const int32_t* WT_row_nnz,
                                  const int32_t* WT_row_capacity, int64_t capT, float* WT_values,
                                  int32_t* WT_col_indices, int64_t* perm, void* stream) {
    using namespace slk;
    clear_error();
    if (int rc = validate_csr(W, "transpose")) return rc;
    const int64_t M = W->nrows, K = W->ncols;
    if (K == 0 || capT == 0) return SLK_OK;
    if (capT > INT32_MAX) {
        return fail(SLK_EINVAL, "transpose: WT capacity " + std::to_string(capT) +
                                    " exceeds the int32 slot index range");
    }
    if (WT_values == nullptr || WT_col_indices == nullptr || perm == nullptr) {
        return fail(SLK_EINVAL, "transpose: NULL WT slot arrays");
    }
    hipStream_t st = as_stream(stream);
    if (rx_chosen(W)) {
        return rx_fill(W, workspace, workspace_bytes, WT_row_start, WT_row_nnz, WT_row_capacity,
                       WT_values, WT_col_indices, perm, st);
    }
    const BlockPlan p = plan_blocks(M, K);
    const int64_t need = p.nblk * K * static_cast<int64_t>(sizeof(int32_t));
    if (workspace_bytes < need || (need > 0 && workspace == nullptr)) {
        return fail(SLK_EINVAL, "transpose: workspace too small");
    }
    hipLaunchKernelGGL(tr_pad_kernel, dim3(static_cast<unsigned>(ceil_div(K, 256 / kWave))),
                       dim3(256), 0, st, K, WT_row_start, WT_row_nnz, WT_row_capacity, WT_values,
                       WT_col_indices, perm);
    if (int rc = check_launch("transpose_fill/pad")) return rc;
    if (p.nblk == 0) return SLK_OK;
    const size_t lds = static_cast<size_t>(K < kColChunk ? K : kColChunk) * sizeof(int32_t);
    // tiles where a row block spans many columns' worth of WT rows
    if (p.rows_per_block <= kParScatterMaxRows && K >= kTileCols &&
        tuning(SLK_TUNE_TRANSPOSE_TILE) != 0) {
        const int64_t ntc = ceil_div(K, int64_t{kTileCols});
        const int64_t tiles = ceil_div(p.nblk, int64_t{kTileSub}) * ntc;
        if (tiles <= INT32_MAX) {
            hipLaunchKernelGGL(tr_scatter_tile_kernel, dim3(static_cast<unsigned>(tiles)),
                               dim3(kTileThreads), 0, st, M, K, p.rows_per_block, p.nblk, ntc,
                               W->row_start, W->row_nnz, W->col_indices, W->values,
                               static_cast<const int32_t*>(workspace), WT_row_start, WT_values,
                               WT_col_indices, perm);
            return check_launch("transpose_fill/scatter");
        }
    }
    if (p.rows_per_block <= kParScatterMaxRows) {
        hipLaunchKernelGGL(tr_scatter_par_kernel, dim3(static_cast<unsigned>(p.nblk)),
                           dim3(kParScatterThreads), lds, st, M, K, p.rows_per_block,
                           W->row_start, W->row_nnz, W->col_indices, W->values,
                           static_cast<const int32_t*>(workspace), WT_row_start, WT_values,
                           WT_col_indices, perm);
        return check_launch("transpose_fill/scatter");
    }
    hipLaunchKernelGGL(tr_scatter_kernel, dim3(static_cast<unsigned>(p.nblk)), dim3(kWave), lds,
                       st, M, K, p.rows_per_block, W->row_start, W->row_nnz, W->col_indices,
                       W->values, static_cast<const int32_t*>(workspace), WT_row_start, WT_values,
                       WT_col_indices, perm);
    return check_launch("transpose_fill/scatter");
}

extern "C" int slk_transpose_refresh(const float* W_values, int64_t W_capacity,
                                     const int64_t* perm, int64_t capT, float* WT_values,
                                     void* stream) {
    using namespace slk;
    clear_error();
    if (capT < 0 || W_capacity < 0) return fail(SLK_EINVAL, "transpose_refresh: negative size");
    if (capT == 0) return SLK_OK;
    if (perm == nullptr || WT_values == nullptr || (W_capacity > 0 && W_values == nullptr)) {
        return fail(SLK_EINVAL, "transpose_refresh: NULL pointer");
    }
    int64_t blocks = ceil_div(capT, 256);
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(tr_refresh_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       as_stream(stream), W_values, W_capacity, perm, capT, WT_values);
    return check_launch("transpose_refresh");
}

extern "C" int slk_row_hints(const int32_t* row_nnz, int64_t n, double heavy_bar,
                             double dense_bar, int64_t dense_min_rows, int64_t* out,
                             void* stream) {
    using namespace slk;
    clear_error();
    if (n < 0) return fail(SLK_EINVAL, "row_hints: negative length");
    if (out == nullptr || (n > 0 && row_nnz == nullptr)) {
        return fail(SLK_EINVAL, "row_hints: NULL pointer");
    }
    hipLaunchKernelGGL(row_hints_kernel, dim3(1), dim3(kHintThreads), 0, as_stream(stream),
                       row_nnz, n, heavy_bar, dense_bar, dense_min_rows, out);
    return check_launch("row_hints");
}
