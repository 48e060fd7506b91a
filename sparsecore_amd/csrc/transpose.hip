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
    int32_t* __restrict__ nnz_t, int32_t* __restrict__ cap_t) {
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
        for (int64_t b = b0; b < b1; ++b) sum += bh[b * K + c];
    }
    part[w][lane] = sum;
    __syncthreads();
    int32_t run = 0;
    for (int v = 0; v < w; ++v) run += part[v][lane];
    if (ok) {
        for (int64_t b = b0; b < b1; ++b) {
            const int32_t t = bh[b * K + c];
            bh[b * K + c] = run;
            run += t;
        }
    }
    if (ok && w == kColScanWaves - 1) {  // the last share ends at the column total
        nnz_t[c] = run;
        // layout.py:66-67: np.maximum(1, np.ceil(nnz.astype(float64) * (1 + pr))).astype(int32)
        const double scaled = ceil(static_cast<double>(run) * one_plus_pr);
        cap_t[c] = scaled < 1.0 ? 1 : static_cast<int32_t>(scaled);
    }
}

constexpr int kScanThreads = 1024;

__global__ __launch_bounds__(kScanThreads) void tr_scan_kernel(int64_t K,
                                                               const int32_t* __restrict__ cap_t,
                                                               int32_t* __restrict__ start_t,
                                                               int64_t* __restrict__ cap_total) {
    __shared__ int64_t part[kScanThreads];
    const int t = threadIdx.x;
    const int64_t per = ceil_div(K, kScanThreads);
    const int64_t a = t * per;
    const int64_t e = (a + per < K) ? a + per : K;
    int64_t sum = 0;
    for (int64_t c = a; c < e; ++c) sum += cap_t[c];
    part[t] = sum;
    __syncthreads();
    // Hillis-Steele inclusive scan over the per-thread sums.
    for (int off = 1; off < kScanThreads; off <<= 1) {
        const int64_t add = (t >= off) ? part[t - off] : 0;
        __syncthreads();
        part[t] += add;
        __syncthreads();
    }
    int64_t run = part[t] - sum;
    for (int64_t c = a; c < e; ++c) {
        start_t[c] = static_cast<int32_t>(run);
        run += cap_t[c];
    }
    if (t == kScanThreads - 1) *cap_total = part[t];
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

extern "C" int64_t slk_transpose_workspace_bytes(const slk_csr* W) {
    if (W == nullptr || W->nrows <= 0 || W->ncols <= 0) return 0;
    const slk::BlockPlan p = slk::plan_blocks(W->nrows, W->ncols);
    return p.nblk * W->ncols * static_cast<int64_t>(sizeof(int32_t));
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
                           WT_row_capacity, WT_row_start, capT_dev);
        return check_launch("transpose_count");
    }
    if (WT_row_start == nullptr || WT_row_nnz == nullptr || WT_row_capacity == nullptr) {
        return fail(SLK_EINVAL, "transpose: NULL WT row arrays");
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
                       WT_row_nnz, WT_row_capacity);
    if (int rc = check_launch("transpose_count/colscan")) return rc;
    hipLaunchKernelGGL(tr_scan_kernel, dim3(1), dim3(kScanThreads), 0, st, K, WT_row_capacity,
                       WT_row_start, capT_dev);
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
    const BlockPlan p = plan_blocks(M, K);
    const int64_t need = p.nblk * K * static_cast<int64_t>(sizeof(int32_t));
    if (workspace_bytes < need || (need > 0 && workspace == nullptr)) {
        return fail(SLK_EINVAL, "transpose: workspace too small");
    }
    hipStream_t st = as_stream(stream);
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
