// Visiting schedules for slk_sddmm (segment list) and slk_spmm (phase
// bounds) on large layers. Neither changes any slot's arithmetic; they only
// decide which wave computes which slots, and when.
//
// Within a row the live columns ascend, so the row's slots in column block b
// (columns [b·C, (b+1)·C)) are one run [lo(r, b), lo(r, b+1)), lo(r, b) =
// first live slot of row r with column >= b·C. The segment list is a
// counting sort of these runs on (block, row), without atomics:
//
//   S1 bounds   one thread per (row, block boundary): lo(r, b) by binary
//               search over the row's columns.
//   S2 rowscan  one workgroup per block: exclusive scan over rows of the
//               run's segment counts (a run of n slots is ceil(n / S)
//               segments of at most S consecutive slots) -> each run's
//               offset inside its block, and the block total.
//   S3 blkscan  one workgroup: exclusive scan of the block totals, each
//               padded to a multiple of SLK_SEG_GROUP (a group of segments
//               never straddles two blocks); the number of groups in use is
//               written to device memory.
//   S4 scatter  one thread per (row, block): writes its run's segments.
//   S5 order    one workgroup per group: a stable sort of the group's
//               segments by count, largest first, so the 16 segments a
//               wave of slk_sddmm takes have close counts and the wave skips
//               the steps none of them has (C5 at 95%: 31% fewer steps).
//
// The padding is left as empty segments by a fill pass that runs first. The
// list's length is an upper bound the host can compute without a device read.
// The phase bounds are S1 with the phase width as the block.
#include "common.hpp"

#include <algorithm>

namespace slk {
namespace {

constexpr int kSchedThreads = 256;
constexpr int kScanBlock = 1024;

__global__ __launch_bounds__(kSchedThreads) void sl_bounds_kernel(
    int64_t M, int64_t nb, int64_t C, const int32_t* __restrict__ row_start,
    const int32_t* __restrict__ row_nnz, const int32_t* __restrict__ col,
    int32_t* __restrict__ lo) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kSchedThreads + threadIdx.x;
    if (t >= M * (nb + 1)) return;
    const int64_t r = t / (nb + 1);
    const int64_t b = t - r * (nb + 1);
    const int64_t s0 = row_start[r];
    int64_t a = 0, e = row_nnz[r];  // first live slot of row r with col >= b*C
    const int64_t key = b * C;
    while (a < e) {
        const int64_t mid = (a + e) >> 1;
        if (col[s0 + mid] < key) a = mid + 1; else e = mid;
    }
    lo[t] = static_cast<int32_t>(s0 + a);
}

// One workgroup per block b: off[r*nb + b] = sum of run lengths of rows < r,
// total[b] = the block's entry count. With S > 1 a run counts as its
// ceil(length / S) segments.
template <int S>
__global__ __launch_bounds__(kScanBlock) void sl_rowscan_kernel(
    int64_t M, int64_t nb, const int32_t* __restrict__ lo, int32_t* __restrict__ off,
    int32_t* __restrict__ total) {
    __shared__ int32_t part[kScanBlock];
    const int64_t b = blockIdx.x;
    const int t = threadIdx.x;
    const int64_t per = ceil_div(M, kScanBlock);
    const int64_t r0 = min(M, t * per), r1 = min(M, r0 + per);
    auto len = [&](int64_t r) {
        const int32_t n = lo[r * (nb + 1) + b + 1] - lo[r * (nb + 1) + b];
        return S == 1 ? n : (n + S - 1) / S;
    };
    int32_t sum = 0;
    for (int64_t r = r0; r < r1; ++r) sum += len(r);
    part[t] = sum;
    __syncthreads();
    for (int d = 1; d < kScanBlock; d <<= 1) {  // inclusive Hillis-Steele scan
        const int32_t add = t >= d ? part[t - d] : 0;
        __syncthreads();
        part[t] += add;
        __syncthreads();
    }
    int32_t run = part[t] - sum;
    for (int64_t r = r0; r < r1; ++r) {
        off[r * nb + b] = run;
        run += len(r);
    }
    if (t == kScanBlock - 1) total[b] = part[t];
}

// start[b] = exclusive scan of the block totals, each rounded up to a
// multiple of PAD; with PAD > 1 *groups = the padded sum / PAD.
template <int PAD>
__global__ __launch_bounds__(kScanBlock) void sl_blkscan_kernel(int64_t nb,
                                                               const int32_t* __restrict__ total,
                                                               int32_t* __restrict__ start,
                                                               int32_t* __restrict__ groups) {
    __shared__ int32_t part[kScanBlock];
    const int t = threadIdx.x;
    const int64_t per = ceil_div(nb, kScanBlock);
    const int64_t a = min(nb, t * per), e = min(nb, a + per);
    auto padded = [&](int64_t b) { return PAD == 1 ? total[b] : (total[b] + PAD - 1) / PAD * PAD; };
    int32_t sum = 0;
    for (int64_t b = a; b < e; ++b) sum += padded(b);
    part[t] = sum;
    __syncthreads();
    for (int d = 1; d < kScanBlock; d <<= 1) {
        const int32_t add = t >= d ? part[t - d] : 0;
        __syncthreads();
        part[t] += add;
        __syncthreads();
    }
    int32_t run = part[t] - sum;
    for (int64_t b = a; b < e; ++b) {
        start[b] = run;
        run += padded(b);
    }
    if (PAD > 1 && t == kScanBlock - 1) groups[0] = part[t] / PAD;
}

// The rows order[0 .. T) left out of the list: every bound of such a row is
// its first slot, so all its runs are empty.
__global__ __launch_bounds__(kSchedThreads) void sl_skip_rows_kernel(
    int64_t T, int64_t nb, const int32_t* __restrict__ order,
    const int32_t* __restrict__ row_start, int32_t* __restrict__ lo) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kSchedThreads + threadIdx.x;
    if (t >= T * (nb + 1)) return;
    const int64_t p = t / (nb + 1);
    const int64_t r = order[p];
    lo[r * (nb + 1) + (t - p * (nb + 1))] = row_start[r];
}

// Segments of run (r, b): seg_start = first slot, seg_row = r, seg_count <= S.
template <int S>
__global__ __launch_bounds__(kSchedThreads) void sg_scatter_kernel(
    int64_t M, int64_t nb, const int32_t* __restrict__ lo, const int32_t* __restrict__ off,
    const int32_t* __restrict__ start, int32_t* __restrict__ seg_start,
    int32_t* __restrict__ seg_row, int32_t* __restrict__ seg_count) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kSchedThreads + threadIdx.x;
    if (t >= M * nb) return;
    const int64_t r = t / nb;
    const int64_t b = t - r * nb;
    const int32_t a = lo[r * (nb + 1) + b];
    const int32_t e = lo[r * (nb + 1) + b + 1];
    const int64_t dst = static_cast<int64_t>(start[b]) + off[t];
    for (int32_t s = a, k = 0; s < e; s += S, ++k) {
        seg_start[dst + k] = s;
        seg_row[dst + k] = static_cast<int32_t>(r);
        seg_count[dst + k] = min(S, e - s);
    }
}

// S5: each group of SLK_SEG_GROUP segments in use, stably sorted by count,
// largest first (padding, count 0, last). A segment's rank is the number of
// segments with a larger count plus those before it with the same count.
__global__ __launch_bounds__(SLK_SEG_GROUP) void sg_order_kernel(
    const int32_t* __restrict__ groups, int32_t* __restrict__ seg_start,
    int32_t* __restrict__ seg_row, int32_t* __restrict__ seg_count) {
    if (static_cast<int64_t>(blockIdx.x) >= groups[0]) return;  // block-uniform
    __shared__ int32_t cn[SLK_SEG_GROUP];
    const int64_t e = static_cast<int64_t>(blockIdx.x) * SLK_SEG_GROUP + threadIdx.x;
    const int32_t s = seg_start[e], r = seg_row[e], c = seg_count[e];
    cn[threadIdx.x] = c;
    __syncthreads();
    int rank = 0;
    for (int j = 0; j < SLK_SEG_GROUP; ++j) {
        const int32_t o = cn[j];
        rank += (o > c || (o == c && j < static_cast<int>(threadIdx.x))) ? 1 : 0;
    }
    __syncthreads();  // every entry of the group is read before any is written
    const int64_t d = static_cast<int64_t>(blockIdx.x) * SLK_SEG_GROUP + rank;
    seg_start[d] = s;
    seg_row[d] = r;
    seg_count[d] = c;
}

// Every entry an empty segment (row 0, slot 0, count 0): the padding.
__global__ __launch_bounds__(kSchedThreads) void sg_fill_kernel(int64_t n,
                                                                int32_t* __restrict__ seg_start,
                                                                int32_t* __restrict__ seg_row,
                                                                int32_t* __restrict__ seg_count) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kSchedThreads + threadIdx.x;
    if (t >= n) return;
    seg_start[t] = 0;
    seg_row[t] = 0;
    seg_count[t] = 0;
}

struct ListPlan {
    int64_t nb;        // column blocks
    int64_t lo_ints;   // M * (nb + 1)
    int64_t off_ints;  // M * nb
    int64_t bytes;     // lo + off + total + start
};

ListPlan plan_list(int64_t M, int64_t K, int64_t C) {
    ListPlan p{};
    p.nb = ceil_div(K, C);
    p.lo_ints = M * (p.nb + 1);
    p.off_ints = M * p.nb;
    p.bytes = static_cast<int64_t>(sizeof(int32_t)) * (p.lo_ints + p.off_ints + 2 * p.nb);
    return p;
}

}  // namespace
}  // namespace slk

extern "C" int64_t slk_seg_list_capacity(const slk_csr* W, int64_t block_cols, int64_t seg_slots) {
    if (W == nullptr || W->nrows <= 0 || W->ncols <= 0 || block_cols <= 0 || seg_slots <= 0) return 0;
    // every run of n slots makes ceil(n/S) <= n/S + 1 segments, and only
    // non-empty runs make any: at most min(cap, M*nb) of them; each block's
    // padding adds fewer than SLK_SEG_GROUP
    const int64_t nb = slk::ceil_div(W->ncols, block_cols);
    const int64_t cap = W->total_capacity;
    return cap / seg_slots + std::min(cap, W->nrows * nb) + nb * (SLK_SEG_GROUP - 1) + SLK_SEG_GROUP;
}

extern "C" int64_t slk_seg_list_workspace_bytes(const slk_csr* W, int64_t block_cols) {
    if (W == nullptr || W->nrows <= 0 || W->ncols <= 0 || block_cols <= 0) return 0;
    return slk::plan_list(W->nrows, W->ncols, block_cols).bytes;
}

extern "C" int slk_seg_list_build(const slk_csr* W, int64_t block_cols, int64_t seg_slots,
                                  void* workspace, int64_t workspace_bytes, int32_t* seg_start,
                                  int32_t* seg_row, int32_t* seg_count, int64_t n_seg,
                                  int32_t* seg_groups, void* stream) {
    using namespace slk;
    clear_error();
    if (int rc = validate_csr(W, "seg_list")) return rc;
    if (block_cols != 64 && block_cols != 128) {
        return fail(SLK_EINVAL, "seg_list: block_cols must be 64 or 128, got " +
                                    std::to_string(block_cols));
    }
    if (seg_slots != 4 && seg_slots != 8) {
        return fail(SLK_EINVAL, "seg_list: seg_slots must be 4 or 8, got " +
                                    std::to_string(seg_slots));
    }
    const int64_t M = W->nrows, K = W->ncols;
    if (seg_groups == nullptr) return fail(SLK_EINVAL, "seg_list: NULL seg_groups");
    hipStream_t st = as_stream(stream);
    if (M == 0 || K == 0) {
        hipLaunchKernelGGL(sl_blkscan_kernel<SLK_SEG_GROUP>, dim3(1), dim3(kScanBlock), 0, st,
                           int64_t{0}, nullptr, nullptr, seg_groups);
        return check_launch("seg_list/blkscan");
    }
    const int64_t need = slk_seg_list_capacity(W, block_cols, seg_slots);
    if (n_seg < need) {
        return fail(SLK_EINVAL, "seg_list: n_seg=" + std::to_string(n_seg) +
                                    " is below the required " + std::to_string(need));
    }
    if (seg_start == nullptr || seg_row == nullptr || seg_count == nullptr) {
        return fail(SLK_EINVAL, "seg_list: NULL output");
    }
    if (n_seg > INT32_MAX) return fail(SLK_EINVAL, "seg_list: matrix too large");
    const ListPlan p = plan_list(M, K, block_cols);
    if (workspace == nullptr || workspace_bytes < p.bytes) {
        return fail(SLK_EINVAL, "seg_list: workspace of " + std::to_string(workspace_bytes) +
                                    " bytes is smaller than the required " +
                                    std::to_string(p.bytes));
    }
    if (p.nb > INT32_MAX || ceil_div(p.lo_ints, kSchedThreads) > INT32_MAX) {
        return fail(SLK_EINVAL, "seg_list: matrix too large");
    }
    int32_t* lo = static_cast<int32_t*>(workspace);
    int32_t* off = lo + p.lo_ints;
    int32_t* total = off + p.off_ints;
    int32_t* start = total + p.nb;
    hipLaunchKernelGGL(sg_fill_kernel, dim3(static_cast<unsigned>(ceil_div(n_seg, kSchedThreads))),
                       dim3(kSchedThreads), 0, st, n_seg, seg_start, seg_row, seg_count);
    if (int rc = check_launch("seg_list/fill")) return rc;
    hipLaunchKernelGGL(sl_bounds_kernel, dim3(static_cast<unsigned>(ceil_div(p.lo_ints, kSchedThreads))),
                       dim3(kSchedThreads), 0, st, M, p.nb, block_cols, W->row_start, W->row_nnz,
                       W->col_indices, lo);
    if (int rc = check_launch("seg_list/bounds")) return rc;
    if (W->seg_dense_rows > 0) {
        const int64_t n = W->seg_dense_rows * (p.nb + 1);
        hipLaunchKernelGGL(sl_skip_rows_kernel, dim3(static_cast<unsigned>(ceil_div(n, kSchedThreads))),
                           dim3(kSchedThreads), 0, st, W->seg_dense_rows, p.nb, W->row_order,
                           W->row_start, lo);
        if (int rc = check_launch("seg_list/skip")) return rc;
    }
    if (seg_slots == 4) {
        hipLaunchKernelGGL(sl_rowscan_kernel<4>, dim3(static_cast<unsigned>(p.nb)), dim3(kScanBlock),
                           0, st, M, p.nb, lo, off, total);
    } else {
        hipLaunchKernelGGL(sl_rowscan_kernel<8>, dim3(static_cast<unsigned>(p.nb)), dim3(kScanBlock),
                           0, st, M, p.nb, lo, off, total);
    }
    if (int rc = check_launch("seg_list/rowscan")) return rc;
    hipLaunchKernelGGL(sl_blkscan_kernel<SLK_SEG_GROUP>, dim3(1), dim3(kScanBlock), 0, st, p.nb,
                       total, start, seg_groups);
    if (int rc = check_launch("seg_list/blkscan")) return rc;
    const dim3 sgrid(static_cast<unsigned>(ceil_div(p.off_ints, kSchedThreads)));
    if (seg_slots == 4) {
        hipLaunchKernelGGL(sg_scatter_kernel<4>, sgrid, dim3(kSchedThreads), 0, st, M, p.nb, lo,
                           off, start, seg_start, seg_row, seg_count);
    } else {
        hipLaunchKernelGGL(sg_scatter_kernel<8>, sgrid, dim3(kSchedThreads), 0, st, M, p.nb, lo,
                           off, start, seg_start, seg_row, seg_count);
    }
    if (int rc = check_launch("seg_list/scatter")) return rc;
    // groups past the ones in use (read on the device) exit at once
    hipLaunchKernelGGL(sg_order_kernel, dim3(static_cast<unsigned>(n_seg / SLK_SEG_GROUP)),
                       dim3(SLK_SEG_GROUP), 0, st, seg_groups, seg_start, seg_row, seg_count);
    return check_launch("seg_list/order");
}

extern "C" int slk_phase_bounds_build(const slk_csr* W, int64_t n_phases, int32_t* phase_lo,
                                      void* stream) {
    using namespace slk;
    clear_error();
    if (int rc = validate_csr(W, "phase_bounds")) return rc;
    if (n_phases < 1) {
        return fail(SLK_EINVAL, "phase_bounds: n_phases must be >= 1, got " +
                                    std::to_string(n_phases));
    }
    const int64_t M = W->nrows, K = W->ncols;
    if (M == 0) return SLK_OK;
    if (phase_lo == nullptr) return fail(SLK_EINVAL, "phase_bounds: NULL phase_lo");
    const int64_t n = M * (n_phases + 1);
    if (ceil_div(n, kSchedThreads) > INT32_MAX) return fail(SLK_EINVAL, "phase_bounds: too large");
    // the slot list's first pass with blocks of ceil(K / n_phases) columns
    const int64_t C = std::max<int64_t>(1, ceil_div(K, n_phases));
    hipLaunchKernelGGL(sl_bounds_kernel, dim3(static_cast<unsigned>(ceil_div(n, kSchedThreads))),
                       dim3(kSchedThreads), 0, as_stream(stream), M, n_phases, C, W->row_start,
                       W->row_nnz, W->col_indices, phase_lo);
    return check_launch("phase_bounds");
}
