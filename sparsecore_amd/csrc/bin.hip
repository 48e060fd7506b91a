// Binned slot streams for slk_spmm's LDS-staged kernel (slk_csr.bin_*).
//
// The LDS-staged SpMM streams X through LDS in chunks of KC = 80 / H rows;
// each wave owns RW rows of its workgroup's 16·RW and, chunk by chunk,
// applies the slots of its rows whose column falls in the chunk. The binned
// stream lists, for every wave unit u (its RW rows) and chunk ch, the unit's
// slots of that chunk row by row in slot order, so the kernel reads a
// chunk's work as one contiguous run whose per-row counts it knows in
// advance: no per-row search for where the chunk ends in the row, no
// per-row window of (column, value) pairs. Columns ascend within a row, so
// chunk order is slot order and every fma chain is unchanged.
//
//   B1 totals  one workgroup: each unit's slot count (the row_nnz of its
//              rows), exclusive scan -> bin_start.
//   B2 fill    one workgroup per unit: per-(chunk, row) counts in LDS,
//              written as bytes (bin_cnt); two scans give each (chunk, row)
//              run's place in the unit's stream and its first slot inside
//              its row; every slot is then written at its place: bin_off =
//              the byte offset of its X row inside the staged chunk
//              ((c mod KC)·H KiB), bin_slot = its slot index (the kernel
//              reads the value through it, so the stream does not go stale
//              when the values change).
#include "common.hpp"

namespace slk {
namespace {

constexpr int kBinWaves = 16;      // waves per workgroup of the LDS kernel
constexpr int kBinChunkRows = 80;  // X rows per chunk at one column half
constexpr int kB1Threads = 1024;
constexpr int kB2Threads = 256;

struct BinShape {
    int64_t P;        // positions covered (nrows - first)
    int64_t units;    // 16 per block of 16·rw positions
    int64_t nchunks;  // X chunks of KC rows
    int64_t kc;
};

int bin_shape(const slk_csr* W, int64_t first, int64_t rw, int64_t h, BinShape* s,
              const char* who) {
    if (int rc = validate_csr(W, who)) return rc;
    if (rw != 1 && rw != 2 && rw != 4 && rw != 8)
        return fail(SLK_EINVAL, std::string(who) + ": rw must be 1, 2, 4 or 8, got " +
                                    std::to_string(rw));
    if (h != 1 && h != 2)
        return fail(SLK_EINVAL, std::string(who) + ": h must be 1 or 2, got " + std::to_string(h));
    if (first < 0 || first > W->nrows)
        return fail(SLK_EINVAL, std::string(who) + ": first=" + std::to_string(first) +
                                    " outside [0, nrows]");
    if (first > 0 && W->row_order == nullptr)
        return fail(SLK_EINVAL, std::string(who) + ": first > 0 needs row_order");
    s->kc = kBinChunkRows / h;
    s->P = W->nrows - first;
    s->units = ceil_div(s->P, kBinWaves * rw) * kBinWaves;
    s->nchunks = ceil_div(W->ncols, s->kc);
    if (s->nchunks > SLK_BIN_MAX_CHUNKS)
        return fail(SLK_EINVAL, std::string(who) + ": " + std::to_string(s->nchunks) +
                                    " chunks of X rows exceed SLK_BIN_MAX_CHUNKS");
    if (s->units + 1 > INT32_MAX || 2 * s->units * s->nchunks > INT32_MAX)
        return fail(SLK_EINVAL, std::string(who) + ": matrix too large");
    return SLK_OK;
}

// Row of unit u's row j, or -1 past the covered positions.
__device__ __forceinline__ int64_t bin_row(int64_t u, int j, int rw, int64_t P,
                                           const int32_t* __restrict__ order) {
    const int64_t q = (u / kBinWaves) * (kBinWaves * rw) + (u % kBinWaves) + kBinWaves * j;
    if (q >= P) return -1;
    return order != nullptr ? order[q] : q;
}

// B1: start[u] = slots of units before u; start[units] = the total.
__global__ __launch_bounds__(kB1Threads) void bin_total_kernel(
    int64_t units, int rw, int64_t P, const int32_t* __restrict__ order,
    const int32_t* __restrict__ row_nnz, int32_t* __restrict__ start) {
    __shared__ int64_t part[kB1Threads];
    const int t = threadIdx.x;
    const int64_t per = ceil_div(units, kB1Threads);
    const int64_t a = min(units, t * per), e = min(units, a + per);
    auto slots = [&](int64_t u) {
        int64_t n = 0;
        for (int j = 0; j < rw; ++j) {
            const int64_t r = bin_row(u, j, rw, P, order);
            if (r >= 0) n += row_nnz[r];
        }
        return n;
    };
    int64_t sum = 0;
    for (int64_t u = a; u < e; ++u) sum += slots(u);
    part[t] = sum;
    __syncthreads();
    for (int d = 1; d < kB1Threads; d <<= 1) {  // inclusive Hillis-Steele scan
        const int64_t add = t >= d ? part[t - d] : 0;
        __syncthreads();
        part[t] += add;
        __syncthreads();
    }
    int64_t run = part[t] - sum;
    for (int64_t u = a; u < e; ++u) {
        start[u] = static_cast<int32_t>(run);
        run += slots(u);
    }
    if (t == kB1Threads - 1) start[units] = static_cast<int32_t>(part[t]);
}

// Exclusive scan over LDS entries v[i·stride], i < n, by the threads
// [t0, t0 + T) of the workgroup (T a power of two <= 256), each taking a
// contiguous range; part is T ints of scratch. Ends with a barrier of the
// whole workgroup (every thread must call it).
template <int T>
__device__ __forceinline__ void lds_exclusive_scan(int32_t* v, int64_t n, int stride, int t,
                                                   bool mine, int32_t* part) {
    const int64_t per = ceil_div(n, T);
    const int64_t a = mine ? min(n, t * per) : 0, e = mine ? min(n, a + per) : 0;
    int32_t sum = 0;
    for (int64_t i = a; i < e; ++i) sum += v[i * stride];
    if (mine) part[t] = sum;
    __syncthreads();
    for (int d = 1; d < T; d <<= 1) {
        const int32_t add = (mine && t >= d) ? part[t - d] : 0;
        __syncthreads();
        if (mine) part[t] += add;
        __syncthreads();
    }
    if (mine) {
        int32_t run = part[t] - sum;
        for (int64_t i = a; i < e; ++i) {
            const int32_t c = v[i * stride];
            v[i * stride] = run;
            run += c;
        }
    }
    __syncthreads();
}

// B2: one workgroup per unit. LDS: cnt -> P (nchunks·8, the (chunk, row)
// runs' places in the unit's stream) and Q (nchunks·8, each run's first
// slot relative to its row's start).
__global__ __launch_bounds__(kB2Threads) void bin_fill_kernel(
    int rw, int h, int64_t P, int64_t nch, int64_t n_bin, const int32_t* __restrict__ order,
    const int32_t* __restrict__ row_start, const int32_t* __restrict__ row_nnz,
    const int32_t* __restrict__ col, const int32_t* __restrict__ start,
    uint32_t* __restrict__ bin_cnt, int32_t* __restrict__ bin_off,
    int32_t* __restrict__ bin_slot) {
    extern __shared__ int32_t lds[];
    int32_t* cnt = lds;              // [nch][8]
    int32_t* Q = lds + nch * 8;      // [nch][8]
    __shared__ int32_t part[kB2Threads];
    __shared__ int32_t rs_s[8], nz_s[8];
    const int64_t u = blockIdx.x;
    const int t = threadIdx.x;
    const int kc = kBinChunkRows / h;
    const int32_t row_bytes = h * 1024;
    if (t < 8) {
        const int64_t r = t < rw ? bin_row(u, t, rw, P, order) : -1;
        rs_s[t] = r >= 0 ? row_start[r] : 0;
        nz_s[t] = r >= 0 ? row_nnz[r] : 0;
    }
    for (int64_t i = t; i < nch * 8; i += kB2Threads) cnt[i] = 0;
    __syncthreads();
    for (int j = 0; j < rw; ++j) {
        const int32_t s0 = rs_s[j], n = nz_s[j];
        for (int32_t s = t; s < n; s += kB2Threads) atomicAdd(&cnt[(col[s0 + s] / kc) * 8 + j], 1);
    }
    __syncthreads();
    // counts as bytes: word 2ch holds rows 0..3, word 2ch + 1 rows 4..7
    uint32_t* out = bin_cnt + u * nch * 2;
    for (int64_t i = t; i < nch * 2; i += kB2Threads) {
        const int32_t* c = cnt + i * 4;
        out[i] = static_cast<uint32_t>(c[0]) | static_cast<uint32_t>(c[1]) << 8 |
                 static_cast<uint32_t>(c[2]) << 16 | static_cast<uint32_t>(c[3]) << 24;
    }
    for (int64_t i = t; i < nch * 8; i += kB2Threads) Q[i] = cnt[i];
    __syncthreads();
    // Q: per row j, exclusive scan over the chunks (32 threads per row)
    lds_exclusive_scan<32>(Q + (t >> 5), nch, 8, t & 31, true, part + (t >> 5) * 32);
    // cnt -> P: exclusive scan in (chunk, row) order
    lds_exclusive_scan<kB2Threads>(cnt, nch * 8, 1, t, true, part);
    const int64_t e0 = start[u];
    for (int j = 0; j < rw; ++j) {
        const int32_t s0 = rs_s[j], n = nz_s[j];
        for (int32_t s = t; s < n; s += kB2Threads) {
            const int32_t c = col[s0 + s];
            const int32_t ch = c / kc;
            const int64_t pos = e0 + cnt[ch * 8 + j] + (s - Q[ch * 8 + j]);
            if (pos >= n_bin) continue;
            bin_off[pos] = (c - ch * kc) * row_bytes;
            bin_slot[pos] = s0 + s;
        }
    }
}

}  // namespace
}  // namespace slk

extern "C" int slk_bin_sizes(const slk_csr* W, int64_t first, int64_t rw, int64_t h,
                             int64_t* units, int64_t* nchunks) {
    using namespace slk;
    clear_error();
    BinShape s{};
    if (int rc = bin_shape(W, first, rw, h, &s, "bin_sizes")) return rc;
    if (units != nullptr) *units = s.units;
    if (nchunks != nullptr) *nchunks = s.nchunks;
    return SLK_OK;
}

extern "C" int slk_bin_build(const slk_csr* W, int64_t first, int64_t rw, int64_t h,
                             int32_t* bin_off, int32_t* bin_slot, int64_t n_bin,
                             uint32_t* bin_cnt, int32_t* bin_start, void* stream) {
    using namespace slk;
    clear_error();
    BinShape s{};
    if (int rc = bin_shape(W, first, rw, h, &s, "bin_build")) return rc;
    if (n_bin < 0) return fail(SLK_EINVAL, "bin_build: negative n_bin");
    if (bin_start == nullptr || (s.units > 0 && bin_cnt == nullptr) ||
        (n_bin > 0 && (bin_off == nullptr || bin_slot == nullptr)))
        return fail(SLK_EINVAL, "bin_build: NULL output");
    hipStream_t st = as_stream(stream);
    const int32_t* order = first > 0 ? W->row_order + first : nullptr;
    hipLaunchKernelGGL(bin_total_kernel, dim3(1), dim3(kB1Threads), 0, st, s.units,
                       static_cast<int>(rw), s.P, order, W->row_nnz, bin_start);
    if (int rc = check_launch("bin_build/totals")) return rc;
    if (s.units == 0) return SLK_OK;
    // The covered slot count is not read back: the fill writes only entries
    // below n_bin (a short buffer gives a short stream, never a stray write).
    const size_t lds = static_cast<size_t>(2 * s.nchunks * 8) * sizeof(int32_t);
    hipLaunchKernelGGL(bin_fill_kernel, dim3(static_cast<unsigned>(s.units)), dim3(kB2Threads), lds,
                       st, static_cast<int>(rw), static_cast<int>(h), s.P, s.nchunks, n_bin, order,
                       W->row_start, W->row_nnz, W->col_indices, bin_start, bin_cnt, bin_off,
                       bin_slot);
    return check_launch("bin_build/fill");
}
