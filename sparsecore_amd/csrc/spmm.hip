// Forward SpMM  Y = W·X  for a padded-CSR W (gfx950).
//
// Reference semantics (csrc/kernels/spmm_avx2.cpp:123-262, spmm.cpp:84-104):
// Y is zeroed, then for every row i and live slot s (in slot order) the
// write-through update  y[i,j] = fma(v_s, X[c_s, j], y[i,j])  is applied to
// all j. Every output element is therefore an ordered fused multiply-add
// chain starting at +0.0. Both kernels here evaluate exactly that chain per
// element, so results are bit-identical to the reference CPU kernels.
//
// Work decomposition: one "item" is (row, column tile). Items are ordered
// tile-major (item = tile * M + r) so that waves resident at the same time
// gather from the same K x tile slab of X, which stays in L2. Within a tile,
// r indexes W->row_order when the caller supplies it (rows by descending
// nnz): the longest rows of every tile start first, so a few heavy rows of a
// skewed matrix do not run alone at the end of the grid, and the rows that
// share a wave in spmm_group_kernel have similar lengths. The order changes
// only which wave computes a row, never the arithmetic.
//
//  * spmm_wave_kernel — one item per wave (64 lanes x VEC columns). The
//    row's (col, value) stream is fetched 64 slots at a time with one
//    coalesced load into lane registers (the next chunk is requested as soon
//    as the current one starts) and broadcast slot by slot with readlane, so
//    the X gathers use a scalar base address. Gathers are issued U slots at
//    a time into two register buffers that alternate (the next batch — the
//    next chunk's first one at a chunk's end — is in flight while the current
//    one is consumed), so a wave keeps 2U gathers outstanding instead of
//    waiting once per slot, and never drains at a chunk boundary.
//  * spmm_group_kernel — several items per wave (L < 64 lanes each) for
//    narrow X (N < 64): each lane streams its row's metadata itself.
//
// VEC (floats per lane) is chosen so that small problems still launch
// enough waves to hide gather latency; large problems use 16-byte gathers.
#include "common.hpp"

#include <cstdlib>

namespace slk {
namespace {

constexpr int kSpmmBlock = 256;  // 4 waves per workgroup

template <int VEC>
struct VecIO;

template <>
struct VecIO<4> {
    typedef f32x4 T;
    static __device__ __forceinline__ T load(const float* p) {
        return *reinterpret_cast<const f32x4*>(p);
    }
    static __device__ __forceinline__ void store(float* p, const float* a) {
        f32x4 v = {a[0], a[1], a[2], a[3]};
        *reinterpret_cast<f32x4*>(p) = v;
    }
    static __device__ __forceinline__ float get(const T& v, int k) { return v[k]; }
};

template <>
struct VecIO<2> {
    typedef float T __attribute__((ext_vector_type(2)));
    static __device__ __forceinline__ T load(const float* p) {
        return *reinterpret_cast<const T*>(p);
    }
    static __device__ __forceinline__ void store(float* p, const float* a) {
        T v = {a[0], a[1]};
        *reinterpret_cast<T*>(p) = v;
    }
    static __device__ __forceinline__ float get(const T& v, int k) { return v[k]; }
};

template <>
struct VecIO<1> {
    typedef float T;
    static __device__ __forceinline__ T load(const float* p) { return *p; }
    static __device__ __forceinline__ void store(float* p, const float* a) { *p = a[0]; }
    static __device__ __forceinline__ float get(const T& v, int) { return v; }
};

__device__ __forceinline__ int32_t bcast_i(int32_t v, int32_t lane) {
    return __builtin_amdgcn_readlane(v, lane);
}
__device__ __forceinline__ float bcast_f(float v, int32_t lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Gathers X rows of slots [k, k + U) of the staged metadata chunk (n = slots
// of the chunk). A full batch is unguarded; the chunk's last batch checks k.
// The X row base is wave-uniform (scalar) and the lane offset a 32-bit
// vector offset, so each gather is one load with no per-slot vector math.
template <int VEC>
__device__ __forceinline__ typename VecIO<VEC>::T gather(const float* __restrict__ X, int32_t c,
                                                         int64_t N, uint32_t off_bytes) {
    const char* rowp = reinterpret_cast<const char*>(X + static_cast<int64_t>(c) * N);
    return VecIO<VEC>::load(reinterpret_cast<const float*>(rowp + off_bytes));
}

template <int VEC, int U>
__device__ __forceinline__ void issue(typename VecIO<VEC>::T (&x)[U], int32_t mc, int32_t k,
                                      int32_t n, const float* __restrict__ X, int64_t N,
                                      uint32_t n0, bool active) {
    if (!active) return;
    if (k + U <= n) {
#pragma unroll
        for (int u = 0; u < U; ++u) x[u] = gather<VEC>(X, bcast_i(mc, k + u), N, n0);
    } else {
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (k + u < n) x[u] = gather<VEC>(X, bcast_i(mc, k + u), N, n0);
    }
}

template <int VEC, int U>
__device__ __forceinline__ void consume(const typename VecIO<VEC>::T (&x)[U], float mv, int32_t k,
                                        int32_t n, float (&acc)[VEC], bool active) {
    if (!active) return;
    if (k + U <= n) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float v = bcast_f(mv, k + u);
#pragma unroll
            for (int e = 0; e < VEC; ++e) acc[e] = __builtin_fmaf(v, VecIO<VEC>::get(x[u], e), acc[e]);
        }
    } else {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (k + u < n) {
                const float v = bcast_f(mv, k + u);
#pragma unroll
                for (int e = 0; e < VEC; ++e)
                    acc[e] = __builtin_fmaf(v, VecIO<VEC>::get(x[u], e), acc[e]);
            }
        }
    }
}

// Bias epilogue: y = fl(chain + b), one rounding after the finished chain —
// what the reference's separate `y + bias` (sparselab/nn.py:237-241) gives.
template <int VEC>
__device__ __forceinline__ void add_bias(float (&acc)[VEC], float b) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = acc[e] + b;
}

__device__ __forceinline__ void load_meta(const int32_t* __restrict__ col,
                                          const float* __restrict__ val, int32_t start,
                                          int32_t base, int32_t nnz, int lane, int32_t& mc,
                                          float& mv) {
    mc = 0;
    mv = 0.0f;
    if (base + lane < nnz) {
        mc = col[start + base + lane];
        mv = val[start + base + lane];
    }
}

template <int VEC, int U>
__global__ __launch_bounds__(kSpmmBlock) void spmm_wave_kernel(
    int64_t M, int64_t N, int64_t nitems, const int32_t* __restrict__ order,
    const int32_t* __restrict__ row_start, const int32_t* __restrict__ row_nnz,
    const int32_t* __restrict__ col, const float* __restrict__ val,
    const float* __restrict__ X, const float* __restrict__ bias, float* __restrict__ Y) {
    typedef typename VecIO<VEC>::T T;
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t item = wave_id();
    if (item >= nitems) return;  // wave-uniform; no barriers below
    const int64_t tile = item / M;
    const int64_t r = item - tile * M;
    const int64_t row = order != nullptr ? order[r] : r;
    const int64_t n0 = (tile * kWave + lane) * VEC;
    const bool active = n0 < N;  // N % VEC == 0, so n0 + VEC <= N
    const int32_t start = row_start[row];
    const int32_t nnz = row_nnz[row];
    const uint32_t off = static_cast<uint32_t>(n0) * 4u;  // 4N < 2^31 (launcher check)

    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.0f;

    static_assert(kWave % (2 * U) == 0, "a full chunk holds an even number of batches");
    int32_t mc, nmc = 0;
    float mv, nmv = 0.0f;
    load_meta(col, val, start, 0, nnz, lane, mc, mv);
    if (nnz > kWave) load_meta(col, val, start, kWave, nnz, lane, nmc, nmv);
    T xa[U], xc[U];
    issue<VEC, U>(xa, mc, 0, nnz < kWave ? nnz : kWave, X, N, off, active);
    int32_t base = 0;
    // Full 64-slot chunks: batches alternate xa, xc, xa, ... and the chunk's
    // last step already issues the next chunk's first batch into xa, so the
    // gathers never drain at a chunk boundary.
    for (; base + kWave <= nnz; base += kWave) {
#pragma unroll
        for (int32_t k = 0; k < kWave; k += 2 * U) {
            issue<VEC, U>(xc, mc, k + U, kWave, X, N, off, active);
            consume<VEC, U>(xa, mv, k, kWave, acc, active);
            if (k + 2 * U < kWave) {
                issue<VEC, U>(xa, mc, k + 2 * U, kWave, X, N, off, active);
            } else if (base + kWave < nnz) {
                const int32_t nn = nnz - base - kWave;
                issue<VEC, U>(xa, nmc, 0, nn < kWave ? nn : kWave, X, N, off, active);
            }
            consume<VEC, U>(xc, mv, k + U, kWave, acc, active);
        }
        mc = nmc;
        mv = nmv;
        if (base + 2 * kWave < nnz) load_meta(col, val, start, base + 2 * kWave, nnz, lane, nmc, nmv);
    }
    // Last, partial chunk (xa already holds its first batch).
    if (base < nnz) {
        const int32_t n = nnz - base;
        for (int32_t k = 0;;) {
            issue<VEC, U>(xc, mc, k + U, n, X, N, off, active && k + U < n);
            consume<VEC, U>(xa, mv, k, n, acc, active);
            k += U;
            if (k >= n) break;
            issue<VEC, U>(xa, mc, k + U, n, X, N, off, active && k + U < n);
            consume<VEC, U>(xc, mv, k, n, acc, active);
            k += U;
            if (k >= n) break;
        }
    }
    if (active) {
        if (bias != nullptr) add_bias<VEC>(acc, bias[row]);
        VecIO<VEC>::store(Y + row * N + n0, acc);
    }
}

template <int L, int VEC>
__global__ __launch_bounds__(kSpmmBlock) void spmm_group_kernel(
    int64_t M, int64_t N, int64_t nitems, const int32_t* __restrict__ order,
    const int32_t* __restrict__ row_start, const int32_t* __restrict__ row_nnz,
    const int32_t* __restrict__ col, const float* __restrict__ val,
    const float* __restrict__ X, const float* __restrict__ bias, float* __restrict__ Y) {
    typedef VecIO<VEC> IO;
    constexpr int kUnroll = 8;
    constexpr int kItemsPerWave = kWave / L;
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t item = wave_id() * kItemsPerWave + lane / L;
    if (item >= nitems) return;
    const int64_t tile = item / M;
    const int64_t r = item - tile * M;
    const int64_t row = order != nullptr ? order[r] : r;
    const int64_t n0 = (tile * L + (lane % L)) * VEC;
    const bool active = n0 < N;

    const int32_t start = row_start[row];
    const int32_t nnz = row_nnz[row];
    const int32_t* c_ptr = col + start;
    const float* v_ptr = val + start;
    const float* xb = X + n0;

    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.0f;

    int32_t s = 0;
    for (; s + kUnroll <= nnz; s += kUnroll) {
        int32_t c[kUnroll];
        float v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            c[u] = c_ptr[s + u];
            v[u] = v_ptr[s + u];
        }
        typename IO::T x[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u)
            if (active) x[u] = IO::load(xb + static_cast<int64_t>(c[u]) * N);
        if (active) {
#pragma unroll
            for (int u = 0; u < kUnroll; ++u)
#pragma unroll
                for (int e = 0; e < VEC; ++e) acc[e] = __builtin_fmaf(v[u], IO::get(x[u], e), acc[e]);
        }
    }
    for (; s < nnz; ++s) {
        const int32_t c = c_ptr[s];
        const float v = v_ptr[s];
        if (active) {
            const typename IO::T x = IO::load(xb + static_cast<int64_t>(c) * N);
#pragma unroll
            for (int e = 0; e < VEC; ++e) acc[e] = __builtin_fmaf(v, IO::get(x, e), acc[e]);
        }
    }
    if (active) {
        if (bias != nullptr) add_bias<VEC>(acc, bias[row]);
        IO::store(Y + row * N + n0, acc);
    }
}

// ───────────────────────── LDS-tiled kernel ─────────────────────────────────
//
// spmm_tile_kernel — for large problems. A workgroup of 8 waves owns a
// 64-row x 128-column output tile: each wave holds 8 rows, each lane two
// adjacent columns, accumulators in registers. X is streamed through LDS in
// chunks of kTileK rows (the next chunk is prefetched into registers while
// the current one is consumed). For each chunk every row consumes its slots
// whose column falls in the chunk; columns ascend within a row, so walking
// the chunks in order visits each row's slots in slot order and the fma chain
// of every element is exactly the reference's. Each X element is fetched
// from L2/HBM once per workgroup and read from LDS by every row of the tile
// that uses it, instead of being gathered through L1 once per slot.
//
// A wave advances its 8 rows in lockstep (one slot of every row per step), so
// eight independent LDS reads are in flight per step. A row's (col, value)
// stream sits in registers 64 slots at a time and is reloaded when less than
// half of the batch is left; a row with more slots in one chunk than its
// batch holds (a near-dense row) finishes the chunk in a per-row loop.
constexpr int kTileCols = 128;                     // 64 lanes x 2 columns
constexpr int kTileK = 64;                         // X rows per LDS chunk
constexpr int kRowsPerWave = 8;
constexpr int kTileWaves = 8;
constexpr int kTileRows = kRowsPerWave * kTileWaves;  // 64
constexpr int kTileThreads = kTileWaves * kWave;      // 512
constexpr int kTilePrefetch = kTileK * kTileCols / (2 * kTileThreads);  // float2 per thread

typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void tile_reload(int32_t& base, int32_t pos, int32_t end, int lane,
                                            const int32_t* __restrict__ col,
                                            const float* __restrict__ val, int32_t& mc,
                                            float& mv) {
    base = pos;
    const int32_t sl = pos + lane;
    mc = sl < end ? col[sl] : INT32_MAX;
    mv = sl < end ? val[sl] : 0.0f;
}

__global__ __launch_bounds__(kTileThreads) void spmm_tile_kernel(
    int64_t M, int64_t K, int64_t N, int64_t nrowblk, const int32_t* __restrict__ row_start,
    const int32_t* __restrict__ row_nnz, const int32_t* __restrict__ col,
    const float* __restrict__ val, const float* __restrict__ X, const float* __restrict__ bias,
    float* __restrict__ Y) {
    __shared__ f32x2 xs[kTileK][kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t lb = xcd_logical_block(blockIdx.x, gridDim.x);
    const int64_t ntile = lb / nrowblk;
    const int64_t rb = lb - ntile * nrowblk;
    const int64_t n = ntile * kTileCols + 2 * lane;  // N is even for this kernel
    const bool n_ok = n < N;
    const int64_t r0 = rb * kTileRows + static_cast<int64_t>(w) * kRowsPerWave;

    int32_t pos[kRowsPerWave], end[kRowsPerWave], base[kRowsPerWave];
    int32_t mc[kRowsPerWave];
    float mv[kRowsPerWave];
    f32x2 acc[kRowsPerWave];
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) {
        const int64_t row = r0 + r;
        const int32_t s = row < M ? row_start[row] : 0;
        const int32_t e = row < M ? s + row_nnz[row] : 0;
        pos[r] = s;
        end[r] = e;
        tile_reload(base[r], s, e, lane, col, val, mc[r], mv[r]);
        acc[r] = f32x2{0.0f, 0.0f};
    }

    // thread t stages chunk rows (t / 64) + 8j, j < kTilePrefetch, at its two columns
    const int krow0 = threadIdx.x >> 6;
    f32x2 pre[kTilePrefetch];
    auto prefetch = [&](int64_t k0) {
#pragma unroll
        for (int j = 0; j < kTilePrefetch; ++j) {
            const int64_t k = k0 + krow0 + j * kTileWaves;
            pre[j] = (k < K && n_ok) ? *reinterpret_cast<const f32x2*>(X + k * N + n)
                                     : f32x2{0.0f, 0.0f};
        }
    };
    const int64_t nchunks = ceil_div(K, kTileK);
    prefetch(0);
    for (int64_t ch = 0; ch < nchunks; ++ch) {
        __syncthreads();  // every wave is done reading the previous chunk
#pragma unroll
        for (int j = 0; j < kTilePrefetch; ++j) xs[krow0 + j * kTileWaves][lane] = pre[j];
        __syncthreads();
        const int32_t k0 = static_cast<int32_t>(ch * kTileK);
        const int32_t k1 = k0 + kTileK;
        if (ch + 1 < nchunks) prefetch(k1);

        int32_t first[kRowsPerWave], cnt[kRowsPerWave];
        int32_t lo = kWave, hi = 0;
#pragma unroll
        for (int r = 0; r < kRowsPerWave; ++r) {
            if (pos[r] < end[r] && pos[r] > base[r] + kWave / 2)
                tile_reload(base[r], pos[r], end[r], lane, col, val, mc[r], mv[r]);
            first[r] = pos[r] - base[r];
            cnt[r] = __popcll(__ballot(lane >= first[r] && mc[r] < k1));
            lo = cnt[r] < lo ? cnt[r] : lo;
            hi = cnt[r] > hi ? cnt[r] : hi;
        }
        int32_t k = 0;
        for (; k < lo; ++k) {  // every row has a slot at step k
            f32x2 x[kRowsPerWave];
#pragma unroll
            for (int r = 0; r < kRowsPerWave; ++r) x[r] = xs[bcast_i(mc[r], first[r] + k) - k0][lane];
#pragma unroll
            for (int r = 0; r < kRowsPerWave; ++r) {
                const float v = bcast_f(mv[r], first[r] + k);
                acc[r][0] = __builtin_fmaf(v, x[r][0], acc[r][0]);
                acc[r][1] = __builtin_fmaf(v, x[r][1], acc[r][1]);
            }
        }
        for (; k < hi; ++k) {
#pragma unroll
            for (int r = 0; r < kRowsPerWave; ++r) {
                if (k < cnt[r]) {
                    const f32x2 x = xs[bcast_i(mc[r], first[r] + k) - k0][lane];
                    const float v = bcast_f(mv[r], first[r] + k);
                    acc[r][0] = __builtin_fmaf(v, x[0], acc[r][0]);
                    acc[r][1] = __builtin_fmaf(v, x[1], acc[r][1]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < kRowsPerWave; ++r) {
            pos[r] += cnt[r];
            // batch used up while the row may still have slots in this chunk
            while (pos[r] < end[r] && pos[r] == base[r] + kWave) {
                tile_reload(base[r], pos[r], end[r], lane, col, val, mc[r], mv[r]);
                const int32_t c2 = __popcll(__ballot(mc[r] < k1));
                for (int32_t q = 0; q < c2; ++q) {
                    const f32x2 x = xs[bcast_i(mc[r], q) - k0][lane];
                    const float v = bcast_f(mv[r], q);
                    acc[r][0] = __builtin_fmaf(v, x[0], acc[r][0]);
                    acc[r][1] = __builtin_fmaf(v, x[1], acc[r][1]);
                }
                pos[r] += c2;
            }
        }
    }
    if (n_ok) {
#pragma unroll
        for (int r = 0; r < kRowsPerWave; ++r)
            if (r0 + r < M) {
                if (bias != nullptr) {
                    const float b = bias[r0 + r];
                    acc[r][0] = acc[r][0] + b;
                    acc[r][1] = acc[r][1] + b;
                }
                *reinterpret_cast<f32x2*>(Y + (r0 + r) * N + n) = acc[r];
            }
    }
}

int launch_blocks(int64_t waves, int64_t* blocks) {
    *blocks = ceil_div(waves, kSpmmBlock / kWave);
    if (*blocks > INT32_MAX) return fail(SLK_EINVAL, "spmm: problem too large for one launch");
    return SLK_OK;
}

int launch_tile(const slk_csr* W, const float* X, int64_t N, const float* bias, float* Y,
                hipStream_t st) {
    const int64_t M = W->nrows;
    const int64_t nrowblk = ceil_div(M, kTileRows);
    const int64_t blocks = nrowblk * ceil_div(N, kTileCols);
    if (blocks > INT32_MAX) return fail(SLK_EINVAL, "spmm: problem too large for one launch");
    hipLaunchKernelGGL(spmm_tile_kernel, dim3(static_cast<unsigned>(blocks)),
                       dim3(kTileThreads), 0, st, M, W->ncols, N, nrowblk, W->row_start,
                       W->row_nnz, W->col_indices, W->values, X, bias, Y);
    return check_launch("spmm");
}

template <int VEC>
int launch_wave(const slk_csr* W, const float* X, int64_t N, const float* bias, float* Y,
                hipStream_t st) {
    constexpr int U = VEC == 4 ? 8 : 16;
    const int64_t M = W->nrows;
    const int64_t nitems = M * ceil_div(N, int64_t{kWave} * VEC);
    int64_t blocks;
    if (int rc = launch_blocks(nitems, &blocks)) return rc;
    hipLaunchKernelGGL((spmm_wave_kernel<VEC, U>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kSpmmBlock), 0, st, M, N, nitems, W->row_order, W->row_start,
                       W->row_nnz, W->col_indices, W->values, X, bias, Y);
    return check_launch("spmm");
}

template <int L, int VEC>
int launch_group(const slk_csr* W, const float* X, int64_t N, const float* bias, float* Y,
                 hipStream_t st) {
    const int64_t M = W->nrows;
    const int64_t nitems = M * ceil_div(N, static_cast<int64_t>(L) * VEC);
    int64_t blocks;
    if (int rc = launch_blocks(ceil_div(nitems, kWave / L), &blocks)) return rc;
    hipLaunchKernelGGL((spmm_group_kernel<L, VEC>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kSpmmBlock), 0, st, M, N, nitems, W->row_order, W->row_start,
                       W->row_nnz, W->col_indices, W->values, X, bias, Y);
    return check_launch("spmm");
}

int launch_group_L(int L, const slk_csr* W, const float* X, int64_t N, const float* bias,
                   float* Y, hipStream_t st) {
    switch (L) {
        case 1: return launch_group<1, 1>(W, X, N, bias, Y, st);
        case 2: return launch_group<2, 1>(W, X, N, bias, Y, st);
        case 4: return launch_group<4, 1>(W, X, N, bias, Y, st);
        case 8: return launch_group<8, 1>(W, X, N, bias, Y, st);
        case 16: return launch_group<16, 1>(W, X, N, bias, Y, st);
        default: return launch_group<32, 1>(W, X, N, bias, Y, st);
    }
}

// Waves worth launching: enough to give every CU several to switch between.
constexpr int64_t kTargetWaves = 4096;

// Y = W·X (+ bias per row): the shared body of slk_spmm and slk_spmm_bias.
int spmm_impl(const slk_csr* W, const float* X, int64_t K, int64_t N, const float* bias,
              float* Y, void* stream) {
    clear_error();
    if (int rc = validate_csr(W, "spmm")) return rc;
    if (N < 0 || K < 0) return fail(SLK_EINVAL, "spmm: negative X shape");
    if (W->ncols != K) {
        return fail(SLK_EINVAL, "spmm: shape mismatch. W has ncols=" + std::to_string(W->ncols) +
                                    " but X has shape[0]=" + std::to_string(K) +
                                    ". Inner dimensions must match for matmul.");
    }
    if (W->nrows == 0 || N == 0) return SLK_OK;
    if (Y == nullptr || (K > 0 && X == nullptr)) return fail(SLK_EINVAL, "spmm: NULL X or Y");
    if (N > INT32_MAX / 4) return fail(SLK_EINVAL, "spmm: N exceeds the 32-bit lane offset range");
    hipStream_t st = as_stream(stream);
    const uintptr_t align = reinterpret_cast<uintptr_t>(X) | reinterpret_cast<uintptr_t>(Y);
    const int64_t M = W->nrows;

    // Kernel choice: the per-wave gather kernels. The LDS-tiled kernel is
    // opt-in (SLK_SPMM_KERNEL=tile, where its layout needs — even N, 8-byte
    // aligned X and Y — hold): on the measured workloads it does not beat the
    // wave kernel, whose X gathers already hit L2 for the tile-major order.
    bool tile = false;
    if (const char* e = std::getenv("SLK_SPMM_KERNEL")) {
        if (e[0] == 't') tile = N % 2 == 0 && align % 8 == 0;
    }
    if (tile) return launch_tile(W, X, N, bias, Y, st);

    int vec = 1;
    if (const char* e = std::getenv("SLK_SPMM_VEC")) vec = std::atoi(e);
    else if (N % 4 == 0 && align % 16 == 0 && M * ceil_div(N, 256) >= kTargetWaves) vec = 4;
    else if (N % 2 == 0 && align % 8 == 0 && M * ceil_div(N, 128) >= kTargetWaves) vec = 2;
    if ((vec == 4 && (N % 4 || align % 16)) || (vec == 2 && (N % 2 || align % 8)) ||
        (vec != 1 && vec != 2 && vec != 4)) {
        vec = 1;
    }
    if (N < kWave * vec) {
        // Narrow X: pack several rows per wave.
        int L = 1;
        while (L < 32 && L < N) L <<= 1;
        if (L < kWave && L >= N) return launch_group_L(L, W, X, N, bias, Y, st);
        vec = 1;
    }
    if (vec == 4) return launch_wave<4>(W, X, N, bias, Y, st);
    if (vec == 2) return launch_wave<2>(W, X, N, bias, Y, st);
    return launch_wave<1>(W, X, N, bias, Y, st);
}

}  // namespace
}  // namespace slk

extern "C" int slk_spmm(const slk_csr* W, const float* X, int64_t K, int64_t N, float* Y,
                        void* stream) {
    return slk::spmm_impl(W, X, K, N, nullptr, Y, stream);
}

extern "C" int slk_spmm_bias(const slk_csr* W, const float* X, int64_t K, int64_t N,
                             const float* bias, float* Y, void* stream) {
    if (bias == nullptr && W != nullptr && W->nrows > 0) {
        slk::clear_error();
        return slk::fail(SLK_EINVAL, "spmm_bias: NULL bias");
    }
    return slk::spmm_impl(W, X, K, N, bias, Y, stream);
}
