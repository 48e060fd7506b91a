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
#include "dense_rows.hpp"

#include <cstdlib>
#include <mutex>
#include <type_traits>
#include <utility>

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
// The broadcast value is copied into a vector register: a VALU instruction
// that reads a scalar operand issues at about half the rate of one whose
// operands are all vector registers (measured on gfx950: 2.0 against 3.3
// wave-wide fmas per ns per CU), so one copy per slot makes its 4·H fmas the
// fast form.
__device__ __forceinline__ float bcast_f(float v, int32_t lane) {
    const float s = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
    float r;
    asm("v_mov_b32 %0, %1" : "=v"(r) : "s"(s));
    return r;
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

// TOUT: Y is stored token-major, Y[i, n] at Y[n·M + i] (slk_spmm_t).
// PH: phase `ph` of `nph` (slk_csr.phase_lo): the row's slots
// [plo[row·(nph+1) + ph], plo[row·(nph+1) + ph + 1]) continue the fma chain
// from the partial sums the previous phase stored in Y (from +0.0 in phase
// 0); the caller passes bias only with the last phase.
template <int VEC, int U, bool TOUT = false, bool PH = false>
__global__ __launch_bounds__(kSpmmBlock) void spmm_wave_kernel(
    int64_t M, int64_t N, int64_t nitems, const int32_t* __restrict__ order,
    const int32_t* __restrict__ row_start, const int32_t* __restrict__ row_nnz,
    const int32_t* __restrict__ col, const float* __restrict__ val,
    const float* __restrict__ X, const float* __restrict__ bias, float* __restrict__ Y,
    const int32_t* __restrict__ plo = nullptr, int64_t nph = 1, int64_t ph = 0) {
    typedef typename VecIO<VEC>::T T;
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t item = wave_id();
    if (item >= nitems) return;  // wave-uniform; no barriers below
    const int64_t tile = item / M;
    const int64_t r = item - tile * M;
    const int64_t row = order != nullptr ? order[r] : r;
    const int64_t n0 = (tile * kWave + lane) * VEC;
    const bool active = n0 < N;  // N % VEC == 0, so n0 + VEC <= N
    int32_t start, nnz;
    if constexpr (PH) {
        start = plo[row * (nph + 1) + ph];
        nnz = plo[row * (nph + 1) + ph + 1] - start;
    } else {
        start = row_start[row];
        nnz = row_nnz[row];
    }
    const uint32_t off = static_cast<uint32_t>(n0) * 4u;  // 4N < 2^31 (launcher check)

    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.0f;
    if constexpr (PH) {
        if (ph > 0 && active) {
            const typename VecIO<VEC>::T y = VecIO<VEC>::load(Y + row * N + n0);
#pragma unroll
            for (int e = 0; e < VEC; ++e) acc[e] = VecIO<VEC>::get(y, e);
        }
    }

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
        if constexpr (TOUT) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) Y[(n0 + e) * M + row] = acc[e];
        } else {
            VecIO<VEC>::store(Y + row * N + n0, acc);
        }
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

// ───────────────────────── LDS-staged kernel ────────────────────────────────
//
// spmm_lds_kernel — for large problems, where every X element is used by
// several rows of a workgroup. A workgroup of 16 waves owns R = 16·RW rows x
// 256·H columns of Y: each lane holds 4 adjacent columns of each of H
// 256-column halves for RW rows in registers (H = 2 halves the readlane,
// address and loop work per fma; measured 5-17% faster on the denser GPT
// layers). X is streamed through LDS in chunks of 80/H rows x 256·H columns
// (1 KB per X row and half), double-buffered: chunk c+1 is loaded straight
// into the other buffer (direct global-to-LDS loads) while chunk c is read,
// so one barrier per chunk orders both. For each chunk every row consumes its slots
// whose column falls in the chunk; columns ascend within a row, so walking
// the chunks in order visits each row's slots in slot order and every
// element's fma chain is exactly the reference's. Each X element is fetched
// from L2/HBM once per workgroup and then read from LDS — about eight times
// the bandwidth of global gathers on gfx950 — by every row that uses it.
//
// Row metadata: each row keeps two 64-slot windows of (column, value) in lane
// registers, the current one and the next, which is requested as soon as the
// current one is entered, so a row never waits on its stream inside a chunk.
// The row's slots that fall in a chunk are a run of the window: a ballot gives
// its length and readlane broadcasts each slot's column and value. Rows are
// dealt to waves round-robin (position r0 + w + 16j of the P positions). A
// position is a row, or with `order` (a range of the longest-rows-first
// schedule) the row order[position]: the launcher runs a skewed matrix's
// heavy rows and the rest as two such ranges, so that each workgroup holds
// rows of similar length (see spmm_impl).
constexpr int kLdsWaves = 16;
constexpr int kLdsThreads = kLdsWaves * kWave;          // 1024
constexpr int kLdsK = 80;                               // X rows per chunk
constexpr int kLdsCols = 4 * kWave;                     // 256 columns per workgroup

__device__ __forceinline__ void lds_window(const int32_t* __restrict__ col,
                                           const float* __restrict__ val, int32_t at,
                                           int32_t end, int lane, int32_t& c, float& v) {
    const int32_t s = at + lane;
    c = s < end ? col[s] : INT32_MAX;  // past the row: never below a chunk end
    v = s < end ? val[s] : 0.0f;
}

// One wave's direct load of 64 x 16 bytes into LDS (global_load_lds_dwordx4):
// lane l's 16 bytes from src go to row + l (row: the wave's common LDS
// address, 1 KB).
__device__ __forceinline__ void lds_load_row(const void* src, f32x4* row) {
    __builtin_amdgcn_global_load_lds(src, row, 16, 0, 0);
}

__device__ __forceinline__ void fma4(float v, const f32x4& x, f32x4& acc) {
    acc[0] = __builtin_fmaf(v, x[0], acc[0]);
    acc[1] = __builtin_fmaf(v, x[1], acc[1]);
    acc[2] = __builtin_fmaf(v, x[2], acc[2]);
    acc[3] = __builtin_fmaf(v, x[3], acc[3]);
}

// X chunk staging of the LDS kernels. A chunk is KC = kLdsK / H X rows x
// 256·H columns of column tile `tile`, 1 KiB per X row and half; it goes
// straight from global memory into LDS (global_load_lds_dwordx4: lane l of
// a wave writes its 16 bytes at the instruction's LDS base + 16 l), so wave
// w's load i fills row-half w + 16 i, i.e. X row (w + 16 i) / H, half
// (w + 16 i) mod H: no registers hold the next chunk and no LDS stores copy
// it. Each load is a scalar X row address (64-bit, computed per chunk; rows
// past K, in the last chunk, are clamped to row K - 1: no slot has a column
// >= K) plus the lane's 32-bit byte offset inside the row, clamped to the
// row's last 16 bytes where the lane's columns pass N (those lanes never
// store theirs); the offset is below 4N < 2^31 (the launcher's bound on N).
template <int H>
struct ChunkStager {
    static constexpr int KC = kLdsK / H;
    static constexpr int kStage = KC * H * kWave / kLdsThreads;  // 16-byte loads per thread
    static_assert(kStage * kLdsWaves == KC * H, "whole X rows per thread group");
    // 16 i is a multiple of H, so every load of wave w stages half w mod H:
    // cb is the lane's byte offset inside the X row for that half
    uint32_t cb;
    __device__ __forceinline__ ChunkStager(int64_t tile, int64_t N, int lane, int w) {
        const int64_t nn = tile * (H * kLdsCols) + (w % H) * kLdsCols + 4 * lane;
        cb = static_cast<uint32_t>((nn < N ? nn : N - 4) * 4);
    }
    // The chunk at X row k0 into xs[buf], by wave w.
    __device__ __forceinline__ void load(f32x4 (&xs)[2][KC][H][kWave], int buf,
                                         const float* __restrict__ X, int64_t k0, int64_t K,
                                         int64_t N, int w) const {
#pragma unroll
        for (int i = 0; i < kStage; ++i) {
            const int q = w + i * kLdsWaves;  // the wave's row-half: wave-uniform
            const int64_t kr = k0 + q / H;
            const char* row = reinterpret_cast<const char*>(X + (kr < K ? kr : K - 1) * N);
            lds_load_row(row + cb, &xs[buf][q / H][q % H][0]);
        }
    }
};

// One workgroup's share of the LDS kernel: logical block lb of a launch over
// positions [0, P) of `order` with nrowblk row blocks per column tile; xs is
// the workgroup's X double buffer.
template <int RW, int H>
__device__ __forceinline__ void spmm_lds_body(
    f32x4 (&xs)[2][kLdsK / H][H][kWave], int64_t lb, int64_t P, int64_t K, int64_t N,
    int64_t nrowblk, const int32_t* __restrict__ order, const int32_t* __restrict__ row_start,
    const int32_t* __restrict__ row_nnz, const int32_t* __restrict__ col,
    const float* __restrict__ val, const float* __restrict__ X, const float* __restrict__ bias,
    float* __restrict__ Y) {
    // H halves of 256 columns per workgroup, each lane 4 columns of each half;
    // chunks of KC X rows keep the double buffer at 160 KiB, all of a CU's LDS
    constexpr int KC = kLdsK / H;
    const int lane = threadIdx.x & (kWave - 1);
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t tile = lb / nrowblk;  // tile-major: a tile's row blocks share X chunks in L2
    const int64_t rb = lb - tile * nrowblk;
    int64_t n[H];
    bool n_ok[H];
#pragma unroll
    for (int h = 0; h < H; ++h) {
        n[h] = tile * (H * kLdsCols) + h * kLdsCols + 4 * lane;
        n_ok[h] = n[h] < N;  // N % 4 == 0 for this kernel
    }
    const int64_t r0 = rb * (kLdsWaves * RW) + w;

    // The next window is requested as soon as a window is entered, so a row
    // never waits on its stream inside a chunk (a wait there holds all 16
    // waves at the next barrier). The 8-row, 8-column-per-lane variant keeps
    // two slots' reads in flight instead of four to stay within 128 VGPRs
    // (four spill).
    constexpr int G = (RW == 8 && H == 2) ? 2 : 4;  // slots per group of LDS reads
    int32_t rows[RW], pos[RW], end[RW], base[RW], mc[RW], nmc[RW];  // rows[j] < 0: none
    float mv[RW], nmv[RW];
    f32x4 acc[RW][H];
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        const int64_t p = r0 + static_cast<int64_t>(kLdsWaves) * j;
        rows[j] = p < P ? (order != nullptr ? order[p] : static_cast<int32_t>(p)) : -1;
        const int32_t row = rows[j];
        const int32_t s = row >= 0 ? row_start[row] : 0;
        const int32_t e = row >= 0 ? s + row_nnz[row] : 0;
        pos[j] = base[j] = s;
        end[j] = e;
        lds_window(col, val, s, e, lane, mc[j], mv[j]);
        lds_window(col, val, s + kWave, e, lane, nmc[j], nmv[j]);
#pragma unroll
        for (int h = 0; h < H; ++h) acc[j][h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }

    const ChunkStager<H> stager(tile, N, lane, w);
    auto prefetch = [&](int buf, int64_t k0) { stager.load(xs, buf, X, k0, K, N, w); };
    const int64_t nchunks = ceil_div(K, KC);
    prefetch(0, 0);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's direct loads have landed
    __syncthreads();
    for (int64_t ch = 0; ch < nchunks; ++ch) {
        const int b = static_cast<int>(ch & 1);
        const bool more = ch + 1 < nchunks;
        // the other buffer's last readers (chunk ch - 1) passed the barrier
        if (more) prefetch(b ^ 1, (ch + 1) * KC);
        const int32_t k0 = static_cast<int32_t>(ch * KC);
        const int32_t k1 = k0 + KC;
#pragma unroll
        for (int j = 0; j < RW; ++j) {
            int32_t first = pos[j] - base[j];
            while (true) {
                // slots of the window at or after `first` (first < 64) below the chunk end:
                // one compare on the VALU, the mask on the scalar unit
                const uint64_t run = __ballot(mc[j] < k1) & (~0ull << first);
                // (two 32-bit counts keep the loop bounds 32-bit scalar compares)
                const int32_t cnt = __popc(static_cast<uint32_t>(run)) +
                                    __popc(static_cast<uint32_t>(run >> 32));
                int32_t k = 0;
                for (; k + G <= cnt; k += G) {  // G slots' LDS reads in flight
                    const int32_t s0 = first + k;
                    int32_t c[G];
#pragma unroll
                    for (int g = 0; g < G; ++g) c[g] = bcast_i(mc[j], s0 + g) - k0;
#pragma unroll
                    for (int h = 0; h < H; ++h) {
                        f32x4 x[G];
#pragma unroll
                        for (int g = 0; g < G; ++g) x[g] = xs[b][c[g]][h][lane];
#pragma unroll
                        for (int g = 0; g < G; ++g) fma4(bcast_f(mv[j], s0 + g), x[g], acc[j][h]);
                    }
                }
                if (G > 2 && k + 2 <= cnt) {  // a pair: both reads in flight
                    const int32_t s0 = first + k;
                    const int32_t c0 = bcast_i(mc[j], s0) - k0, c1 = bcast_i(mc[j], s0 + 1) - k0;
#pragma unroll
                    for (int h = 0; h < H; ++h) {
                        const f32x4 x0 = xs[b][c0][h][lane];
                        const f32x4 x1 = xs[b][c1][h][lane];
                        fma4(bcast_f(mv[j], s0), x0, acc[j][h]);
                        fma4(bcast_f(mv[j], s0 + 1), x1, acc[j][h]);
                    }
                    k += 2;
                }
                if (k < cnt) {
                    const int32_t c0 = bcast_i(mc[j], first + k) - k0;
                    const float v = bcast_f(mv[j], first + k);
#pragma unroll
                    for (int h = 0; h < H; ++h) fma4(v, xs[b][c0][h][lane], acc[j][h]);
                }
                pos[j] += cnt;
                if (first + cnt < kWave) break;  // the run ended inside this window
                // window used up: shift the next one in and request the one after
                base[j] += kWave;
                mc[j] = nmc[j];
                mv[j] = nmv[j];
                lds_window(col, val, base[j] + kWave, end[j], lane, nmc[j], nmv[j]);
                first = 0;
            }
        }
        __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of chunk ch + 1 have landed
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        if (rows[j] < 0) continue;
        const int64_t row = rows[j];
        const float bb = bias != nullptr ? bias[row] : 0.0f;
#pragma unroll
        for (int h = 0; h < H; ++h) {
            if (!n_ok[h]) continue;
            f32x4 a = acc[j][h];
            if (bias != nullptr) {
                a[0] = a[0] + bb;
                a[1] = a[1] + bb;
                a[2] = a[2] + bb;
                a[3] = a[3] + bb;
            }
            *reinterpret_cast<f32x4*>(Y + row * N + n[h]) = a;
        }
    }
}

template <int RW, int H>
__global__ __launch_bounds__(kLdsThreads) void spmm_lds_kernel(
    int64_t P, int64_t K, int64_t N, int64_t nrowblk, const int32_t* __restrict__ order,
    const int32_t* __restrict__ row_start, const int32_t* __restrict__ row_nnz,
    const int32_t* __restrict__ col, const float* __restrict__ val, const float* __restrict__ X,
    const float* __restrict__ bias, float* __restrict__ Y) {
    __shared__ f32x4 xs[2][kLdsK / H][H][kWave];  // 160 KiB
    spmm_lds_body<RW, H>(xs, xcd_logical_block(blockIdx.x, gridDim.x), P, K, N, nrowblk, order,
                         row_start, row_nnz, col, val, X, bias, Y);
}

// A skewed matrix's heavy rows (positions [0, T) of the longest-first order)
// and the rest (positions [T, M), RW rows per wave, 4 columns per lane) in one
// grid: the few workgroups of heavy rows would otherwise leave CUs idle in
// their launch's last round. Heavy rows run two per wave with 8 columns per
// lane (kHeavyH = 2 halves): their long runs of slots amortize a slot's
// readlane and address work over 8 fmas instead of 4 (16384^2 Zipf(1.1) at
// 95%: 8.03 -> 7.35 ms; 4 halves or 1 or 4 rows per wave were slower). Every
// XCD starts its share of the grid with its share of the heavy workgroups (the
// longest), then its share of the rest, each in the tile-major order of its
// own part.
constexpr int kHeavyRW = 2;
constexpr int kHeavyH = 2;
template <int RW>
__global__ __launch_bounds__(kLdsThreads) void spmm_lds_split_kernel(
    int64_t T, int64_t M, int64_t K, int64_t N, int64_t nblk_a, int64_t nrowblk_a,
    int64_t nrowblk_b, const int32_t* __restrict__ order, const int32_t* __restrict__ row_start,
    const int32_t* __restrict__ row_nnz, const int32_t* __restrict__ col,
    const float* __restrict__ val, const float* __restrict__ X, const float* __restrict__ bias,
    float* __restrict__ Y) {
    __shared__ f32x4 xraw[2 * kLdsK * kWave];  // 160 KiB, shaped by each part below
    const int64_t nb = gridDim.x;
    const int64_t x = blockIdx.x % kXcds, q = blockIdx.x / kXcds;
    // blocks of XCD x: q < count_x; heavy ones first: q < ha_x
    const int64_t ha = nblk_a / kXcds + (x < nblk_a % kXcds ? 1 : 0);
    const int64_t a0 = x * (nblk_a / kXcds) + (x < nblk_a % kXcds ? x : nblk_a % kXcds);
    const int64_t nblk_b = nb - nblk_a;
    // XCD x holds count_x = ceil((nb - x) / 8) blocks, ha of them heavy
    const int64_t count_x = (nb - x + kXcds - 1) / kXcds;
    const int64_t hb_lo = x * (nb / kXcds) + (x < nb % kXcds ? x : nb % kXcds) - a0;  // rest before
    if (q < ha) {
        auto& xs = *reinterpret_cast<f32x4(*)[2][kLdsK / kHeavyH][kHeavyH][kWave]>(xraw);
        spmm_lds_body<kHeavyRW, kHeavyH>(xs, a0 + q, T, K, N, nrowblk_a, order, row_start,
                                         row_nnz, col, val, X, bias, Y);
    } else {
        const int64_t lb = hb_lo + (q - ha);
        if (lb < nblk_b && q < count_x) {
            auto& xs = *reinterpret_cast<f32x4(*)[2][kLdsK][1][kWave]>(xraw);
            spmm_lds_body<RW, 1>(xs, lb, M - T, K, N, nrowblk_b, order + T, row_start, row_nnz,
                                 col, val, X, bias, Y);
        }
    }
}

// ───────────────────────── binned-stream kernel ─────────────────────────────
//
// The LDS kernel above finds, per row and chunk, the run of the row's slots
// that falls in the chunk (a ballot over the row's window of columns) and
// keeps two windows of (column, value) per row. With a binned slot stream
// (slk_csr.bin_*, built per topology) each wave's work for a chunk is one
// contiguous run of the stream, row by row, with the rows' counts known:
//   * per wave and chunk, one 64-entry window of (LDS offset, value): the
//     chunk's entries, loaded during the previous chunk (values read through
//     the slot index then, so they are never stale), and the per-row counts
//     from a window of 32 chunks' count records;
//   * each slot costs a readlane of its offset, one address add, H LDS
//     reads, a readlane of its value and 4·H fmas; no per-row search;
//   * the first G slots of row j+1 are read from LDS before row j's fmas,
//     so one row's reads are in flight while the previous row computes (the
//     reads are issued unconditionally — a slot past the row's count reads a
//     valid offset and is not used — so the wait counts are static).
// A chunk whose entries pass the window (more than 64 for the wave: dense
// rows) takes them one by one from the stream.

// One wave's share of workgroup lb of a binned launch over positions [0, P)
// (rows order[p], or p when order is NULL), nrowblk row blocks per column
// tile; the stream's unit u = (row block) * 16 + wave.
template <int RW, int H, int G>
__device__ __forceinline__ void spmm_bin_body(
    f32x4 (&xs)[2][kLdsK / H][H][kWave], int64_t lb, int64_t P, int64_t K, int64_t N,
    int64_t nrowblk, const int32_t* __restrict__ order, const float* __restrict__ val,
    const int32_t* __restrict__ bin_off, const int32_t* __restrict__ bin_slot,
    const uint32_t* __restrict__ bin_cnt, const int32_t* __restrict__ bin_start, int64_t n_bin,
    const float* __restrict__ X, const float* __restrict__ bias, float* __restrict__ Y) {
    constexpr int KC = kLdsK / H;
    constexpr int kHalfBytes = kWave * 16;  // one staged X row half
    const int lane = threadIdx.x & (kWave - 1);
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t tile = lb / nrowblk;
    const int64_t rb = lb - tile * nrowblk;
    const int64_t u = rb * kLdsWaves + w;
    const int64_t nch = ceil_div(K, KC);
    f32x4 acc[RW][H];
#pragma unroll
    for (int j = 0; j < RW; ++j)
#pragma unroll
        for (int h = 0; h < H; ++h) acc[j][h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const uint32_t* cnt = bin_cnt + u * nch * 2;
    const int64_t e_lim = bin_start[u + 1] < n_bin ? bin_start[u + 1] : n_bin;
    // chunk c's count record (wave-uniform address: scalar loads, issued a
    // chunk ahead and first read after the barrier's wait)
    auto rec = [&](int64_t c, uint32_t& a, uint32_t& b) {
        a = cnt[2 * c];
        b = cnt[2 * c + 1];
    };
    auto load_idx = [&](int64_t at, int32_t& o, int32_t& s) {
        const int64_t i = at + lane;
        o = 0;
        s = -1;
        if (i < e_lim) {
            o = bin_off[i];
            s = bin_slot[i];
        }
    };
    auto gather = [&](int32_t s) -> float { return s >= 0 ? val[s] : 0.0f; };
    auto rec_total = [](uint32_t a, uint32_t b) -> int32_t {
        return static_cast<int32_t>((a & 0xff) + ((a >> 8) & 0xff) + ((a >> 16) & 0xff) + (a >> 24) +
                                    (b & 0xff) + ((b >> 8) & 0xff) + ((b >> 16) & 0xff) + (b >> 24));
    };
    // chunk ch's entries (cur_*) and counts (rc*), chunk ch+1's indices
    // (nxt_*) and counts (rn*); e_cur / e_nxt their first entries
    int64_t e_cur = bin_start[u];
    uint32_t rc0, rc1, rn0 = 0, rn1 = 0;
    rec(0, rc0, rc1);
    int64_t e_nxt = e_cur + rec_total(rc0, rc1);
    int32_t cur_off, cur_slot, nxt_off = 0, nxt_slot = -1;
    load_idx(e_cur, cur_off, cur_slot);
    float cur_val = gather(cur_slot);
    if (nch > 1) {
        rec(1, rn0, rn1);
        load_idx(e_nxt, nxt_off, nxt_slot);
    }

    const ChunkStager<H> stager(tile, N, lane, w);
    stager.load(xs, 0, X, 0, K, N, w);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's direct loads have landed
    __syncthreads();
    for (int64_t ch = 0; ch < nch; ++ch) {
        const int b = static_cast<int>(ch & 1);
        const bool more = ch + 1 < nch;
        // the other buffer's last readers (chunk ch - 1) passed the barrier
        if (more) stager.load(xs, b ^ 1, X, (ch + 1) * KC, K, N, w);
        // chunk ch+1's values, chunk ch+2's indices and counts
        float nxt_val = 0.0f;
        int32_t nn_off = 0, nn_slot = -1;
        uint32_t rnn0 = 0, rnn1 = 0;
        int64_t e_nn = e_nxt;
        if (more) {
            nxt_val = gather(nxt_slot);
            e_nn = e_nxt + rec_total(rn0, rn1);
            if (ch + 2 < nch) {
                rec(ch + 2, rnn0, rnn1);
                load_idx(e_nn, nn_off, nn_slot);
            }
        }

        const char* lbase = reinterpret_cast<const char*>(&xs[b][0][0][lane]);
        const int32_t tot = rec_total(rc0, rc1);
        int32_t nr[RW];
#pragma unroll
        for (int j = 0; j < RW; ++j)
            nr[j] = static_cast<int32_t>(((j < 4 ? rc0 : rc1) >> (8 * (j & 3))) & 0xff);
        // One pass per 64 entries of the chunk (one pass unless the wave's
        // rows are dense): each row's part of its run inside the pass's
        // window, rows in order, each row's slots in order.
        auto pass = [&](int32_t wb) {
            f32x4 xa[G][H], xb[G][H];
            // the X rows of the G slots from window position r0 (positions
            // past 63 wrap: their reads are valid and unused)
            auto issue = [&](f32x4 (&x)[G][H], int32_t r0) {
#pragma unroll
                for (int k = 0; k < G; ++k) {
                    const int32_t o = bcast_i(cur_off, (r0 + k) & (kWave - 1));
#pragma unroll
                    for (int h = 0; h < H; ++h)
                        x[k][h] = *reinterpret_cast<const f32x4*>(lbase + o + h * kHalfBytes);
                }
                // keep the reads here: the compiler would otherwise sink each
                // into the branch that uses it, after the previous row's fmas
                asm volatile("" ::: "memory");
            };
            // row j's run [rs, rs + nr) clipped to the window [wb, wb + 64)
            // (no clipping in the usual single window)
            int32_t pj[RW], nj[RW];
            {
                const bool whole = wb == 0 && tot <= kWave;
                int32_t rs = 0;
#pragma unroll
                for (int j = 0; j < RW; ++j) {
                    if (whole) {
                        pj[j] = rs;
                        nj[j] = nr[j];
                    } else {
                        const int32_t lo = rs > wb ? rs : wb;
                        const int32_t hi = rs + nr[j] < wb + kWave ? rs + nr[j] : wb + kWave;
                        pj[j] = lo - wb;
                        nj[j] = max(hi - lo, 0);
                    }
                    rs += nr[j];
                }
            }
            auto consume = [&](const f32x4 (&x)[G][H], f32x4 (&a)[H], int32_t p0, int32_t n) {
#pragma unroll
                for (int k = 0; k < G; ++k) {
                    if (k < n) {
                        const float v = bcast_f(cur_val, p0 + k);
#pragma unroll
                        for (int h = 0; h < H; ++h) fma4(v, x[k][h], a[h]);
                    }
                }
            };
            // pass 1, straight-line: each row's first G slots, row j+1's
            // reads issued before row j's fmas
            issue(xa, pj[0]);
            static_for<RW>([&](auto J) {
                constexpr int j = decltype(J)::value;
                f32x4(&xj)[G][H] = (j & 1) ? xb : xa;
                f32x4(&xo)[G][H] = (j & 1) ? xa : xb;
                if constexpr (j + 1 < RW) issue(xo, pj[j + 1]);
                consume(xj, acc[j], pj[j], nj[j]);
            });
            // pass 2: the rest of the rows with more than G slots here
            static_for<RW>([&](auto J) {
                constexpr int j = decltype(J)::value;
                for (int32_t t = G; t < nj[j]; t += G) {
                    issue(xa, pj[j] + t);
                    consume(xa, acc[j], pj[j] + t, nj[j] - t);
                }
            });
        };
        // the first window outside any loop, so its reads wait only on LDS
        // (a loop with the reload below would make them wait for the next
        // chunk's loads too)
        pass(0);
        for (int32_t wb = kWave; wb < tot; wb += kWave) {
            int32_t sl;  // the next 64 entries into the current window
            load_idx(e_cur + wb, cur_off, sl);
            cur_val = gather(sl);
            pass(wb);
        }
        __builtin_amdgcn_s_waitcnt(0);  // chunk ch+1 and the next windows have landed
        __syncthreads();
        cur_off = nxt_off;
        cur_val = nxt_val;
        nxt_off = nn_off;
        nxt_slot = nn_slot;
        rc0 = rn0;
        rc1 = rn1;
        rn0 = rnn0;
        rn1 = rnn1;
        e_cur = e_nxt;
        e_nxt = e_nn;
    }
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        const int64_t q = rb * (kLdsWaves * RW) + w + kLdsWaves * j;
        if (q >= P) continue;
        const int64_t row = order != nullptr ? order[q] : q;
        const float bb = bias != nullptr ? bias[row] : 0.0f;
#pragma unroll
        for (int h = 0; h < H; ++h) {
            const int64_t nn = tile * (H * kLdsCols) + h * kLdsCols + 4 * lane;
            if (nn >= N) continue;  // N % 4 == 0 for this kernel
            f32x4 a = acc[j][h];
            if (bias != nullptr) {
                a[0] = a[0] + bb;
                a[1] = a[1] + bb;
                a[2] = a[2] + bb;
                a[3] = a[3] + bb;
            }
            *reinterpret_cast<f32x4*>(Y + row * N + nn) = a;
        }
    }
}

template <int RW, int H, int G>
__global__ __launch_bounds__(kLdsThreads) void spmm_bin_kernel(
    int64_t P, int64_t K, int64_t N, int64_t nrowblk, const int32_t* __restrict__ order,
    const float* __restrict__ val, const int32_t* __restrict__ bin_off,
    const int32_t* __restrict__ bin_slot, const uint32_t* __restrict__ bin_cnt,
    const int32_t* __restrict__ bin_start, int64_t n_bin, const float* __restrict__ X,
    const float* __restrict__ bias, float* __restrict__ Y) {
    __shared__ f32x4 xs[2][kLdsK / H][H][kWave];  // 160 KiB
    spmm_bin_body<RW, H, G>(xs, xcd_logical_block(blockIdx.x, gridDim.x), P, K, N, nrowblk, order,
                            val, bin_off, bin_slot, bin_cnt, bin_start, n_bin, X, bias, Y);
}

// The heavy rows (positions [0, T) of the longest-first order, two per wave,
// 8 columns per lane, on the LDS kernel) and the binned rest in one grid,
// each XCD starting its share with its share of the heavy workgroups (as
// spmm_lds_split_kernel).
template <int RW, int H, int G>
__global__ __launch_bounds__(kLdsThreads) void spmm_bin_split_kernel(
    int64_t T, int64_t M, int64_t K, int64_t N, int64_t nblk_a, int64_t nrowblk_a,
    int64_t nrowblk_b, const int32_t* __restrict__ order, const int32_t* __restrict__ row_start,
    const int32_t* __restrict__ row_nnz, const int32_t* __restrict__ col,
    const float* __restrict__ val, const int32_t* __restrict__ bin_off,
    const int32_t* __restrict__ bin_slot, const uint32_t* __restrict__ bin_cnt,
    const int32_t* __restrict__ bin_start, int64_t n_bin, const float* __restrict__ X,
    const float* __restrict__ bias, float* __restrict__ Y) {
    __shared__ f32x4 xraw[2 * kLdsK * kWave];  // 160 KiB, shaped by each part below
    const int64_t nb = gridDim.x;
    const int64_t x = blockIdx.x % kXcds, q = blockIdx.x / kXcds;
    const int64_t ha = nblk_a / kXcds + (x < nblk_a % kXcds ? 1 : 0);
    const int64_t a0 = x * (nblk_a / kXcds) + (x < nblk_a % kXcds ? x : nblk_a % kXcds);
    const int64_t nblk_b = nb - nblk_a;
    const int64_t count_x = (nb - x + kXcds - 1) / kXcds;
    const int64_t hb_lo = x * (nb / kXcds) + (x < nb % kXcds ? x : nb % kXcds) - a0;
    if (q < ha) {
        auto& xs = *reinterpret_cast<f32x4(*)[2][kLdsK / kHeavyH][kHeavyH][kWave]>(xraw);
        spmm_lds_body<kHeavyRW, kHeavyH>(xs, a0 + q, T, K, N, nrowblk_a, order, row_start,
                                         row_nnz, col, val, X, bias, Y);
    } else {
        const int64_t lb = hb_lo + (q - ha);
        if (lb < nblk_b && q < count_x) {
            auto& xs = *reinterpret_cast<f32x4(*)[2][kLdsK / H][H][kWave]>(xraw);
            spmm_bin_body<RW, H, G>(xs, lb, M - T, K, N, nrowblk_b, order + T, val, bin_off,
                                    bin_slot, bin_cnt, bin_start, n_bin, X, bias, Y);
        }
    }
}

int launch_blocks(int64_t waves, int64_t* blocks) {
    *blocks = ceil_div(waves, kSpmmBlock / kWave);
    if (*blocks > INT32_MAX) return fail(SLK_EINVAL, "spmm: problem too large for one launch");
    return SLK_OK;
}

// Rows at positions [0, P) of `order` (NULL: rows 0..P-1).
template <int RW, int H = 1>
int launch_lds_rw(const slk_csr* W, const int32_t* order, int64_t P, const float* X, int64_t N,
                  const float* bias, float* Y, hipStream_t st) {
    if (P == 0) return SLK_OK;
    const int64_t nrowblk = ceil_div(P, int64_t{kLdsWaves} * RW);
    const int64_t blocks = nrowblk * ceil_div(N, int64_t{kLdsCols} * H);
    if (blocks > INT32_MAX) return fail(SLK_EINVAL, "spmm: problem too large for one launch");
    hipLaunchKernelGGL((spmm_lds_kernel<RW, H>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kLdsThreads), 0, st, P, W->ncols, N, nrowblk, order, W->row_start,
                       W->row_nnz, W->col_indices, W->values, X, bias, Y);
    return check_launch("spmm");
}

// Heavy rows (positions [0, T) of W->row_order, kHeavyRW per wave, kHeavyH
// halves) and the rest (rw per wave, one half) in one grid
// (spmm_lds_split_kernel).
template <int RW>
int launch_lds_split_rw(const slk_csr* W, int64_t T, const float* X, int64_t N,
                        const float* bias, float* Y, hipStream_t st) {
    const int64_t M = W->nrows;
    const int64_t tiles_a = ceil_div(N, int64_t{kLdsCols} * kHeavyH);
    const int64_t tiles_b = ceil_div(N, int64_t{kLdsCols});
    const int64_t nrowblk_a = ceil_div(T, int64_t{kLdsWaves} * kHeavyRW);
    const int64_t nrowblk_b = ceil_div(M - T, int64_t{kLdsWaves} * RW);
    const int64_t na = nrowblk_a * tiles_a, nb = nrowblk_b * tiles_b;
    if (na + nb > INT32_MAX) return fail(SLK_EINVAL, "spmm: problem too large for one launch");
    hipLaunchKernelGGL((spmm_lds_split_kernel<RW>), dim3(static_cast<unsigned>(na + nb)),
                       dim3(kLdsThreads), 0, st, T, M, W->ncols, N, na, nrowblk_a, nrowblk_b,
                       W->row_order, W->row_start, W->row_nnz, W->col_indices, W->values, X, bias,
                       Y);
    return check_launch("spmm");
}

int launch_lds(int h, int rw, const slk_csr* W, const int32_t* order, int64_t P, const float* X,
               int64_t N, const float* bias, float* Y, hipStream_t st) {
    if (h == 2) {
        switch (rw) {
            case 2: return launch_lds_rw<2, 2>(W, order, P, X, N, bias, Y, st);
            case 3: return launch_lds_rw<3, 2>(W, order, P, X, N, bias, Y, st);
            case 4: return launch_lds_rw<4, 2>(W, order, P, X, N, bias, Y, st);
            case 6: return launch_lds_rw<6, 2>(W, order, P, X, N, bias, Y, st);
            default: return launch_lds_rw<8, 2>(W, order, P, X, N, bias, Y, st);
        }
    }
    switch (rw) {
        case 2: return launch_lds_rw<2>(W, order, P, X, N, bias, Y, st);
        case 3: return launch_lds_rw<3>(W, order, P, X, N, bias, Y, st);
        case 4: return launch_lds_rw<4>(W, order, P, X, N, bias, Y, st);
        case 6: return launch_lds_rw<6>(W, order, P, X, N, bias, Y, st);
        default: return launch_lds_rw<8>(W, order, P, X, N, bias, Y, st);
    }
}

template <int VEC>
int launch_wave(const slk_csr* W, const float* X, int64_t N, const float* bias, float* Y,
                hipStream_t st) {
    constexpr int U = VEC == 4 ? 8 : VEC == 2 ? 16 : 32;  // 2U gathers in flight per wave
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

// The binned rows (positions [T, M), T = W->bin_first) on the binned
// kernel, with the heavy rows before them on the LDS kernel in the same grid
// when T > 0 (one grid needs the rest to fill a workgroup per XCD; else two
// launches).
template <int RW, int H, int G>
int launch_bin_cfg(const slk_csr* W, const float* X, int64_t N, const float* bias, float* Y,
                   hipStream_t st) {
    const int64_t M = W->nrows, K = W->ncols, T = W->bin_first;
    const int64_t nrowblk_b = ceil_div(M - T, int64_t{kLdsWaves} * RW);
    const int64_t nb = nrowblk_b * ceil_div(N, int64_t{kLdsCols} * H);
    const int32_t* order = T > 0 ? W->row_order + T : nullptr;
    if (T > 0) {
        const int64_t nrowblk_a = ceil_div(T, int64_t{kLdsWaves} * kHeavyRW);
        const int64_t na = nrowblk_a * ceil_div(N, int64_t{kLdsCols} * kHeavyH);
        if (na + nb > INT32_MAX) return fail(SLK_EINVAL, "spmm: problem too large for one launch");
        if (nb >= kXcds) {
            hipLaunchKernelGGL((spmm_bin_split_kernel<RW, H, G>), dim3(static_cast<unsigned>(na + nb)),
                               dim3(kLdsThreads), 0, st, T, M, K, N, na, nrowblk_a, nrowblk_b,
                               W->row_order, W->row_start, W->row_nnz, W->col_indices, W->values,
                               W->bin_off, W->bin_slot, W->bin_cnt, W->bin_start, W->n_bin, X, bias,
                               Y);
            return check_launch("spmm");
        }
        if (int rc = launch_lds_rw<kHeavyRW, kHeavyH>(W, W->row_order, T, X, N, bias, Y, st))
            return rc;
    }
    if (nb == 0) return SLK_OK;
    if (nb > INT32_MAX) return fail(SLK_EINVAL, "spmm: problem too large for one launch");
    hipLaunchKernelGGL((spmm_bin_kernel<RW, H, G>), dim3(static_cast<unsigned>(nb)),
                       dim3(kLdsThreads), 0, st, M - T, K, N, nrowblk_b, order, W->values,
                       W->bin_off, W->bin_slot, W->bin_cnt, W->bin_start, W->n_bin, X, bias, Y);
    return check_launch("spmm");
}

// Slots of a binned row read ahead (G): about one per expected slot of a row
// in a chunk, so few reads go unused.
int bin_group(const slk_csr* W) {
    if (const int64_t t = tuning(SLK_TUNE_SPMM_G); t == 1 || t == 2 || t == 4)
        return static_cast<int>(t);
    const int64_t rows = W->nrows - W->bin_first;
    const double per_chunk = rows > 0 && W->ncols > 0
                                 ? static_cast<double>(W->n_bin) / (static_cast<double>(rows) *
                                                                    W->ncols) *
                                       (kLdsK / W->bin_h)
                                 : 0.0;
    return per_chunk < 1.5 ? 1 : per_chunk < 3.0 ? 2 : 4;
}

// (8 rows x 2 halves reads at most 2 slots ahead: 4 would not fit 128 VGPRs)
template <int RW, int H>
int launch_bin_g(int g, const slk_csr* W, const float* X, int64_t N, const float* bias, float* Y,
                 hipStream_t st) {
    if constexpr (RW * H >= 16) {
        if (g == 1) return launch_bin_cfg<RW, H, 1>(W, X, N, bias, Y, st);
        return launch_bin_cfg<RW, H, 2>(W, X, N, bias, Y, st);
    } else {
        switch (g) {
            case 1: return launch_bin_cfg<RW, H, 1>(W, X, N, bias, Y, st);
            case 2: return launch_bin_cfg<RW, H, 2>(W, X, N, bias, Y, st);
            default: return launch_bin_cfg<RW, H, 4>(W, X, N, bias, Y, st);
        }
    }
}

int launch_bin(const slk_csr* W, const float* X, int64_t N, const float* bias, float* Y,
               hipStream_t st) {
    const int g = bin_group(W);
    const int64_t cfg = W->bin_h * 10 + W->bin_rw;
    switch (cfg) {
        case 28: return launch_bin_g<8, 2>(g, W, X, N, bias, Y, st);
        case 24: return launch_bin_g<4, 2>(g, W, X, N, bias, Y, st);
        case 22: return launch_bin_g<2, 2>(g, W, X, N, bias, Y, st);
        case 21: return launch_bin_g<1, 2>(g, W, X, N, bias, Y, st);
        case 18: return launch_bin_g<8, 1>(g, W, X, N, bias, Y, st);
        case 14: return launch_bin_g<4, 1>(g, W, X, N, bias, Y, st);
        default:
            return fail(SLK_EINVAL, "spmm: binned stream of " + std::to_string(W->bin_rw) +
                                        " rows per wave and " + std::to_string(W->bin_h) +
                                        " halves has no kernel");
    }
}

// Waves worth launching: enough to give every CU several to switch between.
constexpr int64_t kTargetWaves = 4096;
// LDS kernel: N from which it is considered, and expected uses of each staged
// X element (density x rows per workgroup) below which direct gathers are as
// fast (both measured on the C3/C4/C5 layer shapes).
constexpr int64_t kLdsMinN = 1024;
// Dense rows run on the matrix cores in the forward only from this many: each
// dense wave's chain is K steps long whatever the row count (16384 columns:
// about 0.5 ms), so a few rows cannot fill the chip, and the dense waves'
// X reads compete with the gather kernel's for the L2s (16384^2 Zipf(1.1):
// at 95%, 622 rows, 5.80 -> 5.28 ms; at 99%, 102 rows, 2.50 -> 3.0 ms).
constexpr int64_t kDenseFwdMinRows = 256;
constexpr double kLdsMinReuse = 4.0;
constexpr int64_t kCUs = 256;  // MI355X; one LDS-kernel workgroup per CU at a time

// Workgroups of the LDS kernel (one per CU at a time: 160 KiB of LDS each).
int64_t lds_blocks(int64_t M, int64_t N, int h, int rw) {
    return ceil_div(M, int64_t{kLdsWaves} * rw) * ceil_div(N, int64_t{kLdsCols} * h);
}
// With fewer workgroups than this, CUs idle while each workgroup streams all
// of K, and the wave kernels, which spread the same work over every CU, are
// faster. Measured on 10%-dense layers with 64-2048 rows and 512-784 columns:
// 32 workgroups 44 us against 15 us for the wave kernel, 128 workgroups 46
// against 29 us, 208 even (33 us), 256 51 against 54 us; the 10M-GPT layers
// that the LDS kernel wins have 192.
constexpr int64_t kLdsMinBlocks = 3 * kCUs / 4;

// Estimated time of the LDS kernel with H halves of 256 columns per lane and
// RW rows per wave: rounds of workgroups x X chunks x (barrier + rows x (row
// overhead + expected slots per row and chunk x per-slot cost)). The constants
// (40, 2, 4 and 6 per slot) were fitted to the measured times of all five
// configurations on the 10M- and 60M-GPT and 16384^2 layer shapes, forward and
// transpose, where the choice they give is the fastest measured in every case.
double lds_cost(int64_t M, int64_t K, int64_t N, double density, int h, int rw) {
    const int64_t kc = kLdsK / h;
    const int64_t blocks = lds_blocks(M, N, h, rw);
    const double rounds = static_cast<double>(ceil_div(blocks, kCUs));
    const double chunks = static_cast<double>(ceil_div(K, kc));
    return rounds * chunks * (40.0 + rw * (2.0 + density * kc * (h == 1 ? 4.0 : 6.0)));
}

// Y = W·X (+ bias per row): the shared body of slk_spmm and slk_spmm_bias.
// Y^T for slk_spmm_t: one-row-per-wave kernel, one float per lane, each
// lane writing its token's row of Yt (narrow layers; the stores of a wave are
// M floats apart).
int launch_wave_t(const slk_csr* W, const float* X, int64_t N, const float* bias, float* Yt,
                  hipStream_t st) {
    const int64_t M = W->nrows;
    const int64_t nitems = M * ceil_div(N, int64_t{kWave});
    int64_t blocks;
    if (int rc = launch_blocks(nitems, &blocks)) return rc;
    hipLaunchKernelGGL((spmm_wave_kernel<1, 32, true>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kSpmmBlock), 0, st, M, N, nitems, W->row_order, W->row_start,
                       W->row_nnz, W->col_indices, W->values, X, bias, Yt);
    return check_launch("spmm_t");
}

// The phased gather sweep with 16-byte lanes: one launch per column phase,
// stream-ordered, so each phase reads the partial sums its predecessor stored.
int launch_phased4(const slk_csr* W, const float* X, int64_t N, const float* bias, float* Y,
                   hipStream_t st) {
    constexpr int U = 8;
    const int64_t nitems = W->nrows * ceil_div(N, int64_t{kWave} * 4);
    int64_t blocks;
    if (int rc = launch_blocks(nitems, &blocks)) return rc;
    for (int64_t ph = 0; ph < W->n_phases; ++ph) {
        const float* b = ph + 1 == W->n_phases ? bias : nullptr;
        hipLaunchKernelGGL((spmm_wave_kernel<4, U, false, true>),
                           dim3(static_cast<unsigned>(blocks)), dim3(kSpmmBlock), 0, st,
                           W->nrows, N, nitems, W->row_order, W->row_start, W->row_nnz,
                           W->col_indices, W->values, X, b, Y, W->phase_lo, W->n_phases, ph);
        if (int rc = check_launch("spmm")) return rc;
    }
    return SLK_OK;
}

// Heavy rows (positions [0, T) of W->row_order) on the LDS kernel on the
// caller's stream, the rest on the phased gather kernel on the side stream,
// concurrently: the heavy rows' workgroups alone leave CUs idle in their last
// rounds, which the gather launches fill. Rows are disjoint, so the two write
// disjoint rows of Y. With `dense` (a view whose n_dense_rows rows precede
// W's in the order), those dense rows run first on the caller's stream, on the
// matrix cores, beside the gather: the gather's waves use the vector units
// and leave most registers free, the dense waves the matrix cores. Returns
// SLK_OK with *done = false if no side queue (nothing launched then).
int spmm_split_two_queues(const slk_csr* W, int64_t T, const float* X, int64_t N,
                          const float* bias, float* Y, hipStream_t st, bool* done,
                          const slk_csr* dense = nullptr) {
    std::lock_guard<std::mutex> lock(side_mutex());
    SideQueue* q = side_queue(st);
    *done = q != nullptr;
    if (q == nullptr) return SLK_OK;
    if (hipEventRecord(q->fork, st) != hipSuccess || hipStreamWaitEvent(q->s, q->fork, 0) != hipSuccess)
        return fail(SLK_EDEVICE, "spmm: fork to the side stream failed");
    int rc = dense != nullptr ? spmm_dense_rows(dense, X, dense->ncols, N, bias, Y, st) : SLK_OK;
    if (rc == SLK_OK && T > 0)
        rc = launch_lds_rw<kHeavyRW, kHeavyH>(W, W->row_order, T, X, N, bias, Y, st);
    if (rc == SLK_OK) {
        slk_csr rest = *W;
        rest.nrows = W->nrows - T;
        rest.row_order = W->row_order + T;
        rest.n_heavy_rows = 0;
        rc = launch_phased4(&rest, X, N, bias, Y, q->s);
    }
    // joined back even after a failed launch, so the caller's stream stays ordered
    if (hipEventRecord(q->join, q->s) != hipSuccess || hipStreamWaitEvent(st, q->join, 0) != hipSuccess)
        return fail(SLK_EDEVICE, "spmm: join from the side stream failed");
    return rc;
}

int spmm_impl(const slk_csr* W, const float* X, int64_t K, int64_t N, const float* bias,
              float* Y, void* stream, bool transposed_out = false) {
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
    if (transposed_out) return launch_wave_t(W, X, N, bias, Y, st);
    // Dense rows (the head of row_order) on the matrix cores, then the rest
    // of the rows as a view of their own. SLK_TUNE_DENSE_ROWS = 0 keeps them
    // with the rest.
    if (W->n_dense_rows >= kDenseFwdMinRows && tuning(SLK_TUNE_DENSE_ROWS) != 0 &&
        dense_rows_apply(W->n_dense_rows, K, N)) {
        const int64_t T = W->n_dense_rows;
        slk_csr rest = *W;
        rest.nrows = W->nrows - T;
        rest.row_order = W->row_order + T;
        rest.n_heavy_rows = W->n_heavy_rows > T ? W->n_heavy_rows - T : 0;
        rest.n_dense_rows = 0;
        rest.dense_ws = nullptr;
        if (rest.bin_off != nullptr) {
            if (W->bin_first >= T) rest.bin_first = W->bin_first - T;
            else rest.bin_off = nullptr;  // a stream that covers dense rows is not used
        }
        if (rest.nrows == 0) return SLK_OK;
        // With phase bounds (X far beyond the L2s), the dense rows run on the
        // caller's stream beside the phased gather of the light rows on the
        // side stream (the two-queue path below; the rest's heavy rows, if
        // any, on the LDS kernel after the dense ones): the gather waves use
        // the vector units, the dense waves the matrix cores, and the
        // longest rows, whose serial chains set each phase's length, leave
        // the gather.
        const uintptr_t al = reinterpret_cast<uintptr_t>(X) | reinterpret_cast<uintptr_t>(Y);
        if (rest.n_heavy_rows < rest.nrows && rest.phase_lo != nullptr && rest.n_phases > 1 &&
            N % 4 == 0 && al % 16 == 0 && N >= kLdsMinN && tuning(SLK_TUNE_SPMM_SPLIT) < 0 &&
            tuning(SLK_TUNE_SPMM_KERNEL) != 0 && tuning(SLK_TUNE_SPMM_BIN) <= 0 &&
            rest.bin_off == nullptr) {
            bool done = false;
            const int rc = spmm_split_two_queues(&rest, rest.n_heavy_rows, X, N, bias, Y, st, &done, W);
            if (done || rc != SLK_OK) return rc;
        }
        if (int rc = spmm_dense_rows(W, X, K, N, bias, Y, st)) return rc;
        return spmm_impl(&rest, X, K, N, bias, Y, stream);
    }
    const uintptr_t align = reinterpret_cast<uintptr_t>(X) | reinterpret_cast<uintptr_t>(Y);
    const int64_t M = W->nrows;
    // A binned slot stream (built by the caller where it pays) takes the LDS
    // path with its own kernel. SLK_TUNE_SPMM_BIN = 0 ignores it, and so does
    // a forced choice of the other kernels unless SLK_TUNE_SPMM_BIN = 1.
    const int64_t tb = tuning(SLK_TUNE_SPMM_BIN);
    const bool forced = tuning(SLK_TUNE_SPMM_KERNEL) >= 0 || tuning(SLK_TUNE_SPMM_H) >= 0 ||
                        tuning(SLK_TUNE_SPMM_RW) >= 0 || tuning(SLK_TUNE_SPMM_VEC) >= 0;
    if (W->bin_off != nullptr && (tb > 0 || (tb < 0 && !forced)) && K > 0 && N % 4 == 0 &&
        align % 16 == 0 && ceil_div(K, kLdsK / W->bin_h) <= SLK_BIN_MAX_CHUNKS)
        return launch_bin(W, X, N, bias, Y, st);

    // Kernel choice. The LDS-staged kernel needs 16-byte lanes (N % 4 == 0,
    // aligned X and Y) and pays off when each staged X element feeds several
    // rows of a workgroup: expected uses = density x rows per workgroup, and
    // when it has enough workgroups to occupy the chip. Among the
    // configurations that pass both bars, lds_cost picks one. The per-wave
    // gather kernels cover everything else (small N is latency-bound).
    // SLK_TUNE_SPMM_KERNEL, SLK_TUNE_SPMM_H and SLK_TUNE_SPMM_RW override.
    const bool lds_ok = N % 4 == 0 && align % 16 == 0;
    int rw = 0, h = 1;
    if (lds_ok && N >= kLdsMinN) {
        const double density =
            K > 0 ? static_cast<double>(W->total_capacity) / (1.2 * M * K) : 0.0;
        double best = 0.0;
        // (3 and 6 rows per wave fit row counts such as 768 and 2304 to whole
        // rounds of 256 workgroups: the 60M-GPT QKV input gradient, 768 rows,
        // is 192 workgroups at 4 rows and 256 at 3)
        for (const int cfg : {18, 16, 14, 13, 12, 28, 26, 24, 23, 22}) {  // h * 10 + rw
            const int ch = cfg / 10, crw = cfg % 10;
            // 8 rows x 8 columns per lane: rows of uniform length only (the
            // light rows of a skewed matrix run slower with it: 16384^2
            // Zipf(1.1) at 95%, forward as one split grid 6.97 -> 7.94 ms
            // against 8 rows x 4 columns, while its transpose runs 6.91 ->
            // 5.69 ms)
            if (cfg == 28 && W->n_heavy_rows > 0) continue;
            if (density * kLdsWaves * crw < kLdsMinReuse) continue;
            if (lds_blocks(M, N, ch, crw) < kLdsMinBlocks) continue;
            const double c = lds_cost(M, K, N, density, ch, crw);
            if (rw == 0 || c < best) {
                best = c;
                rw = crw;
                h = ch;
            }
        }
    }
    if (const int64_t t = tuning(SLK_TUNE_SPMM_KERNEL); t >= 0) {
        if (t == 0) rw = 0;
        if (t == 1 && lds_ok && rw == 0) rw = 8;
    }
    if (rw != 0) {
        if (const int64_t t = tuning(SLK_TUNE_SPMM_H); t >= 0) h = t == 2 ? 2 : 1;
        if (const int64_t t = tuning(SLK_TUNE_SPMM_RW); t >= 0) rw = static_cast<int>(t);
        if (rw != 2 && rw != 3 && rw != 4 && rw != 6 && rw != 8) rw = 8;
        // Heavy rows (the head of the longest-rows-first order) in workgroups
        // of their own with two rows per wave and 8 columns per lane, then the
        // rest in that order, so every workgroup holds rows of similar length:
        // on the 16384^2 Zipf(1.1) layer at 95% sparsity 12.6 -> 9.1 ms (heavy
        // rows with the rest, a long row stalls its workgroup at every chunk;
        // all rows in one sorted launch, the few workgroups of full rows
        // outlast the rest).
        // SLK_TUNE_SPMM_SPLIT = 0 runs one launch in natural row order.
        const int64_t T = W->n_heavy_rows;
        const int64_t split_t = tuning(SLK_TUNE_SPMM_SPLIT);
        const bool split = T > 0 && split_t != 0;
        // With phase bounds (X far beyond the L2s) the rows after the heavy
        // ones run on the phased gather kernel, concurrently with the heavy
        // rows' LDS launch (spmm_split_two_queues): 16384^2 Zipf(1.1) at 95%
        // 7.05 -> 6.0 ms against the one-grid LDS split. SLK_TUNE_SPMM_SPLIT =
        // 1 keeps the LDS split, 0 runs one launch in natural row order.
        if (split && split_t < 0 && T < M && W->phase_lo != nullptr && W->n_phases > 1 &&
            N >= kWave * 4) {
            bool done = false;
            const int rc = spmm_split_two_queues(W, T, X, N, bias, Y, st, &done);
            if (done || rc != SLK_OK) return rc;
        }
        if (split) {
            // one grid when the rest fills at least one workgroup per XCD (the
            // split kernel's XCD shares need it): 16384^2 Zipf(1.1) at 95%
            // forward 8.27 -> 8.03 ms against two launches
            const int64_t nb_rest = ceil_div(M - T, int64_t{kLdsWaves} * rw) * ceil_div(N, int64_t{kLdsCols});
            if (h == 1 && nb_rest >= kXcds) {
                switch (rw) {  // every rw the checks above admit
                    case 2: return launch_lds_split_rw<2>(W, T, X, N, bias, Y, st);
                    case 3: return launch_lds_split_rw<3>(W, T, X, N, bias, Y, st);
                    case 4: return launch_lds_split_rw<4>(W, T, X, N, bias, Y, st);
                    case 6: return launch_lds_split_rw<6>(W, T, X, N, bias, Y, st);
                    default: return launch_lds_split_rw<8>(W, T, X, N, bias, Y, st);
                }
            }
            if (int rc = launch_lds_rw<kHeavyRW, kHeavyH>(W, W->row_order, T, X, N, bias, Y, st))
                return rc;
            return launch_lds(h, rw, W, W->row_order + T, M - T, X, N, bias, Y, st);
        }
        return launch_lds(h, rw, W, nullptr, M, X, N, bias, Y, st);
    }

    int vec = 1;
    if (const int64_t t = tuning(SLK_TUNE_SPMM_VEC); t >= 0) vec = static_cast<int>(t);
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
    if (vec == 4 && W->phase_lo != nullptr && W->n_phases > 1) return launch_phased4(W, X, N, bias, Y, st);
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

extern "C" int slk_spmm_t(const slk_csr* W, const float* X, int64_t K, int64_t N,
                          const float* bias, float* Yt, void* stream) {
    return slk::spmm_impl(W, X, K, N, bias, Yt, stream, true);
}
