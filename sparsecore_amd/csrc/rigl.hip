// RigL's grow choice from an approximate dense gradient with a certified
// error bound, so that the grown columns are the reference's bit for bit
// without computing G = dY·X^T exactly everywhere.
//
// The reference ranks a row's empty columns by |G[i, c]| with G from its own
// dense_grad (csrc/kernels/dense_grad.cpp:57-83: per element one running sum
// over j, products rounded, then added; the last N mod 4 terms fused) and
// grows the n_grow largest (sparselab/router.py:698-721). Computing that G on
// the VALU costs M·K·N sequential multiply-adds (40 ms at 16384^2 x 4096).
// Here:
//
//   norms    n_i >= ||dY_i||_2 and n_k >= ||X_k||_2 (float64 sums, rounded up).
//   approx   G' = dY·X^T on the matrix cores: every fp32 operand is split into
//            bf16 parts, x = x_h + x_l + r (|r| <= 2^-16 |x|, round to nearest
//            even), and G' = Σ x_h y_h + Σ (x_h y_l + x_l y_h), three
//            bf16 MFMA products per term in fp32. The x_h y_h products are
//            summed in chunks of 512 j on the matrix cores and the chunk sums
//            added on the VALU, so no product passes through more than
//            511 + N/512 additions.
//   bound    |G'[i,k] - G[i,k]| <= E[i,k] = c_N·n_i·n_k + δ, where
//            c_N covers the reference's own rounding (γ_N), the matrix-core
//            sums (≤ 2u per addition, to cover any rounding mode), the dropped
//            x_l y_l and r terms, the final add, plus a 1% margin; and δ the
//            flushing of subnormal bf16 parts and products (2^-100·(1+n_i+n_k)).
//            Σ_j |x_j y_j| <= n_i·n_k by Cauchy-Schwarz.
//   count    per row: survivors as in the exact kernel; n_grow = min(dropped,
//            empty columns); among the empty columns, lower = |G'| - E and
//            upper = |G'| + E (rounded outward); T_lo / T_hi = the n_grow-th
//            largest lower / upper. A column with lower > T_hi is certainly
//            grown (|G| > T_hi >= the exact n_grow-th largest |G|), one with
//            upper < T_lo certainly not; the rest are undecided. Counts them.
//   finish   per row: lists the undecided columns (ascending), computes their
//            exact G with the reference's arithmetic (dY_i staged in LDS, X_k
//            streamed), takes the n_grow - (certain) smallest exact keys
//            ~bits(|G|) among them (ties to the lower column), and rewrites
//            the row exactly as the exact drop/grow kernel does.
//
// A row whose norms are not finite or too large (n_i·n_k beyond 2^120, where
// G could overflow) is an exact row: every empty column is undecided, and NaN
// columns are excluded from the grow count as in the exact kernel.
#include "common.hpp"
#include "row_rewrite.hpp"

namespace slk {
namespace {

// ───────────────────────────── row norms ───────────────────────────────────

// nrm[r] >= ||A_r||_2 for the R rows of the row-major R x N matrix A; +inf if
// the row is not finite. One wave per row.
__global__ __launch_bounds__(256) void rigl_norm_kernel(const float* __restrict__ A, int64_t R,
                                                         int64_t N, float* __restrict__ nrm) {
    const int64_t r = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) >> 6;
    if (r >= R) return;
    const int lane = threadIdx.x & 63;
    const float* p = A + r * N;
    double s = 0.0;
    for (int64_t j = lane; j < N; j += 64) {
        const double v = p[j];
        s += v * v;  // exact square; the sum's relative error is below N·2^-53
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if (lane == 0) {
        const double n = sqrt(s) * (1.0 + 0x1p-30);
        nrm[r] = (s == s && s < 0x1p1000) ? __double2float_ru(n) : __builtin_inff();
    }
}

// ───────────────────────────── approximate G ───────────────────────────────

constexpr int kAT = 128;        // output tile edge (rows of dY, rows of X)
constexpr int kAJ = 32;         // j per LDS stage: two MFMA k-steps of 16
constexpr int kARow = 40;       // bf16 per LDS row: 32 + 8 padding (80 bytes)
constexpr int kAChunk = 512;    // j per matrix-core partial sum of x_h·y_h
constexpr int kAThreads = 256;  // 4 waves, 2 x 2, each 64 x 64 of the tile
constexpr int kAGroup = 8;      // tile rows per group of the tile order

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// bf16 bits of x rounded to nearest even (x finite; non-finite x keeps its
// class: the bound of any row or column holding one is infinite anyway).
__device__ __forceinline__ uint32_t bf16_rne(float x) {
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7f800000u) == 0x7f800000u) return (u >> 16) | ((u & 0xffffu) ? 0x40u : 0u);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// Splits four floats into packed bf16 high parts and packed low parts.
__device__ __forceinline__ void split4(f32x4 v, uint2& hi, uint2& lo) {
    uint32_t h[4], l[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        h[q] = bf16_rne(v[q]);
        const float rest = v[q] - __uint_as_float(h[q] << 16);  // exact
        l[q] = bf16_rne(rest);
    }
    hi = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
    lo = make_uint2(l[0] | (l[1] << 16), l[2] | (l[3] << 16));
}

// Operand layout of the matrix-core pass: every row of dY and of X cut into
// stages of kAJ j, each stage stored as kAJ bf16 high parts then kAJ bf16 low
// parts (128 contiguous bytes), zero beyond N. Split once per call, so the
// tiles that share a row read it ready-made.
constexpr int kAStageBytes = 2 * kAJ * 2;

// P[r][s] = the stage s of row r (R rows of N floats, nst stages). One thread
// per 4 floats.
__global__ __launch_bounds__(256) void rigl_split_kernel(const float* __restrict__ A, int64_t R,
                                                          int64_t N, int64_t nst,
                                                          uint16_t* __restrict__ P) {
    const int64_t q = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // 4-float piece
    const int64_t per_row = nst * (kAJ / 4);
    if (q >= R * per_row) return;
    const int64_t r = q / per_row;
    const int64_t j = (q - r * per_row) * 4;
    f32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = j + e < N ? A[r * N + j + e] : 0.0f;
    uint2 hi, lo;
    split4(v, hi, lo);
    const int64_t s = j / kAJ, js = j - s * kAJ;
    uint16_t* blk = P + (r * nst + s) * (2 * kAJ);
    *reinterpret_cast<uint2*>(blk + js) = hi;
    *reinterpret_cast<uint2*>(blk + kAJ + js) = lo;
}

constexpr int kALdsRow = kAStageBytes + 16;  // bytes per staged row (padded)

__global__ __launch_bounds__(kAThreads) void rigl_approx_kernel(int64_t M, int64_t K, int64_t nst,
                                                                const uint16_t* __restrict__ PA,
                                                                const uint16_t* __restrict__ PB,
                                                                float* __restrict__ G) {
    __shared__ __align__(16) unsigned char sA[2][kAT * kALdsRow];
    __shared__ __align__(16) unsigned char sB[2][kAT * kALdsRow];

    // grouped, XCD-contiguous tile order: consecutive tiles share dY and X rows
    const int64_t nTi = ceil_div(M, kAT), nTk = ceil_div(K, kAT);
    const int64_t L = xcd_logical_block(blockIdx.x, gridDim.x);
    const int64_t grp = L / (kAGroup * nTk);
    const int64_t first = grp * kAGroup;
    const int64_t gsize = nTi - first < kAGroup ? nTi - first : kAGroup;
    const int64_t in_grp = L - grp * kAGroup * nTk;
    const int64_t i0 = (first + in_grp % gsize) * kAT;
    const int64_t k0 = (in_grp / gsize) * kAT;

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wv = t >> 6;
    const int wm = wv >> 1, wn = wv & 1;
    // staging: thread t moves bytes [64h, 64h + 64) of staged row t/2
    const int lr = t >> 1, lh = (t & 1) * 64;
    const unsigned char* ga = reinterpret_cast<const unsigned char*>(
        PA + (i0 + lr < M ? i0 + lr : M - 1) * nst * (2 * kAJ)) + lh;
    const unsigned char* gb = reinterpret_cast<const unsigned char*>(
        PB + (k0 + lr < K ? k0 + lr : K - 1) * nst * (2 * kAJ)) + lh;

    f32x16 cm[2][2], mm[2][2], cx[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) cm[a][b][r] = mm[a][b][r] = cx[a][b][r] = 0.0f;

    f32x4 ra[4], rb[4];
    auto fetch = [&](int64_t st) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            ra[q] = *reinterpret_cast<const f32x4*>(ga + st * kAStageBytes + 16 * q);
            rb[q] = *reinterpret_cast<const f32x4*>(gb + st * kAStageBytes + 16 * q);
        }
    };
    if (nst > 0) fetch(0);
    const int half = 16 * (lane >> 5);
    for (int64_t st = 0; st < nst; ++st) {
        const int buf = static_cast<int>(st & 1);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            *reinterpret_cast<f32x4*>(&sA[buf][lr * kALdsRow + lh + 16 * q]) = ra[q];
            *reinterpret_cast<f32x4*>(&sB[buf][lr * kALdsRow + lh + 16 * q]) = rb[q];
        }
        __syncthreads();
        if (st + 1 < nst) fetch(st + 1);  // in flight during this stage's MFMAs
        // both k-steps' fragments: [k-step][block][high, low]
        bf16x8 af[2][2][2], bf[2][2][2];
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    const int ra_ = wm * 64 + b * 32 + (lane & 31);
                    const int rb_ = wn * 64 + b * 32 + (lane & 31);
                    const int o = p * (kAStageBytes / 2) + 32 * s + half;
                    af[s][b][p] = *reinterpret_cast<const bf16x8*>(&sA[buf][ra_ * kALdsRow + o]);
                    bf[s][b][p] = *reinterpret_cast<const bf16x8*>(&sB[buf][rb_ * kALdsRow + o]);
                }
#pragma unroll
        for (int s = 0; s < 2; ++s) {
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b)
                    cm[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[s][a][0], bf[s][b][0],
                                                                        cm[a][b], 0, 0, 0);
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b)
                    cx[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[s][a][0], bf[s][b][1],
                                                                        cx[a][b], 0, 0, 0);
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b)
                    cx[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[s][a][1], bf[s][b][0],
                                                                        cx[a][b], 0, 0, 0);
        }
        if ((st + 1) % (kAChunk / kAJ) == 0 || st + 1 == nst) {
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        mm[a][b][r] = mm[a][b][r] + cm[a][b][r];
                        cm[a][b][r] = 0.0f;
                    }
        }
    }
    // lane l, register 4g + q of a 32x32 block: row 8g + 4(l/32) + q, column l % 32
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int64_t col = k0 + wn * 64 + b * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = i0 + wm * 64 + a * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row < M && col < K) G[row * K + col] = mm[a][b][r] + cx[a][b][r];
            }
        }
}

// ───────────────────────────── certified selection ─────────────────────────

struct RowInfo {
    int32_t n_grow;  // grows of the row (exact rows: decided in finish)
    int32_t n_in;    // columns certainly grown
    float t_lo;      // the n_grow-th largest lower bound
    float t_hi;      // the n_grow-th largest upper bound
    int32_t flags;   // kRowExact, kRowKeep
    int32_t n_keep;
    int32_t pad[2];
};
constexpr int32_t kRowExact = 1;  // every empty column undecided
constexpr int32_t kRowKeep = 2;   // nothing to grow: the row is left as it is
static_assert(sizeof(RowInfo) == 32, "RowInfo is 32 bytes");

// Certified bounds of |G[i, c]| from |G'[i, c]|: false if the column must be
// decided exactly (norms not finite or too large).
__device__ __forceinline__ bool bounds_of(float g, float ni, float nk, double c_bound, float& lo,
                                          float& hi) {
    if (!(ni <= 0x1p60f) || !(nk <= 0x1p60f)) return false;
    const double e = c_bound * static_cast<double>(ni) * static_cast<double>(nk) *
                         (1.0 + 0x1p-30) +
                     0x1p-100 * (1.0 + static_cast<double>(ni) + static_cast<double>(nk));
    const double a = fabs(static_cast<double>(g));
    if (!(a <= 0x1p125)) return false;  // G' not finite (cannot happen below the norm cap)
    const double l = (a - e) * (1.0 - 0x1p-40), h = (a + e) * (1.0 + 0x1p-40);
    lo = l > 0.0 ? __double2float_rd(l) : 0.0f;
    hi = __double2float_ru(h);
    return true;
}

// Largest-first selection keys of a non-negative float.
__device__ __forceinline__ uint32_t desc_key(float v) { return ~__float_as_uint(v); }

// The need-th smallest key among n candidates (cand(e, key) -> bool): a radix
// select with 8-bit digits; need in [1, count of candidates].
template <class Cand>
__device__ uint32_t kth_smallest_key(Cand cand, int64_t n, int64_t need, uint32_t* hist,
                                     uint32_t* s_digit, int64_t* s_below, int64_t* tmp) {
    const int t = threadIdx.x;
    uint32_t prefix = 0;
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        hist[t] = 0;
        __syncthreads();
        for (int64_t e = t; e < n; e += kRowThreads) {
            uint32_t u;
            if (!cand(e, u)) continue;
            if (pass == 0 || (u >> (shift + 8)) == prefix) atomicAdd(&hist[(u >> shift) & 255u], 1u);
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
    return prefix;
}

__global__ __launch_bounds__(kRowThreads) void rigl_count_kernel(
    int64_t K, int64_t Kw, const int32_t* __restrict__ row_start,
    const int32_t* __restrict__ row_nnz, const float* __restrict__ values,
    const int32_t* __restrict__ cols, const float* __restrict__ thr_ptr,
    const float* __restrict__ Gp, int64_t ldg, const float* __restrict__ nrm_r,
    const float* __restrict__ nrm_c, double c_bound, RowInfo* __restrict__ info,
    int64_t* __restrict__ amb_count) {
    extern __shared__ uint32_t lds[];
    uint32_t* keep = lds;
    __shared__ int64_t tmp[kRowThreads];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_digit;
    __shared__ int64_t s_below;
    __shared__ unsigned long long s_best;

    const int64_t i = blockIdx.x;
    const int t = threadIdx.x;
    RowInfo ri{};
    const int32_t n_live = row_nnz[i];
    if (n_live <= 0) {  // the reference skips empty rows
        if (t == 0) {
            ri.flags = kRowKeep;
            info[i] = ri;
            amb_count[i] = 0;
        }
        return;
    }
    const int32_t start = row_start[i];
    for (int64_t w = t; w < Kw; w += kRowThreads) keep[w] = 0;
    __syncthreads();
    const int64_t n_keep = mark_survivors(values, cols, start, n_live, thr_ptr[0], keep, tmp,
                                          &s_best);
    const int64_t n_drop = n_live - n_keep;
    ri.n_keep = static_cast<int32_t>(n_keep);
    if (n_drop == 0) {
        if (t == 0) {
            ri.flags = kRowKeep;
            info[i] = ri;
            amb_count[i] = 0;
        }
        return;
    }
    const float ni = nrm_r[i];
    const float* g_row = Gp + i * ldg;
    // a column without a certified bound makes the whole row exact
    int64_t unbounded = 0;
    for (int64_t c = t; c < K; c += kRowThreads) {
        float lo, hi;
        if (!bit_of(keep, c) && !bounds_of(g_row[c], ni, nrm_c[c], c_bound, lo, hi)) ++unbounded;
    }
    block_inclusive_scan(unbounded, tmp);
    unbounded = tmp[kRowThreads - 1];
    __syncthreads();
    const int64_t n_empty = K - n_keep;
    if (unbounded > 0) {
        if (t == 0) {
            ri.flags = kRowExact;
            info[i] = ri;
            amb_count[i] = n_empty;
        }
        return;
    }
    const int64_t n_grow = n_drop < n_empty ? n_drop : n_empty;
    auto lower = [&](int64_t c, uint32_t& key) -> bool {
        if (bit_of(keep, c)) return false;
        float lo, hi;
        bounds_of(g_row[c], ni, nrm_c[c], c_bound, lo, hi);
        key = desc_key(lo);
        return true;
    };
    auto upper = [&](int64_t c, uint32_t& key) -> bool {
        if (bit_of(keep, c)) return false;
        float lo, hi;
        bounds_of(g_row[c], ni, nrm_c[c], c_bound, lo, hi);
        key = desc_key(hi);
        return true;
    };
    const float t_lo = __uint_as_float(~kth_smallest_key(lower, K, n_grow, hist, &s_digit,
                                                         &s_below, tmp));
    const float t_hi = __uint_as_float(~kth_smallest_key(upper, K, n_grow, hist, &s_digit,
                                                         &s_below, tmp));
    int64_t n_in = 0, n_amb = 0;
    for (int64_t c = t; c < K; c += kRowThreads) {
        if (bit_of(keep, c)) continue;
        float lo, hi;
        bounds_of(g_row[c], ni, nrm_c[c], c_bound, lo, hi);
        if (lo > t_hi) ++n_in;
        else if (hi >= t_lo) ++n_amb;
    }
    block_inclusive_scan(n_in, tmp);
    n_in = tmp[kRowThreads - 1];
    __syncthreads();
    block_inclusive_scan(n_amb, tmp);
    n_amb = tmp[kRowThreads - 1];
    if (t == 0) {
        ri.n_grow = static_cast<int32_t>(n_grow);
        ri.n_in = static_cast<int32_t>(n_in);
        ri.t_lo = t_lo;
        ri.t_hi = t_hi;
        info[i] = ri;
        amb_count[i] = n_amb;
    }
}

// off[0..M] = exclusive scan of cnt[0..M-1]; *total = off[M]. One workgroup.
__global__ __launch_bounds__(1024) void rigl_scan_kernel(int64_t M, const int64_t* __restrict__ cnt,
                                                         int64_t* __restrict__ off,
                                                         int64_t* __restrict__ total) {
    __shared__ int64_t part[1024];
    const int t = threadIdx.x;
    const int64_t per = ceil_div(M, 1024);
    const int64_t a = t * per < M ? t * per : M, e = a + per < M ? a + per : M;
    int64_t s = 0;
    for (int64_t r = a; r < e; ++r) s += cnt[r];
    part[t] = s;
    __syncthreads();
    for (int d = 1; d < 1024; d <<= 1) {
        const int64_t add = t >= d ? part[t - d] : 0;
        __syncthreads();
        part[t] += add;
        __syncthreads();
    }
    int64_t run = part[t] - s;
    for (int64_t r = a; r < e; ++r) {
        off[r] = run;
        run += cnt[r];
    }
    if (t == 1023) {
        off[M] = part[t];
        *total = part[t];
    }
}

constexpr int64_t kStageMaxN = 8192;     // dY rows up to this length are staged in LDS
constexpr int64_t kRiglMaxCols = 131072;  // bitmaps of 3 x 16 KiB in LDS

// Exact G[i, c] with the reference's arithmetic: one running sum over j,
// products rounded then added, the last N mod 4 terms fused. y: dY_i (LDS
// or global), x: X_c (global); V4: both 16-byte aligned and N % 4 == 0.
template <bool V4>
__device__ __forceinline__ float exact_dot(const float* y, const float* __restrict__ x, int64_t N) {
    float acc = 0.0f;
    const int64_t n4 = N & ~int64_t{3};
    int64_t j = 0;
    if (V4) {
        for (; j < n4; j += 4) {
            const f32x4 a = *reinterpret_cast<const f32x4*>(y + j);
            const f32x4 b = *reinterpret_cast<const f32x4*>(x + j);
            acc = acc + a[0] * b[0];
            acc = acc + a[1] * b[1];
            acc = acc + a[2] * b[2];
            acc = acc + a[3] * b[3];
        }
    } else {
        for (; j < n4; ++j) {
            const float p = y[j] * x[j];
            acc = acc + p;
        }
    }
    for (; j < N; ++j) acc = __builtin_fmaf(y[j], x[j], acc);
    return acc;
}

template <bool V4>
__global__ __launch_bounds__(kRowThreads) void rigl_finish_kernel(
    int64_t K, int64_t Kw, int64_t N, const int32_t* __restrict__ row_start,
    int32_t* __restrict__ row_nnz, float* __restrict__ values, int32_t* __restrict__ cols,
    const float* __restrict__ thr_ptr, const float* __restrict__ Gp, int64_t ldg,
    const float* __restrict__ nrm_r, const float* __restrict__ nrm_c, double c_bound,
    const RowInfo* __restrict__ info, const int64_t* __restrict__ amb_off,
    int32_t* __restrict__ amb_col, uint32_t* __restrict__ amb_key,
    const float* __restrict__ dY, const float* __restrict__ X,
    int32_t* __restrict__ stage_col, float* __restrict__ stage_val,
    unsigned long long* __restrict__ removed) {
    extern __shared__ uint32_t lds[];
    uint32_t* keep = lds;
    uint32_t* grow = lds + Kw;
    uint32_t* wpre = lds + 2 * Kw;
    float* ys = reinterpret_cast<float*>(lds + ((3 * Kw + 3) & ~int64_t{3}));  // 16-byte aligned
    __shared__ int64_t tmp[kRowThreads];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_digit;
    __shared__ int64_t s_below;
    __shared__ unsigned long long s_best;

    const int64_t i = blockIdx.x;
    const int t = threadIdx.x;
    const RowInfo ri = info[i];
    if (ri.flags & kRowKeep) return;
    const int32_t n_live = row_nnz[i];
    const int32_t start = row_start[i];
    for (int64_t w = t; w < Kw; w += kRowThreads) keep[w] = grow[w] = 0;
    __syncthreads();
    const int64_t n_keep = mark_survivors(values, cols, start, n_live, thr_ptr[0], keep, tmp,
                                          &s_best);
    const int64_t n_drop = n_live - n_keep;
    const bool exact_row = (ri.flags & kRowExact) != 0;
    const float ni = nrm_r[i];
    const float* g_row = Gp + i * ldg;
    const int64_t off = amb_off[i];
    const int64_t n_amb = amb_off[i + 1] - off;

    // undecided columns, ascending; certainly grown ones straight into `grow`
    int64_t run = 0;
    for (int64_t c0 = 0; c0 < K; c0 += kRowThreads) {
        const int64_t c = c0 + t;
        bool amb = false;
        if (c < K && !bit_of(keep, c)) {
            if (exact_row) {
                amb = true;
            } else {
                float lo, hi;
                bounds_of(g_row[c], ni, nrm_c[c], c_bound, lo, hi);
                if (lo > ri.t_hi) atomicOr(&grow[c >> 5], 1u << (c & 31));
                else amb = hi >= ri.t_lo;
            }
        }
        const int64_t incl = block_inclusive_scan(amb ? 1 : 0, tmp);
        // (the count pass classified the same columns the same way, so
        // run + incl <= n_amb; the guard keeps a mismatch inside the row)
        if (amb && run + incl - 1 < n_amb) amb_col[off + run + incl - 1] = static_cast<int32_t>(c);
        run += tmp[kRowThreads - 1];
        __syncthreads();
    }

    // exact keys of the undecided columns (0 marks a NaN |G|)
    const float* y = dY + i * N;
    const bool staged = V4 && N <= kStageMaxN;
    if (staged) {
        for (int64_t j = 4 * t; j < N; j += 4 * kRowThreads)
            *reinterpret_cast<f32x4*>(ys + j) = *reinterpret_cast<const f32x4*>(y + j);
        __syncthreads();
    }
    for (int64_t e = t; e < n_amb; e += kRowThreads) {
        const int64_t c = amb_col[off + e];
        const float g = staged ? exact_dot<true>(ys, X + c * N, N)
                               : exact_dot<V4>(y, X + c * N, N);
        const float a = fabsf(g);
        amb_key[off + e] = a == a ? desc_key(a) : 0u;
    }
    __syncthreads();

    int64_t n_grow = ri.n_grow, need = ri.n_grow - ri.n_in;
    if (exact_row) {  // NaN columns are not growable
        int64_t ok = 0;
        for (int64_t e = t; e < n_amb; e += kRowThreads) ok += amb_key[off + e] != 0u;
        block_inclusive_scan(ok, tmp);
        ok = tmp[kRowThreads - 1];
        __syncthreads();
        n_grow = need = n_drop < ok ? n_drop : ok;
    }
    auto cand = [&](int64_t e, int64_t& col, uint32_t& key) -> bool {
        col = amb_col[off + e];
        key = amb_key[off + e];
        return key != 0u;
    };
    select_smallest_keys(cand, n_amb, need, grow, hist, &s_digit, &s_below, tmp);
    write_back_row(keep, grow, wpre, Kw, i, start, n_live, n_keep, n_grow, values, cols, row_nnz,
                   stage_col, stage_val, removed, tmp);
}

__global__ void rigl_clear_kernel(unsigned long long* __restrict__ c) { *c = 0; }

// c_N of the bound (see the file comment): the reference's γ_N, the matrix
// cores' sums at <= 2u per addition (chunks of kAChunk, chunk sums added on
// the VALU at <= u), the cross products' sums, the dropped parts, the final
// add; times 1.01.
double certified_c(int64_t N) {
    const double u = 0x1p-24;
    auto gam = [&](double n, double uu) { return n * uu / (1.0 - n * uu); };
    const double n = static_cast<double>(N > 0 ? N : 1);
    const double chunks = ceil(n / kAChunk) + 1.0;
    const double g_ref = gam(n, u);
    const double g_main = (gam(kAChunk, 2 * u) + gam(chunks, u)) * (1.0 + 0x1p-7);
    const double g_cross = gam(2 * n, 2 * u) * 2 * 0x1p-8 * (1.0 + 0x1p-7);
    const double dropped = 3.1 * 0x1p-16;
    const double fin = 1.01 * u;
    return (g_ref + g_main + g_cross + dropped + fin) * 1.01;
}

}  // namespace
}  // namespace slk

extern "C" int slk_rigl_norms(const float* dY, int64_t M, const float* X, int64_t K, int64_t N,
                              float* nrm_dY, float* nrm_X, void* stream) {
    using namespace slk;
    clear_error();
    if (M < 0 || K < 0 || N < 0) return fail(SLK_EINVAL, "rigl_norms: negative shape");
    if ((M > 0 && (dY == nullptr || nrm_dY == nullptr)) ||
        (K > 0 && (X == nullptr || nrm_X == nullptr)))
        return fail(SLK_EINVAL, "rigl_norms: NULL pointer");
    hipStream_t st = as_stream(stream);
    if (M > 0) {
        hipLaunchKernelGGL(rigl_norm_kernel, dim3(static_cast<unsigned>(ceil_div(M, 4))), dim3(256),
                           0, st, dY, M, N, nrm_dY);
    }
    if (K > 0) {
        hipLaunchKernelGGL(rigl_norm_kernel, dim3(static_cast<unsigned>(ceil_div(K, 4))), dim3(256),
                           0, st, X, K, N, nrm_X);
    }
    return check_launch("rigl_norms");
}

extern "C" int64_t slk_dense_grad_approx_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    if (M < 0 || K < 0 || N < 0) return 0;
    return (M + K) * slk::ceil_div(N, slk::kAJ) * slk::kAStageBytes;
}

extern "C" int slk_dense_grad_approx(const float* dY, const float* X, int64_t M, int64_t K,
                                     int64_t N, float* G, void* workspace,
                                     int64_t workspace_bytes, void* stream) {
    using namespace slk;
    clear_error();
    if (M < 0 || K < 0 || N < 0)
        return fail(SLK_EINVAL, "dense_grad_approx: shape params must be non-negative");
    if (M == 0 || K == 0) return SLK_OK;
    if (G == nullptr || (N > 0 && (dY == nullptr || X == nullptr)))
        return fail(SLK_EINVAL, "dense_grad_approx: NULL pointer");
    const int64_t nst = ceil_div(N, kAJ);
    const int64_t need = (M + K) * nst * kAStageBytes;
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
        return fail(SLK_EINVAL, "dense_grad_approx: workspace smaller than "
                                "slk_dense_grad_approx_workspace_bytes");
    const int64_t tiles = ceil_div(M, kAT) * ceil_div(K, kAT);
    if (tiles > INT32_MAX || ceil_div((M + K) * nst * (kAJ / 4), 256) > INT32_MAX)
        return fail(SLK_EINVAL, "dense_grad_approx: problem too large");
    hipStream_t st = as_stream(stream);
    uint16_t* PA = static_cast<uint16_t*>(workspace);
    uint16_t* PB = PA + M * nst * (2 * kAJ);
    if (nst > 0) {
        hipLaunchKernelGGL(rigl_split_kernel,
                           dim3(static_cast<unsigned>(ceil_div(M * nst * (kAJ / 4), 256))),
                           dim3(256), 0, st, dY, M, N, nst, PA);
        hipLaunchKernelGGL(rigl_split_kernel,
                           dim3(static_cast<unsigned>(ceil_div(K * nst * (kAJ / 4), 256))),
                           dim3(256), 0, st, X, K, N, nst, PB);
        if (int rc = check_launch("dense_grad_approx/split")) return rc;
    }
    hipLaunchKernelGGL(rigl_approx_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kAThreads), 0,
                       st, M, K, nst, PA, PB, G);
    return check_launch("dense_grad_approx");
}

extern "C" double slk_rigl_bound_factor(int64_t N) { return slk::certified_c(N); }

extern "C" int slk_rigl_count(const slk_csr* W, const float* thr_dev, const float* G_approx,
                              int64_t ldg, const float* nrm_dY, const float* nrm_X, int64_t N,
                              void* info, int64_t* amb_off, int64_t* amb_total, void* stream) {
    using namespace slk;
    clear_error();
    if (int rc = validate_csr(W, "rigl_count")) return rc;
    if (W->ncols > kRiglMaxCols)
        return fail(SLK_EINVAL, "rigl_count: ncols=" + std::to_string(W->ncols) +
                                    " exceeds the supported maximum " +
                                    std::to_string(kRiglMaxCols));
    if (W->nrows > INT32_MAX) return fail(SLK_EINVAL, "rigl_count: too many rows for one launch");
    if (N < 0) return fail(SLK_EINVAL, "rigl_count: negative N");
    if (amb_off == nullptr || amb_total == nullptr)
        return fail(SLK_EINVAL, "rigl_count: NULL output");
    if (W->nrows > 0 && (thr_dev == nullptr || G_approx == nullptr || ldg < W->ncols ||
                         nrm_dY == nullptr || nrm_X == nullptr || info == nullptr))
        return fail(SLK_EINVAL, "rigl_count: NULL input or ldg < ncols");
    hipStream_t st = as_stream(stream);
    const int64_t M = W->nrows, K = W->ncols;
    const int64_t Kw = ceil_div(K, 32) > 0 ? ceil_div(K, 32) : 1;
    // amb_off doubles as the per-row counts before the scan
    if (M > 0) {
        hipLaunchKernelGGL(rigl_count_kernel, dim3(static_cast<unsigned>(M)), dim3(kRowThreads),
                           static_cast<size_t>(Kw) * 4, st, K, Kw, W->row_start, W->row_nnz,
                           W->values, W->col_indices, thr_dev, G_approx, ldg, nrm_dY, nrm_X,
                           certified_c(N), static_cast<RowInfo*>(info), amb_off + M + 1);
        if (int rc = check_launch("rigl_count")) return rc;
    }
    hipLaunchKernelGGL(rigl_scan_kernel, dim3(1), dim3(1024), 0, st, M, amb_off + M + 1, amb_off,
                       amb_total);
    return check_launch("rigl_count/scan");
}

extern "C" int slk_rigl_finish(const slk_csr* W, float* values, int32_t* col_indices,
                               int32_t* row_nnz, const float* thr_dev, const float* G_approx,
                               int64_t ldg, const float* nrm_dY, const float* nrm_X,
                               const float* dY, const float* X, int64_t N, const void* info,
                               const int64_t* amb_off, void* amb_ws, int64_t amb_ws_bytes,
                               void* workspace, int64_t workspace_bytes, int64_t* removed,
                               void* stream) {
    using namespace slk;
    clear_error();
    if (int rc = validate_csr(W, "rigl_finish")) return rc;
    if (values != W->values || col_indices != W->col_indices || row_nnz != W->row_nnz)
        return fail(SLK_EINVAL, "rigl_finish: values/col_indices/row_nnz must be W's own arrays");
    if (W->ncols > kRiglMaxCols)
        return fail(SLK_EINVAL, "rigl_finish: ncols=" + std::to_string(W->ncols) +
                                    " exceeds the supported maximum " +
                                    std::to_string(kRiglMaxCols));
    if (removed == nullptr) return fail(SLK_EINVAL, "rigl_finish: NULL removed-slot counter");
    const int64_t M = W->nrows, K = W->ncols;
    if (M > 0 && (thr_dev == nullptr || G_approx == nullptr || ldg < K || nrm_dY == nullptr ||
                  nrm_X == nullptr || info == nullptr || amb_off == nullptr ||
                  (N > 0 && (dY == nullptr || X == nullptr))))
        return fail(SLK_EINVAL, "rigl_finish: NULL input or ldg < ncols");
    if (M > 0 && W->total_capacity > 0 &&
        (workspace == nullptr || workspace_bytes < W->total_capacity * 8))
        return fail(SLK_EINVAL, "rigl_finish: workspace smaller than slk_drop_grow_workspace_bytes");
    if (amb_ws_bytes < 0 || (amb_ws_bytes > 0 && amb_ws == nullptr))
        return fail(SLK_EINVAL, "rigl_finish: bad undecided-column workspace");
    hipStream_t st = as_stream(stream);
    unsigned long long* removed_u = reinterpret_cast<unsigned long long*>(removed);
    hipLaunchKernelGGL(rigl_clear_kernel, dim3(1), dim3(1), 0, st, removed_u);
    if (int rc = check_launch("rigl_finish")) return rc;
    if (M == 0 || W->total_capacity == 0) return SLK_OK;
    // undecided columns: int32 columns, then as many uint32 keys; sized by the
    // caller from slk_rigl_count's total (8 bytes per column)
    const int64_t n_amb_max = amb_ws_bytes / 8;
    int32_t* amb_col = static_cast<int32_t*>(amb_ws);
    uint32_t* amb_key = reinterpret_cast<uint32_t*>(amb_col + n_amb_max);
    const int64_t Kw = ceil_div(K, 32) > 0 ? ceil_div(K, 32) : 1;
    const bool v4 = N % 4 == 0 && reinterpret_cast<uintptr_t>(dY) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(X) % 16 == 0;
    const int64_t words = ((3 * Kw + 3) & ~int64_t{3}) + (v4 && N <= kStageMaxN ? N : 0);
    const size_t lds = static_cast<size_t>(words) * 4;
    int32_t* stage_col = static_cast<int32_t*>(workspace);
    float* stage_val = reinterpret_cast<float*>(stage_col + W->total_capacity);
    if (v4) {
        hipLaunchKernelGGL(rigl_finish_kernel<true>, dim3(static_cast<unsigned>(M)),
                           dim3(kRowThreads), lds, st, K, Kw, N, W->row_start, row_nnz, values,
                           col_indices, thr_dev, G_approx, ldg, nrm_dY, nrm_X, certified_c(N),
                           static_cast<const RowInfo*>(info), amb_off, amb_col, amb_key, dY, X,
                           stage_col, stage_val, removed_u);
    } else {
        hipLaunchKernelGGL(rigl_finish_kernel<false>, dim3(static_cast<unsigned>(M)),
                           dim3(kRowThreads), lds, st, K, Kw, N, W->row_start, row_nnz, values,
                           col_indices, thr_dev, G_approx, ldg, nrm_dY, nrm_X, certified_c(N),
                           static_cast<const RowInfo*>(info), amb_off, amb_col, amb_key, dY, X,
                           stage_col, stage_val, removed_u);
    }
    return check_launch("rigl_finish");
}
