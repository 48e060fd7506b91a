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
//            bf16 MFMA products per term, all accumulated into one running
//            fp32 sum per element over the whole of N (each MFMA adds 16
//            exact products to it). Beside it the kernel samples the running
//            sum's magnitude at the end of every chunk of 128 j and keeps
//            pm = the sum of those magnitudes, written as a byte code per
//            element.
//   bound    |G'[i,k] - G[i,k]| <= E[i,k] = c1·n_i·n_k + c2·pm[i,k] + δ
//            (certified_factors below, which derives each term): the matrix
//            cores' rounding (<= 2u per addition, any order and rounding
//            mode, relative to the running sum and the products added) and
//            the reference's own rounding (relative to its running sums) are
//            both bounded through the partial sums at the chunk ends, so pm
//            carries them; the dropped x_l y_l and r terms; a 1% margin; and
//            δ the flushing of subnormal bf16 parts and products
//            (2^-100·(1+n_i+n_k)). Σ_j |x_j y_j| <= n_i·n_k by Cauchy-Schwarz.
//            slk_rigl_mfma_probe runs the instruction on chosen operands, so
//            a test can check the 2u-per-addition model against exact sums.
//   count    per row: survivors as in the exact kernel; n_grow = min(dropped,
//            empty columns); T' = the n_grow-th largest |G'| of the empty
//            columns and E_max = the row's largest E_k, so the exact n_grow-th
//            largest |G| lies in [T' - E_max, T' + E_max]. A column with
//            |G'| - E_k above that is certainly grown, one with |G'| + E_k
//            below it certainly not; the rest are undecided. Counts them.
//   finish   per row, the undecided columns listed (ascending); over all
//            undecided (row, column) pairs, their exact G with the reference's
//            arithmetic (a wave per 64 pairs, both rows streamed through LDS);
//            per row, the n_grow - (certain) smallest exact keys ~bits(|G|)
//            among them (ties to the lower column) grown, and the row
//            rewritten exactly as the exact drop/grow kernel does.
//
// A row whose norms are not finite or too large (n_i·n_k beyond 2^120, where
// G could overflow) is an exact row: every empty column is undecided, and NaN
// columns are excluded from the grow count as in the exact kernel.
#include "common.hpp"
#include "row_rewrite.hpp"

#include <cmath>
#include <type_traits>

namespace slk {
namespace {

// ───────────────────────────── row norms ───────────────────────────────────

// nrm[r] >= ||A_r||_2 for the R rows of the row-major R x N matrix A; +inf if
// the row is not finite. One wave per row.
__global__ __launch_bounds__(256) void rigl_norm_kernel(const float* __restrict__ A, int64_t R,
                                                         const float* __restrict__ B, int64_t S,
                                                         int64_t N, float* __restrict__ nrm_a,
                                                         float* __restrict__ nrm_b) {
    // rows [0, R) of A, then rows [0, S) of B: one wave per row, each lane
    // four floats at a time (16-byte loads where N % 4 == 0), four float64
    // partial sums per lane
    int64_t r = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) >> 6;
    if (r >= R + S) return;
    const bool second = r >= R;
    if (second) r -= R;
    const float* p = (second ? B : A) + r * N;
    float* nrm = second ? nrm_b : nrm_a;
    const int lane = threadIdx.x & 63;
    double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;  // exact squares; the sum's relative
                                                   // error is below N·2^-53
    if (N % 4 == 0 && (reinterpret_cast<uintptr_t>(p) & 15) == 0) {
        const f32x4* p4 = reinterpret_cast<const f32x4*>(p);
        const int64_t n4 = N / 4;
        for (int64_t j = lane; j < n4; j += 64) {
            const f32x4 v = p4[j];
            s0 += static_cast<double>(v[0]) * v[0];
            s1 += static_cast<double>(v[1]) * v[1];
            s2 += static_cast<double>(v[2]) * v[2];
            s3 += static_cast<double>(v[3]) * v[3];
        }
    } else {
        for (int64_t j = lane; j < N; j += 64) {
            const double v = p[j];
            s0 += v * v;
        }
    }
    double s = (s0 + s1) + (s2 + s3);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if (lane == 0) {
        const double n = sqrt(s) * (1.0 + 0x1p-30);
        nrm[r] = (s == s && s < 0x1p1000) ? __double2float_ru(n) : __builtin_inff();
    }
}

// ───────────────────────────── approximate G ───────────────────────────────

constexpr int kATI = 128;       // output tile rows (rows of dY)
constexpr int kATK = 128;       // output tile columns (rows of X)
constexpr int kAJ = 32;         // j per LDS stage: two MFMA k-steps of 16
constexpr int kAChunk = 128;    // j per matrix-core partial sum
constexpr int kAThreads = 256;  // 4 waves, 2 x 2, each 64 x 64 of the tile
constexpr int kAGroup = 8;      // tile rows per group of the tile order

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// s_waitcnt operand: vector-memory count <= n and no LDS or scalar access
// outstanding (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt
// 11:8)
constexpr int kVmcntLe(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4); }
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

// The partial-sum code of an element: pm = the sum of |G' partial sums| at
// the chunk ends, stored as the exponent code c with pm < 2^(c - 127)
// (c = biased exponent + 1, at most 255 = +inf for a non-finite pm).
__device__ __forceinline__ uint32_t partial_code(float pm) {
    return min(((__float_as_uint(pm) >> 23) & 0xffu) + 1u, 255u);
}
// 2^(c - 127) for c in [1, 255] (255: +inf)
__device__ __forceinline__ float partial_bound(uint32_t c) { return __uint_as_float(c << 23); }

// Stages per row: N rounded up to whole chunks (zero beyond N).
inline int64_t approx_stages(int64_t N) { return ceil_div(N, kAChunk) * (kAChunk / kAJ); }

// G'[i0 + 128, k0 + 128 tile] = Σ (x_h·y_h + x_h·y_l + x_l·y_h), where
// x = dY row i, y = X row k: one fp32 matrix-core sum of the three products
// of every term, and beside it pm = the sum of the running sum's magnitudes
// at the ends of its chunks of kAChunk j, written as the element's partial-sum
// code. The bound uses pm twice: each MFMA's rounding is relative to its
// running sum, and so is each addition of the reference's own sum.
// Four waves in a 2 x 2 grid, each 64 rows x 64 columns (2 x 2 blocks of
// 32 x 32): per k-step of 16 j a wave reads four A and four B fragments from
// LDS for twelve MFMAs (waves of 32 x 64 read six for six). Two workgroups
// per CU (72 KiB of LDS each), so one workgroup's barrier waits are covered
// by the other's MFMAs. (A 256 x 128 tile of eight such waves, one workgroup
// per CU, measured the same: 6.75 against 6.70 ms at 16384^2 x 4096.)
__global__ __launch_bounds__(kAThreads) void rigl_approx_kernel(int64_t M, int64_t K, int64_t nst,
                                                                const uint16_t* __restrict__ PA,
                                                                const uint16_t* __restrict__ PB,
                                                                float* __restrict__ G,
                                                                uint8_t* __restrict__ Gc) {
    __shared__ __align__(16) unsigned char sA[2][kATI * kALdsRow];
    __shared__ __align__(16) unsigned char sB[2][kATK * kALdsRow];

    // grouped, XCD-contiguous tile order: consecutive tiles share dY and X rows
    const int64_t nTi = ceil_div(M, kATI), nTk = ceil_div(K, kATK);
    const int64_t L = xcd_logical_block(blockIdx.x, gridDim.x);
    const int64_t grp = L / (kAGroup * nTk);
    const int64_t first = grp * kAGroup;
    const int64_t gsize = nTi - first < kAGroup ? nTi - first : kAGroup;
    const int64_t in_grp = L - grp * kAGroup * nTk;
    const int64_t i0 = (first + in_grp % gsize) * kATI;
    const int64_t k0 = (in_grp / gsize) * kATK;

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wv = t >> 6;
    const int wm = wv >> 1, wn = wv & 1;  // rows wm*64 .. +64, columns wn*64 .. +64
    // staging: thread t moves bytes [64(t&1), +64) of staged row t/2 of A and of B
    constexpr int kPA = kAStageBytes / 16 * kATI / kAThreads;  // 16-byte pieces per thread
    constexpr int kPB = kAStageBytes / 16 * kATK / kAThreads;
    static_assert(kPA == 4 && kPB == 4, "staging map below");
    const int lra = t >> 1, lha = (t & 1) * 64;
    const int lrb = t >> 1, lhb = (t & 1) * 64;
    const unsigned char* ga = reinterpret_cast<const unsigned char*>(
        PA + (i0 + lra < M ? i0 + lra : M - 1) * nst * (2 * kAJ)) + lha;
    const unsigned char* gb = reinterpret_cast<const unsigned char*>(
        PB + (k0 + lrb < K ? k0 + lrb : K - 1) * nst * (2 * kAJ)) + lhb;

    // [row block][column block]: the running sums, and the sum of their
    // magnitudes at the chunk ends (the partial sums the bound uses)
    f32x16 acc[2][2], pm[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][b][r] = pm[a][b][r] = 0.0f;

    // Pipeline: stage st+2's loads are issued while stage st is computed from
    // LDS buffer st&1; stage st+1 (loaded during stage st-1) is written into
    // the other buffer after this stage's MFMAs; one barrier per stage. nst is
    // a whole number of chunks (the split pads with zero stages), so every
    // load and LDS write is unconditional: past the end a stage reloads the
    // last one, unused. (A conditional load would leave the wait before the
    // LDS write covering the newer loads as well.)
    f32x4 ra[2][kPA], rb[2][kPB];
    auto fetch = [&](int reg, int64_t st) {
        const unsigned char* pa = ga + st * kAStageBytes;
        const unsigned char* pb = gb + st * kAStageBytes;
#pragma unroll
        for (int q = 0; q < kPA; ++q) ra[reg][q] = *reinterpret_cast<const f32x4*>(pa + 16 * q);
#pragma unroll
        for (int q = 0; q < kPB; ++q) rb[reg][q] = *reinterpret_cast<const f32x4*>(pb + 16 * q);
    };
    const int sta = lra * kALdsRow + lha, stb = lrb * kALdsRow + lhb;
    auto stage_to_lds = [&](int reg, int b) {
#pragma unroll
        for (int q = 0; q < kPA; ++q)
            *reinterpret_cast<f32x4*>(&sA[b][sta + 16 * q]) = ra[reg][q];
#pragma unroll
        for (int q = 0; q < kPB; ++q)
            *reinterpret_cast<f32x4*>(&sB[b][stb + 16 * q]) = rb[reg][q];
    };
    const int half = 16 * (lane >> 5);
    const int ra0 = (wm * 64 + (lane & 31)) * kALdsRow + half;
    const int rb0 = (wn * 64 + (lane & 31)) * kALdsRow + half;
    // stage st lives in register set st & 1 and LDS buffer st & 1; the two
    // parities are unrolled so both indexes are compile-time constants.
    auto stage = [&](auto R, int64_t st) {
        constexpr int reg = decltype(R)::value;
        fetch(reg, st + 2 < nst ? st + 2 : nst - 1);  // set of stage st: already in LDS
        const unsigned char* la = sA[reg];
        const unsigned char* lb = sB[reg];
#pragma unroll
        for (int s = 0; s < kAJ / 16; ++s) {
            bf16x8 af[2][2], bf[2][2];  // [block][high, low]
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const int o = p * (kAStageBytes / 2) + 32 * s;
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    af[b][p] = *reinterpret_cast<const bf16x8*>(la + ra0 + b * 32 * kALdsRow + o);
                    bf[b][p] = *reinterpret_cast<const bf16x8*>(lb + rb0 + b * 32 * kALdsRow + o);
                }
            }
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[a][0], bf[b][0], acc[a][b], 0, 0, 0);
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[a][0], bf[b][1], acc[a][b], 0, 0, 0);
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[a][1], bf[b][0], acc[a][b], 0, 0, 0);
        }
        // stage st+1 into the other buffer (its last readers, stage st-1,
        // passed the previous barrier)
        stage_to_lds(reg ^ 1, reg ^ 1);
        __syncthreads();
    };
    static_assert((kAChunk / kAJ) % 2 == 0, "whole pairs of stages per chunk below");
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    if (nst > 0) {  // workgroup-uniform
        fetch(0, 0);
        fetch(1, 1);
        stage_to_lds(0, 0);
        __syncthreads();
        for (int64_t c0 = 0; c0 < nst; c0 += kAChunk / kAJ) {
            for (int k = 0; k < kAChunk / kAJ; k += 2) {
                stage(I0{}, c0 + k);
                stage(I1{}, c0 + k + 1);
            }
            // a chunk done: the running sum's magnitude to pm
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int r = 0; r < 16; ++r) pm[a][b][r] = pm[a][b][r] + fabsf(acc[a][b][r]);
        }
    }
    // lane l, register 4g + q of a 32x32 block: row 8g + 4(l/32) + q, column l % 32
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const int64_t col = k0 + wn * 64 + b * 32 + (lane & 31);
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = i0 + wm * 64 + a * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row < M && col < K) {
                    G[row * K + col] = acc[a][b][r];
                    Gc[row * K + col] = static_cast<uint8_t>(partial_code(pm[a][b][r]));
                }
            }
    }
}

// The same G' and codes from larger tiles fed by direct loads into LDS.
// A workgroup of 8 waves (4 x 2, each 64 x 64 as above) takes a 256 x 128
// tile, so every staged B row serves twice the rows of A. Stages reach LDS by
// global_load_lds_dwordx4 (no registers, no LDS stores) in a ring of three,
// issued two stages ahead, with one barrier per stage. A staged row is its
// 128 bytes unpadded: piece c (16 bytes) of row r sits at slot r·8 + (c ^
// ((r >> 1) & 7)), so the 16 lanes of an LDS pass, reading one piece of 16
// consecutive rows, hit 16 distinct slot columns (all 64 banks once). Each
// element's MFMA sequence (per k-step: hi·hi, hi·lo, lo·hi; k-steps in j
// order; |running sum| added to pm at every chunk end) is the 128 x 128
// kernel's, so G' and the codes are bit for bit the same.
constexpr int kGTI = 256;                      // output tile rows (rows of dY)
constexpr int kGTK = 128;                      // output tile columns (rows of X)
constexpr int kGThreads = 512;                 // 8 waves
constexpr int kGBufs = 3;                      // LDS ring of stages
// Tile rows per group of the tile order: an XCD's 32 concurrent tiles are then
// 4 tile rows x 8 tile columns, 256 KiB of distinct operands per stage
// against 320 KiB at 8 x 4 (C5: 5.75 -> 5.37 ms; 2: 5.42, 16: 5.80).
constexpr int kGGroup = 4;
constexpr int kGPerA = kGTI * 8 / 64 / 8;      // A loads per wave and stage (64 pieces each)
constexpr int kGPerB = kGTK * 8 / 64 / 8;      // B loads per wave and stage
static_assert(kAStageBytes == 128, "eight 16-byte pieces per staged row");

__device__ __forceinline__ int g_slot(int r, int c) { return r * 8 + (c ^ ((r >> 1) & 7)); }

__global__ __launch_bounds__(kGThreads) void rigl_approx_dma_kernel(
    int64_t M, int64_t K, int64_t nst, const uint16_t* __restrict__ PA,
    const uint16_t* __restrict__ PB, float* __restrict__ G, uint8_t* __restrict__ Gc) {
    // one LDS array (A rows, then B rows, per ring buffer): 3 x 48 KiB
    __shared__ __align__(16) unsigned char sAB[kGBufs][(kGTI + kGTK) * kAStageBytes];

    const int64_t nTi = ceil_div(M, kGTI), nTk = ceil_div(K, kGTK);
    const int64_t L = xcd_logical_block(blockIdx.x, gridDim.x);
    const int64_t grp = L / (kGGroup * nTk);
    const int64_t first = grp * kGGroup;
    const int64_t gsize = nTi - first < kGGroup ? nTi - first : kGGroup;
    const int64_t in_grp = L - grp * kGGroup * nTk;
    const int64_t i0 = (first + in_grp % gsize) * kGTI;
    const int64_t k0 = (in_grp / gsize) * kGTK;

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wv >> 1, wn = wv & 1;  // rows wm*64 .. +64, columns wn*64 .. +64

    // Staging. Load i of a stage fills slots [64 i, 64 i + 64) of its matrix's
    // buffer: rows 8 i .. 8 i + 7; lane l fetches piece (l mod 8) ^ swizzle of
    // row 8 i + l / 8, so it lands at its swizzled slot. Wave wv issues loads
    // wv, wv + 8, ...: per lane a fixed 32-bit offset from a scalar row base
    // (rows past the matrix clamped to its last row), plus 128 bytes a stage.
    const char* baseA[kGPerA];
    const char* baseB[kGPerB];
    uint32_t offA[kGPerA], offB[kGPerB];
    auto plan = [&](const uint16_t* P, int64_t R, int64_t r0, int i, const char*& base,
                    uint32_t& off) {
        const int64_t rb = min(r0 + 8 * i, R - 1);
        const int64_t r = min(r0 + 8 * i + lane / 8, R - 1);
        const int rr = 8 * i + lane / 8;  // the row inside the tile
        const int c = (lane & 7) ^ ((rr >> 1) & 7);
        base = reinterpret_cast<const char*>(P) + rb * nst * kAStageBytes;
        off = static_cast<uint32_t>((r - rb) * nst * kAStageBytes + 16 * c);
    };
#pragma unroll
    for (int q = 0; q < kGPerA; ++q) plan(PA, M, i0, wv + 8 * q, baseA[q], offA[q]);
#pragma unroll
    for (int q = 0; q < kGPerB; ++q) plan(PB, K, k0, wv + 8 * q, baseB[q], offB[q]);
    auto issue = [&](int buf, int64_t st) {
        const int64_t so = st * kAStageBytes;
#pragma unroll
        for (int q = 0; q < kGPerA; ++q)
            __builtin_amdgcn_global_load_lds(baseA[q] + so + offA[q],
                                             &sAB[buf][64 * 16 * (wv + 8 * q)], 16, 0, 0);
#pragma unroll
        for (int q = 0; q < kGPerB; ++q)
            __builtin_amdgcn_global_load_lds(baseB[q] + so + offB[q],
                                             &sAB[buf][kGTI * kAStageBytes + 64 * 16 * (wv + 8 * q)],
                                             16, 0, 0);
    };

    f32x16 acc[2][2], pm[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][b][r] = pm[a][b][r] = 0.0f;

    const int half = lane >> 5;
    const int rA = wm * 64 + (lane & 31), rB = wn * 64 + (lane & 31);
    auto frag = [&](const unsigned char* lds, int r, int c) {
        return *reinterpret_cast<const bf16x8*>(lds + 16 * g_slot(r, c));
    };
    constexpr int kLoads = kGPerA + kGPerB;  // this wave's direct loads per stage
    bf16x8 af[kAJ / 16][2][2], bf[kAJ / 16][2][2];  // [k-step][block][high, low]
    auto reads = [&](const unsigned char* buf, int ks) {
        const unsigned char* lb = buf + kGTI * kAStageBytes;
#pragma unroll
        for (int p = 0; p < 2; ++p)
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int c = 4 * p + 2 * ks + half;
                af[ks][b][p] = frag(buf, rA + 32 * b, c);
                bf[ks][b][p] = frag(lb, rB + 32 * b, c);
            }
    };
    auto mfmas = [&](int ks, int pa, int pb) {
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b)
                acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ks][a][pa], bf[ks][b][pb],
                                                                     acc[a][b], 0, 0, 0);
    };
    static_assert(kAJ / 16 == 2, "two k-steps per stage below");
    // Stage st reads ring buffer st mod 3 and loads stage st + 2 into buffer
    // (st + 2) mod 3. The loop is unrolled by three so both indexes are
    // compile-time constants: the compiler then sees that the reads and the
    // direct loads touch different buffers (with run-time indexes it makes
    // every read wait for the loads just issued).
    //
    // The workgroup barrier sits in the middle of a stage, after its last
    // reads, so that the next stage's first reads go out right after it and
    // land while this stage's last twelve MFMAs run: per stage, k-step 0's
    // fragments (read in the previous stage) feed its high x high MFMAs;
    // k-step 1's reads and stage st+2's direct loads go out; the rest of
    // k-step 0; then this wave's loads of stage st+1 have landed (loads
    // complete in order; stage st+2's may still be in flight) and its reads
    // of stage st have returned, and the barrier: every wave's loads of stage
    // st+1 are in LDS and buffer st is free for stage st+3's loads; stage
    // st+1's k-step 0 reads; k-step 1's MFMAs. A bare s_barrier: the
    // workgroup fence of __syncthreads() would also wait for stage st+2's
    // loads; the memory clobber keeps the compiler from moving LDS accesses
    // across it, and scheduling barriers keep it from sinking the reads to
    // their uses. At most 12 LDS reads are outstanding (the wait counter
    // tracks 15). The last two stages load the last stage again (into the
    // buffer that is free), so every stage waits for the same count and
    // passes the barrier, with no branch for the compiler's wait tracking to
    // merge (at a branch join it waits for every outstanding read). Each
    // element's MFMA order is unchanged: per k-step hi·hi, hi·lo, lo·hi,
    // k-steps in j order.
    auto stage = [&](auto I, int64_t st) {
        constexpr int buf = decltype(I)::value;
        mfmas(0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        reads(sAB[buf], 1);
        issue((buf + 2) % kGBufs, st + 2 < nst ? st + 2 : nst - 1);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(0, 0, 1);
        mfmas(0, 1, 0);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(kVmcntLe(kLoads));
        asm volatile("s_barrier" ::: "memory");
        reads(sAB[(buf + 1) % kGBufs], 0);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(1, 0, 0);
        mfmas(1, 0, 1);
        mfmas(1, 1, 0);
        if ((st + 1) % (kAChunk / kAJ) == 0) {  // a chunk done: |running sum| to pm
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int r = 0; r < 16; ++r) pm[a][b][r] = pm[a][b][r] + fabsf(acc[a][b][r]);
        }
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    using B2 = std::integral_constant<int, 2>;
    if (nst > 0) {
        issue(0, 0);
        issue(1, nst > 1 ? 1 : 0);
        // stage 0's loads landed (stage 1's may be in flight), then its k-step 0 reads
        __builtin_amdgcn_s_waitcnt(kVmcntLe(kLoads));
        asm volatile("s_barrier" ::: "memory");
        reads(sAB[0], 0);
        int64_t st = 0;
        for (; st + 3 <= nst; st += 3) {
            stage(B0{}, st);
            stage(B1{}, st + 1);
            stage(B2{}, st + 2);
        }
        if (st < nst) stage(B0{}, st);
        if (st + 1 < nst) stage(B1{}, st + 1);
        __builtin_amdgcn_s_waitcnt(0);  // no direct load still writing LDS when the waves end
    }
    // lane l, register 4g + q of a 32x32 block: row 8g + 4(l/32) + q, column l % 32
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const int64_t col = k0 + wn * 64 + b * 32 + (lane & 31);
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = i0 + wm * 64 + a * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row < M && col < K) {
                    G[row * K + col] = acc[a][b][r];
                    Gc[row * K + col] = static_cast<uint8_t>(partial_code(pm[a][b][r]));
                }
            }
    }
}

// ───────────────────────────── certified selection ─────────────────────────

struct RowInfo {
    int32_t n_grow;  // grows of the row (exact rows: decided in finish)
    int32_t n_in;    // columns certainly grown
    float t_in;      // a column is certainly grown if its lower bound exceeds this
    float t_out;     // a column is certainly not grown if its upper bound is below this
    int32_t flags;   // kRowExact, kRowKeep
    int32_t n_keep;
    float cni;       // an upper bound of c_N·n_i
    float delta;     // the absolute part of the bound, for every column of the row
};
constexpr int32_t kRowExact = 1;  // every empty column undecided
constexpr int32_t kRowKeep = 2;   // nothing to grow: the row is left as it is
static_assert(sizeof(RowInfo) == 32, "RowInfo is 32 bytes");

// Float bounds, each rounded outward by a relative 2^-20 (every float
// operation rounds by at most 2^-24) and an absolute 2^-120 (subnormals).
__device__ __forceinline__ float up_(float x) { return x * (1.0f + 0x1p-20f) + 0x1p-120f; }
__device__ __forceinline__ float dn_(float x) { return x * (1.0f - 0x1p-20f) - 0x1p-120f; }
constexpr float kNormCap = 0x1p60f;  // norms above this make the row exact

// The per-column error E_k >= c_N·n_i·n_k + the absolute part (delta =
// up(2^-100·(1 + n_i + max n_k))) + c2·(the element's sum of |partial
// sums|): two fmas (c2·2^(code - 127) is exact), each rounding by at most u,
// then raised by 2^-20 relative (> 2u) and 2^-120 absolute.
__device__ __forceinline__ float col_err(float cni, float nk, float delta, float c2,
                                         uint32_t code) {
    return fmaf(fmaf(cni, nk, fmaf(c2, partial_bound(code), delta)), 1.0f + 0x1p-20f, 0x1p-120f);
}

// A column's class for the row's thresholds t_in / t_out (kGrowIn: |G| is
// certainly above the n_grow-th largest; kGrowOut: certainly below;
// otherwise undecided; a NaN |G'| is undecided). E_k as in col_err but
// unraised; each sum with it is raised by 2^-20 relative (covering its own
// rounding and E_k's two) and 2^-120 absolute before the compare.
constexpr int kGrowOut = 0, kGrowIn = 1, kGrowUndecided = 2;
__device__ __forceinline__ int classify_col(float a, float cni, float nk, float delta, float c2,
                                            uint32_t code, float t_in, float t_out) {
    const float ek = fmaf(cni, nk, fmaf(c2, partial_bound(code), delta));
    if (a > fmaf(t_in + ek, 1.0f + 0x1p-20f, 0x1p-120f)) return kGrowIn;
    return fmaf(a + ek, 1.0f + 0x1p-20f, 0x1p-120f) < t_out ? kGrowOut : kGrowUndecided;
}

// Largest-first selection key of a non-negative float.
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
        const int64_t n_pad = ceil_div(n, kRowThreads) * kRowThreads;  // uniform trip count
        for (int64_t e = t; e < n_pad; e += kRowThreads) {
            uint32_t u = 0;
            const bool ok = e < n && cand(e, u) && (pass == 0 || (u >> (shift + 8)) == prefix);
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
    return prefix;
}

constexpr int64_t kStageMaxK = 16384;  // G' rows up to this length are staged in LDS
constexpr int kColBlock = 8;            // float4 loads per thread in flight per block

// Calls f(c, g, nk, code) for every column c < K of a row: g = G'[c] of the
// row, nk = nrm_c[c], code = the row's partial-sum code of c. V4 (K % 4 == 0,
// 16-byte aligned rows, 4-byte aligned codes): each thread issues kColBlock
// loads of each before using any, so a row streams with one memory latency
// per block instead of one per column.
template <bool V4, class F>
__device__ __forceinline__ void for_each_col(const float* __restrict__ g_row,
                                             const float* __restrict__ nrm_c,
                                             const uint8_t* __restrict__ code_row, int64_t K,
                                             F f) {
    const int t = threadIdx.x;
    if (V4) {
        constexpr int64_t step = int64_t{kRowThreads} * 4 * kColBlock;
        for (int64_t base = 0; base < K; base += step) {
            f32x4 g[kColBlock], n[kColBlock];
            uint32_t cw[kColBlock];
#pragma unroll
            for (int u = 0; u < kColBlock; ++u) {  // no branch: all loads issued at once
                const int64_t c = base + 4 * (t + int64_t{kRowThreads} * u);
                const int64_t cl = c < K ? c : K - 4;  // in bounds, unused past K
                g[u] = *reinterpret_cast<const f32x4*>(g_row + cl);
                n[u] = *reinterpret_cast<const f32x4*>(nrm_c + cl);
                cw[u] = *reinterpret_cast<const uint32_t*>(code_row + cl);
            }
#pragma unroll
            for (int u = 0; u < kColBlock; ++u) {
                const int64_t c = base + 4 * (t + int64_t{kRowThreads} * u);
                if (c < K) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) f(c + e, g[u][e], n[u][e], (cw[u] >> (8 * e)) & 255u);
                }
            }
        }
    } else {
        for (int64_t c = t; c < K; c += kRowThreads) f(c, g_row[c], nrm_c[c], uint32_t{code_row[c]});
    }
}

constexpr int kCountList = 2048;  // keys of the selected top bin listed in LDS (8 KiB)

// rigl_count_kernel with the row's |G'| in registers, and the list pass
// (rigl_list_kernel) folded in: thread t owns columns 16(t + 256v) + e
// (v < U/4, e < 16), so the radix passes read no memory, and the classes
// found for the counts are the ones listed, with no second pass over G'. For
// K <= 1024·U, K % 16 == 0, 16-byte aligned rows of G', codes and nrm_c.
// Same counts, thresholds and flags as rigl_count_kernel (the select visits
// the same candidates with the same keys), and the same lists as
// rigl_list_kernel: the row's undecided columns ascending at its range of the
// pair list (reserved with one atomic add on the running total amb_off[M],
// which the caller zeroes; amb_off[i] = the row's start, amb_off[M + 1 + i]
// its count; pairs past amb_cap are not written), its certain grows
// ascending in its staging slots.
template <int U>
__global__ __launch_bounds__(kRowThreads) void rigl_count_reg_kernel(
    int64_t K, int64_t M, const int32_t* __restrict__ row_start,
    const int32_t* __restrict__ row_nnz, const float* __restrict__ values,
    const int32_t* __restrict__ cols, const float* __restrict__ thr_ptr,
    const float* __restrict__ Gp, int64_t ldg, const uint8_t* __restrict__ Gc,
    const float* __restrict__ nrm_r, const float* __restrict__ nrm_c, float c_bound, float c2,
    RowInfo* __restrict__ info, int64_t* __restrict__ amb_off, int32_t* __restrict__ amb_col,
    uint32_t* __restrict__ amb_key, int64_t amb_cap, int32_t* __restrict__ stage_col) {
    constexpr int kGroups = U / 4;  // groups of 16 consecutive columns per thread
    static_assert(kGroups >= 1 && kGroups <= 4, "four 16-bit counts per int64");
    __shared__ uint32_t keep[U * kRowThreads * 4 / 32];
    __shared__ int64_t tmp[kRowThreads];
    __shared__ uint32_t hist[2048];
    __shared__ uint32_t lst[kCountList];
    __shared__ uint32_t s_digit;
    __shared__ int64_t s_below;
    __shared__ unsigned long long s_best;
    __shared__ uint32_t s_nmax, s_cmax;
    __shared__ int64_t s_base;

    const int64_t i = blockIdx.x;
    const int t = threadIdx.x;
    // thread t owns the 16 consecutive columns 16(t + 256v) .. + 15 for each
    // v < U/4: register u holds the four columns col_of(u) .. + 3
    auto col_of = [&](int u) -> int64_t {
        return 16 * (t + int64_t{kRowThreads} * (u / 4)) + 4 * (u % 4);
    };
    RowInfo ri{};
    const int32_t n_live = row_nnz[i];
    auto keep_row = [&]() {  // nothing to grow: nothing listed
        if (t == 0) {
            ri.flags = kRowKeep;
            info[i] = ri;
            amb_off[i] = 0;
            amb_off[M + 1 + i] = 0;
        }
    };
    if (n_live <= 0) return keep_row();  // the reference skips empty rows
    const int32_t start = row_start[i];
    for (int w = t; w < U * kRowThreads * 4 / 32; w += kRowThreads) keep[w] = 0;
    if (t == 0) s_nmax = s_cmax = 0;
    __syncthreads();
    const int64_t n_keep = mark_survivors(values, cols, start, n_live, thr_ptr[0], keep, tmp,
                                          &s_best);
    const int64_t n_drop = n_live - n_keep;
    ri.n_keep = static_cast<int32_t>(n_keep);
    if (n_drop == 0) return keep_row();
    const int64_t n_empty = K - n_keep;
    const float ni = nrm_r[i];
    const float* g_row = Gp + i * ldg;

    // Lists the row (bit 4u + e of a mask is column col_of(u) + e): the
    // undecided columns `amb` and, for a certified row, the certain grows
    // `in`, in ascending column order, i.e. in the order (v, t, u % 4, e).
    // Per-thread counts of each group v, 16 bits apiece in one int64, go
    // through one workgroup scan per list, which gives every thread its start
    // in every group.
    auto emit = [&](int32_t flags, uint64_t amb, uint64_t in) {
        int64_t pa = 0, pi = 0;
#pragma unroll
        for (int v = 0; v < kGroups; ++v) {
            pa |= static_cast<int64_t>(__popcll((amb >> (16 * v)) & 0xFFFFull)) << (16 * v);
            pi |= static_cast<int64_t>(__popcll((in >> (16 * v)) & 0xFFFFull)) << (16 * v);
        }
        const int64_t xa = block_inclusive_scan(pa, tmp) - pa;
        const int64_t ta = tmp[kRowThreads - 1];
        const int64_t xi = block_inclusive_scan(pi, tmp) - pi;
        const int64_t ti = tmp[kRowThreads - 1];
        int64_t n_amb = 0, n_in = 0;
#pragma unroll
        for (int v = 0; v < kGroups; ++v) {
            n_amb += (ta >> (16 * v)) & 0xFFFF;
            n_in += (ti >> (16 * v)) & 0xFFFF;
        }
        if (t == 0) {
            const int64_t base =
                n_amb > 0 ? static_cast<int64_t>(atomicAdd(
                                reinterpret_cast<unsigned long long*>(amb_off + M),
                                static_cast<unsigned long long>(n_amb)))
                          : 0;
            s_base = base;
            ri.flags = flags;
            ri.n_in = static_cast<int32_t>(n_in);
            info[i] = ri;
            amb_off[i] = base;
            amb_off[M + 1 + i] = n_amb;
        }
        __syncthreads();
        // field v of cum(x) << 16: the counts of the groups before v (each
        // field sum stays below 2^16: at most 16384 columns a row)
        auto cum = [](int64_t x) { return x + (x << 16) + (x << 32) + (x << 48); };
        const int64_t sa = (cum(ta) << 16) + xa, si = (cum(ti) << 16) + xi;
        // column of bit q: 16(t + 256(q / 16)) + q % 16; its position: its
        // group's start for this thread + the earlier bits of its group
        auto place = [&](uint64_t m, int64_t starts, auto put) {
            const uint64_t all = m;
            while (m) {
                const int q = __builtin_ctzll(m);
                m &= m - 1;
                const int v = q >> 4;
                const uint64_t below = all & ((1ull << q) - 1ull) & (0xFFFFull << (16 * v));
                put(((starts >> (16 * v)) & 0xFFFF) + __popcll(below),
                    16 * (t + int64_t{kRowThreads} * v) + (q & 15));
            }
        };
        place(amb, sa, [&](int64_t pos, int64_t c) {
            const int64_t at = s_base + pos;
            if (at < amb_cap) {
                amb_col[at] = static_cast<int32_t>(c);
                amb_key[at] = static_cast<uint32_t>(i);
            }
        });
        place(in, si, [&](int64_t pos, int64_t c) {
            if (pos < n_live) stage_col[start + pos] = static_cast<int32_t>(c);
        });
    };

    // the row's |G'| and empty-column mask (bit 4u + e) (every load issued
    // before the first use: clamped addresses instead of branches, the
    // columns past K masked out of `cand`); the norms are read after the
    // select, so the two sets of 4U registers are never live together
    // (held as selection keys, ~bits(|g|), one register per column: |g|
    // is ~key's float, so the keys and the values are never both live)
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 a[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t c = col_of(u);
        a[u] = *reinterpret_cast<const u32x4*>(g_row + (c < K ? c : K - 4));
    }
    // the columns' partial-sum codes (one 16-byte load per 16 columns: K %
    // 16 == 0 for this kernel; past K a clamped load, its columns not
    // candidates), requested now so that they arrive while the select runs
    const uint8_t* c_row = Gc + i * K;
    typedef uint32_t u32x4c __attribute__((ext_vector_type(4)));
    u32x4c cw4[kGroups];
#pragma unroll
    for (int v = 0; v < kGroups; ++v) {
        const int64_t c = 16 * (t + int64_t{kRowThreads} * v);
        cw4[v] = *reinterpret_cast<const u32x4c*>(c_row + (c < K ? c : K - 16));
    }
    asm volatile("" ::: "memory");  // all these loads in flight before the first use
    uint64_t cand = 0;
    int64_t unbounded = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t c = col_of(u);
        const uint32_t kw = c < K ? keep[c >> 5] >> (c & 31) : 15u;  // c % 4 == 0: one word
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            a[u][e] = desc_key(fabsf(__uint_as_float(a[u][e])));
            if ((kw >> e) & 1u) continue;
            cand |= 1ull << (4 * u + e);
            if (!(__uint_as_float(~a[u][e]) <= 0x1p125f)) ++unbounded;
        }
    }
    block_inclusive_scan(unbounded, tmp);
    unbounded = tmp[kRowThreads - 1];
    if (unbounded > 0 || !(ni <= kNormCap)) return emit(kRowExact, cand, 0);
    const int64_t n_grow = n_drop < n_empty ? n_drop : n_empty;

    // T' = the n_grow-th largest |G'| of the empty columns: the n_grow-th
    // smallest key, by a radix select over the registers: the top 11 bits
    // (2048 bins), then the remaining 21 in passes of 8, 8 and 5 bits over
    // the keys that share the prefix found so far. Any exact selection gives
    // the same key.
    uint32_t prefix = 0;
    int64_t need = n_grow;
    auto pick = [&](int64_t h_of_thread_lo, int per) {
        // thread t holds bins [t*per, t*per + per); finds the bin of the
        // need-th key and the count below it
        const int64_t incl = block_inclusive_scan(h_of_thread_lo, tmp);
        if (incl - h_of_thread_lo < need && need <= incl) {
            int64_t run = incl - h_of_thread_lo;
            for (int q = 0; q < per; ++q) {
                const int64_t hq = hist[t * per + q];
                if (run + hq >= need) {
                    s_digit = static_cast<uint32_t>(t * per + q);
                    s_below = run;
                    break;
                }
                run += hq;
            }
        }
        __syncthreads();
    };
    {
        constexpr int kTopBits = 11, kTopBins = 1 << kTopBits, kPer = kTopBins / kRowThreads;
        for (int q = 0; q < kPer; ++q) hist[t * kPer + q] = 0;
        __syncthreads();
        // (one LDS atomic per key: 2048 bins spread a wave's keys enough that
        // hist_add's folding does not pay for its registers)
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if ((cand >> (4 * u + e)) & 1ull) atomicAdd(&hist[a[u][e] >> (32 - kTopBits)], 1u);
        __syncthreads();
        int64_t hs = 0;
        for (int q = 0; q < kPer; ++q) hs += hist[t * kPer + q];
        pick(hs, kPer);
        prefix = s_digit;
        need -= s_below;
        const int64_t n_bin = hist[prefix];
        __syncthreads();
        int shift = 32 - kTopBits;
        if (n_bin <= kCountList) {
            // the bin's keys listed in LDS (per-thread counts, one scan for
            // the offsets); the passes then read only them
            uint64_t in_bin = 0;
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if ((a[u][e] >> shift) == prefix) in_bin |= 1ull << (4 * u + e);
            in_bin &= cand;
            const int64_t mine = __popcll(in_bin);
            const int32_t at = static_cast<int32_t>(block_inclusive_scan(mine, tmp) - mine);
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int bit = 4 * u + e;
                    if ((in_bin >> bit) & 1ull)
                        lst[at + __popcll(in_bin & ((1ull << bit) - 1ull))] = a[u][e];
                }
            __syncthreads();
            auto pass = [&](int width) {
                hist[t] = 0;
                __syncthreads();
                for (int64_t e = t; e < n_bin; e += kRowThreads) {
                    const uint32_t key = lst[e];
                    if ((key >> shift) == prefix)
                        atomicAdd(&hist[(key >> (shift - width)) & ((1u << width) - 1u)], 1u);
                }
                shift -= width;
                __syncthreads();
                pick(hist[t], 1);
                prefix = (prefix << width) | s_digit;
                need -= s_below;
                __syncthreads();
            };
            pass(8);
            pass(8);
            pass(5);
        } else {  // a crowded bin: the passes over the registers
            auto pass = [&](int width) {
                hist[t] = 0;
                __syncthreads();
#pragma unroll
                for (int u = 0; u < U; ++u)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (((cand >> (4 * u + e)) & 1ull) && (a[u][e] >> shift) == prefix)
                            atomicAdd(&hist[(a[u][e] >> (shift - width)) & ((1u << width) - 1u)],
                                      1u);
                shift -= width;
                __syncthreads();
                pick(hist[t], 1);
                prefix = (prefix << width) | s_digit;
                need -= s_below;
                __syncthreads();
            };
            pass(8);
            pass(8);
            pass(5);
        }
    }
    const float Tp = __uint_as_float(~prefix);
    // the candidates' norms: the largest, and whether every bound exists
    f32x4 nr[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t c = col_of(u);
        nr[u] = *reinterpret_cast<const f32x4*>(nrm_c + (c < K ? c : K - 4));
    }
    asm volatile("" ::: "memory");  // all U loads in flight before the first use
    uint32_t nmax = 0, cmax = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t cw = cw4[u / 4][u % 4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (!((cand >> (4 * u + e)) & 1ull)) continue;
            if (!(nr[u][e] <= kNormCap)) ++unbounded;
            else nmax = max(nmax, __float_as_uint(nr[u][e]));
            cmax = max(cmax, (cw >> (8 * e)) & 255u);
        }
    }
    atomicMax(&s_nmax, nmax);
    atomicMax(&s_cmax, cmax);
    block_inclusive_scan(unbounded, tmp);
    if (tmp[kRowThreads - 1] > 0) return emit(kRowExact, cand, 0);
    const float nm = __uint_as_float(s_nmax);
    const float cni = up_(c_bound * ni);
    const float delta = up_(0x1p-100f * up_(1.0f + ni + nm));
    const float e_max = col_err(cni, nm, delta, c2, s_cmax);
    const float t_in = up_(Tp + e_max);
    const float t_out = dn_(Tp - e_max);
    uint64_t amb = 0, in = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t cw = cw4[u / 4][u % 4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (!((cand >> (4 * u + e)) & 1ull)) continue;
            const int cls = classify_col(__uint_as_float(~a[u][e]), cni, nr[u][e], delta, c2,
                                         (cw >> (8 * e)) & 255u, t_in, t_out);
            // (both ORs unconditional: with one under each class the compiler
            // merged them into a store to a class-indexed array in scratch)
            const uint64_t bit = 1ull << (4 * u + e);
            in |= cls == kGrowIn ? bit : 0ull;
            amb |= cls == kGrowUndecided ? bit : 0ull;
        }
    }
    ri.n_grow = static_cast<int32_t>(n_grow);
    ri.t_in = t_in;
    ri.t_out = t_out;
    ri.cni = cni;
    ri.delta = delta;
    emit(0, amb, in);
}

// Per row: survivors (as the exact kernel), then, over the empty columns,
// T' = the n_grow-th largest |G'| and E_max = the largest E_k. Every |G_k|
// lies below |G'_k| + E_max, so the n_grow-th largest |G| is at most
// t_in = T' + E_max; and |G'_k| >= T' holds for n_grow columns, so it is at
// least t_out = T' - E_max. A column is certainly grown if |G'_k| - E_k >
// t_in (at most n_grow - 1 of them: they all have |G'_k| > T'), certainly
// not grown if |G'_k| + E_k < t_out, and undecided otherwise (with the
// certain ones, at least n_grow: every column with |G'_k| >= T' is one).
template <bool STAGED, bool V4>
__global__ __launch_bounds__(kRowThreads) void rigl_count_kernel(
    int64_t K, int64_t Kw, const int32_t* __restrict__ row_start,
    const int32_t* __restrict__ row_nnz, const float* __restrict__ values,
    const int32_t* __restrict__ cols, const float* __restrict__ thr_ptr,
    const float* __restrict__ Gp, int64_t ldg, const uint8_t* __restrict__ Gc,
    const float* __restrict__ nrm_r, const float* __restrict__ nrm_c, float c_bound, float c2,
    RowInfo* __restrict__ info,
    int64_t* __restrict__ amb_count) {
    extern __shared__ uint32_t lds[];
    uint32_t* keep = lds;
    float* ag = reinterpret_cast<float*>(lds + Kw);  // |G'| of the row (STAGED)
    __shared__ int64_t tmp[kRowThreads];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_digit;
    __shared__ int64_t s_below;
    __shared__ unsigned long long s_best;
    __shared__ uint32_t s_nmax, s_cmax;

    const int64_t i = blockIdx.x;
    const int t = threadIdx.x;
    RowInfo ri{};
    const int32_t n_live = row_nnz[i];
    auto finish_row = [&](int32_t flags, int64_t n_amb) {
        if (t == 0) {
            ri.flags = flags;
            info[i] = ri;
            amb_count[i] = n_amb;
        }
    };
    if (n_live <= 0) return finish_row(kRowKeep, 0);  // the reference skips empty rows
    const int32_t start = row_start[i];
    for (int64_t w = t; w < Kw; w += kRowThreads) keep[w] = 0;
    if (t == 0) s_nmax = s_cmax = 0;
    __syncthreads();
    const int64_t n_keep = mark_survivors(values, cols, start, n_live, thr_ptr[0], keep, tmp,
                                          &s_best);
    const int64_t n_drop = n_live - n_keep;
    ri.n_keep = static_cast<int32_t>(n_keep);
    if (n_drop == 0) return finish_row(kRowKeep, 0);
    const int64_t n_empty = K - n_keep;
    const float ni = nrm_r[i];
    const float* g_row = Gp + i * ldg;

    // stage |G'|, the largest candidate norm, and whether every bound exists
    int64_t unbounded = 0;
    uint32_t nmax = 0, cmax = 0;
    const uint8_t* c_row = Gc + i * K;
    for_each_col<V4>(g_row, nrm_c, c_row, K, [&](int64_t c, float g, float nk, uint32_t code) {
        const float a = fabsf(g);
        if (STAGED) ag[c] = a;
        if (bit_of(keep, c)) return;
        if (!(nk <= kNormCap) || !(a <= 0x1p125f)) ++unbounded;
        else nmax = max(nmax, __float_as_uint(nk));
        cmax = max(cmax, code);
    });
    atomicMax(&s_nmax, nmax);
    atomicMax(&s_cmax, cmax);
    block_inclusive_scan(unbounded, tmp);
    unbounded = tmp[kRowThreads - 1];
    if (unbounded > 0 || !(ni <= kNormCap)) return finish_row(kRowExact, n_empty);
    const float nm = __uint_as_float(s_nmax);
    const int64_t n_grow = n_drop < n_empty ? n_drop : n_empty;
    auto absg = [&](int64_t c) -> float { return STAGED ? ag[c] : fabsf(g_row[c]); };
    auto key_of = [&](int64_t c, uint32_t& key) -> bool {
        if (bit_of(keep, c)) return false;
        key = desc_key(absg(c));
        return true;
    };
    const float Tp = __uint_as_float(~kth_smallest_key(key_of, K, n_grow, hist, &s_digit,
                                                       &s_below, tmp));
    const float cni = up_(c_bound * ni);
    const float delta = up_(0x1p-100f * up_(1.0f + ni + nm));
    const float e_max = col_err(cni, nm, delta, c2, s_cmax);
    const float t_in = up_(Tp + e_max);
    const float t_out = dn_(Tp - e_max);
    int64_t n_in = 0, n_amb = 0;
    for_each_col<V4>(g_row, nrm_c, c_row, K, [&](int64_t c, float g, float nk, uint32_t code) {
        if (bit_of(keep, c)) return;
        const int cls = classify_col(fabsf(g), cni, nk, delta, c2, code, t_in, t_out);
        n_in += cls == kGrowIn;
        n_amb += cls == kGrowUndecided;
    });
    block_inclusive_scan(n_in, tmp);
    n_in = tmp[kRowThreads - 1];
    block_inclusive_scan(n_amb, tmp);
    n_amb = tmp[kRowThreads - 1];
    ri.n_grow = static_cast<int32_t>(n_grow);
    ri.n_in = static_cast<int32_t>(n_in);
    ri.t_in = t_in;
    ri.t_out = t_out;
    ri.cni = cni;
    ri.delta = delta;
    finish_row(0, n_amb);
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
constexpr int kDotBlock = 8;  // float4 of X in flight per block of the exact dot

// Exact G[i, c] with the reference's arithmetic: one running sum over j,
// products rounded then added, the last N mod 4 terms fused. y: dY_i (LDS
// or global), x: X_c (global); V4: both 16-byte aligned and N % 4 == 0, and
// the next block of x is loaded while the current one is summed.
template <bool V4>
__device__ __forceinline__ float exact_dot(const float* y, const float* __restrict__ x, int64_t N) {
    float acc = 0.0f;
    const int64_t n4 = N & ~int64_t{3};
    int64_t j = 0;
    if (V4) {
        const int64_t nb = n4 / (4 * kDotBlock);
        f32x4 cur[kDotBlock], nxt[kDotBlock];
        if (nb > 0) {
#pragma unroll
            for (int u = 0; u < kDotBlock; ++u) cur[u] = *reinterpret_cast<const f32x4*>(x + 4 * u);
        }
        for (int64_t b = 0; b < nb; ++b) {
            if (b + 1 < nb) {
#pragma unroll
                for (int u = 0; u < kDotBlock; ++u)
                    nxt[u] = *reinterpret_cast<const f32x4*>(x + 4 * (kDotBlock * (b + 1) + u));
            }
#pragma unroll
            for (int u = 0; u < kDotBlock; ++u) {
                const f32x4 a = *reinterpret_cast<const f32x4*>(y + 4 * (kDotBlock * b + u));
                acc = acc + a[0] * cur[u][0];
                acc = acc + a[1] * cur[u][1];
                acc = acc + a[2] * cur[u][2];
                acc = acc + a[3] * cur[u][3];
            }
#pragma unroll
            for (int u = 0; u < kDotBlock; ++u) cur[u] = nxt[u];
        }
        for (j = nb * 4 * kDotBlock; j < n4; j += 4) {
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

// Lists the set columns of the bitmap bm (Kw words) in ascending order:
// emit(position, column) for every one, positions from 0. One workgroup.
template <class Emit>
__device__ void list_bitmap(const uint32_t* bm, int64_t Kw, int64_t* tmp, Emit emit) {
    const int t = threadIdx.x;
    const int64_t per = ceil_div(Kw, kRowThreads);
    const int64_t w0 = t * per < Kw ? t * per : Kw, w1 = w0 + per < Kw ? w0 + per : Kw;
    int64_t cnt = 0;
    for (int64_t w = w0; w < w1; ++w) cnt += __popc(bm[w]);
    int64_t pos = block_inclusive_scan(cnt, tmp) - cnt;
    for (int64_t w = w0; w < w1; ++w) {
        uint32_t bits = bm[w];
        while (bits) {
            const int b = __builtin_ctz(bits);
            bits &= bits - 1;
            emit(pos, w * 32 + b);
            ++pos;
        }
    }
}

// Finish, step 1, per row: the undecided columns in ascending order into
// amb_col[amb_off[i] ..] with the row index in amb_key (the exact step turns
// it into the key), and the columns certainly grown into the row's own
// staging slots stage_col[row_start ..] (there are n_in < row_nnz of them;
// the select step reads them before it stages the new row there).
template <bool VG>
__global__ __launch_bounds__(kRowThreads) void rigl_list_kernel(
    int64_t K, int64_t Kw, const int32_t* __restrict__ row_start,
    const int32_t* __restrict__ row_nnz, const float* __restrict__ values,
    const int32_t* __restrict__ cols, const float* __restrict__ thr_ptr,
    const float* __restrict__ Gp, int64_t ldg, const uint8_t* __restrict__ Gc, float c2,
    const float* __restrict__ nrm_c, const RowInfo* __restrict__ info,
    const int64_t* __restrict__ amb_off, int32_t* __restrict__ amb_col,
    uint32_t* __restrict__ amb_key, int64_t amb_cap,
    int32_t* __restrict__ stage_col) {
    extern __shared__ uint32_t lds[];
    uint32_t* keep = lds;
    uint32_t* grow = lds + Kw;
    uint32_t* ambm = lds + 2 * Kw;
    __shared__ int64_t tmp[kRowThreads];
    __shared__ unsigned long long s_best;

    const int64_t i = blockIdx.x;
    const int t = threadIdx.x;
    const RowInfo ri = info[i];
    if (ri.flags & kRowKeep) return;
    const int32_t n_live = row_nnz[i];
    const int32_t start = row_start[i];
    for (int64_t w = t; w < Kw; w += kRowThreads) keep[w] = grow[w] = ambm[w] = 0;
    __syncthreads();
    mark_survivors(values, cols, start, n_live, thr_ptr[0], keep, tmp, &s_best);
    const int64_t off = amb_off[i];
    const int64_t n_amb = amb_off[gridDim.x + 1 + i];
    if (ri.flags & kRowExact) {
        for (int64_t c = t; c < K; c += kRowThreads)
            if (!bit_of(keep, c)) atomicOr(&ambm[c >> 5], 1u << (c & 31));
    } else {
        for_each_col<VG>(Gp + i * ldg, nrm_c, Gc + i * K, K,
                         [&](int64_t c, float g, float nk, uint32_t code) {
            if (bit_of(keep, c)) return;
            const int cls = classify_col(fabsf(g), ri.cni, nk, ri.delta, c2, code, ri.t_in, ri.t_out);
            if (cls == kGrowIn) atomicOr(&grow[c >> 5], 1u << (c & 31));
            else if (cls == kGrowUndecided) atomicOr(&ambm[c >> 5], 1u << (c & 31));
        });
    }
    __syncthreads();
    // (the count pass classified the same columns the same way, so every
    // position is below n_amb and n_in; the guards keep a mismatch inside the row)
    list_bitmap(ambm, Kw, tmp, [&](int64_t pos, int64_t c) {
        if (pos < n_amb && off + pos < amb_cap) {
            amb_col[off + pos] = static_cast<int32_t>(c);
            amb_key[off + pos] = static_cast<uint32_t>(i);
        }
    });
    __syncthreads();
    const int64_t n_in = (ri.flags & kRowExact) ? 0 : ri.n_in;
    list_bitmap(grow, Kw, tmp, [&](int64_t pos, int64_t c) {
        if (pos < n_in && pos < n_live) stage_col[start + pos] = static_cast<int32_t>(c);
    });
}

// Finish, step 2, over all P undecided (row, column) pairs: the exact G with
// the reference's arithmetic (exact_dot), as the key ~bits(|G|) (0 for NaN).
// amb_key holds the row on entry. A wave takes 64 consecutive pairs, one per
// lane; the X rows of its pairs and its distinct dY rows (a row's pairs are
// consecutive, so a wave's 64 pairs usually span a few rows) are streamed
// through the wave's own LDS rows in chunks of kExJ floats, eight lanes
// loading one 128-byte piece of a row (so a pair's 16 KB X row is 128
// coalesced loads of the wave, two chunks ahead in registers, instead of one
// thread's dependent stream). Each lane then runs its pair's sum over the
// chunk from LDS. N % 4 == 0 and 16-byte aligned rows; the four waves of a
// workgroup run in step (barriers).
constexpr int kExJ = 32;               // floats per chunk
constexpr int kExRow = kExJ / 4 + 1;   // 16-byte pieces per LDS row (one padding)
constexpr int kExThreads = 256;
__global__ __launch_bounds__(kExThreads) void rigl_exact_kernel(
    const int64_t* __restrict__ total, int64_t cap, int64_t M, int64_t K, int64_t N,
    const int32_t* __restrict__ amb_col, uint32_t* __restrict__ amb_key,
    const float* __restrict__ dY, const float* __restrict__ X) {
    __shared__ f32x4 xs[kExThreads / kWave][kWave][kExRow];
    __shared__ f32x4 ys[kExThreads / kWave][kWave][kExRow];
    __shared__ int32_t drow[kExThreads / kWave][kWave];
    const int64_t P = *total < cap ? *total : cap;  // the grid covers the capacity
    if (static_cast<int64_t>(blockIdx.x) * kExThreads >= P) return;  // workgroup-uniform
    const int w = threadIdx.x >> 6;
    const int l = threadIdx.x & 63;
    const int64_t p = static_cast<int64_t>(blockIdx.x) * kExThreads + threadIdx.x;
    const int64_t pc = p < P ? p : P - 1;
    // (rows and columns clamped into the matrices: a list that disagreed
    // with the count would give wrong keys, never an out-of-bounds read)
    const int32_t my_col = min(max(amb_col[pc], 0), static_cast<int32_t>(K - 1));
    const int32_t my_row = static_cast<int32_t>(min<uint32_t>(amb_key[pc], static_cast<uint32_t>(M - 1)));
    // the wave's distinct rows: a lane whose row differs from its left
    // neighbour's starts one; its rank among them indexes the LDS rows of dY
    const int32_t left = __shfl_up(my_row, 1);
    const bool first = l == 0 || left != my_row;
    const uint64_t starts = __ballot(first);
    const int rank = __popcll(starts & ((2ull << l) - 1ull)) - 1;
    const int nd = __popcll(starts);  // wave-uniform
    if (first) drow[w][rank] = my_row;
    __syncthreads();
    // staging: load u of lane l is piece l % 8 of pair 8u + l / 8's X row
    // and, for the first ceil(nd / 8) loads, of distinct row 8u + l / 8 of dY
    constexpr int kU = kWave * (kExJ / 4) / kWave;  // loads per lane per chunk and matrix
    static_assert(kU == 8, "eight lanes per 128-byte piece of a row");
    const int nu = (nd + 7) / 8;
    const int pe = l & 7;
    const float* xsrc[kU];
    const float* ysrc[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
        const int src = 8 * u + (l >> 3);
        xsrc[u] = X + static_cast<int64_t>(__shfl(my_col, src)) * N;
        ysrc[u] = dY + static_cast<int64_t>(drow[w][src < nd ? src : nd - 1]) * N;
    }
    const int64_t nch = ceil_div(N, kExJ);
    f32x4 rx[2][kU], ry[2][kU];
    // chunks past the last reload the last one, and a piece past N loads
    // the row's last piece: every load is in bounds and unconditional
    auto load = [&](int set, int64_t ch) {
        const int64_t c = ch < nch ? ch : nch - 1;
        const int64_t j0 = c * kExJ + 4 * pe;
        const int64_t j = j0 + 4 <= N ? j0 : N - 4;
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            rx[set][u] = *reinterpret_cast<const f32x4*>(xsrc[u] + j);
            if (u < nu) ry[set][u] = *reinterpret_cast<const f32x4*>(ysrc[u] + j);
        }
    };
    float acc = 0.0f;
    auto chunk = [&](auto S, int64_t ch) {
        constexpr int set = decltype(S)::value;
        __syncthreads();  // every lane has read the previous chunk
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            xs[w][8 * u + (l >> 3)][pe] = rx[set][u];
            if (u < nu) ys[w][8 * u + (l >> 3)][pe] = ry[set][u];
        }
        __syncthreads();
        load(set, ch + 2);
        const int64_t left_j = N - ch * kExJ;  // workgroup-uniform
        const int terms = left_j <= 0 ? 0 : left_j < kExJ ? static_cast<int>(left_j) : kExJ;
#pragma unroll
        for (int q = 0; q < kExJ / 4; ++q) {
            if (4 * q < terms) {
                const f32x4 a = ys[w][rank][q];
                const f32x4 b = xs[w][l][q];
                acc = acc + a[0] * b[0];
                acc = acc + a[1] * b[1];
                acc = acc + a[2] * b[2];
                acc = acc + a[3] * b[3];
            }
        }
    };
    load(0, 0);
    load(1, 1);
    for (int64_t ch = 0; ch < nch; ch += 2) {
        chunk(std::integral_constant<int, 0>{}, ch);
        chunk(std::integral_constant<int, 1>{}, ch + 1);
    }
    if (p < P) {
        const float a = fabsf(acc);
        amb_key[p] = a == a ? desc_key(a) : 0u;
    }
}

// The same for any N and alignment: one thread per pair, from global memory.
__global__ __launch_bounds__(256) void rigl_exact_simple_kernel(
    const int64_t* __restrict__ total, int64_t cap, int64_t M, int64_t K, int64_t N,
    const int32_t* __restrict__ amb_col, uint32_t* __restrict__ amb_key,
    const float* __restrict__ dY, const float* __restrict__ X) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (p >= *total || p >= cap) return;
    const int64_t c = min(max(amb_col[p], 0), static_cast<int32_t>(K - 1));
    const int64_t r = min<uint32_t>(amb_key[p], static_cast<uint32_t>(M - 1));
    const float a = fabsf(exact_dot<false>(dY + r * N, X + c * N, N));
    amb_key[p] = a == a ? desc_key(a) : 0u;
}

// Finish, step 3, per row: survivors, the certain grows (from the row's
// staging slots), the need = n_grow - n_in smallest exact keys among the
// undecided (ties to the lower column; for an exact row n_grow counts only
// non-NaN columns), and the row rewritten as the exact drop/grow kernel
// writes it.
__global__ __launch_bounds__(kRowThreads) void rigl_select_kernel(
    int64_t Kw, const int32_t* __restrict__ row_start, int32_t* __restrict__ row_nnz,
    float* __restrict__ values, int32_t* __restrict__ cols, const float* __restrict__ thr_ptr,
    const RowInfo* __restrict__ info, const int64_t* __restrict__ amb_off,
    const int32_t* __restrict__ amb_col, const uint32_t* __restrict__ amb_key, int64_t amb_cap,
    int32_t* __restrict__ stage_col, float* __restrict__ stage_val,
    unsigned long long* __restrict__ removed) {
    extern __shared__ uint32_t lds[];
    uint32_t* keep = lds;
    uint32_t* grow = lds + Kw;
    uint32_t* wpre = lds + 2 * Kw;
    __shared__ int64_t tmp[kRowThreads];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_digit;
    __shared__ int64_t s_below;
    __shared__ unsigned long long s_best;

    const int64_t i = blockIdx.x;
    const int t = threadIdx.x;
    const RowInfo ri = info[i];
    if (ri.flags & kRowKeep) return;
    // more undecided columns than the lists hold: no row is rewritten (the
    // caller reads the count afterwards and takes the exact path instead)
    if (amb_off[gridDim.x] > amb_cap) return;
    const int32_t n_live = row_nnz[i];
    const int32_t start = row_start[i];
    for (int64_t w = t; w < Kw; w += kRowThreads) keep[w] = grow[w] = 0;
    __syncthreads();
    const int64_t n_keep = mark_survivors(values, cols, start, n_live, thr_ptr[0], keep, tmp,
                                          &s_best);
    const int64_t n_drop = n_live - n_keep;
    const bool exact_row = (ri.flags & kRowExact) != 0;
    const int64_t n_in = exact_row ? 0 : ri.n_in;
    for (int64_t e = t; e < n_in && e < n_live; e += kRowThreads) {
        const int32_t c = stage_col[start + e];
        atomicOr(&grow[c >> 5], 1u << (c & 31));
    }
    __syncthreads();
    const int64_t off = amb_off[i];
    const int64_t n_amb = min(off + amb_off[gridDim.x + 1 + i], amb_cap) - min(off, amb_cap);
    // (a workspace smaller than the contract asks leaves columns out, never
    // reads past it)
    int64_t n_grow = ri.n_grow, need = ri.n_grow - n_in;
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

// One 32 x 32 x 16 bf16 MFMA per wave on given operands
// (slk_rigl_mfma_probe), with the operand and accumulator layout
// rigl_approx_kernel uses: lane l holds row l % 32 of A and of B at k = 8 (l /
// 32) .. + 8, and accumulator register 4 g + q holds row 8 g + 4 (l / 32) + q,
// column l % 32.
__global__ __launch_bounds__(64) void rigl_mfma_probe_kernel(const uint16_t* __restrict__ A,
                                                             const uint16_t* __restrict__ B,
                                                             const float* __restrict__ C,
                                                             float* __restrict__ D, int64_t n) {
    const int64_t t = blockIdx.x;
    if (t >= n) return;
    const int lane = threadIdx.x;
    const int r = lane & 31, k0 = 8 * (lane >> 5);
    const bf16x8 a = *reinterpret_cast<const bf16x8*>(A + (t * 32 + r) * 16 + k0);
    const bf16x8 b = *reinterpret_cast<const bf16x8*>(B + (t * 32 + r) * 16 + k0);
    f32x16 acc;
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int q = 0; q < 4; ++q)
            acc[4 * g + q] = C[(t * 32 + 8 * g + 4 * (lane >> 5) + q) * 32 + r];
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int q = 0; q < 4; ++q)
            D[(t * 32 + 8 * g + 4 * (lane >> 5) + q) * 32 + r] = acc[4 * g + q];
}

__global__ void rigl_clear_kernel(unsigned long long* __restrict__ c) { *c = 0; }
__global__ void rigl_copy_kernel(const int64_t* __restrict__ s, int64_t* __restrict__ d) { *d = *s; }

// U of the row-in-registers count kernel for this problem, or 0 for the
// generic count kernel (whose lists the finish's list pass writes). Both
// slk_rigl_count and slk_rigl_finish decide with it.
int count_reg_units(int64_t K, int64_t ldg, const float* G, const uint8_t* Gc, const float* nrm_X) {
    const bool vr = K % 16 == 0 && ldg % 4 == 0 && reinterpret_cast<uintptr_t>(G) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(Gc) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(nrm_X) % 16 == 0;
    if (!vr) return 0;
    if (K <= 4 * kRowThreads * 4) return 4;
    if (K <= 4 * kRowThreads * 8) return 8;
    if (K <= 4 * kRowThreads * 16) return 16;
    return 0;
}

// The bound's factors: |G'[i,k] - G[i,k]| <= c1·n_i·n_k + c2·pm[i,k] + δ,
// pm = the element's sum of |running sums of G'| at the chunk ends (its
// code's power of two bounds it). u = 2^-24, u' = u / (1 - u), L = kAChunk,
// C = ceil(N / L) chunks, I = 3L/16 MFMAs per chunk, g = γ_16(2u).
//  * G' against the exact sum S_N = Σ x_j y_j: each MFMA adds 16 exact bf16
//    products to its running sum R, at <= 2u per addition in any order and
//    rounding mode: error <= g·(|R| + Σ|t|). Inside chunk c, |R| <= |S_{a_c}| +
//    Σ_{chunk c}|t| + (the error so far <= c_run·Σ|x y|), so the matrix-core
//    error is <= g·I·Σ_c |S_{a_c}| + g·(I + 1 + (3N/16)·c_run)·Σ|t|, with
//    Σ|t| = Σ|x_h y_h| + |x_h y_l| + |x_l y_h| <= (1 + 2^-6)·Σ|x y|; plus the
//    dropped x_l y_l and r terms, 3.1·2^-16·Σ|x y|.
//  * The reference's sum G = ŝ_N (products rounded, then added in order)
//    against S_N: |ŝ_N - S_N| <= u·Σ|p| + u'·Σ_j |ŝ_j|, Σ_j |ŝ_j| <=
//    Σ_j |S_j| + N·γ_N·Σ|p|, and inside chunk c |S_j| <= |S_{a_c}| +
//    Σ_{chunk c}|p|: Σ_j |S_j| <= L·Σ_c |S_{a_c}| + L·Σ|p|.
//  * Σ_c |S_{a_c}| <= (1 + 2Cu)·pm + C·c_run·Σ|x y| (pm: C positive terms
//    summed in fp32, over running sums within c_run·Σ|x y| of the exact
//    partial sums; c_run = g·(3N/16)·2·(1 + 2^-6) + 3.1·2^-16, a crude bound
//    that only ever multiplies small factors).
//  * Σ|x y| <= n_i·n_k (Cauchy-Schwarz); everything times 1.01.
// Against γ_N·Σ|x y| for the reference's rounding alone this is L instead of
// N per unit of Σ|x y|, plus the partial sums' magnitudes, which grow like a
// random walk, not like Σ|x y| (16384^2 x 4096: c1 = 1.14e-4 against the
// 3.43e-4 of a bound without pm, and c2·pm is about a tenth of the bound).
struct BoundFactors {
    double c1, c2;
};
BoundFactors certified_factors(int64_t N) {
    const double u = 0x1p-24, u1 = u / (1.0 - u);
    auto gam = [&](double n, double uu) { return n * uu / (1.0 - n * uu); };
    const double n = static_cast<double>(N > 0 ? N : 1);
    const double L = kAChunk;
    const double C = ceil(n / L);
    const double I = 3.0 * L / 16.0;
    const double ninstr = 3.0 * C * L / 16.0;  // MFMAs per element, padded chunks included
    const double g = gam(16.0, 2 * u);
    const double sums = 1.0 + 0x1p-6;
    const double dropped = 3.1 * 0x1p-16;
    const double c_run = g * ninstr * 2.0 * sums + dropped;
    const double c_mc = g * (I + 1.0 + ninstr * c_run) * sums + dropped;
    const double c_ref = u + u1 * (L + n * gam(n, u));
    const double part = g * I + u1 * L;  // per unit of Σ_c |S_{a_c}|
    const double c1 = (c_mc + c_ref + part * C * c_run + 1.01 * u) * 1.01;
    const double c2 = part * (1.0 + 2.0 * C * u) * 1.01;
    return {c1, c2};
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
    if (M + K > 0) {
        hipLaunchKernelGGL(rigl_norm_kernel, dim3(static_cast<unsigned>(ceil_div(M + K, 4))),
                           dim3(256), 0, st, dY, M, X, K, N, nrm_dY, nrm_X);
    }
    return check_launch("rigl_norms");
}

extern "C" int64_t slk_dense_grad_approx_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    if (M < 0 || K < 0 || N < 0) return 0;
    return (M + K) * slk::approx_stages(N) * slk::kAStageBytes;
}

extern "C" int slk_dense_grad_approx(const float* dY, const float* X, int64_t M, int64_t K,
                                     int64_t N, float* G, uint8_t* G_code, void* workspace,
                                     int64_t workspace_bytes, void* stream) {
    using namespace slk;
    clear_error();
    if (M < 0 || K < 0 || N < 0)
        return fail(SLK_EINVAL, "dense_grad_approx: shape params must be non-negative");
    if (M == 0 || K == 0) return SLK_OK;
    if (G == nullptr || G_code == nullptr || (N > 0 && (dY == nullptr || X == nullptr)))
        return fail(SLK_EINVAL, "dense_grad_approx: NULL pointer");
    const int64_t nst = approx_stages(N);
    const int64_t need = (M + K) * nst * kAStageBytes;
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
        return fail(SLK_EINVAL, "dense_grad_approx: workspace smaller than "
                                "slk_dense_grad_approx_workspace_bytes");
    const int64_t tiles = ceil_div(M, kATI) * ceil_div(K, kATK);
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
    if (tuning(SLK_TUNE_RIGL_TILE) == 128) {
        hipLaunchKernelGGL(rigl_approx_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kAThreads),
                           0, st, M, K, nst, PA, PB, G, G_code);
    } else {
        const int64_t big = ceil_div(M, kGTI) * ceil_div(K, kGTK);
        hipLaunchKernelGGL(rigl_approx_dma_kernel, dim3(static_cast<unsigned>(big)),
                           dim3(kGThreads), 0, st, M, K, nst, PA, PB, G, G_code);
    }
    return check_launch("dense_grad_approx");
}

extern "C" double slk_rigl_bound_factor(int64_t N) { return slk::certified_factors(N).c1; }

extern "C" double slk_rigl_partial_factor(int64_t N) { return slk::certified_factors(N).c2; }

extern "C" int slk_rigl_count(const slk_csr* W, const float* thr_dev, const float* G_approx,
                              int64_t ldg, const uint8_t* G_code, const float* nrm_dY,
                              const float* nrm_X, int64_t N, void* info, int64_t* amb_off,
                              int64_t* amb_total, void* amb_ws, int64_t amb_ws_bytes,
                              void* workspace, int64_t workspace_bytes, void* stream) {
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
    if (W->nrows > 0 && (thr_dev == nullptr || G_approx == nullptr || G_code == nullptr ||
                         ldg < W->ncols || nrm_dY == nullptr || nrm_X == nullptr ||
                         info == nullptr))
        return fail(SLK_EINVAL, "rigl_count: NULL input or ldg < ncols");
    if (amb_ws_bytes < 0 || (amb_ws_bytes > 0 && amb_ws == nullptr))
        return fail(SLK_EINVAL, "rigl_count: bad undecided-column workspace");
    if (W->nrows > 0 && W->total_capacity > 0 &&
        (workspace == nullptr || workspace_bytes < W->total_capacity * 8))
        return fail(SLK_EINVAL, "rigl_count: workspace smaller than slk_drop_grow_workspace_bytes");
    hipStream_t st = as_stream(stream);
    const int64_t M = W->nrows, K = W->ncols;
    const int64_t Kw = ceil_div(K, 32) > 0 ? ceil_div(K, 32) : 1;
    const int U = M > 0 ? count_reg_units(K, ldg, G_approx, G_code, nrm_X) : 0;
    if (U > 0) {
        // the lists written here: the running total amb_off[M] from zero
        hipLaunchKernelGGL(rigl_clear_kernel, dim3(1), dim3(1), 0, st,
                           reinterpret_cast<unsigned long long*>(amb_off + M));
        if (int rc = check_launch("rigl_count")) return rc;
    }
    if (M > 0) {
        // the factors rounded up to floats
        const BoundFactors bf = certified_factors(N);
        const float c_f = std::nextafter(static_cast<float>(bf.c1), INFINITY);
        const float c2_f = std::nextafter(static_cast<float>(bf.c2), INFINITY);
        const bool vg = K % 4 == 0 && ldg % 4 == 0 &&
                        reinterpret_cast<uintptr_t>(G_approx) % 16 == 0 &&
                        reinterpret_cast<uintptr_t>(G_code) % 4 == 0 &&
                        reinterpret_cast<uintptr_t>(nrm_X) % 16 == 0;
        const dim3 grid(static_cast<unsigned>(M));
        const size_t lds_st = static_cast<size_t>(Kw + K) * 4, lds_un = static_cast<size_t>(Kw) * 4;
        const int64_t n_amb_max = amb_ws_bytes / 8;
        int32_t* amb_col = static_cast<int32_t*>(amb_ws);
        uint32_t* amb_key = reinterpret_cast<uint32_t*>(amb_col + n_amb_max);
        int32_t* stage_col = static_cast<int32_t*>(workspace);
#define SLK_COUNT_REG_ARGS                                                                      K, M, W->row_start, W->row_nnz, W->values, W->col_indices, thr_dev, G_approx, ldg, G_code,         nrm_dY, nrm_X, c_f, c2_f, static_cast<RowInfo*>(info), amb_off, amb_col, amb_key,            n_amb_max, stage_col
        // (amb_off + M + 1: the per-row counts, which the scan turns into offsets)
#define SLK_COUNT_ARGS                                                                           K, Kw, W->row_start, W->row_nnz, W->values, W->col_indices, thr_dev, G_approx, ldg, G_code,         nrm_dY, nrm_X, c_f, c2_f, static_cast<RowInfo*>(info), amb_off + M + 1
        if (U == 4) {
            hipLaunchKernelGGL(rigl_count_reg_kernel<4>, grid, dim3(kRowThreads), 0, st,
                               SLK_COUNT_REG_ARGS);
        } else if (U == 8) {
            hipLaunchKernelGGL(rigl_count_reg_kernel<8>, grid, dim3(kRowThreads), 0, st,
                               SLK_COUNT_REG_ARGS);
        } else if (U == 16) {
            hipLaunchKernelGGL(rigl_count_reg_kernel<16>, grid, dim3(kRowThreads), 0, st,
                               SLK_COUNT_REG_ARGS);
        } else if (K <= kStageMaxK && vg) {
            hipLaunchKernelGGL((rigl_count_kernel<true, true>), grid, dim3(kRowThreads), lds_st, st,
                               SLK_COUNT_ARGS);
        } else if (K <= kStageMaxK) {
            hipLaunchKernelGGL((rigl_count_kernel<true, false>), grid, dim3(kRowThreads), lds_st, st,
                               SLK_COUNT_ARGS);
        } else if (vg) {
            hipLaunchKernelGGL((rigl_count_kernel<false, true>), grid, dim3(kRowThreads), lds_un, st,
                               SLK_COUNT_ARGS);
        } else {
            hipLaunchKernelGGL((rigl_count_kernel<false, false>), grid, dim3(kRowThreads), lds_un,
                               st, SLK_COUNT_ARGS);
        }
#undef SLK_COUNT_ARGS
#undef SLK_COUNT_REG_ARGS
        if (int rc = check_launch("rigl_count")) return rc;
    }
    if (U > 0) {
        hipLaunchKernelGGL(rigl_copy_kernel, dim3(1), dim3(1), 0, st, amb_off + M, amb_total);
    } else {
        hipLaunchKernelGGL(rigl_scan_kernel, dim3(1), dim3(1024), 0, st, M, amb_off + M + 1,
                           amb_off, amb_total);
    }
    return check_launch("rigl_count/scan");
}

extern "C" int slk_rigl_finish(const slk_csr* W, float* values, int32_t* col_indices,
                               int32_t* row_nnz, const float* thr_dev, const float* G_approx,
                               int64_t ldg, const uint8_t* G_code, const float* nrm_dY,
                               const float* nrm_X,
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
    if (M > 0 && (thr_dev == nullptr || G_approx == nullptr || G_code == nullptr || ldg < K ||
                  nrm_dY == nullptr ||
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
    // the exact step's grid covers the workspace's capacity; the pairs in
    // use are amb_off[M] (slk_rigl_count's total), read on the device
    const int64_t P = n_amb_max;
    const size_t lds = static_cast<size_t>(3 * Kw) * 4;
    int32_t* stage_col = static_cast<int32_t*>(workspace);
    float* stage_val = reinterpret_cast<float*>(stage_col + W->total_capacity);
    const bool vg = K % 4 == 0 && ldg % 4 == 0 && reinterpret_cast<uintptr_t>(G_approx) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(G_code) % 4 == 0 &&
                    reinterpret_cast<uintptr_t>(nrm_X) % 16 == 0;
    const float c2_f = std::nextafter(static_cast<float>(certified_factors(N).c2), INFINITY);
    const dim3 grid(static_cast<unsigned>(M));
    // the lists: written by the count kernel where it held the row in
    // registers, else by the list pass
#define SLK_LIST_ARGS                                                                      \
    K, Kw, W->row_start, row_nnz, values, col_indices, thr_dev, G_approx, ldg, G_code, c2_f, \
        nrm_X, static_cast<const RowInfo*>(info), amb_off, amb_col, amb_key, n_amb_max, stage_col
    if (count_reg_units(K, ldg, G_approx, G_code, nrm_X) == 0) {
        if (vg) {
            hipLaunchKernelGGL(rigl_list_kernel<true>, grid, dim3(kRowThreads), lds, st,
                               SLK_LIST_ARGS);
        } else {
            hipLaunchKernelGGL(rigl_list_kernel<false>, grid, dim3(kRowThreads), lds, st,
                               SLK_LIST_ARGS);
        }
        if (int rc = check_launch("rigl_finish/list")) return rc;
    }
#undef SLK_LIST_ARGS
    if (P > 0) {
        if (ceil_div(P, 256) > INT32_MAX) return fail(SLK_EINVAL, "rigl_finish: too many undecided columns");
        const bool v4 = N > 0 && N % 4 == 0 && reinterpret_cast<uintptr_t>(dY) % 16 == 0 &&
                        reinterpret_cast<uintptr_t>(X) % 16 == 0;
        if (v4) {
            hipLaunchKernelGGL(rigl_exact_kernel, dim3(static_cast<unsigned>(ceil_div(P, kExThreads))),
                               dim3(kExThreads), 0, st, amb_off + M, P, M, K, N, amb_col, amb_key, dY, X);
        } else {  // any N (N = 0: every G is +0.0)
            hipLaunchKernelGGL(rigl_exact_simple_kernel, dim3(static_cast<unsigned>(ceil_div(P, 256))),
                               dim3(256), 0, st, amb_off + M, P, M, K, N, amb_col, amb_key, dY, X);
        }
        if (int rc = check_launch("rigl_finish/exact")) return rc;
    }
    hipLaunchKernelGGL(rigl_select_kernel, grid, dim3(kRowThreads), lds, st, Kw, W->row_start,
                       row_nnz, values, col_indices, thr_dev, static_cast<const RowInfo*>(info),
                       amb_off, amb_col, amb_key, n_amb_max, stage_col, stage_val, removed_u);
    return check_launch("rigl_finish");
}

extern "C" int slk_rigl_mfma_probe(const uint16_t* A, const uint16_t* B, const float* C, float* D,
                                   int64_t n, void* stream) {
    using namespace slk;
    clear_error();
    if (n < 0 || n > INT32_MAX) return fail(SLK_EINVAL, "rigl_mfma_probe: n outside [0, 2^31)");
    if (n == 0) return SLK_OK;
    if (A == nullptr || B == nullptr || C == nullptr || D == nullptr)
        return fail(SLK_EINVAL, "rigl_mfma_probe: NULL pointer");
    hipLaunchKernelGGL(rigl_mfma_probe_kernel, dim3(static_cast<unsigned>(n)), dim3(64), 0,
                       as_stream(stream), A, B, C, D, n);
    return check_launch("rigl_mfma_probe");
}
