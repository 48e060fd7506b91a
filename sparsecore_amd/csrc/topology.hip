// Topology mutation on the device: the drop/grow pass of SET and RigL, the
// global drop threshold they share, and the dense gradient RigL ranks its
// grow candidates by.
//
// Reference (sparselab/router.py:378-478 SET, :598-732 RigL): per layer,
//   threshold = k-th smallest |v| over all live slots, k = max(1, int(f*nnz));
//   per row: keep |v| > threshold (at least the largest slot), then grow as
//   many columns as were dropped, outside the kept set, zero-initialised, and
//   rewrite the row sorted by column (PaddedCSR.rewrite_row).
// A row regrows what it dropped (ncols - kept >= dropped), so row_start and
// the capacities never change and row_nnz changes only in RigL's one
// exception: columns whose |G| is NaN are never grown (the reference counts
// `available` as the empty columns with |G| > -inf, router.py:704-705), and a
// row that runs out of such columns shrinks by the difference.
//
//   kth_*        radix select (digits of 11, 10, 10 bits) over the bit
//                patterns of |v| of the live slots: for non-negative floats
//                the unsigned order of the bits is the numeric order, so the
//                result is exact. Three histogram launches plus three
//                one-workgroup pick launches; no host synchronisation.
//   drop_grow    one workgroup per row. Survivors and grows are marked in
//                LDS bitmaps over the row's columns; grows are the n_grow
//                smallest 32-bit keys among the unmarked columns (a per-row
//                radix select with 8-bit digits, ties to the lower column).
//                RigL keys are ~bits(|G|) (largest |G| first); SET keys are
//                splitmix64 hashes (a uniform random subset). A column's new
//                slot is its rank in the union bitmap; the row is staged in a
//                workspace and copied back.
//   dense_grad   128x128 output tile per workgroup, 8x8 per thread, j staged
//                through LDS 16 at a time (the next 16 loaded into registers
//                while the current 16 are summed). Each output element is one
//                running sum over j in order with the reference build's
//                arithmetic.
#include "common.hpp"
#include "row_rewrite.hpp"

#include <mutex>

namespace slk {
namespace {

// ───────────────────────── global k-th |value| ─────────────────────────────

constexpr int kSelBins = 2048;
constexpr int kSelThreads = 256;

struct SelState {
    uint32_t prefix;
    uint32_t found;
    int64_t need;
    uint32_t hist[kSelBins];
};
static_assert(sizeof(SelState) <= SLK_KTH_WORKSPACE_BYTES, "workspace too small");

// Digit p covers bits [shift, shift + width) of the 31-bit key (bit 31 of
// |v| is always 0).
__host__ __device__ constexpr int sel_shift(int p) { return p == 0 ? 20 : (p == 1 ? 10 : 0); }
__host__ __device__ constexpr int sel_width(int p) { return p == 0 ? 11 : 10; }

__global__ __launch_bounds__(kSelThreads) void kth_init_kernel(SelState* st, int64_t k) {
    for (int b = threadIdx.x; b < kSelBins; b += kSelThreads) st->hist[b] = 0;
    if (threadIdx.x == 0) {
        st->prefix = 0;
        st->found = 1;
        st->need = k;
    }
}

__global__ __launch_bounds__(kSelThreads) void kth_hist_kernel(
    int64_t cap, const int32_t* __restrict__ col, const float* __restrict__ val,
    SelState* __restrict__ st, int pass) {
    __shared__ uint32_t h[kSelBins];
    for (int b = threadIdx.x; b < kSelBins; b += kSelThreads) h[b] = 0;
    __syncthreads();
    const int shift = sel_shift(pass);
    const uint32_t mask = (1u << sel_width(pass)) - 1u;
    const uint32_t prefix = st->prefix;
    const int hi = shift + sel_width(pass);
    // kSelUnroll slots per thread at a time, all loads issued before any use
    constexpr int kSelUnroll = 8;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kSelThreads;
    for (int64_t s0 = static_cast<int64_t>(blockIdx.x) * kSelThreads + threadIdx.x; s0 < cap;
         s0 += kSelUnroll * stride) {
        int32_t c[kSelUnroll];
        float v[kSelUnroll];
#pragma unroll
        for (int q = 0; q < kSelUnroll; ++q) {
            const int64_t s = s0 + q * stride;
            c[q] = s < cap ? col[s] : -1;
            v[q] = s < cap ? val[s] : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < kSelUnroll; ++q) {
            if (c[q] < 0) continue;  // padding (or past the end)
            const uint32_t u = __float_as_uint(fabsf(v[q]));
            if (pass == 0 || (u >> hi) == prefix) atomicAdd(&h[(u >> shift) & mask], 1u);
        }
    }
    __syncthreads();
    for (int b = threadIdx.x; b < kSelBins; b += kSelThreads)
        if (h[b] != 0) atomicAdd(&st->hist[b], h[b]);
}

__global__ __launch_bounds__(kSelThreads) void kth_pick_kernel(SelState* __restrict__ st, int pass,
                                                              float* __restrict__ thr_out) {
    __shared__ int64_t tmp[kSelThreads];
    __shared__ uint32_t digit;
    __shared__ int64_t below;
    __shared__ int hit;
    constexpr int kPer = kSelBins / kSelThreads;
    const int t = threadIdx.x;
    const int nbins = 1 << sel_width(pass);
    int64_t local = 0;
    for (int q = 0; q < kPer; ++q) {
        const int b = t * kPer + q;
        if (b < nbins) local += st->hist[b];
    }
    if (t == 0) hit = 0;
    const int64_t incl = block_inclusive_scan(local, tmp);
    const int64_t excl = incl - local;
    const int64_t need = st->need;
    if (excl < need && need <= incl) {
        int64_t c = excl;
        for (int q = 0; q < kPer; ++q) {
            const int b = t * kPer + q;
            const int64_t h = b < nbins ? st->hist[b] : 0;
            if (c + h >= need) {
                digit = static_cast<uint32_t>(b);
                below = c;
                hit = 1;
                break;
            }
            c += h;
        }
    }
    __syncthreads();
    for (int b = t; b < kSelBins; b += kSelThreads) st->hist[b] = 0;
    if (t == 0) {
        if (!hit) st->found = 0;  // k exceeded the live count: caller's contract broken
        const uint32_t p = hit ? ((st->prefix << sel_width(pass)) | digit) : st->prefix;
        st->prefix = p;
        st->need = need - (hit ? below : 0);
        if (pass == 2) thr_out[0] = st->found ? __uint_as_float(p) : __builtin_nanf("");
    }
}

// ───────────────────────── drop / grow ─────────────────────────────────────

constexpr int kDgThreads = kRowThreads;
constexpr int64_t kDgMaxCols = 131072;

__device__ __forceinline__ uint32_t set_key(uint64_t seed, int64_t row, int64_t K, int64_t c) {
    // splitmix64: output number (row*K + c + 1) of the stream seeded by `seed`
    uint64_t z = seed + static_cast<uint64_t>(row * K + c + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return static_cast<uint32_t>(z >> 32);
}

// RigL: ~bits(|G|), largest |G| first (NaN columns are skipped before any
// key is taken); SET: the splitmix64 key.
template <bool RIGL>
__device__ __forceinline__ uint32_t grow_key(const float* __restrict__ g_row, uint64_t seed,
                                             int64_t row, int64_t K, int64_t c) {
    if (RIGL) return ~__float_as_uint(fabsf(g_row[c]));
    return set_key(seed, row, K, c);
}

// A column RigL may not grow into: |G| is NaN.
template <bool RIGL>
__device__ __forceinline__ bool never_grown(const float* __restrict__ g_row, int64_t c) {
    if (!RIGL) return false;
    const float g = g_row[c];
    return g != g;
}


template <bool RIGL>
__global__ __launch_bounds__(kDgThreads) void drop_grow_kernel(
    int64_t K, int64_t Kw, const int32_t* __restrict__ row_start,
    int32_t* __restrict__ row_nnz, float* __restrict__ values, int32_t* __restrict__ cols,
    const float* __restrict__ thr_ptr, const float* __restrict__ G, int64_t ldg, uint64_t seed,
    int32_t* __restrict__ stage_col, float* __restrict__ stage_val,
    unsigned long long* __restrict__ removed) {
    extern __shared__ uint32_t lds[];
    uint32_t* keep = lds;         // survivors
    uint32_t* grow = lds + Kw;    // grown columns
    uint32_t* wpre = lds + 2 * Kw;  // exclusive prefix of popcounts of keep|grow
    __shared__ int64_t tmp[kDgThreads];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_digit;
    __shared__ int64_t s_below;
    __shared__ unsigned long long s_best;

    const int64_t i = blockIdx.x;
    const int t = threadIdx.x;
    const int32_t n_live = row_nnz[i];
    if (n_live <= 0) return;  // the reference skips empty rows
    const int32_t start = row_start[i];

    for (int64_t w = t; w < Kw; w += kDgThreads) keep[w] = grow[w] = 0;
    __syncthreads();
    const int64_t n_keep = mark_survivors(values, cols, start, n_live, thr_ptr[0], keep, tmp,
                                          &s_best);
    const int64_t n_drop = n_live - n_keep;
    const float* g_row = RIGL ? G + i * ldg : nullptr;
    int64_t n_grow = 0;
    if (n_drop > 0) {
        // n_grow = min(dropped, growable columns); RigL never grows a column
        // whose |G| is NaN
        int64_t growable = K - n_keep;
        if (RIGL) {
            int64_t skipped = 0;
            for (int64_t c = t; c < K; c += kDgThreads)
                if (!bit_of(keep, c) && never_grown<RIGL>(g_row, c)) ++skipped;
            block_inclusive_scan(skipped, tmp);
            growable -= tmp[kDgThreads - 1];
            __syncthreads();
        }
        n_grow = n_drop < growable ? n_drop : growable;
        // the n_grow smallest keys among the growable columns, ties to the
        // lower column
        auto cand = [&](int64_t c, int64_t& col, uint32_t& key) -> bool {
            col = c;
            if (bit_of(keep, c) || never_grown<RIGL>(g_row, c)) return false;
            key = grow_key<RIGL>(g_row, seed, i, K, c);
            return true;
        };
        select_smallest_keys(cand, K, n_grow, grow, hist, &s_digit, &s_below, tmp);
    }
    write_back_row(keep, grow, wpre, Kw, i, start, n_live, n_keep, n_grow, values, cols, row_nnz,
                   stage_col, stage_val, removed, tmp);
}

__global__ void clear_counter_kernel(unsigned long long* __restrict__ c) { *c = 0; }

// ───────────────────────── dense gradient ──────────────────────────────────

constexpr int kGT = 128;  // output tile edge (rows of G and columns of G)
constexpr int kGJ = 16;   // j values staged per step
constexpr int kGThreads = 256;
constexpr int kGPad = 4;

// Slab staging: a kGT x kGJ slab (rows r0.., j0..) of a matrix whose element
// (r, j) sits at p[r*N + j] (TOKEN_MAJOR = false) or p[j*R + r] (TOKEN_MAJOR =
// true) goes to s[j][r] in two halves: fetch_slab loads a thread's kGSlab
// elements into registers (every load unconditional at a clamped, in-bounds
// index, so all are in flight together; out-of-range entries become 0 and are
// never summed), store_slab writes them to LDS. The kernel fetches slab s+1
// while it computes slab s.
constexpr int kGSlab = kGT * kGJ / kGThreads;  // elements per thread per slab (8)

template <bool TOKEN_MAJOR>
__device__ __forceinline__ void fetch_slab(float (&v)[kGSlab], const float* __restrict__ p,
                                           int64_t R, int64_t N, int64_t r0, int64_t j0) {
    const int t = threadIdx.x;
#pragma unroll
    for (int q = 0; q < kGSlab; ++q) {
        // TOKEN_MAJOR: consecutive threads read consecutive r of one j;
        // otherwise consecutive j of one row
        const int r = TOKEN_MAJOR ? (t & (kGT - 1)) : (t >> 4) + 16 * q;
        const int j = TOKEN_MAJOR ? (t >> 7) + 2 * q : (t & (kGJ - 1));
        const int64_t rr = r0 + r, jj = j0 + j;
        const bool ok = rr < R && jj < N;
        const int64_t rc = rr < R ? rr : R - 1, jc = jj < N ? jj : N - 1;
        const float x = TOKEN_MAJOR ? p[jc * R + rc] : p[rc * N + jc];
        v[q] = ok ? x : 0.0f;
    }
}

template <bool TOKEN_MAJOR>
__device__ __forceinline__ void store_slab(float (*s)[kGT + kGPad], const float (&v)[kGSlab]) {
    const int t = threadIdx.x;
#pragma unroll
    for (int q = 0; q < kGSlab; ++q) {
        const int r = TOKEN_MAJOR ? (t & (kGT - 1)) : (t >> 4) + 16 * q;
        const int j = TOKEN_MAJOR ? (t >> 7) + 2 * q : (t & (kGJ - 1));
        s[j][r] = v[q];
    }
}

template <bool TOKEN_MAJOR>
__global__ __launch_bounds__(kGThreads) void dense_grad_kernel(
    int64_t M, int64_t K, int64_t N, int64_t N4, const float* __restrict__ dY,
    const float* __restrict__ X, float* __restrict__ G) {
    __shared__ float As[kGJ][kGT + kGPad];
    __shared__ float Bs[kGJ][kGT + kGPad];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int64_t i0 = static_cast<int64_t>(blockIdx.y) * kGT;
    const int64_t k0 = static_cast<int64_t>(blockIdx.x) * kGT;

    float acc[8][8];
#pragma unroll
    for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[r][c] = 0.0f;

    float va[kGSlab], vb[kGSlab];
    if (N > 0) {
        fetch_slab<TOKEN_MAJOR>(va, dY, M, N, i0, 0);
        fetch_slab<TOKEN_MAJOR>(vb, X, K, N, k0, 0);
    }
    for (int64_t j0 = 0; j0 < N; j0 += kGJ) {
        store_slab<TOKEN_MAJOR>(As, va);
        store_slab<TOKEN_MAJOR>(Bs, vb);
        __syncthreads();
        if (j0 + kGJ < N) {  // the next slab's loads fly while this one is summed
            fetch_slab<TOKEN_MAJOR>(va, dY, M, N, i0, j0 + kGJ);
            fetch_slab<TOKEN_MAJOR>(vb, X, K, N, k0, j0 + kGJ);
        }
        const int jn = N - j0 < kGJ ? static_cast<int>(N - j0) : kGJ;
        // j < N4: product rounded, then added; j >= N4: fused (the reference
        // build's evaluation of `acc += a*b`).
        int jsplit = N4 - j0 < 0 ? 0 : (N4 - j0 > jn ? jn : static_cast<int>(N4 - j0));
        for (int jj = 0; jj < jsplit; ++jj) {
            float a[8], b[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) a[r] = As[jj][ty * 8 + r];
#pragma unroll
            for (int c = 0; c < 8; ++c) b[c] = Bs[jj][tx * 8 + c];
#pragma unroll
            for (int r = 0; r < 8; ++r)
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    const float p = a[r] * b[c];
                    acc[r][c] = acc[r][c] + p;
                }
        }
        for (int jj = jsplit; jj < jn; ++jj) {
            float a[8], b[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) a[r] = As[jj][ty * 8 + r];
#pragma unroll
            for (int c = 0; c < 8; ++c) b[c] = Bs[jj][tx * 8 + c];
#pragma unroll
            for (int r = 0; r < 8; ++r)
#pragma unroll
                for (int c = 0; c < 8; ++c) acc[r][c] = __builtin_fmaf(a[r], b[c], acc[r][c]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        const int64_t i = i0 + ty * 8 + r;
        if (i >= M) break;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const int64_t k = k0 + tx * 8 + c;
            if (k < K) G[i * K + k] = acc[r][c];
        }
    }
}

__global__ __launch_bounds__(kGThreads) void zero_kernel(float* __restrict__ p, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kGThreads;
    for (int64_t q = static_cast<int64_t>(blockIdx.x) * kGThreads + threadIdx.x; q < n; q += stride)
        p[q] = 0.0f;
}

}  // namespace
}  // namespace slk

extern "C" int slk_live_abs_kth(const slk_csr* W, int64_t k, void* workspace,
                                int64_t workspace_bytes, float* thr_dev, void* stream) {
    using namespace slk;
    clear_error();
    if (int rc = validate_csr(W, "live_abs_kth")) return rc;
    if (workspace == nullptr || workspace_bytes < SLK_KTH_WORKSPACE_BYTES)
        return fail(SLK_EINVAL, "live_abs_kth: workspace smaller than SLK_KTH_WORKSPACE_BYTES");
    if (thr_dev == nullptr) return fail(SLK_EINVAL, "live_abs_kth: NULL threshold output");
    if (k < 1 || k > W->total_capacity)
        return fail(SLK_EINVAL, "live_abs_kth: k=" + std::to_string(k) +
                                    " outside [1, live slots]");
    hipStream_t st = as_stream(stream);
    SelState* s = static_cast<SelState*>(workspace);
    hipLaunchKernelGGL(kth_init_kernel, dim3(1), dim3(kSelThreads), 0, st, s, k);
    const int64_t cap = W->total_capacity;
    // at most 1024 workgroups: each one's histogram goes to the global one by
    // atomics on the same few bins (16384^2 at 95%: the select 162 -> 139 us
    // against 2048; 512: 163, 256: 242)
    int64_t blocks = ceil_div(cap, int64_t{kSelThreads} * 16);
    if (blocks > 1024) blocks = 1024;
    if (blocks < 1) blocks = 1;
    for (int pass = 0; pass < 3; ++pass) {
        hipLaunchKernelGGL(kth_hist_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kSelThreads),
                           0, st, cap, W->col_indices, W->values, s, pass);
        hipLaunchKernelGGL(kth_pick_kernel, dim3(1), dim3(kSelThreads), 0, st, s, pass, thr_dev);
    }
    return check_launch("live_abs_kth");
}

extern "C" int64_t slk_drop_grow_workspace_bytes(const slk_csr* W) {
    if (W == nullptr || W->total_capacity < 0) return 0;
    return W->total_capacity * 8;
}

namespace slk {
namespace {

// The shared body of slk_drop_grow and slk_drop_grow_noalloc: `stage` holds
// the row staging (total_capacity int32 columns, then as many floats).
int drop_grow_impl(const slk_csr* W, float* values, int32_t* col_indices, int32_t* row_nnz,
                   const float* thr_dev, int rule, const float* G, int64_t ldg, uint64_t seed,
                   void* stage, int64_t stage_bytes, int64_t* removed, void* stream,
                   const char* stage_what) {
    if (int rc = validate_csr(W, "drop_grow")) return rc;
    if (values != W->values || col_indices != W->col_indices || row_nnz != W->row_nnz)
        return fail(SLK_EINVAL, "drop_grow: values/col_indices/row_nnz must be W's own arrays");
    if (rule != SLK_GROW_RANDOM && rule != SLK_GROW_GRADIENT)
        return fail(SLK_EINVAL, "drop_grow: unknown grow rule " + std::to_string(rule));
    if (W->ncols > kDgMaxCols)
        return fail(SLK_EINVAL, "drop_grow: ncols=" + std::to_string(W->ncols) +
                                    " exceeds the supported maximum " + std::to_string(kDgMaxCols));
    if (removed == nullptr) return fail(SLK_EINVAL, "drop_grow: NULL removed-slot counter");
    const bool empty = W->nrows == 0 || W->total_capacity == 0;
    if (!empty) {
        if (thr_dev == nullptr) return fail(SLK_EINVAL, "drop_grow: NULL threshold");
        if (rule == SLK_GROW_GRADIENT && (G == nullptr || ldg < W->ncols))
            return fail(SLK_EINVAL, "drop_grow: the gradient rule needs G with ldg >= ncols");
        if (stage == nullptr || stage_bytes < W->total_capacity * 8)
            return fail(SLK_EINVAL, std::string("drop_grow: ") + stage_what);
        if (W->nrows > INT32_MAX) return fail(SLK_EINVAL, "drop_grow: too many rows for one launch");
    }
    hipStream_t st = as_stream(stream);
    unsigned long long* removed_u = reinterpret_cast<unsigned long long*>(removed);
    hipLaunchKernelGGL(clear_counter_kernel, dim3(1), dim3(1), 0, st, removed_u);
    if (int rc = check_launch("drop_grow")) return rc;
    if (empty) return SLK_OK;
    const int64_t K = W->ncols;
    const int64_t Kw = ceil_div(K, 32) > 0 ? ceil_div(K, 32) : 1;
    const size_t lds = static_cast<size_t>(3 * Kw) * sizeof(uint32_t);
    int32_t* stage_col = static_cast<int32_t*>(stage);
    float* stage_val = reinterpret_cast<float*>(stage_col + W->total_capacity);
    const dim3 grid(static_cast<unsigned>(W->nrows));
    if (rule == SLK_GROW_GRADIENT) {
        hipLaunchKernelGGL(drop_grow_kernel<true>, grid, dim3(kDgThreads), lds, st, K, Kw,
                           W->row_start, row_nnz, values, col_indices, thr_dev, G, ldg, seed,
                           stage_col, stage_val, removed_u);
    } else {
        hipLaunchKernelGGL(drop_grow_kernel<false>, grid, dim3(kDgThreads), lds, st, K, Kw,
                           W->row_start, row_nnz, values, col_indices, thr_dev, G, ldg, seed,
                           stage_col, stage_val, removed_u);
    }
    return check_launch("drop_grow");
}

// Row staging of slk_drop_grow_noalloc: a file-scope device array, one copy
// per GPU, held until the process ends. Host code never passes the array's
// name to a kernel (on the host it is only a stand-in for the symbol): the
// device address of each GPU's copy is looked up once per device with
// hipGetSymbolAddress and kept in scratch_dev[].
constexpr int64_t kNoallocMaxSlots = SLK_DROP_GROW_NOALLOC_MAX_SLOTS;
__device__ __align__(256) unsigned char scratch[kNoallocMaxSlots * 8];

constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void* scratch_dev[kMaxDevices] = {};

// This device's address of `scratch` (the current device's), or NULL with
// the error recorded.
void* scratch_for_current_device() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        fail(SLK_EDEVICE, "drop_grow_noalloc: no current HIP device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (scratch_dev[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            fail(SLK_EDEVICE, std::string("drop_grow_noalloc: hipGetSymbolAddress(scratch) "
                                          "failed: ") + hipGetErrorString(e));
            return nullptr;
        }
        scratch_dev[dev] = p;
    }
    return scratch_dev[dev];
}

}  // namespace
}  // namespace slk

extern "C" int slk_drop_grow(const slk_csr* W, float* values, int32_t* col_indices,
                             int32_t* row_nnz, const float* thr_dev, int rule, const float* G,
                             int64_t ldg, uint64_t seed, void* workspace,
                             int64_t workspace_bytes, int64_t* removed, void* stream) {
    slk::clear_error();
    return slk::drop_grow_impl(W, values, col_indices, row_nnz, thr_dev, rule, G, ldg, seed,
                               workspace, workspace_bytes, removed, stream,
                               "workspace smaller than slk_drop_grow_workspace_bytes");
}

extern "C" int slk_drop_grow_noalloc(const slk_csr* W, float* values, int32_t* col_indices,
                                     int32_t* row_nnz, const float* thr_dev, int rule,
                                     const float* G, int64_t ldg, uint64_t seed,
                                     int64_t* removed, void* stream) {
    using namespace slk;
    clear_error();
    if (W != nullptr && W->total_capacity > kNoallocMaxSlots) {
        return fail(SLK_EINVAL, "drop_grow_noalloc: total_capacity=" +
                                    std::to_string(W->total_capacity) +
                                    " exceeds the static scratch of " +
                                    std::to_string(kNoallocMaxSlots) +
                                    " slots; use slk_drop_grow with a workspace");
    }
    if (int rc = validate_csr(W, "drop_grow")) return rc;
    void* stage = nullptr;
    if (W->nrows > 0 && W->total_capacity > 0) {
        stage = scratch_for_current_device();
        if (stage == nullptr) return SLK_EDEVICE;
    }
    return drop_grow_impl(W, values, col_indices, row_nnz, thr_dev, rule, G, ldg, seed, stage,
                          kNoallocMaxSlots * 8, removed, stream, "static scratch unavailable");
}

extern "C" int slk_dense_grad(const float* dY, const float* X, int64_t M, int64_t K, int64_t N,
                              int token_major, float* G, void* stream) {
    using namespace slk;
    clear_error();
    if (M < 0 || K < 0 || N < 0) return fail(SLK_EINVAL, "dense_grad: shape params must be non-negative");
    if (M == 0 || K == 0) return SLK_OK;
    if (G == nullptr) return fail(SLK_EINVAL, "dense_grad: NULL G");
    hipStream_t st = as_stream(stream);
    if (N == 0) {  // empty sums: G = 0 (a kernel, not a memset, so graph capture stays safe)
        const int64_t n = M * K;
        int64_t blocks = ceil_div(n, kGThreads);
        if (blocks > 65536) blocks = 65536;
        hipLaunchKernelGGL(zero_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kGThreads), 0, st,
                           G, n);
        return check_launch("dense_grad");
    }
    if (dY == nullptr || X == nullptr) return fail(SLK_EINVAL, "dense_grad: NULL dY or X");
    const int64_t gx = ceil_div(K, kGT), gy = ceil_div(M, kGT);
    if (gx > INT32_MAX || gy > 65535) return fail(SLK_EINVAL, "dense_grad: problem too large for one launch");
    const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
    const int64_t N4 = N & ~int64_t{3};
    if (token_major) {
        hipLaunchKernelGGL(dense_grad_kernel<true>, grid, dim3(kGThreads), 0, st, M, K, N, N4, dY,
                           X, G);
    } else {
        hipLaunchKernelGGL(dense_grad_kernel<false>, grid, dim3(kGThreads), 0, st, M, K, N, N4, dY,
                           X, G);
    }
    return check_launch("dense_grad");
}
