/*
 * sparsecore_amd.h — C-ABI of the MI355X (gfx950) padded-CSR training path.
 *
 * This is the drop-in boundary that replaces the reference's pybind11 module
 * `sparselab._core` (csrc/bindings.cpp:494-745) for the hot path: forward
 * SpMM, the live-slot weight gradient (SDDMM), the CSR transpose build used
 * for dX = W^T·dY, the transpose-cache value refresh, and the PaddedCSR
 * invariant checker.
 *
 * Conventions
 *   - Every pointer is a DEVICE pointer (HBM) unless the name ends in _host.
 *   - No entry point allocates memory: callers pass outputs and workspaces
 *     (the Python host layer allocates them through torch's caching
 *     allocator).
 *   - Every call is stream-ordered on `stream` (a hipStream_t passed as
 *     void*; NULL means the legacy default stream) and returns without
 *     synchronizing.
 *   - Return value: SLK_OK (0) on success; on failure a non-zero code and a
 *     thread-local message available from slk_last_error(). Messages keep
 *     the substrings the reference raises as ValueError ("shape mismatch",
 *     "ncols", "dY.shape", "X.shape", "shared inner dim N", ...).
 *   - Shapes follow the reference: W is M x K (nrows x ncols), X is K x N
 *     row-major, Y is M x N row-major, dY is M x N, dW has total_capacity
 *     entries aligned with W.values.
 */
#ifndef SPARSECORE_AMD_H
#define SPARSECORE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SLK_ABI_VERSION 16

#if defined(__GNUC__)
#define SLK_API __attribute__((visibility("default")))
#else
#define SLK_API
#endif

enum slk_status {
    SLK_OK = 0,
    SLK_EINVAL = 1,   /* bad shape / argument: the reference raises ValueError  */
    SLK_EDEVICE = 2,  /* HIP runtime error (launch failure, bad device pointer) */
};

/* Order of the per-slot dot products in slk_sddmm.
 *   SLK_DW_SIMD   — the reference AVX2 kernel's order: two 8-wide
 *                   accumulators over 16-float steps, an 8-wide step, a
 *                   3-level horizontal add, then a scalar tail
 *                   (csrc/kernels/spmm_grad_avx2.cpp:112-258).
 *   SLK_DW_SCALAR — the reference scalar kernel's single sequential chain
 *                   (csrc/kernels/spmm_grad.cpp:89-108).                     */
enum slk_dw_order { SLK_DW_SIMD = 0, SLK_DW_SCALAR = 1 };

/* Device view of a PaddedCSR (reference struct: csrc/kernels/padded_csr.hpp:47-74).
 * values/col_indices have total_capacity entries; the three row arrays have
 * nrows entries. Within row i, slots [row_start[i], row_start[i]+row_nnz[i])
 * are live with strictly ascending columns; the rest of the row's capacity is
 * padding (col = -1).                                                        */
typedef struct slk_csr {
    int64_t nrows;
    int64_t ncols;
    int64_t total_capacity;
    const float*   values;
    const int32_t* col_indices;
    const int32_t* row_start;
    const int32_t* row_nnz;
    const int32_t* row_capacity;
    /* Optional (may be NULL): a permutation of [0, nrows) listing rows by
     * descending row_nnz. slk_spmm then starts the longest rows of every
     * column tile first, so skewed rows do not straggle at the end of the
     * grid; results are the same either way. Not part of the reference
     * layout — a schedule the caller caches per topology. */
    const int32_t* row_order;
    /* Rows at the head of row_order that are long against the rest (0 = none;
     * needs row_order; at most nrows). When slk_spmm runs its LDS-staged
     * kernel it runs them as a launch of their own, with fewer rows per
     * wave, and then the rest: a workgroup's waves wait on each other at
     * every staged chunk, so rows much longer than their workgroup's others
     * stall it. Results are the same either way. */
    int64_t n_heavy_rows;
    /* Optional (may be NULL): the live slots of every (row, column block) run
     * cut into segments of at most seg_slots consecutive slots (block b =
     * columns [b*seg_block, (b+1)*seg_block)), as built by
     * slk_seg_list_build: segment e covers slots seg_start[e] ..
     * seg_start[e] + seg_count[e] - 1 of row seg_row[e]. Segments go block by
     * block, then by row; each block's list is padded with empty segments
     * (count 0) to a multiple of SLK_SEG_GROUP, each such group of segments
     * is then stably sorted by count, largest first (so a wave of slk_sddmm
     * takes segments of close counts), and *seg_groups (a device
     * int32) holds the number of such groups in use; n_seg is the arrays'
     * length. slk_sddmm then gives each group of segments one workgroup that
     * stages the block's X rows in LDS and keeps each segment's dY row in
     * registers, consecutive groups on one XCD; results are the same either
     * way. A schedule the caller caches per topology. */
    const int32_t* seg_start;
    const int32_t* seg_row;
    const int32_t* seg_count;
    const int32_t* seg_groups;
    int64_t n_seg;
    int64_t seg_block;
    int64_t seg_slots;
    /* Optional (may be NULL): phase bounds for slk_spmm's gather kernel, as
     * built by slk_phase_bounds_build: phase_lo[r*(n_phases+1) + p] is the
     * first live slot of row r whose column is >= p*ceil(ncols/n_phases). The
     * kernel then sweeps the columns in n_phases launches, each row's fma
     * chain continuing from the partial sum the previous phase left in Y, so
     * the X rows that one phase gathers fit the L2s; the chain, and so every
     * bit, is the same. A schedule the caller caches per topology. */
    const int32_t* phase_lo;
    int64_t n_phases;
    /* Optional (may be NULL): the binned slot stream of slk_spmm's
     * LDS-staged kernel, as built by slk_bin_build for bin_rw rows per wave
     * and bin_h column halves (X staged in chunks of 80 / bin_h rows). It
     * covers positions p in [bin_first, nrows): rows row_order[p] when
     * bin_first > 0 (the rows after the heavy ones), else rows p. Position
     * p goes to unit u = (q / (16 bin_rw)) * 16 + q % 16 as its row j =
     * (q / 16) % bin_rw, q = p - bin_first (a unit is one wave's rows).
     * For unit u and chunk ch, the bytes of bin_cnt[(u * nchunks + ch) * 2]
     * and [.. + 1] (byte j at bits 8 (j mod 4) of word j / 4) count row j's
     * live slots whose column lies in the chunk, and the unit's slots are
     * listed from bin_start[u] on (bin_start[units] = n_bin), chunk by chunk,
     * row by row, in slot order: bin_off = the byte offset of the slot's X
     * row inside the staged chunk, bin_slot = the slot's index into values
     * (read through it, so the stream stays valid when values change). With
     * it, slk_spmm runs those rows on the binned kernel, which reads each
     * chunk's work of a wave as one run with its row counts known, and the
     * rows before bin_first on the LDS-staged kernel; results are the same.
     * A schedule the caller caches per topology. */
    const int32_t* bin_off;
    const int32_t* bin_slot;
    const uint32_t* bin_cnt;
    const int32_t* bin_start;
    int64_t bin_first;
    int64_t bin_rw;
    int64_t bin_h;
    int64_t n_bin;
    /* Optional (0 = none): dense rows. The first n_dense_rows rows of
     * row_order (which must then be given) are the densest, and slk_spmm
     * computes them as a dense product on the matrix cores: the row spread
     * over all ncols columns (0 where no live slot is), and one fp32 K=1
     * MFMA outer product per column in ascending column order. Each such
     * product adds w·x to its sum with one rounding, exactly the fma of the
     * slot-order chain, and an absent column adds 0·x, which leaves the sum
     * as it is; a non-finite X (0·inf is NaN) is caught and the dense rows
     * are then recomputed slot by slot. Results equal the reference's under
     * == (a zero sum may differ in sign). dense_ws is device scratch of at
     * least slk_dense_rows_workspace_bytes(n_dense_rows, ncols) bytes that
     * every call overwrites (calls that share it must be ordered on one
     * stream). Not part of the reference layout: a schedule the caller caches
     * per topology. */
    int64_t n_dense_rows;
    void* dense_ws;
    /* With a segment list (seg_start ...): the rows order[0 ..
     * seg_dense_rows) are left out of the list, and slk_sddmm computes their
     * live slots as dense rows on the matrix cores: per slot the reference's
     * SIMD-order dot product (16 fma chains, then its add tree), each fma a
     * K=1 fp32 MFMA step — the same bits. Needs seg_dense_rows ==
     * n_dense_rows, dense_ws, SLK_DW_SIMD and N a multiple of 64.
     * slk_seg_list_build reads it too and builds the list without those
     * rows. 0 = none. */
    int64_t seg_dense_rows;
} slk_csr;

/* Bytes of slk_csr.dense_ws for n_dense_rows dense rows of an ncols-column
 * matrix (the rows spread densely, padded, plus a status word). No
 * counterpart in the reference; 0 for n_dense_rows <= 0. */
SLK_API int64_t slk_dense_rows_workspace_bytes(int64_t n_dense_rows, int64_t ncols);

/* Padding unit of a segment list: each column block's segments are padded
 * to a multiple of this. slk_sddmm workgroups take 64 or 128 segments. */
#define SLK_SEG_GROUP 128

/* Thread-local description of the last failure of this thread ("" if none). */
SLK_API const char* slk_last_error(void);

/* SLK_ABI_VERSION of the loaded library. */
SLK_API int slk_abi_version(void);

/* Kernel-choice overrides, process-wide, for tests and measurement. No
 * counterpart in the reference (its dispatch is the compile-time
 * AVX2/NEON/scalar choice of csrc/bindings.cpp). Every launcher chooses its
 * kernel variant from the problem shape; a knob set to a value >= 0 replaces
 * that choice for every later launch until it is set back to -1
 * (automatic). Results are the same bits under every setting; only the
 * schedule changes. Values:
 *   SLK_TUNE_SPMM_KERNEL  0 = per-wave gather kernel, 1 = LDS-staged kernel
 *   SLK_TUNE_SPMM_H       LDS kernel: 1 or 2 column halves per lane
 *   SLK_TUNE_SPMM_RW      LDS kernel: rows per wave (2, 4 or 8)
 *   SLK_TUNE_SPMM_SPLIT   LDS kernel: 0 = no separate launch for heavy rows,
 *                         1 = heavy rows and the rest as LDS launches on the
 *                         caller's stream only (automatic: with phase bounds
 *                         the rest runs on the gather kernel on a second
 *                         stream, see slk_spmm)
 *   SLK_TUNE_SPMM_VEC     gather kernel: floats per lane (1, 2 or 4)
 *   SLK_TUNE_SDDMM_G      windowed dW kernel: groups per wave (1, 2 or 4)
 *   SLK_TUNE_SEG_LEAN     segment dW kernel: 1 = lean variant, 0 = not
 *   SLK_TUNE_SEG_GROUP    segment dW kernel: segments per workgroup (64 or 128)
 *   SLK_TUNE_TRANSPOSE_TILE transpose fill: 0 = one workgroup per row block over
 *                         all columns instead of row x column tiles
 *   SLK_TUNE_SPMM_BIN     0 = ignore a binned slot stream (slk_csr.bin_off)
 *   SLK_TUNE_SPMM_G       binned kernel: slots of a row read ahead (1, 2 or 4)
 *   SLK_TUNE_RIGL_TILE    slk_dense_grad_approx: 128 = 128 x 128 tiles staged
 *                         through registers (else 256 x 128 tiles, direct loads)
 *   SLK_TUNE_DENSE_ROWS   0 = run a view's dense rows (slk_csr.n_dense_rows)
 *                         with the other rows instead of on the matrix cores
 *   SLK_TUNE_TRANSPOSE_RADIX transpose: 0 = the counting sort (row-block
 *                         histograms and scatter) everywhere, 1 = the radix
 *                         sort by column wherever ncols <= 65535 (automatic:
 *                         there, for total_capacity >= 2^20)
 * Returns SLK_EINVAL for an unknown knob.                                   */
enum slk_tune_knob {
    SLK_TUNE_SPMM_KERNEL = 0,
    SLK_TUNE_SPMM_H = 1,
    SLK_TUNE_SPMM_RW = 2,
    SLK_TUNE_SPMM_SPLIT = 3,
    SLK_TUNE_SPMM_VEC = 4,
    SLK_TUNE_SDDMM_G = 5,
    SLK_TUNE_SEG_LEAN = 6,
    SLK_TUNE_SEG_GROUP = 7,
    SLK_TUNE_TRANSPOSE_TILE = 8,
    SLK_TUNE_SPMM_BIN = 9,
    SLK_TUNE_SPMM_G = 10,
    SLK_TUNE_RIGL_TILE = 11,
    SLK_TUNE_DENSE_ROWS = 12,
    SLK_TUNE_TRANSPOSE_RADIX = 13,
    SLK_TUNE_COUNT = 14
};
SLK_API int slk_set_tuning(int knob, int64_t value);

/* Y = W·X. Replaces `spmm_simd` / `spmm_scalar` (csrc/bindings.cpp:243-272,
 * kernels csrc/kernels/spmm_avx2.cpp:82-263 and spmm.cpp:20-105). Y is fully
 * written (rows without live slots become 0), so it needs no pre-zeroing.
 * Each Y element is the fused multiply-add chain over the row's live slots in
 * slot order, starting from +0.0 — the same arithmetic as the reference.
 * For a skewed matrix with phase bounds on the LDS-staged path, the rows
 * after the heavy ones run concurrently on a second stream of the library's
 * own, forked from and joined back to `stream` with events (capture-safe:
 * the second stream joins the caller's capture); it and its two events are
 * created on the first such call on a device that is not under capture.      */
SLK_API int slk_spmm(const slk_csr* W, const float* X, int64_t K, int64_t N,
             float* Y, void* stream);

/* Y[i,:] = (W·X)[i,:] + bias[i]: slk_spmm with SparseLinear's bias add
 * (sparselab/nn.py:237-241, `y_flat + self.bias`) fused into the store. Each
 * element is the same fma chain as slk_spmm, then one float32 add of
 * bias[i] — the rounding of the reference's separate add. bias is a device
 * array of W->nrows floats.                                                 */
SLK_API int slk_spmm_bias(const slk_csr* W, const float* X, int64_t K, int64_t N,
                  const float* bias, float* Y, void* stream);

/* dW[s] = dot(dY[i,:], X[col[s],:]) for every live slot s of row i, and
 * dW[s] = 0 for every padding slot. Replaces `spmm_grad_w_simd` /
 * `spmm_grad_w` (csrc/bindings.cpp:318-431). `order` is an slk_dw_order.
 * dY is M x N, X is K x N; dW has W->total_capacity entries.                */
SLK_API int slk_sddmm(const slk_csr* W, const float* dY, int64_t dY_rows,
              const float* X, int64_t X_rows, int64_t N, float* dW,
              int order, void* stream);

/* slk_sddmm plus dbias[i] = sum_j dY[i,j] (W->nrows floats) in the same
 * launch: the gradient of SparseLinear's bias add (sparselab/nn.py:237-241),
 * which the reference gets from torch autograd as a separate reduction. dW
 * is bit-identical to slk_sddmm's; each dbias element is a fixed-order sum
 * (lane-strided partials, then a butterfly), repeatable run to run.         */
SLK_API int slk_sddmm_bias(const slk_csr* W, const float* dY, int64_t dY_rows,
                   const float* X, int64_t X_rows, int64_t N, float* dW,
                   float* dbias, int order, void* stream);

/* Transpose build, part 1 of 2 (replaces the index work of
 * `transpose_with_perm`, sparselab/layout.py:460-536).
 * Bytes of device workspace slk_transpose_count needs for W.                */
SLK_API int64_t slk_transpose_workspace_bytes(const slk_csr* W);

/* Counting pass: per-row-block column histograms, WT row_nnz, WT
 * row_capacity = max(1, ceil(nnz * (1 + padding_ratio))) evaluated in
 * float64 (layout.py:46-68), WT row_start = exclusive scan of the
 * capacities, and *capT_dev = total WT capacity (one int64 on the device).
 * WT arrays have W->ncols entries.                                          */
SLK_API int slk_transpose_count(const slk_csr* W, double padding_ratio,
                        void* workspace, int64_t workspace_bytes,
                        int32_t* WT_row_start, int32_t* WT_row_nnz,
                        int32_t* WT_row_capacity, int64_t* capT_dev,
                        void* stream);

/* Fill pass: stable scatter of W's live slots into WT (each WT row lists its
 * source rows in ascending order), padding = (col -1, value 0, perm -1).
 * perm[t] = slot of W whose value sits at WT slot t (int64, -1 on padding).
 * `workspace` must be the one slk_transpose_count filled for this W.       */
SLK_API int slk_transpose_fill(const slk_csr* W, const void* workspace,
                       int64_t workspace_bytes,
                       const int32_t* WT_row_start, const int32_t* WT_row_nnz,
                       const int32_t* WT_row_capacity, int64_t capT,
                       float* WT_values, int32_t* WT_col_indices,
                       int64_t* perm, void* stream);

/* Cache-hit refresh: WT_values[t] = W_values[perm[t]] where perm[t] >= 0;
 * padding slots are left as they are. Replaces the numpy gather of
 * `_cached_transpose` (sparselab/ops.py:83-94).                              */
SLK_API int slk_transpose_refresh(const float* W_values, int64_t W_capacity,
                          const int64_t* perm, int64_t capT,
                          float* WT_values, void* stream);

/* Counts of a row_nnz array (n entries, int32) written to device memory:
 * out[0] = entries with (double)row_nnz[i] > heavy_bar, out[1] = entries
 * with (double)row_nnz[i] >= dense_bar, or 0 when fewer than
 * dense_min_rows. No counterpart in the reference: it computes the heavy-
 * and dense-row hints of a freshly built transpose (the rules of
 * layout.heavy_row_count / layout.dense_row_count in this package) on the
 * device, so the host reads them with the transpose's capacity in one read. */
SLK_API int slk_row_hints(const int32_t* row_nnz, int64_t n, double heavy_bar,
                          double dense_bar, int64_t dense_min_rows, int64_t* out, void* stream);

/* Invariant scan of a device PaddedCSR (the checks of
 * csrc/kernels/padded_csr.cpp:79-196, invariants 3-7). Writes
 * SLK_CHECK_WORDS int64 words to result_dev:
 *   [0] sum of row_capacity
 *   [1] first row violating invariant 3 (INT64_MAX if none)
 *   [2] first row violating invariant 4 (INT64_MAX if none)
 *   [3] first (row << 32 | slot-in-row) with a live-column violation
 *       (invariant 6), INT64_MAX if none
 *   [4] first (row << 32 | slot-in-row) with a padding column != -1
 *       (invariants 5+7), INT64_MAX if none
 * Slot checks are only evaluated for rows whose [row_start, row_start+cap)
 * lies inside the arrays, so a malformed CSR never causes an out-of-bounds
 * read. The caller formats the reference's message from these words.       */
#define SLK_CHECK_WORDS 5
SLK_API int slk_check_invariants(const slk_csr* W, int64_t col_indices_len,
                         int64_t* result_dev, void* stream);

/* ─── Topology mutation (SET / RigL) and the dense gradient ───────────── */

/* Bytes of device workspace slk_live_abs_kth needs (independent of W). */
#define SLK_KTH_WORKSPACE_BYTES 8448

/* *thr_dev = the k-th smallest |values[s]| over W's live slots (1 <= k <=
 * number of live slots), i.e. np.partition(np.abs(live), k-1)[k-1] — the
 * global drop threshold of SET and RigL (sparselab/router.py:394-412 and
 * :648-661). Exact: a radix select on the float bits, no rounding.        */
SLK_API int slk_live_abs_kth(const slk_csr* W, int64_t k, void* workspace,
                             int64_t workspace_bytes, float* thr_dev, void* stream);

/* Grow rule of slk_drop_grow. */
enum slk_grow_rule {
    SLK_GROW_RANDOM = 0,   /* SET: uniform over the row's empty columns       */
    SLK_GROW_GRADIENT = 1, /* RigL: largest |G[i, c]| over the empty columns  */
};

/* Bytes of device workspace slk_drop_grow needs for W (row staging).       */
SLK_API int64_t slk_drop_grow_workspace_bytes(const slk_csr* W);

/* One SET / RigL drop-and-grow pass over every row of W, in place
 * (replaces the per-row loop of sparselab/router.py:414-478 for SET and
 * :663-732 for RigL, with its PaddedCSR.rewrite_row calls,
 * csrc/kernels/padded_csr.cpp:219-296). For each row with live slots:
 *   keep the slots with |v| > *thr_dev (if none, the first slot of largest
 *   |v|); grow n_grow = min(dropped, growable columns) columns outside the
 *   kept set with value 0 and write the row back sorted by column.
 * Growable columns: SLK_GROW_RANDOM, every column outside the kept set;
 * SLK_GROW_GRADIENT, those whose |G[i*ldg + c]| is not NaN (the reference
 * counts only |G| > -inf as available, router.py:704-705). Grow choice:
 * SLK_GROW_GRADIENT takes the n_grow largest |G| (ties: lower column
 * first); SLK_GROW_RANDOM takes the n_grow smallest 32-bit keys
 * splitmix64(seed, i*ncols + c), which is a uniform random subset (the
 * reference draws it with numpy's Generator.choice, a stream this cannot
 * reproduce). row_start and the capacities never change. A row regrows what
 * it dropped, except a RigL row that runs out of growable columns: it
 * shrinks, its trailing slots become padding and row_nnz[i] is lowered.
 * values, col_indices and row_nnz must be W's own arrays. *removed (a
 * device int64) receives the number of live slots the pass removed in total
 * (0 unless some row shrank). ncols is at most 131072.                       */
SLK_API int slk_drop_grow(const slk_csr* W, float* values, int32_t* col_indices,
                          int32_t* row_nnz, const float* thr_dev, int rule, const float* G,
                          int64_t ldg, uint64_t seed, void* workspace,
                          int64_t workspace_bytes, int64_t* removed, void* stream);

/* slk_drop_grow without a workspace argument and without any allocation:
 * the row staging lives in a static device array of the library ("scratch",
 * SLK_DROP_GROW_NOALLOC_MAX_SLOTS * 8 bytes = 16 MiB, one copy per GPU the
 * library runs on, held until the process ends). No counterpart in the
 * reference: it is for callers that cannot allocate device memory — code
 * under HIP graph capture, tight serving or training loops, harnesses that
 * forbid hipMalloc. Same arguments (minus the workspace), same results bit
 * for bit as slk_drop_grow. W->total_capacity must be at most
 * SLK_DROP_GROW_NOALLOC_MAX_SLOTS (SLK_EINVAL otherwise, before any device
 * work). Every call on one GPU shares that GPU's scratch, which keeps the
 * last call's contents (each call writes what it reads first): calls that
 * overlap on one GPU — on two streams, or from two threads — race, so
 * order them on one stream. The first call on a device looks up that
 * device's address of the array (hipGetSymbolAddress), with the device
 * current.                                                                  */
#define SLK_DROP_GROW_NOALLOC_MAX_SLOTS (1 << 21)
SLK_API int slk_drop_grow_noalloc(const slk_csr* W, float* values, int32_t* col_indices,
                                  int32_t* row_nnz, const float* thr_dev, int rule,
                                  const float* G, int64_t ldg, uint64_t seed, int64_t* removed,
                                  void* stream);

/* G = dY·X^T, G is M x K row-major: G[i,k] = sum_j dY[i,j]·X[k,j], each
 * element one running sum over j in order, with the arithmetic of the
 * reference build (products of whole 4-element groups rounded, then added;
 * the last N mod 4 terms fused). Replaces `_core.dense_grad`
 * (csrc/bindings.cpp:445-485, csrc/kernels/dense_grad.cpp:24-84).
 * token_major = 0: dY is M x N and X is K x N (the reference's layout);
 * token_major = 1: dY is N x M and X is N x K (a layer's (tokens, features)
 * activations, as RigL captures them), read without a transpose copy.     */
SLK_API int slk_dense_grad(const float* dY, const float* X, int64_t M, int64_t K,
                           int64_t N, int token_major, float* G, void* stream);

/* ─── RigL grow choice from a certified approximate gradient ──────────────
 *
 * The same rows as slk_drop_grow with SLK_GROW_GRADIENT on G = dY·X^T (the
 * reference build's dense_grad arithmetic), bit for bit, without computing
 * that G everywhere. No counterpart entry in the reference; replaces its
 * RigL._update_layer (sparselab/router.py:598-732) with _core.dense_grad.
 * Four calls, in stream order:
 *   slk_rigl_norms         row norms of dY (M x N) and X (K x N), row-major;
 *   slk_dense_grad_approx  G' = dY·X^T on the matrix cores (fp32 split into
 *                          bf16 parts), M x K row-major;
 *   slk_rigl_count         per row: survivors, the empty columns whose rank
 *                          |G'| certifies, and those it cannot (undecided);
 *                          their counts, and (for rows of up to 16384
 *                          columns, K % 16 == 0) their lists;
 *   slk_rigl_finish        per row: exact G of the undecided columns, the
 *                          grow choice, the rewrite (as slk_drop_grow).
 * The caller sizes amb_ws before slk_rigl_count (8 bytes per undecided
 * column it accepts) and reads *amb_total after it: a total above that
 * capacity means the lists are incomplete and the finish must not run (the
 * caller computes G exactly instead). |G'[i,k] - G[i,k]| <=
 * slk_rigl_bound_factor(N)·nrm_dY[i]·nrm_X[k] + slk_rigl_partial_factor(N)·
 * 2^(G_code[i,k] - 127) + 2^-100·(1 + nrm_dY[i] + nrm_X[k]) for norms up to
 * 2^60 (larger or non-finite norms make the row exact: every empty column is
 * computed exactly). G_code (one byte per element of G', row-major M x K) is
 * written by slk_dense_grad_approx: 2^(G_code - 127) bounds the element's sum
 * of |partial sums of G'| at the ends of its 128-term chunks, which bounds
 * the reference's own rounding far tighter than a multiple of n_i·n_k.      */

/* nrm_dY[i] >= ||dY_i||_2, nrm_X[k] >= ||X_k||_2 (+inf where not finite). */
SLK_API int slk_rigl_norms(const float* dY, int64_t M, const float* X, int64_t K, int64_t N,
                           float* nrm_dY, float* nrm_X, void* stream);

/* Bytes of device workspace slk_dense_grad_approx needs: both operands split
 * into bf16 parts, (M + K) * ceil(N / 32) * 128.                            */
SLK_API int64_t slk_dense_grad_approx_workspace_bytes(int64_t M, int64_t K, int64_t N);

/* G' = dY·X^T within the bound above, and its partial-sum codes G_code (M x K
 * bytes); dY is M x N and X is K x N, row-major. */
SLK_API int slk_dense_grad_approx(const float* dY, const float* X, int64_t M, int64_t K,
                                  int64_t N, float* G, uint8_t* G_code, void* workspace,
                                  int64_t workspace_bytes, void* stream);

/* The factors of the bound above (host functions, no device work). */
SLK_API double slk_rigl_bound_factor(int64_t N);
SLK_API double slk_rigl_partial_factor(int64_t N);

/* Per row of W: survivors of *thr_dev (the global drop threshold, as for
 * slk_drop_grow) and the empty columns the bound leaves undecided. info:
 * 32 bytes per row (opaque to the caller, read by slk_rigl_finish); amb_off:
 * 2*nrows + 1 int64: row i's undecided columns are pairs
 * [amb_off[i], amb_off[i] + amb_off[nrows + 1 + i]) of the list, and
 * *amb_total = amb_off[nrows] (device int64) their total. amb_ws (8 bytes per
 * pair, amb_ws_bytes of them) and workspace (as slk_drop_grow's) are the
 * ones slk_rigl_finish then receives: the lists go there. ncols at most
 * 131072.                                                                   */
SLK_API int slk_rigl_count(const slk_csr* W, const float* thr_dev, const float* G_approx,
                           int64_t ldg, const uint8_t* G_code, const float* nrm_dY,
                           const float* nrm_X, int64_t N, void* info, int64_t* amb_off,
                           int64_t* amb_total, void* amb_ws, int64_t amb_ws_bytes,
                           void* workspace, int64_t workspace_bytes, void* stream);

/* Finishes the RigL pass slk_rigl_count began: values, col_indices and
 * row_nnz must be W's own arrays (rewritten as slk_drop_grow rewrites them);
 * amb_ws and workspace the ones slk_rigl_count received, with
 * amb_ws_bytes >= 8 * *amb_total; *removed as slk_drop_grow's.             */
SLK_API int slk_rigl_finish(const slk_csr* W, float* values, int32_t* col_indices,
                            int32_t* row_nnz, const float* thr_dev, const float* G_approx,
                            int64_t ldg, const uint8_t* G_code, const float* nrm_dY,
                            const float* nrm_X,
                            const float* dY, const float* X, int64_t N, const void* info,
                            const int64_t* amb_off, void* amb_ws, int64_t amb_ws_bytes,
                            void* workspace, int64_t workspace_bytes, int64_t* removed,
                            void* stream);

/* ─── Dense layout ─────────────────────────────────────────────────────── */

/* dst = src^T for a float32 matrix: src is rows x cols with row stride
 * ld_src (>= cols), dst is cols x rows row-major; a bitwise copy. Replaces
 * the layout copies around the kernels: SparseLinear's `x.t().contiguous()`
 * (sparselab/nn.py:235) and the backward's `dY.contiguous()` of a transposed
 * gradient (sparselab/ops.py:174).                                          */
SLK_API int slk_transpose_dense(const float* src, int64_t rows, int64_t cols,
                                int64_t ld_src, float* dst, void* stream);

/* Yt = (W·X)^T (+ bias[i] on row i): slk_spmm / slk_spmm_bias with the
 * result stored token-major, Yt[n*M + i] = Y[i, n] (N x M row-major) — the
 * layout of SparseLinear's output y = (W·xᵀ)ᵀ (sparselab/nn.py:229-241),
 * written directly for a consumer that needs it contiguous (a loss on a
 * narrow classifier layer). The same fma chain and bias rounding as
 * slk_spmm_bias; bias may be NULL.                                           */
SLK_API int slk_spmm_t(const slk_csr* W, const float* X, int64_t K, int64_t N,
                       const float* bias, float* Yt, void* stream);

/* Largest W slk_backward_narrow takes (rows; slots, staged in LDS).          */
#define SLK_NARROW_MAX_ROWS 64
#define SLK_NARROW_MAX_CAPACITY 8192

/* Backward of a narrow layer (W->nrows <= SLK_NARROW_MAX_ROWS and
 * W->total_capacity <= SLK_NARROW_MAX_CAPACITY) in one launch, from the
 * token-major output gradient dYt (N x M, dY[i, n] = dYt[n*M + i]):
 *   dW    — as slk_sddmm in `order` (live slots; padding 0), if not NULL;
 *   dbias — as slk_sddmm_bias's dbias (M floats), if not NULL;
 *   dX    — W^T·dY, K x N row-major, bit-identical to slk_spmm on the
 *           transpose slk_transpose_fill builds (each element the fma chain
 *           over column c's rows in ascending order from +0.0), if not NULL.
 * X is the layer input, X_rows x N row-major with X_rows == W->ncols (read
 * only for dW). Replaces, for such layers, the dY.contiguous(), the dW call,
 * the transpose-cache refresh and spmm(WT, dY) of the reference backward
 * (sparselab/ops.py:160-210).                                               */
SLK_API int slk_backward_narrow(const slk_csr* W, const float* dYt, int64_t N, const float* X,
                                int64_t X_rows, float* dW, float* dbias, float* dX, int order,
                                void* stream);

/* Backward of a small layer in one launch (the caller chooses it where the
 * three kernels are each a few microseconds of latency), from the row-major
 * output gradient dY (M x N) and the layer input X (K x N):
 *   dW    — as slk_sddmm in the SIMD order (live slots; padding 0);
 *   dbias — as slk_sddmm_bias's dbias (M floats), if not NULL;
 *   dX    — W^T·dY, K x N row-major, bit-identical to slk_spmm(WT, dY) after
 *           slk_transpose_refresh: WT is W's transpose from
 *           slk_transpose_fill (its structure: row_start, row_nnz,
 *           col_indices; its values are not read) and perm its slot map
 *           (WT slot s holds W slot perm[s]); W's values are read through
 *           perm, so no refresh is needed first.
 * Replaces, for such layers, the dW call, the transpose-cache refresh and
 * spmm(WT, dY) of the reference backward (sparselab/ops.py:160-210).       */
SLK_API int slk_backward_fused(const slk_csr* W, const slk_csr* WT, const int64_t* perm,
                               const float* dY, const float* X, int64_t N, float* dW,
                               float* dbias, float* dX, void* stream);

/* Length of the segment arrays slk_seg_list_build needs for W, block_cols
 * and seg_slots (an upper bound on the padded segment count, so the list can
 * be built without reading anything back to the host); 0 on bad arguments. */
SLK_API int64_t slk_seg_list_capacity(const slk_csr* W, int64_t block_cols, int64_t seg_slots);

/* Bytes of device workspace slk_seg_list_build needs for W and block_cols. */
SLK_API int64_t slk_seg_list_workspace_bytes(const slk_csr* W, int64_t block_cols);

/* Builds the optional segment schedule of slk_csr on the device (see
 * seg_start there): block_cols is 64 or 128 columns, seg_slots 4 or 8; the
 * three arrays hold n_seg >= slk_seg_list_capacity entries, and *seg_groups
 * receives the number of SLK_SEG_GROUP-segment groups in use. Entries past
 * the padded list are left as empty segments. Deterministic, no atomics.
 * No counterpart in the reference (csrc/kernels/spmm_grad_avx2.cpp walks
 * slots in capacity order): a visiting order for slk_sddmm that leaves
 * every output bit unchanged.                                               */
SLK_API int slk_seg_list_build(const slk_csr* W, int64_t block_cols, int64_t seg_slots,
                               void* workspace, int64_t workspace_bytes, int32_t* seg_start,
                               int32_t* seg_row, int32_t* seg_count, int64_t n_seg,
                               int32_t* seg_groups, void* stream);

/* Builds the optional phase bounds of slk_csr (see phase_lo there) on the
 * device: phase_lo receives W->nrows * (n_phases + 1) int32 entries, n_phases
 * >= 1. No counterpart in the reference (csrc/kernels/spmm_avx2.cpp walks
 * each row's slots in one pass): a visiting schedule for slk_spmm that leaves
 * every output bit unchanged.                                               */
SLK_API int slk_phase_bounds_build(const slk_csr* W, int64_t n_phases, int32_t* phase_lo,
                                   void* stream);

/* Sizes of the binned slot stream of slk_csr (see bin_off there) for W's
 * positions [first, nrows), rw rows per wave (1, 2, 4 or 8) and h column
 * halves (1 or 2): *units (wave units; bin_start has units + 1 entries,
 * bin_cnt 2 * units * *nchunks words) and *nchunks (X chunks of 80 / h
 * rows). SLK_EINVAL where the stream is not supported: bad arguments, or
 * more than SLK_BIN_MAX_CHUNKS chunks (ncols beyond 80 * that / h).       */
#define SLK_BIN_MAX_CHUNKS 960
SLK_API int slk_bin_sizes(const slk_csr* W, int64_t first, int64_t rw, int64_t h,
                          int64_t* units, int64_t* nchunks);

/* Builds the binned slot stream (see bin_off in slk_csr) on the device: two
 * launches, deterministic, no host read. n_bin (the length of bin_off and
 * bin_slot) must be at least the live slots of the covered rows; bin_start
 * receives units + 1 entries, bin_cnt 2 * units * nchunks words. Rows before
 * `first` are W->row_order's first `first` (first > 0 needs row_order). No
 * counterpart in the reference (csrc/kernels/spmm_avx2.cpp walks each row's
 * slots in one pass): a visiting schedule for slk_spmm that leaves every
 * output bit unchanged.                                                     */
SLK_API int slk_bin_build(const slk_csr* W, int64_t first, int64_t rw, int64_t h,
                          int32_t* bin_off, int32_t* bin_slot, int64_t n_bin,
                          uint32_t* bin_cnt, int32_t* bin_start, void* stream);

/* Diagnostic with no counterpart in the reference: n independent
 * 32 x 32 x 16 bf16 matrix-core products with an fp32 accumulator, the
 * instruction slk_dense_grad_approx accumulates G' with:
 * D[t] = C[t] + A[t]·B[t]^T, A[t] and B[t] 32 x 16 bf16 (raw bits,
 * row-major), C[t] and D[t] 32 x 32 float row-major. For checking the
 * rounding model the certified RigL bound assumes (each accumulation step
 * within 2u of its exact value relative to the magnitudes summed).          */
SLK_API int slk_rigl_mfma_probe(const uint16_t* A, const uint16_t* B, const float* C, float* D,
                                int64_t n, void* stream);

/* Diagnostic with no counterpart in the reference: n independent fp32
 * 32 x 32 x 1 (two-block) matrix-core outer products, the instruction the
 * dense rows of slk_spmm (slk_csr.n_dense_rows) accumulate with, run on
 * given operands in its register layout: for case t and lane l, A[t*64+l]
 * and B[t*64+l] are the lane's A and B values and C[(t*64+l)*32+r] its
 * accumulator register r; D gets the result in the same place. Register r of
 * lane l holds block b = r/16, row 8((r mod 16)/4) + 4(l/32) + r mod 4 of A's
 * lanes 32b.., column l mod 32 of B's lanes 32b..: D = fma(A[32b + row],
 * B[32b + l mod 32], C) there. For checking that the instruction rounds as
 * one fma.                                                                  */
SLK_API int slk_dense_mfma_probe(const float* A, const float* B, const float* C, float* D,
                                 int64_t n, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SPARSECORE_AMD_H */
