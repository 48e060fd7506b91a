// Error state and argument validation shared by every entry point.
#include "common.hpp"

#include <atomic>
#include <mutex>

namespace slk {

namespace {
thread_local std::string g_last_error;
// Kernel-choice overrides, process-wide; -1 = the launcher's own choice
// (every knob, whatever their number: a braced list shorter than the array
// would leave the rest at 0).
struct Tuning {
    std::atomic<int64_t> v[SLK_TUNE_COUNT];
    Tuning() {
        for (auto& x : v) x.store(-1, std::memory_order_relaxed);
    }
};
Tuning g_tuning;
}

int64_t tuning(int knob) { return g_tuning.v[knob].load(std::memory_order_relaxed); }

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_side_mu;
SideQueue g_side[kMaxDevices];
}  // namespace

std::mutex& side_mutex() { return g_side_mu; }

SideQueue* side_queue(hipStream_t st) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        return nullptr;
    }
    SideQueue& q = g_side[dev];
    if (q.s != nullptr) return &q;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
        (void)hipGetLastError();
        return nullptr;
    }
    hipStream_t s = nullptr;
    hipEvent_t f = nullptr, j = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&f, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&j, hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        if (j != nullptr) (void)hipEventDestroy(j);
        if (f != nullptr) (void)hipEventDestroy(f);
        if (s != nullptr) (void)hipStreamDestroy(s);
        return nullptr;
    }
    q.s = s;
    q.fork = f;
    q.join = j;
    return &q;
}

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

void clear_error() { g_last_error.clear(); }

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        return fail(SLK_EDEVICE, std::string(what) + ": kernel launch failed: " +
                                     hipGetErrorString(e));
    }
    return SLK_OK;
}

int validate_csr(const slk_csr* W, const char* who) {
    if (W == nullptr) return fail(SLK_EINVAL, std::string(who) + ": W is NULL");
    if (W->nrows < 0 || W->ncols < 0 || W->total_capacity < 0) {
        return fail(SLK_EINVAL, std::string(who) + ": negative shape (" +
                                    std::to_string(W->nrows) + ", " +
                                    std::to_string(W->ncols) + ")");
    }
    if (W->total_capacity > INT32_MAX) {
        return fail(SLK_EINVAL, std::string(who) +
                                    ": total_capacity exceeds the int32 slot index range");
    }
    if (W->nrows > 0 &&
        (W->row_start == nullptr || W->row_nnz == nullptr || W->row_capacity == nullptr)) {
        return fail(SLK_EINVAL, std::string(who) + ": NULL row array");
    }
    if (W->total_capacity > 0 && (W->values == nullptr || W->col_indices == nullptr)) {
        return fail(SLK_EINVAL, std::string(who) + ": NULL slot array");
    }
    if (W->n_heavy_rows < 0 || W->n_heavy_rows > W->nrows ||
        (W->n_heavy_rows > 0 && W->row_order == nullptr)) {
        return fail(SLK_EINVAL, std::string(who) + ": n_heavy_rows=" +
                                    std::to_string(W->n_heavy_rows) +
                                    " needs row_order and must lie in [0, nrows]");
    }
    if (W->seg_start != nullptr &&
        (W->seg_row == nullptr || W->seg_count == nullptr || W->seg_groups == nullptr ||
         W->n_seg < 0 || (W->seg_block != 64 && W->seg_block != 128) ||
         (W->seg_slots != 4 && W->seg_slots != 8))) {
        return fail(SLK_EINVAL, std::string(who) +
                                    ": a segment list needs seg_row, seg_count, seg_groups, "
                                    "n_seg >= 0, seg_block 64 or 128 and seg_slots 4 or 8");
    }
    if (W->n_dense_rows < 0 || W->n_dense_rows > W->nrows ||
        (W->n_dense_rows > 0 && (W->row_order == nullptr || W->dense_ws == nullptr))) {
        return fail(SLK_EINVAL, std::string(who) + ": n_dense_rows=" +
                                    std::to_string(W->n_dense_rows) +
                                    " needs row_order and dense_ws and must lie in [0, nrows]");
    }
    if (W->seg_dense_rows < 0 || W->seg_dense_rows > W->nrows ||
        (W->seg_dense_rows > 0 && W->row_order == nullptr)) {
        return fail(SLK_EINVAL, std::string(who) + ": seg_dense_rows=" +
                                    std::to_string(W->seg_dense_rows) +
                                    " needs row_order and must lie in [0, nrows]");
    }
    if (W->phase_lo != nullptr && W->n_phases < 1) {
        return fail(SLK_EINVAL, std::string(who) + ": phase_lo needs n_phases >= 1, got " +
                                    std::to_string(W->n_phases));
    }
    if (W->bin_off != nullptr &&
        (W->bin_slot == nullptr || W->bin_cnt == nullptr || W->bin_start == nullptr ||
         W->n_bin < 0 || W->bin_first < 0 || W->bin_first > W->nrows ||
         (W->bin_first > 0 && W->row_order == nullptr) ||
         (W->bin_rw != 1 && W->bin_rw != 2 && W->bin_rw != 4 && W->bin_rw != 8) ||
         (W->bin_h != 1 && W->bin_h != 2))) {
        return fail(SLK_EINVAL, std::string(who) +
                                    ": a binned stream needs bin_slot, bin_cnt, bin_start, "
                                    "n_bin >= 0, bin_first in [0, nrows] (row_order if > 0), "
                                    "bin_rw 1, 2, 4 or 8 and bin_h 1 or 2");
    }
    return SLK_OK;
}

}  // namespace slk

extern "C" const char* slk_last_error(void) { return slk::g_last_error.c_str(); }

extern "C" int slk_abi_version(void) { return SLK_ABI_VERSION; }

extern "C" int slk_set_tuning(int knob, int64_t value) {
    slk::clear_error();
    if (knob < 0 || knob >= SLK_TUNE_COUNT) {
        return slk::fail(SLK_EINVAL, "set_tuning: unknown knob " + std::to_string(knob));
    }
    slk::g_tuning.v[knob].store(value < 0 ? -1 : value, std::memory_order_relaxed);
    return SLK_OK;
}
