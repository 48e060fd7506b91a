// Shared helpers for the gfx950 padded-CSR kernels: error reporting,
// launch checking and small device utilities. Host and device code.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <utility>
#include <string>

#include "sparsecore_amd.h"

namespace slk {

constexpr int kWave = 64;  // CDNA wavefront width

// Records `msg` as this thread's last error and returns `code`.
int fail(int code, const std::string& msg);

// Clears this thread's last error (called at the start of every entry point).
void clear_error();

// Converts a pending launch error into SLK_EDEVICE with context `what`.
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Current value of a kernel-choice override (slk_set_tuning); -1 = automatic.
int64_t tuning(int knob);

// Validates the parts of a CSR view every kernel relies on.
int validate_csr(const slk_csr* W, const char* who);

// A second queue per device, for launchers that run two independent parts
// of one call concurrently (slk_spmm's split forward, slk_sddmm's dense rows):
// one stream (default priority) and the two events that fork it from and join
// it back to the caller's stream. Created on the first such call on the device
// that is not made under graph capture (until then such calls keep to one
// stream) and kept until the process ends. side_mutex() is held from the fork
// to the join, so calls from several host threads cannot interleave their
// event records; side_queue() is called with it held and returns nullptr if no
// queue is available.
struct SideQueue {
    hipStream_t s = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
};
std::mutex& side_mutex();
SideQueue* side_queue(hipStream_t st);

// MI355X has 8 XCDs (each with its own L2); the dispatcher hands workgroup b
// to XCD (b mod 8). This renumbers workgroups so that every XCD receives one
// contiguous range of logical workgroups: consecutive work (same X column
// tile, neighbouring rows) then shares one L2 instead of being spread over
// all eight. A bijection on [0, nb); if the dispatch order differed only
// cache locality would change, never the result.
constexpr int kXcds = 8;

__device__ __forceinline__ int64_t xcd_logical_block(int64_t b, int64_t nb) {
    const int64_t x = b % kXcds, q = b / kXcds;
    const int64_t per = nb / kXcds, extra = nb % kXcds;
    return x * per + (x < extra ? x : extra) + q;
}

// Wave index of the calling thread over XCD-grouped workgroups, made
// wave-uniform so that values derived from it live in scalar registers (and
// row metadata loads become scalar).
__device__ __forceinline__ int64_t wave_id() {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    return xcd_logical_block(blockIdx.x, gridDim.x) * (blockDim.x >> 6) + w;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// f(std::integral_constant<int, j>{}) for j = 0..N-1, unrolled at compile time
// (so array indexes derived from j are constants, never private memory).
template <class F, int... J>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, J...>) {
    (f(std::integral_constant<int, J>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

}  // namespace slk
