// Shared plumbing of libenilnets_amd: status/error reporting, the library
// stream, the per-device workspace and small device helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>
#include <type_traits>

#include "enilnets_amd.h"

namespace enq {

// ---- errors -------------------------------------------------------------
// The last failure message of the calling thread (enq_last_error()).
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
const char* last_error();

// Thrown inside the library and turned into a status at the C boundary.
struct Failure {
  int status;
};

[[noreturn]] void fail(int status, const char* fmt, ...)
    __attribute__((format(printf, 2, 3)));

#define ENQ_HIP(call)                                                      \
  do {                                                                     \
    hipError_t enq_err_ = (call);                                          \
    if (enq_err_ != hipSuccess)                                            \
      ::enq::fail(ENQ_ERR_RUNTIME, "%s failed: %s (%s:%d)", #call,         \
                  hipGetErrorString(enq_err_), __FILE__, __LINE__);        \
  } while (0)

#define ENQ_REQUIRE(cond, ...)                                 \
  do {                                                         \
    if (!(cond)) ::enq::fail(ENQ_ERR_INVALID, __VA_ARGS__);    \
  } while (0)

// Runs `body` and maps a Failure (or any C++ exception) to a status code.
template <class F>
int guarded(F&& body) {
  try {
    body();
    return ENQ_OK;
  } catch (const Failure& f) {
    return f.status;
  } catch (...) {
    set_error("unexpected C++ exception");
    return ENQ_ERR_RUNTIME;
  }
}

// ---- device state -------------------------------------------------------
// Fails with ENQ_ERR_NO_DEVICE unless enq_init() succeeded.
void require_init();
hipStream_t stream();
int device_cu_count();

// Growable per-device scratch memory for partial results.  A call may use
// `bytes` of it until it returns; calls on the library stream are ordered,
// so reuse across calls is safe.  Growing synchronizes the stream first.
// Slot kKernelSlot belongs to the single-operation entry points (dense, W8A8,
// quantize); kLayerSlot to layer-level entry points (attention, MoE) that
// call those operations while their own buffers stay live.
constexpr int kKernelSlot = 0;
constexpr int kLayerSlot = 1;
void* workspace(size_t bytes, int slot = kKernelSlot);

// Fixed device scratch of the allocation-free entry point
// (enq_dense_w8_noalloc): a file-scope device array, one copy per device,
// whose address enq_init looks up once per device.  Returns the current
// device's copy; fails with ENQ_ERR_INVALID when `bytes` exceeds it.  It
// allocates nothing, and every call on a device shares the one array.
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
void* noalloc_scratch(size_t bytes);

// Checks the launch that was just enqueued.
void check_launch(const char* what);

// ---- small helpers ------------------------------------------------------
__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline bool aligned(const void* p, size_t a) {
  return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

}  // namespace enq

// ---- device-side helpers (header-only) ----------------------------------
namespace enq {

// Round half to even, as np.round: rint uses the current rounding mode,
// which is round-to-nearest-even on AMDGPU.
__device__ __forceinline__ float round_even(float v) { return __builtin_rintf(v); }
__device__ __forceinline__ double round_even(double v) { return __builtin_rint(v); }

template <class T>
__device__ __forceinline__ bool is_nan(T v) { return v != v; }

// f(integral_constant<int, I>) for I in [B, E), unrolled at compile time:
// register arrays indexed by I stay in registers where a `#pragma unroll`
// loop whose body is too large to unroll would leave them in scratch.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// np.clip(v, lo, hi): NaN passes through, -0.0 is kept.
template <class T>
__device__ __forceinline__ T clip(T v, T lo, T hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

}  // namespace enq
