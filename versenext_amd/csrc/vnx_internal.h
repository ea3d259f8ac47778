// Host-side helpers shared by the vnx entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/vnx.h"
#include "vnx_common.h"

namespace vnx {

// Records the HIP error text for vnx_last_hip_error() and maps it to a status.
int hip_fail(hipError_t e);

#define VNX_HIP_CHECK(expr)                          \
  do {                                               \
    hipError_t _e = (expr);                          \
    if (_e != hipSuccess) return ::vnx::hip_fail(_e); \
  } while (0)

// Checks the launch that was just enqueued.
#define VNX_LAUNCH_CHECK() VNX_HIP_CHECK(hipGetLastError())

// Builds the temperature-scaling descriptor for T > 0 (see scale_logit):
// mode 0 for T == 1, mode 1 when the Markstein step is exact for every fp32
// significand with this T (checked once per T on the host), else mode 2.
Scale make_scale(float T);

// Bump allocator over a caller-provided workspace (256-byte aligned slices).
struct Carve {
  char* base;
  size_t used = 0;
  explicit Carve(void* p) : base(static_cast<char*>(p)) {}
  template <typename T>
  T* take(size_t n) {
    size_t off = (used + 255) & ~size_t(255);
    used = off + n * sizeof(T);
    return base ? reinterpret_cast<T*>(base + off) : nullptr;
  }
  size_t bytes() const { return (used + 255) & ~size_t(255); }
};

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int elem_size(int dtype) { return dtype == VNX_F32 ? 4 : 2; }

// Zeroes n arrival counters on `st` (a kernel, not a memset, so the call
// stays valid inside captured HIP graphs).
int zero_counters(unsigned* p, int64_t n, hipStream_t st);

// Chunks per row for the streaming row kernels: enough workgroups to cover
// every CU several times, chunks no shorter than one 256-thread x 16-byte pass.
int pick_chunks(int64_t rows, int64_t V, int vec_elems, int max_chunks);

}  // namespace vnx
