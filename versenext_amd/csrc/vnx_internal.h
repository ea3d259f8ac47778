// Helpers shared by the vnx entry points (host side, plus the RoPE / KV-cache
// arguments of the projection epilogue).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/vnx.h"
#include "vnx_common.h"

namespace vnx {

// Records the HIP error text for vnx_last_hip_error() and maps it to a status.
int hip_fail(hipError_t e);

// Resolves this device's copy of the fixed scratch of the allocation-free
// entry point (spec.hip); the device must be current.  Idempotent.
int spec_scratch_init(int device);

#define VNX_HIP_CHECK(expr)                          \
  do {                                               \
    hipError_t _e = (expr);                          \
    if (_e != hipSuccess) return ::vnx::hip_fail(_e); \
  } while (0)

// Checks the launch that was just enqueued.
#define VNX_LAUNCH_CHECK() VNX_HIP_CHECK(hipGetLastError())

// Fills the temperature-scaling descriptor for T > 0 and returns the scaling
// mode (tscale): SM_ID for T == 1, SM_MARK when the Markstein step equals
// RN(l/T) for every fp32 significand with this T (checked once per T on the
// host and cached), else SM_DIV.
int make_scale(float T, TScale* out);

template <int V>
struct IntC { static constexpr int value = V; };
template <bool V>
struct BoolC { static constexpr bool value = V; };

// Calls f(Tin{}, IntC<SM>{}, BoolC<THR>{}) for the runtime (dtype, mode, thr).
template <typename F>
int dispatch_tsm(int dtype, int sm, bool thr, F&& f) {
  auto by_thr = [&](auto tin, auto smc) {
    return thr ? f(tin, smc, BoolC<true>{}) : f(tin, smc, BoolC<false>{});
  };
  auto by_sm = [&](auto tin) {
    switch (sm) {
      case SM_ID: return by_thr(tin, IntC<SM_ID>{});
      case SM_MARK: return by_thr(tin, IntC<SM_MARK>{});
      default: return by_thr(tin, IntC<SM_DIV>{});
    }
  };
  if (dtype == VNX_F32) return by_sm(float{});
  return by_sm(__hip_bfloat16{});
}

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

// Phase profiling (vnx_profile_begin / vnx_profile_end): returns this call's
// kMaxPhases + 1 events while profiling is active and slots remain, else
// nullptr.  The caller records event j before launch j and event nphase after
// the last launch, on its stream.
constexpr int kMaxPhases = 7;
hipEvent_t* profile_slot(int nphase);

// Compute units of the current device (cached per device ordinal).
int device_cus();

// Chunks per row for the streaming row kernels: about target_wgs workgroups
// in the launch, chunks no shorter than one 256-thread x 16-byte pass, at most
// max_chunks per row.
int pick_chunks(int64_t rows, int64_t V, int vec_elems, int max_chunks, int64_t target_wgs);

// Rows (b, i), i < nrows, at x + b*sb + i*ld must not overlap inside a batch
// row (ld >= V) and batch rows must not overlap (sb >= (nrows-1)*ld + V);
// 16-byte vector loads need x, ld and sb aligned to the vector width.
inline int check_rows(const void* x, int dtype, int64_t ld, int64_t sb, int nrows, int64_t V) {
  if (!x) return VNX_ERR_INVALID_ARG;
  if (ld < V || sb < (int64_t)(nrows - 1) * ld + V) return VNX_ERR_INVALID_ARG;
  const int ve = dtype == VNX_F32 ? 4 : 8;
  if (!aligned16(x) || ld % ve != 0 || sb % ve != 0) return VNX_ERR_UNSUPPORTED;
  return VNX_OK;
}

// RoPE + KV-cache store of a q|k|v projection epilogue (the per-row work of
// vnx_rope_kv: TriSparseAttention._apply_rope, tri_sparse_attn.py:182-221,
// and the cache write).  Row m is token (m / n, m % n) at position
// lens[m / n] + m % n; rows at or past cap (the cache, and the RoPE table when
// rope) are skipped.
struct RopeOut {
  const int32_t* lens;
  const float* cos;
  const float* sin;
  uint16_t* q;               // (B, H, n, d) bf16 bits
  uint16_t* kc;              // bf16 caches, strides c_sb, c_sh, c_sr
  uint16_t* vc;
  int64_t c_sb, c_sh, c_sr, cap;
  int n, H, Hkv, d, rope;
};

// Fills a RopeOut from the public argument block; VNX_OK or an error status.
int rope_out_from(const vnx_rope_kv_args* a, int64_t N, RopeOut* out);

}  // namespace vnx
