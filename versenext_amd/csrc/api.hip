// Library-level entry points: version, status text, device init, and the
// host-side temperature check used by every kernel that scales logits.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <unordered_map>
#include <vector>

#include "vnx_internal.h"

namespace vnx {

static thread_local char g_last_hip_error[256] = "";

int hip_fail(hipError_t e) {
  const char* s = hipGetErrorString(e);
  strncpy(g_last_hip_error, s ? s : "unknown HIP error", sizeof(g_last_hip_error) - 1);
  g_last_hip_error[sizeof(g_last_hip_error) - 1] = 0;
  return VNX_ERR_HIP;
}

// True when q1 = RN(q0 + RN-exact(a - q0*T) * y), q0 = RN(a*y), y = RN(1/T),
// equals RN(a/T) for every significand of a in [1, 2).  Scaling a by a power
// of two scales every intermediate exactly (away from overflow/underflow), so
// one binade covers all normal a; a = 0 and +-inf are exact by construction.
static bool markstein_exact(float T) {
  volatile float Tv = T;  // keep the host compiler from folding the loop
  const float t = Tv;
  const float y = 1.0f / t;
  for (uint32_t m = 0; m < (1u << 23); ++m) {
    uint32_t bits = (127u << 23) | m;
    float a;
    memcpy(&a, &bits, 4);
    float q0 = a * y;
    float r = fmaf(-q0, t, a);
    float q1 = fmaf(r, y, q0);
    float ref = a / t;
    if (q1 != ref) return false;
  }
  return true;
}

int make_scale(float T, TScale* out) {
  out->T = T;
  out->y = 1.0f / T;
  if (T == 1.0f) return SM_ID;
  static std::mutex mu;
  static std::unordered_map<uint32_t, bool> cache;
  uint32_t key;
  memcpy(&key, &T, 4);
  bool exact;
  {
    std::lock_guard<std::mutex> g(mu);
    auto it = cache.find(key);
    if (it != cache.end()) {
      exact = it->second;
    } else {
      exact = markstein_exact(T);
      cache.emplace(key, exact);
    }
  }
  return exact ? SM_MARK : SM_DIV;
}

__global__ void k_zero_u32(unsigned* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

int zero_counters(unsigned* p, int64_t n, hipStream_t st) {
  if (n <= 0) return VNX_OK;
  const int nt = 256;
  hipLaunchKernelGGL(k_zero_u32, dim3((unsigned)((n + nt - 1) / nt)), dim3(nt), 0, st, p, n);
  VNX_LAUNCH_CHECK();
  return VNX_OK;
}

int device_cus() {
  static std::mutex mu;
  static std::unordered_map<int, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> g(mu);
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  cache.emplace(dev, n);
  return n;
}

int pick_chunks(int64_t rows, int64_t V, int vec_elems, int max_chunks, int64_t target_wgs) {
  int64_t c = (target_wgs + rows - 1) / rows;
  int64_t max_by_len = V / (256 * (int64_t)vec_elems);
  if (max_by_len < 1) max_by_len = 1;
  if (c > max_by_len) c = max_by_len;
  if (c > max_chunks) c = max_chunks;
  if (c < 1) c = 1;
  return (int)c;
}

// ---------------------------------------------------------------------------
// Phase profiling: while active, entry points record hipEvents around each of
// their launches into one slot per call (slots are handed out in call order).
// ---------------------------------------------------------------------------
namespace {
struct Profile {
  std::mutex mu;
  bool active = false;
  int max_calls = 0, next = 0, nphase = 0;
  std::vector<hipEvent_t> ev;  // max_calls * (kMaxPhases + 1)
};
Profile g_prof;
}  // namespace

hipEvent_t* profile_slot(int nphase) {
  std::lock_guard<std::mutex> g(g_prof.mu);
  if (!g_prof.active || g_prof.next >= g_prof.max_calls || nphase > kMaxPhases) return nullptr;
  if (g_prof.nphase == 0) g_prof.nphase = nphase;
  if (g_prof.nphase != nphase) return nullptr;
  return &g_prof.ev[(size_t)(g_prof.next++) * (kMaxPhases + 1)];
}

}  // namespace vnx

extern "C" {

int vnx_profile_begin(int max_calls) {
  using namespace vnx;
  if (max_calls < 1 || max_calls > (1 << 16)) return VNX_ERR_INVALID_ARG;
  std::lock_guard<std::mutex> g(g_prof.mu);
  if (g_prof.active) return VNX_ERR_INVALID_ARG;
  g_prof.ev.assign((size_t)max_calls * (kMaxPhases + 1), nullptr);
  for (auto& e : g_prof.ev) {
    hipError_t err = hipEventCreate(&e);
    if (err != hipSuccess) {
      for (auto& f : g_prof.ev)
        if (f) (void)hipEventDestroy(f);
      g_prof.ev.clear();
      return hip_fail(err);
    }
  }
  g_prof.active = true;
  g_prof.max_calls = max_calls;
  g_prof.next = 0;
  g_prof.nphase = 0;
  return VNX_OK;
}

int vnx_profile_end(double* phase_ms, int nphase, int* ncalls) {
  using namespace vnx;
  std::lock_guard<std::mutex> g(g_prof.mu);
  if (!g_prof.active) return VNX_ERR_INVALID_ARG;
  int st = VNX_OK;
  const int np = g_prof.nphase;
  if (phase_ms)
    for (int j = 0; j < nphase; ++j) phase_ms[j] = 0.0;
  for (int c = 0; c < g_prof.next && st == VNX_OK; ++c) {
    hipEvent_t* e = &g_prof.ev[(size_t)c * (kMaxPhases + 1)];
    hipError_t err = hipEventSynchronize(e[np]);
    if (err != hipSuccess) { st = hip_fail(err); break; }
    for (int j = 0; j < np && j < nphase; ++j) {
      float ms = 0.0f;
      err = hipEventElapsedTime(&ms, e[j], e[j + 1]);
      if (err != hipSuccess) { st = hip_fail(err); break; }
      if (phase_ms) phase_ms[j] += ms;
    }
  }
  if (ncalls) *ncalls = g_prof.next;
  for (auto& e : g_prof.ev) (void)hipEventDestroy(e);
  g_prof.ev.clear();
  g_prof.active = false;
  return st;
}

int vnx_version(void) { return 100; }

const char* vnx_status_string(int status) {
  switch (status) {
    case VNX_OK: return "ok";
    case VNX_ERR_INVALID_ARG: return "invalid argument";
    case VNX_ERR_WORKSPACE: return "workspace missing or too small";
    case VNX_ERR_UNSUPPORTED: return "unsupported dtype or size";
    case VNX_ERR_HIP: return "HIP runtime error";
    case VNX_ERR_NO_DEVICE: return "no gfx950 device";
    case VNX_ERR_TOO_LARGE: return "size exceeds the fixed scratch of an allocation-free entry point";
    default: return "unknown status";
  }
}

const char* vnx_last_hip_error(void) { return vnx::g_last_hip_error; }

int vnx_init(int device) {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) return vnx::hip_fail(e);
  if (device < 0 || device >= n) return VNX_ERR_NO_DEVICE;
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return vnx::hip_fail(e);
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return VNX_ERR_NO_DEVICE;
  e = hipSetDevice(device);
  if (e != hipSuccess) return vnx::hip_fail(e);
  return vnx::spec_scratch_init(device);
}

}  // extern "C"
