// Shared device helpers for the vnx HIP library (gfx950 / CDNA4, wave64).
//
// Numerical contract shared with the CPU checker in oracle/canon.c:
//   * temperature scaling is the correctly rounded fp32 quotient RN(l / T),
//     the value numpy produces for `logits / temperature` on float32 arrays
//     (packages/verse_infra/verse_infra/verse_inference/sampler.py:95);
//   * vnx_exp_canon() is an exp built only from IEEE-754 fp32 operations
//     (mul, rint, fma) in a fixed order, so the CPU checker reproduces every
//     bit of it; it is used wherever a probability feeds a discrete decision
//     (acceptance test, inverse-CDF search);
//   * sums that feed discrete decisions are carried in fp64.
// The library is compiled with -ffp-contract=off, so every a*b+c written
// without an explicit fma is two rounded operations, as in the C checker.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#define VNX_WAVE 64

namespace vnx {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kNegInf = -__builtin_inff();

// ---------------------------------------------------------------------------
// Temperature scaling: a = RN(l / T), the value numpy gives for float32
// `logits / temperature`.  The scaling mode is a template parameter so the
// streaming loops carry no per-element branch:
//   SM_ID   T == 1: a = l;
//   SM_MARK Markstein correction step, y = RN(1/T):
//             q0 = RN(l*y), r = l - q0*T (exact through fma), a = RN(q0 + r*y);
//           the host selects it only after checking that it equals RN(l/T)
//           for every fp32 significand with this T (api.hip).  r is NaN when
//           l (or q0) is infinite; clamping r to +-FLT_MAX keeps a = q0 there,
//           with one min and one max instead of a compare and select;
//   SM_DIV  IEEE division (compiler's correctly rounded sequence).
// ---------------------------------------------------------------------------
enum ScaleMode { SM_ID = 0, SM_MARK = 1, SM_DIV = 2 };

struct TScale {
  float T;  // temperature
  float y;  // RN(1 / T)
};

template <int SM>
__device__ __forceinline__ float tscale(float l, const TScale& s) {
  if constexpr (SM == SM_ID) {
    return l;
  } else if constexpr (SM == SM_MARK) {
    const float q0 = l * s.y;
    float r = __builtin_fmaf(-q0, s.T, l);
    r = __builtin_fminf(__builtin_fmaxf(r, -3.40282347e38f), 3.40282347e38f);
    return __builtin_fmaf(r, s.y, q0);
  } else {
    return l / s.T;
  }
}

// Scaled logit with the top-k mask (values below thr become -inf).
template <int SM, bool THR>
__device__ __forceinline__ float scaled(float l, const TScale& s, float thr) {
  const float a = tscale<SM>(l, s);
  if constexpr (THR) return (a < thr) ? -__builtin_inff() : a;
  return a;
}

// log2(e) split for the compensated exponent of the LSE sums:
// kL2eHi = RN32(log2 e), kL2eLo = RN32(log2 e - kL2eHi).
constexpr float kL2eHi = 0x1.715476p+0f;
constexpr float kL2eLo = 0x1.4ae0c0p-26f;
constexpr double kLn2 = 0x1.62e42fefa39efp-1;

// ---------------------------------------------------------------------------
// Canonical exp (Cody-Waite reduction by ln2 + degree-7 Taylor polynomial).
// Constants are the fp32 roundings of mathematical constants:
//   kLog2e = RN(log2 e), kLn2Hi = RN(ln 2), kLn2Lo = RN(ln 2 - kLn2Hi),
//   kC[n] = RN(1/n!).
// Domain: t < -86.5 (and NaN) -> 0; t > 88 is clamped to 88.  On the kept
// domain 2^k is a normal number, so the final scaling is exact.
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ float vnx_exp_canon(float t) {
  const float kLog2e = 0x1.715476p+0f;    // 0x3FB8AA3B
  const float kLn2Hi = 0x1.62e430p-1f;    // 0x3F317218
  const float kLn2Lo = -0x1.05c610p-29f;  // 0xB102E308
  const float c7 = 0x1.a01a02p-13f;       // 1/5040, 0x39500D01
  const float c6 = 0x1.6c16c2p-10f;       // 1/720,  0x3AB60B61
  const float c5 = 0x1.111112p-7f;        // 1/120,  0x3C088889
  const float c4 = 0x1.555556p-5f;        // 1/24,   0x3D2AAAAB
  const float c3 = 0x1.555556p-3f;        // 1/6,    0x3E2AAAAB
  const float c2 = 0x1p-1f;
  // Evaluated on t clamped into [-86.5, 88] and replaced by 0 for t < -86.5
  // (and NaN) at the end: the same value as the early-return form, without a
  // divergent branch per element.
  const float tc = __builtin_fminf(__builtin_fmaxf(t, -86.5f), 88.0f);
  float kf = __builtin_rintf(tc * kLog2e);
  float r = __builtin_fmaf(-kf, kLn2Hi, tc);
  r = __builtin_fmaf(-kf, kLn2Lo, r);
  float p = c7;
  p = __builtin_fmaf(p, r, c6);
  p = __builtin_fmaf(p, r, c5);
  p = __builtin_fmaf(p, r, c4);
  p = __builtin_fmaf(p, r, c3);
  p = __builtin_fmaf(p, r, c2);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  // p * 2^k with k in [-125, 127]: 2^k and the product are normal numbers,
  // so the scaling is exact (ldexp, one instruction, equals the multiply)
  const float e = __builtin_ldexpf(p, (int)kf);
  return (t >= -86.5f) ? e : 0.0f;
}

// ---------------------------------------------------------------------------
// Argmax ordering identical to numpy.argmax: NaN counts as the maximum, ties
// (and repeated NaN) go to the lowest index.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool argmax_better(float v, int64_t i, float bv, int64_t bi) {
  bool vn = __builtin_isnan(v), bn = __builtin_isnan(bv);
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

// ---------------------------------------------------------------------------
// Wave / block reductions (blockDim.x == NT, a multiple of 64).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, VNX_WAVE));
  return v;
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, VNX_WAVE);
  return v;
}

__device__ __forceinline__ void wave_argmax(float& v, int64_t& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float ov = __shfl_xor(v, o, VNX_WAVE);
    int64_t oi = __shfl_xor(i, o, VNX_WAVE);
    if (argmax_better(ov, oi, v, i)) { v = ov; i = oi; }
  }
}

template <int NT>
__device__ __forceinline__ float block_max(float v, float* lds) {
  constexpr int NW = NT / VNX_WAVE;
  v = wave_max(v);
  const int w = threadIdx.x / VNX_WAVE, l = threadIdx.x % VNX_WAVE;
  __syncthreads();
  if (l == 0) lds[w] = v;
  __syncthreads();
  float r = lds[0];
#pragma unroll
  for (int j = 1; j < NW; ++j) r = fmaxf(r, lds[j]);
  return r;
}

template <int NT>
__device__ __forceinline__ double block_sum(double v, double* lds) {
  constexpr int NW = NT / VNX_WAVE;
  v = wave_sum(v);
  const int w = threadIdx.x / VNX_WAVE, l = threadIdx.x % VNX_WAVE;
  __syncthreads();
  if (l == 0) lds[w] = v;
  __syncthreads();
  double r = lds[0];
#pragma unroll
  for (int j = 1; j < NW; ++j) r += lds[j];
  return r;
}

template <int NT>
__device__ __forceinline__ void block_argmax(float& v, int64_t& i, float* ldsv, int64_t* ldsi) {
  constexpr int NW = NT / VNX_WAVE;
  wave_argmax(v, i);
  const int w = threadIdx.x / VNX_WAVE, l = threadIdx.x % VNX_WAVE;
  __syncthreads();
  if (l == 0) { ldsv[w] = v; ldsi[w] = i; }
  __syncthreads();
  v = ldsv[0]; i = ldsi[0];
#pragma unroll
  for (int j = 1; j < NW; ++j)
    if (argmax_better(ldsv[j], ldsi[j], v, i)) { v = ldsv[j]; i = ldsi[j]; }
}

// Inclusive scan of one double per lane across the wave (lane order).
__device__ __forceinline__ double wave_inclusive_scan(double v) {
  const int l = threadIdx.x % VNX_WAVE;
#pragma unroll
  for (int o = 1; o < VNX_WAVE; o <<= 1) {
    const double n = __shfl_up(v, o, VNX_WAVE);
    if (l >= o) v += n;
  }
  return v;
}

// Inclusive scan of one double per thread across the block (NT threads).
template <int NT>
__device__ __forceinline__ double block_inclusive_scan(double v, double* lds) {
  constexpr int NW = NT / VNX_WAVE;
  const int w = threadIdx.x / VNX_WAVE, l = threadIdx.x % VNX_WAVE;
#pragma unroll
  for (int o = 1; o < VNX_WAVE; o <<= 1) {
    double n = __shfl_up(v, o, VNX_WAVE);
    if (l >= o) v += n;
  }
  __syncthreads();
  if (l == VNX_WAVE - 1) lds[w] = v;
  __syncthreads();
  double base = 0.0;
#pragma unroll
  for (int j = 0; j < NW; ++j)
    if (j < w) base += lds[j];
  return base + v;
}

// ---------------------------------------------------------------------------
// Element loads.  Rows are read as 16-byte vectors (4 fp32 or 8 bf16).
// ---------------------------------------------------------------------------
template <typename Tin> struct Vec;
template <> struct Vec<float> {
  static constexpr int N = 4;
  __device__ __forceinline__ static void load(const float* p, float* out) {
    f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
  }
  __device__ __forceinline__ static float load1(const float* p) { return *p; }
  // The 16 bytes alone, converted later (a load under a per-lane condition
  // then carries no conversion that would wait for it inside the condition).
  __device__ __forceinline__ static u32x4 load_raw(const float* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  }
  __device__ __forceinline__ static void cvt_raw(const u32x4& v, float* out) {
    out[0] = __uint_as_float(v.x); out[1] = __uint_as_float(v.y);
    out[2] = __uint_as_float(v.z); out[3] = __uint_as_float(v.w);
  }
};
template <> struct Vec<__hip_bfloat16> {
  static constexpr int N = 8;
  __device__ __forceinline__ static float cvt(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
  __device__ __forceinline__ static void load(const __hip_bfloat16* p, float* out) {
    u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      out[2 * j] = __uint_as_float(w[j] << 16);
      out[2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
    }
  }
  __device__ __forceinline__ static float load1(const __hip_bfloat16* p) {
    return __uint_as_float((uint32_t)(*reinterpret_cast<const uint16_t*>(p)) << 16);
  }
  __device__ __forceinline__ static u32x4 load_raw(const __hip_bfloat16* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  }
  __device__ __forceinline__ static void cvt_raw(const u32x4& v, float* out) {
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      out[2 * j] = __uint_as_float(w[j] << 16);
      out[2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
    }
  }
};

}  // namespace vnx
