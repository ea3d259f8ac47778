// One workgroup reduces one chunk [c0, c1) of one vocab row:
//   LSE:    (m, s) with m = max_j a_j and s = sum_j exp(a_j - m) in fp64,
//           a_j = RN(l_j / T), masked to -inf below the row threshold;
//   ARGMAX: first index of the maximum of the raw logits (numpy.argmax order).
// Rows are streamed as 16-byte non-temporal vector loads, NB vectors per
// thread in flight per batch.  Per thread the running max is updated once
// per batch; the fp32 partial of a batch is added to an fp64 accumulator, so
// the row sum is accurate to ~1e-9 relative regardless of V.
#pragma once

#include "vnx_common.h"

namespace vnx {

struct ChunkResult {
  float m;       // max of scaled values (-inf if none)
  double s;      // sum exp(a - m)
  float av;      // argmax value (raw)
  int64_t ai;    // argmax index (INT64_MAX if the chunk is empty)
};

struct ReduceLds {
  float f[16];
  double d[16];
  int64_t i[16];
};

template <typename Tin, int NT, int NB, bool LSE, bool ARGMAX>
__device__ __forceinline__ ChunkResult reduce_chunk(const Tin* __restrict__ row, int64_t c0,
                                                    int64_t c1, const Scale& sc, float thr,
                                                    ReduceLds& lds) {
  constexpr int VE = Vec<Tin>::N;
  const int tid = threadIdx.x;
  float m = kNegInf;
  double s = 0.0;
  float bv = kNegInf;
  int64_t bi = INT64_MAX;

  const int64_t n = c1 - c0;
  const int64_t nvec = n / VE;  // c0 is a multiple of VE
  const Tin* base = row + c0;

  for (int64_t v0 = 0; v0 < nvec; v0 += (int64_t)NT * NB) {
    float x[NB][VE];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int64_t vi = v0 + tid + (int64_t)NT * j;
      if (vi < nvec) {
        Vec<Tin>::load(base + vi * VE, x[j]);
      } else {
#pragma unroll
        for (int e = 0; e < VE; ++e) x[j][e] = __builtin_nanf("");
      }
    }
    if constexpr (ARGMAX) {
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int64_t vi = v0 + tid + (int64_t)NT * j;
        if (vi < nvec) {
#pragma unroll
          for (int e = 0; e < VE; ++e) {
            const int64_t idx = c0 + vi * VE + e;
            if (argmax_better(x[j][e], idx, bv, bi)) { bv = x[j][e]; bi = idx; }
          }
        }
      }
    }
    if constexpr (LSE) {
      float a[NB][VE];
      float bm = kNegInf;
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int64_t vi = v0 + tid + (int64_t)NT * j;
        const bool ok = vi < nvec;
#pragma unroll
        for (int e = 0; e < VE; ++e) {
          float t = scale_logit(x[j][e], sc);
          t = (t < thr) ? kNegInf : t;
          a[j][e] = ok ? t : kNegInf;
          bm = fmaxf(bm, a[j][e]);
        }
      }
      if (bm > m) {
        if (m != kNegInf) s *= exp((double)m - (double)bm);
        m = bm;
      }
      if (m != kNegInf) {
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
          for (int e = 0; e < VE; ++e) acc[(j * VE + e) & 3] += fast_exp(a[j][e] - m);
        s += (double)((acc[0] + acc[1]) + (acc[2] + acc[3]));
      }
    }
  }

  // Tail: fewer than VE elements after the last full vector.
  const int64_t tail0 = nvec * VE;
  if (tid < n - tail0) {
    const int64_t idx = c0 + tail0 + tid;
    const float xv = Vec<Tin>::load1(row + idx);
    if constexpr (ARGMAX) {
      if (argmax_better(xv, idx, bv, bi)) { bv = xv; bi = idx; }
    }
    if constexpr (LSE) {
      float t = scale_logit(xv, sc);
      t = (t < thr) ? kNegInf : t;
      if (t > m) {
        if (m != kNegInf) s *= exp((double)m - (double)t);
        m = t;
      }
      if (m != kNegInf) s += (double)fast_exp(t - m);
    }
  }

  ChunkResult r;
  r.m = kNegInf;
  r.s = 0.0;
  r.av = kNegInf;
  r.ai = INT64_MAX;
  if constexpr (LSE) {
    const float M = block_max<NT>(m, lds.f);
    double sc_s = 0.0;
    if (m != kNegInf) sc_s = (m == M) ? s : s * exp((double)m - (double)M);
    r.m = M;
    r.s = block_sum<NT>(sc_s, lds.d);
  }
  if constexpr (ARGMAX) {
    block_argmax<NT>(bv, bi, lds.f, lds.i);
    r.av = bv;
    r.ai = bi;
  }
  return r;
}

// Merge of chunk partials (m_c, s_c): M = max m_c, S = sum s_c exp(m_c - M).
__device__ __forceinline__ void merge_partial(float& M, double& S, float m, double s) {
  if (m == kNegInf) return;
  if (M == kNegInf) { M = m; S = s; return; }
  if (m > M) { S = S * exp((double)M - (double)m) + s; M = m; }
  else { S += s * exp((double)m - (double)M); }
}

__device__ __forceinline__ double lse_of(float M, double S) {
  if (M == kNegInf) return -__builtin_inf();
  return (double)M + log(S);
}

// Arrival counter for "last workgroup of a group finishes the group".  The
// counter is zeroed by k_zero_u32 at the start of every call.  Partials
// written before this call (by any thread of the block) are published with a
// device-scope release; the last arriving block acquires them.
__device__ __forceinline__ bool arrive_last(unsigned* counter, unsigned total, int* lds_flag) {
  __syncthreads();
  if (threadIdx.x == 0) {
    __threadfence();
    unsigned prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    int last = (prev == total - 1) ? 1 : 0;
    if (last) __threadfence();
    *lds_flag = last;
  }
  __syncthreads();
  return *lds_flag != 0;
}

template <typename T>
__device__ __forceinline__ void st_agent(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T ld_agent(const T* p) {
  return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace vnx
