// One workgroup reduces one chunk [c0, c1) of one vocab row:
//   LSE:    (m, s) with m = max_j a_j and s = sum_j 2^(a_j*log2(e) - mt),
//           mt = RN(m * kL2eHi), a_j = RN(l_j / T) masked to -inf below the
//           row threshold; the row LSE is mt*ln2 + ln(s);
//   ARGMAX: first index of the maximum of the RAW logits (numpy.argmax order,
//           NaN counts as the maximum).
// Rows are streamed as 16-byte non-temporal vector loads, NB vectors per
// thread in flight per batch.  Full batches run without bounds checks; one
// guarded batch and a scalar tail finish the chunk.  Per element the LSE costs
// the exact scaling, one max, two fma (the exponent a*log2(e) - mt with the
// product's rounding compensated) and one v_exp_f32; the running max is
// updated once per batch and the fp32 batch partial is added to an fp64
// accumulator.
#pragma once

#include "vnx_common.h"

namespace vnx {

struct ChunkResult {
  float m;       // max of scaled values (-inf if none)
  double s;      // sum 2^(a*log2e - mt_of(m))
  float av;      // argmax value (raw)
  int64_t ai;    // argmax index (INT64_MAX if the chunk is empty)
};

struct ReduceLds {
  float f[16];
  double d[16];
  int64_t i[16];
};

constexpr float kPosInf = __builtin_inff();

__device__ __forceinline__ float mt_of(float m) { return m * kL2eHi; }

// 2^(a*log2(e) - mt): the first fma rounds a*kL2eHi - mt once, the second
// adds a*kL2eLo, so the exponent carries no systematic error from log2(e).
__device__ __forceinline__ float exp2_term(float a, float mt) {
  float t = __builtin_fmaf(a, kL2eHi, -mt);
  t = __builtin_fmaf(a, kL2eLo, t);
  return __builtin_amdgcn_exp2f(t);
}

// Rescales an fp64 partial from reference mt_from to mt_to (mt_to >= mt_from).
__device__ __forceinline__ double rescale(double s, float mt_from, float mt_to) {
  return s * exp2((double)mt_from - (double)mt_to);
}

// Per-thread state of a chunk reduction.
struct RowAcc {
  float m = kNegInf;
  float mt = kNegInf;
  double s = 0.0;
  float bv = kNegInf;
  int64_t bi = INT64_MAX;
};

// Consumes N raw values x[0..N) whose element indices are idx(q) (increasing
// in q).  The first nvalid entries are real elements; the rest is -inf
// padding, which adds nothing to the LSE and is never an argmax.
template <int SM, bool THR, bool LSE, bool ARGMAX, int N, typename IdxFn>
__device__ __forceinline__ void consume(const float (&x)[N], int nvalid, RowAcc& st, const TScale& sc,
                                        float thr, IdxFn idx) {
  if constexpr (ARGMAX) {
    float bmx = kNegInf;
    bool nan = false;
#pragma unroll
    for (int q = 0; q < N; ++q) {
      bmx = __builtin_fmaxf(bmx, x[q]);
      nan |= __builtin_isnan(x[q]);
    }
    if (nan) {
      if (!__builtin_isnan(st.bv)) {
#pragma unroll
        for (int q = N - 1; q >= 0; --q)
          if (__builtin_isnan(x[q])) { st.bv = x[q]; st.bi = idx(q); }
      }
    } else if (bmx > st.bv) {
#pragma unroll
      for (int q = N - 1; q >= 0; --q)
        if (x[q] == bmx) st.bi = idx(q);
      st.bv = bmx;
    } else if (st.bi == INT64_MAX && nvalid > 0) {
      // Every element so far is -inf: the first one is the argmax.
      st.bv = x[0];
      st.bi = idx(0);
    }
  }
  if constexpr (LSE) {
    float a[N];
    float bm = kNegInf;
#pragma unroll
    for (int q = 0; q < N; ++q) {
      a[q] = scaled<SM, THR>(x[q], sc, thr);
      bm = __builtin_fmaxf(bm, a[q]);
    }
    if (bm > st.m) {
      const float mtn = mt_of(bm);
      if (st.s != 0.0) st.s = rescale(st.s, st.mt, mtn);
      st.m = bm;
      st.mt = mtn;
    }
    if (st.m > kNegInf && st.m < kPosInf) {
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < N; ++q) acc[q & 3] += exp2_term(a[q], st.mt);
      st.s += (double)((acc[0] + acc[1]) + (acc[2] + acc[3]));
    }
  }
}

template <typename Tin, int SM, bool THR, bool LSE, bool ARGMAX, int NT, int NB>
__device__ __forceinline__ ChunkResult reduce_chunk(const Tin* __restrict__ row, int64_t c0,
                                                    int64_t c1, const TScale& sc, float thr,
                                                    ReduceLds& lds) {
  constexpr int VE = Vec<Tin>::N;
  constexpr int64_t STEP = (int64_t)NT * NB;
  const int tid = threadIdx.x;
  RowAcc st;

  const int64_t n = c1 - c0;
  const int64_t nvec = n / VE;  // c0 is a multiple of VE
  const Tin* base = row + c0;
  const int64_t nfull = nvec / STEP * STEP;

  for (int64_t v0 = 0; v0 < nfull; v0 += STEP) {
    float x[NB * VE];
#pragma unroll
    for (int j = 0; j < NB; ++j) Vec<Tin>::load(base + (v0 + tid + (int64_t)NT * j) * VE, &x[j * VE]);
    consume<SM, THR, LSE, ARGMAX>(x, NB * VE, st, sc, thr, [&](int q) {
      return c0 + (v0 + tid + (int64_t)NT * (q / VE)) * VE + (q % VE);
    });
  }
  if (nfull < nvec) {
    // The last, partial batch: every load first (all in flight), then each
    // loaded vector consumed on its own, so a short batch costs its vectors'
    // work only (no -inf padding through the scaling and the exps).
    u32x4 raw[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int64_t vi = nfull + tid + (int64_t)NT * j;
      raw[j] = u32x4{0u, 0u, 0u, 0u};
      if (vi < nvec) raw[j] = Vec<Tin>::load_raw(base + vi * VE);
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int64_t vi = nfull + tid + (int64_t)NT * j;
      if (vi < nvec) {
        float x[VE];
        Vec<Tin>::cvt_raw(raw[j], x);
        consume<SM, THR, LSE, ARGMAX>(x, VE, st, sc, thr, [&](int q) { return c0 + vi * VE + q; });
      }
    }
  }
  // Tail: fewer than VE elements after the last full vector.
  const int64_t tail0 = nvec * VE;
  if (tid < n - tail0) {
    float x[1] = {Vec<Tin>::load1(row + c0 + tail0 + tid)};
    consume<SM, THR, LSE, ARGMAX>(x, 1, st, sc, thr, [&](int) { return c0 + tail0 + tid; });
  }

  ChunkResult r;
  r.m = kNegInf;
  r.s = 0.0;
  r.av = kNegInf;
  r.ai = INT64_MAX;
  if constexpr (LSE) {
    const float M = block_max<NT>(st.m, lds.f);
    double sc_s = 0.0;
    if (M < kPosInf && st.m > kNegInf) sc_s = (st.m == M) ? st.s : rescale(st.s, st.mt, mt_of(M));
    r.m = M;
    r.s = block_sum<NT>(sc_s, lds.d);
  }
  if constexpr (ARGMAX) {
    block_argmax<NT>(st.bv, st.bi, lds.f, lds.i);
    r.av = st.bv;
    r.ai = st.bi;
  }
  return r;
}

// Balanced static split of `rows` rows of nvr vectors each (the rows laid
// end to end, nv = rows*nvr vectors) over G workgroups: workgroup w owns
// vectors [vstart(w), vstart(w+1)), vstart(w) = floor(w*nv/G), so every
// workgroup streams the same number of bytes to within one vector.  A row is
// covered by the workgroups first_wg(r)..last_wg(r), one piece each.  The host
// keeps G <= nv, so no workgroup is empty.
struct Split {
  int64_t rows, nvr, nv, G;
  __host__ __device__ int64_t vstart(int64_t w) const { return w * nv / G; }
  // The workgroup whose range holds vector v.
  __host__ __device__ int64_t wg_of(int64_t v) const { return ((v + 1) * G - 1) / nv; }
  __host__ __device__ int64_t first_wg(int64_t r) const { return wg_of(r * nvr); }
  __host__ __device__ int64_t last_wg(int64_t r) const { return wg_of((r + 1) * nvr - 1); }
  __host__ __device__ int pieces(int64_t r) const { return (int)(last_wg(r) - first_wg(r) + 1); }
  // Upper bound of pieces(r) over all rows.
  __host__ __device__ int max_pieces() const {
    const int64_t q = nv / G;  // >= 1
    return (int)((nvr + q - 1) / q + 1);
  }
};

__host__ inline Split make_split(int64_t rows, int64_t nvr, int64_t G) {
  Split sp;
  sp.rows = rows;
  sp.nvr = nvr;
  sp.nv = rows * nvr;
  sp.G = G < sp.nv ? G : sp.nv;
  if (sp.G < 1) sp.G = 1;
  return sp;
}

// Merge of chunk partials (m_c, s_c) in the exp2 domain.
__device__ __forceinline__ void merge_partial(float& M, double& S, float m, double s) {
  if (m == kNegInf || M == kPosInf) return;
  if (M == kNegInf || m == kPosInf) { M = m; S = s; return; }
  if (m > M) { S = rescale(S, mt_of(M), mt_of(m)) + s; M = m; }
  else { S += rescale(s, mt_of(m), mt_of(M)); }
}

// Row LSE in fp64 from the merged (M, S).
__device__ __forceinline__ double lse_of(float M, double S) {
  if (M == kNegInf) return -__builtin_inf();
  if (M == kPosInf) return __builtin_inf();
  return (double)mt_of(M) * kLn2 + log(S);
}

// Arrival of n pieces at a group counter; true in the workgroup whose
// arrival completes the group (total pieces).  Same publication contract as
// arrive_last.
__device__ __forceinline__ bool arrive_n(unsigned* counter, unsigned n, unsigned total, int* lds_flag) {
  __syncthreads();
  if (threadIdx.x == 0) {
    __builtin_amdgcn_s_waitcnt(0);
    const unsigned prev = __hip_atomic_fetch_add(counter, n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *lds_flag = (prev + n == total) ? 1 : 0;
  }
  __syncthreads();
  return *lds_flag != 0;
}

// Arrival counter for "last workgroup of a group finishes the group".
// Contract: the data a group publishes is written by thread 0 of each
// workgroup with st_agent (agent-scope atomic stores) before it arrives, and
// read by the last workgroup with ld_agent (agent-scope atomic loads).  Those
// accesses are coherent across the XCDs by themselves, so no fence is needed,
// only ordering: s_waitcnt(0) completes thread 0's stores before its counter
// increment issues.  (A __threadfence here would write back and invalidate
// the whole L2 of the XCD for every workgroup; with thousands of workgroups
// per launch that costs more than streaming the rows.)  The counter is zeroed
// by k_zero_u32 at the start of every call.
__device__ __forceinline__ bool arrive_last(unsigned* counter, unsigned total, int* lds_flag) {
  __syncthreads();
  if (threadIdx.x == 0) {
    __builtin_amdgcn_s_waitcnt(0);
    const unsigned prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *lds_flag = (prev == total - 1) ? 1 : 0;
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
