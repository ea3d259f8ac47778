// Sampler.sample on the GPU (packages/verse_infra/verse_infra/verse_inference/
// sampler.py:70-138) and the logit calibration of VMPC-compressed models
// (packages/verse_nex/verse_nex/cometspark.py:922-948).
//
// k_sampler: one workgroup of kST threads per row, every step of the
// reference in one launch, nothing outside LDS:
//   calibrate   (CometSpark mode) l = RN(RN(l / s) * f), s = RN(sqrt(RN32(var)
//               + eps)) with var the fp64 population variance of the row
//               (cometspark.py:922-948), two extra passes;
//   T == 0      numpy.argmax of the row;
//   a = RN(l/T) (the exact scaling of vnx_common.h);
//   top-k       kth = the kth largest a by a radix select over order-preserving
//               32-bit keys, four 8-bit digits, per-wave LDS histograms.
//               Sampler rule (sampler.py:96-102): NaN ranks largest
//               (numpy.partition) and a = a >= kth ? a : -inf keeps every tie.
//               Exactly-k rule (cometspark.py:896-904, argpartition(-a)[:k]):
//               NaN ranks smallest and the ties at kth are taken by lower id
//               until k are kept (a rank pass finds the last one, k*);
//   softmax     M = max a (not finite -> numpy.argmax of the raw row), the row
//               LSE in fp64, L32 = RN32(LSE), p = vnx_exp_canon(a - L32);
//   top-p       the nucleus on p ordered by (p descending, id ascending), with
//               cumulative sums in exact fixed point floor(p * 2^60) (integer
//               adds, so every order gives the same sums): a radix select on
//               the keys of p with (count, mass) histograms finds the last
//               kept value p*, the number m of its ties that the sums need,
//               and a rank pass over the row in id order finds the id j* of
//               the m-th tie; kept iff p > p* or (p == p* and id <= j*);
//   draw        the inverse CDF with the row's uniform over the kept p in id
//               order (first j with C_j > u * C_V, fp64 sums): sub-block
//               masses in LDS, a thread-order scan to the sub-block, one wave
//               rescans it.
// The CPU checker oracle/sampler.py restates the same rules.  The exactly-k
// draw runs over the kept tokens in id order: argpartition's output order,
// which the reference draws over, is implementation-defined.
#include <algorithm>

#include "rowred.h"
#include "vnx_internal.h"

namespace vnx {

constexpr int kST = 1024;            // threads per row
constexpr int kSW = kST / VNX_WAVE;  // waves per row
constexpr int kSNB = 4;              // vectors in flight per thread
constexpr int kBins = 256;           // 8-bit digits
constexpr int kHist = 8;             // private histograms (wave w uses w % kHist)
constexpr int kSampDraw = 4096;      // sub-blocks of 64 vectors held in LDS

struct SamplerParams {
  const void* x;
  int64_t B, V, ld;
  TScale sc;
  int greedy;
  int64_t top_k;           // 0: off
  int exact_k;             // CometSpark's exactly-k rule
  int calib;               // fused logit calibration
  float cf, ceps;          // calibration factor and eps
  int use_p;               // top_p < 1
  uint64_t p_target;       // floor(top_p * 2^60)
  const float* u;
  int64_t* out;
  uint8_t* flags;
  float* lse;
  float* kth;
  float* p_star;
  int64_t* j_star;
  int64_t* k_star;
};

struct SamplerLds {
  union {
    struct {  // radix passes
      unsigned cnt[kHist][kBins];
      unsigned long long mass[kHist][kBins];
    } h;
    struct {  // rank pass and draw
      double T[kST], E[kST];
      unsigned long long seg[kST];
    } d;
  } u;
  unsigned tot_cnt[kBins];
  unsigned long long tot_mass[kBins];
  float f[kSW];
  double dd[kSW];
  int64_t i[kSW];
  double scan[kSW];
  // row state
  uint32_t prefix, pmask;
  unsigned long long rem;
  int64_t jstar;
  unsigned long long rank;
  double total, target, base;
  int64_t sb;
  int tstar, tlast;
  int done;
};

// Order-preserving key of a float: larger value, larger key; NaN above all
// (numpy.partition's order).
__device__ __forceinline__ uint32_t okey(float a) {
  if (__builtin_isnan(a)) return 0xFFFFFFFFu;
  const uint32_t u = __float_as_uint(a);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// The exactly-k order (argpartition of -a): NaN below every value, -0 and +0
// one value (a + 0 turns -0 into +0), so equal values tie and go by id.
__device__ __forceinline__ uint32_t okey_lo(float a) { return __builtin_isnan(a) ? 0u : okey(a + 0.0f); }

__device__ __forceinline__ float okey_value(uint32_t k) {
  if (k == 0xFFFFFFFFu || k == 0u) return __builtin_nanf("");
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  return __uint_as_float(u);
}

__device__ __forceinline__ unsigned long long fix60(float p) {
  // floor(p * 2^60) for 0 <= p <= 2 (exact: scaling by a power of two)
  return (unsigned long long)((double)p * 1152921504606846976.0);
}

// Calls f(j, raw) for every element of the row, each thread its vectors
// tid, tid + kST, ... with kSNB loads in flight, then the tail.
template <typename Tin, typename F>
__device__ __forceinline__ void for_row(const Tin* row, int64_t V, F&& f) {
  constexpr int VE = Vec<Tin>::N;
  const int64_t nv = V / VE;
  const int tid = threadIdx.x;
  int64_t v0 = 0;
  for (; v0 + (int64_t)kST * kSNB <= nv; v0 += (int64_t)kST * kSNB) {
    float x[kSNB][VE];
#pragma unroll
    for (int j = 0; j < kSNB; ++j) Vec<Tin>::load(row + (v0 + tid + (int64_t)kST * j) * VE, x[j]);
#pragma unroll
    for (int j = 0; j < kSNB; ++j)
#pragma unroll
      for (int e = 0; e < VE; ++e) f((v0 + tid + (int64_t)kST * j) * VE + e, x[j][e]);
  }
  for (int64_t v = v0 + tid; v < nv; v += kST) {
    float x[VE];
    Vec<Tin>::load(row + v * VE, x);
#pragma unroll
    for (int e = 0; e < VE; ++e) f(v * VE + e, x[e]);
  }
  const int64_t t0 = nv * VE;
  if (tid < V - t0) f(t0 + tid, Vec<Tin>::load1(row + t0 + tid));
}

// Calls f(j, raw) for j in [j0, j1) in increasing order (j0 a multiple of the
// vector width), kSNB * 2 vector loads in flight.
template <typename Tin, typename F>
__device__ __forceinline__ void seg_visit(const Tin* row, int64_t j0, int64_t j1, F&& f) {
  constexpr int VE = Vec<Tin>::N;
  constexpr int NB = 2 * kSNB;
  const int64_t nv = (j1 - j0) / VE;
  int64_t v = 0;
  for (; v + NB <= nv; v += NB) {
    float x[NB][VE];
#pragma unroll
    for (int q = 0; q < NB; ++q) Vec<Tin>::load(row + j0 + (v + q) * VE, x[q]);
#pragma unroll
    for (int q = 0; q < NB; ++q)
#pragma unroll
      for (int e = 0; e < VE; ++e) f(j0 + (v + q) * VE + e, x[q][e]);
  }
  for (; v < nv; ++v) {
    float x[VE];
    Vec<Tin>::load(row + j0 + v * VE, x);
#pragma unroll
    for (int e = 0; e < VE; ++e) f(j0 + v * VE + e, x[e]);
  }
  for (int64_t j = j0 + nv * VE; j < j1; ++j) f(j, Vec<Tin>::load1(row + j));
}

__device__ __forceinline__ void hist_clear(SamplerLds& L) {
  __syncthreads();
  for (int i = threadIdx.x; i < kHist * kBins; i += kST) {
    (&L.u.h.cnt[0][0])[i] = 0u;
    (&L.u.h.mass[0][0])[i] = 0ull;
  }
  __syncthreads();
}

// Sums the per-wave histograms into tot_cnt / tot_mass.
__device__ __forceinline__ void hist_merge(SamplerLds& L) {
  __syncthreads();
  const int t = threadIdx.x;
  if (t < kBins) {
    unsigned c = 0;
    unsigned long long m = 0;
#pragma unroll
    for (int w = 0; w < kHist; ++w) {
      c += L.u.h.cnt[w][t];
      m += L.u.h.mass[w][t];
    }
    L.tot_cnt[t] = c;
    L.tot_mass[t] = m;
  }
  __syncthreads();
}

// numpy.argmax of the row g(l) (NaN first, then the lowest index of the max).
template <typename Tin, typename G>
__device__ __forceinline__ int64_t row_argmax(const Tin* row, int64_t V, SamplerLds& L, G&& g) {
  float bv = kNegInf;
  int64_t bi = INT64_MAX;
  for_row<Tin>(row, V, [&](int64_t j, float x) {
    const float v = g(x);
    if (bi == INT64_MAX || argmax_better(v, j, bv, bi)) { bv = v; bi = j; }
  });
  block_argmax<kST>(bv, bi, L.f, L.i);
  return bi == INT64_MAX ? 0 : bi;
}

// The id of the m-th element (1-based, id order) of the row for which
// pred(j, raw) holds, -1 if there are fewer.  Thread t owns the contiguous
// range [t*seg, (t+1)*seg) (seg a multiple of the vector width): counts, a
// scan in thread order, then the owner of the m-th match walks its range.
template <typename Tin, typename P>
__device__ __forceinline__ int64_t nth_match(const Tin* row, int64_t V, unsigned long long m, SamplerLds& L, P&& pred) {
  constexpr int VE = Vec<Tin>::N;
  const int tid = threadIdx.x;
  const int64_t seg = ((V + kST - 1) / kST + VE - 1) / VE * VE;
  const int64_t j0 = min((int64_t)tid * seg, V), j1 = min(j0 + seg, V);
  unsigned long long c = 0;
  seg_visit<Tin>(row, j0, j1, [&](int64_t j, float x) { c += pred(j, x) ? 1ull : 0ull; });
  __syncthreads();
  L.u.d.seg[tid] = c;
  __syncthreads();
  if (tid == 0) {
    unsigned long long run = 0;
    int owner = -1;
    for (int t = 0; t < kST; ++t) {
      if (run + L.u.d.seg[t] >= m) { owner = t; break; }
      run += L.u.d.seg[t];
    }
    L.tstar = owner;
    L.rank = m - run;  // rank of the match inside the owner's range
    L.jstar = -1;
  }
  __syncthreads();
  if (tid == L.tstar) {
    const unsigned long long want = L.rank;
    unsigned long long r = 0;
    int64_t found = -1;
    seg_visit<Tin>(row, j0, j1, [&](int64_t j, float x) {
      if (found < 0 && pred(j, x) && ++r == want) found = j;
    });
    L.jstar = found;
  }
  __syncthreads();
  const int64_t res = L.jstar;
  __syncthreads();
  return res;
}

template <typename Tin, int SM>
__global__ __launch_bounds__(kST) void k_sampler(SamplerParams p) {
  __shared__ SamplerLds L;
  extern __shared__ double sh_m[];  // draw: sub-block masses
  constexpr int VE = Vec<Tin>::N;
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  const int wave = tid / VNX_WAVE, lane = tid % VNX_WAVE;
  const Tin* row = static_cast<const Tin*>(p.x) + b * p.ld;
  const int64_t V = p.V;
  int fl = 0;
  int64_t kstar = -1;
  auto finish = [&](int64_t token, float lse, float kth, float ps, int64_t js) {
    if (tid == 0) {
      p.out[b] = token;
      if (p.flags) p.flags[b] = (uint8_t)fl;
      if (p.lse) p.lse[b] = lse;
      if (p.kth) p.kth[b] = kth;
      if (p.p_star) p.p_star[b] = ps;
      if (p.j_star) p.j_star[b] = js;
      if (p.k_star) p.k_star[b] = kstar;
    }
  };
  // ---- calibration: s = sqrt(RN32(var) + eps), l -> RN(RN(l / s) * f) ----
  float sd = 1.0f;
  if (p.calib) {
    double s1 = 0.0;
    for_row<Tin>(row, V, [&](int64_t, float x) { s1 += (double)x; });
    const double mean = block_sum<kST>(s1, L.dd) / (double)V;
    double s2 = 0.0;
    for_row<Tin>(row, V, [&](int64_t, float x) {
      const double d = (double)x - mean;
      s2 += d * d;
    });
    const double var = block_sum<kST>(s2, L.dd) / (double)V;
    sd = sqrtf((float)var + p.ceps);
  }
  // small lambdas capture by value so every closure stays in registers
  auto val = [calib = p.calib != 0, sd, cf = p.cf](float x) -> float { return calib ? (x / sd) * cf : x; };
  if (p.greedy) {
    finish(row_argmax<Tin>(row, V, L, val), __builtin_nanf(""), kNegInf, -1.0f, -1);
    return;
  }
  auto scaled = [val, sc = p.sc](float x) -> float { return tscale<SM>(val(x), sc); };
  const bool exact = p.exact_k != 0;
  auto key = [exact](float a) -> uint32_t { return exact ? okey_lo(a) : okey(a); };
  // ---- top-k: radix select of the kth largest scaled value ----
  const bool use_thr = p.top_k > 0 && p.top_k < V;
  float thr = kNegInf;
  uint32_t tkey = 0u;
  if (use_thr) {
    if (tid == 0) { L.prefix = 0u; L.pmask = 0u; L.rem = (unsigned long long)p.top_k; }
    for (int pass = 0; pass < 4; ++pass) {
      hist_clear(L);
      const int shift = 24 - 8 * pass;
      const uint32_t prefix = L.prefix, pmask = L.pmask;
      for_row<Tin>(row, V, [&](int64_t, float x) {
        const uint32_t k = key(scaled(x));
        if ((k & pmask) == prefix) atomicAdd(&L.u.h.cnt[wave % kHist][(k >> shift) & 0xFFu], 1u);
      });
      hist_merge(L);
      if (tid == 0) {
        unsigned long long above = 0;
        int bin = 0;
        for (int d = kBins - 1; d >= 0; --d) {
          if (above + L.tot_cnt[d] >= L.rem) { bin = d; break; }
          above += L.tot_cnt[d];
        }
        L.rem -= above;
        L.prefix = prefix | ((uint32_t)bin << shift);
        L.pmask = pmask | (0xFFu << shift);
      }
      __syncthreads();
    }
    tkey = L.prefix;
    thr = okey_value(tkey);
    if (exact) {
      // L.rem ties at the kth key complete the k: the last kept one is the
      // L.rem-th tie in id order
      const unsigned long long m = L.rem;
      kstar = nth_match<Tin>(row, V, m, L, [key, scaled, tkey](int64_t, float x) { return key(scaled(x)) == tkey; });
    }
  }
  auto masked = [scaled, key, use_thr, exact, thr, tkey, kstar](int64_t j, float x) -> float {
    const float a = scaled(x);
    if (!use_thr) return a;
    if (!exact) return a >= thr ? a : kNegInf;
    const uint32_t k = key(a);
    return (k > tkey || (k == tkey && j <= kstar)) ? a : kNegInf;
  };
  // ---- softmax: max, row LSE (fp64), L32 ----
  float M = kNegInf;
  bool nan = false;
  for_row<Tin>(row, V, [&](int64_t j, float x) {
    const float a = masked(j, x);
    nan |= __builtin_isnan(a);
    M = fmaxf(M, a);
  });
  {
    const float bm = block_max<kST>(nan ? kPosInf : M, L.f);
    M = bm;
  }
  if (!(M > kNegInf && M < kPosInf)) {  // np.max not finite: numpy.argmax of the row
    __syncthreads();
    finish(row_argmax<Tin>(row, V, L, val), __builtin_nanf(""), thr, -1.0f, -1);
    return;
  }
  const float mt = mt_of(M);
  double s = 0.0;
  for_row<Tin>(row, V, [&](int64_t j, float x) {
    const float a = masked(j, x);
    if (a > kNegInf) s += (double)exp2_term(a, mt);
  });
  s = block_sum<kST>(s, L.dd);
  const double Lr = lse_of(M, s);
  const float L32 = (float)Lr;
  {
    const double up = (double)nextafterf(L32, kPosInf), dn = (double)nextafterf(L32, kNegInf);
    const double mu = 0.5 * ((double)L32 + up), md = 0.5 * ((double)L32 + dn);
    if (fabs(Lr - mu) < 1e-7 || fabs(Lr - md) < 1e-7) fl |= VNX_FLAG_LSE_EDGE;
  }
  auto prob = [masked, L32](int64_t j, float x) -> float { return vnx_exp_canon(masked(j, x) - L32); };
  // ---- top-p: nucleus value p*, tie count, j* ----
  float pstar = -1.0f;
  int64_t jstar = -1;
  if (p.use_p) {
    if (tid == 0) { L.prefix = 0u; L.pmask = 0u; L.rem = p.p_target; L.done = 0; }
    for (int pass = 0; pass < 4; ++pass) {
      hist_clear(L);
      const int shift = 24 - 8 * pass;
      const uint32_t prefix = L.prefix, pmask = L.pmask;
      for_row<Tin>(row, V, [&](int64_t j, float x) {
        const float pp = prob(j, x);
        const uint32_t k = __float_as_uint(pp);
        if ((k & pmask) == prefix) {
          const int d = (k >> shift) & 0xFFu;
          atomicAdd(&L.u.h.cnt[wave % kHist][d], 1u);
          atomicAdd(&L.u.h.mass[wave % kHist][d], fix60(pp));
        }
      });
      hist_merge(L);
      if (tid == 0 && !L.done) {
        unsigned long long above = 0;
        int bin = -1;
        for (int d = kBins - 1; d >= 0; --d) {
          if (above + L.tot_mass[d] >= L.rem) { bin = d; break; }
          above += L.tot_mass[d];
        }
        if (bin < 0) {
          L.done = 1;  // the whole mass stays below top_p: every token is kept
        } else {
          L.rem -= above;
          L.prefix = prefix | ((uint32_t)bin << shift);
          L.pmask = pmask | (0xFFu << shift);
        }
      }
      __syncthreads();
      if (L.done) break;
    }
    if (!L.done) {
      pstar = __uint_as_float(L.prefix);
      // m = the smallest number of ties whose fixed-point mass reaches rem
      const unsigned long long P = fix60(pstar);  // > 0: a zero-mass bin is never chosen
      const unsigned long long m = (L.rem + P - 1) / P;
      jstar = nth_match<Tin>(row, V, m, L, [prob, pstar](int64_t j, float x) { return prob(j, x) == pstar; });
    }
    __syncthreads();
  }
  auto weight = [prob, pstar, jstar](int64_t j, float x) -> float {
    const float pp = prob(j, x);
    if (pstar >= 0.0f && !(pp > pstar || (pp == pstar && j <= jstar))) return 0.0f;
    return pp;
  };
  // ---- draw ----
  const int64_t sbl = (int64_t)VNX_WAVE * VE;
  const int64_t nsb = (V + sbl - 1) / sbl;  // <= kSampDraw (host check)
  auto lane_w = [&](int64_t sbi, float (&w)[VE]) -> double {
    const int64_t e0 = (sbi * VNX_WAVE + lane) * VE;
    float x[VE];
    if (e0 + VE <= V) {
      Vec<Tin>::load(row + e0, x);
    } else {
#pragma unroll
      for (int i = 0; i < VE; ++i) x[i] = 0.0f;
    }
    double m = 0.0;
#pragma unroll
    for (int i = 0; i < VE; ++i) {
      w[i] = (e0 + i < V) ? weight(e0 + i, e0 + VE <= V ? x[i] : Vec<Tin>::load1(row + e0 + i)) : 0.0f;
      m += (double)w[i];
    }
    return m;
  };
  constexpr int kDNB = 4;  // sub-blocks in flight per wave
  for (int64_t s0 = wave; s0 < nsb; s0 += (int64_t)kSW * kDNB) {
    double m[kDNB];
#pragma unroll
    for (int j = 0; j < kDNB; ++j) {
      float w[VE];
      const int64_t sbi = s0 + (int64_t)kSW * j;
      m[j] = sbi < nsb ? lane_w(sbi, w) : 0.0;
    }
#pragma unroll
    for (int j = 0; j < kDNB; ++j) {
      const int64_t sbi = s0 + (int64_t)kSW * j;
      const double t = wave_sum(m[j]);
      if (lane == 0 && sbi < nsb) sh_m[sbi] = t;
    }
  }
  __syncthreads();
  const int64_t q = (nsb + kST - 1) / kST;
  {
    double t = 0.0;
    for (int64_t i = (int64_t)tid * q; i < min((int64_t)(tid + 1) * q, nsb); ++i) t += sh_m[i];
    const double incl = block_inclusive_scan<kST>(t, L.scan);
    L.u.d.T[tid] = t;
    L.u.d.E[tid] = incl;
    __syncthreads();
    if (tid == kST - 1) L.total = incl;
    if (tid == 0) { L.tstar = kST; L.tlast = -1; }
    __syncthreads();
  }
  const double total = L.total;
  const double target = (double)p.u[b] * total;
  {
    const double T = L.u.d.T[tid], end = L.u.d.E[tid];
    const double start = tid ? L.u.d.E[tid - 1] : 0.0;
    if (T > 0.0 && start <= target && target < end) atomicMin(&L.tstar, tid);
    if (T > 0.0) atomicMax(&L.tlast, tid);
  }
  __syncthreads();
  if (tid == 0) {
    int ts = L.tstar;
    if (ts == kST) ts = L.tlast;
    int64_t sstar = -1;
    double base = 0.0;
    if (ts >= 0) {
      const double b0 = ts ? L.u.d.E[ts - 1] : 0.0;
      double r2 = b0, b_last = b0;
      int64_t slast = -1;
      for (int64_t i = (int64_t)ts * q; i < min((int64_t)(ts + 1) * q, nsb); ++i) {
        const double m = sh_m[i];
        if (m > 0.0) {
          if (sstar < 0 && r2 + m > target) { sstar = i; base = r2; }
          slast = i;
          b_last = r2;
        }
        r2 += m;
      }
      if (sstar < 0) { sstar = slast; base = b_last; }
    }
    L.sb = sstar;
    L.target = target;
    L.base = base;
  }
  __syncthreads();
  const int64_t sstar = L.sb;
  if (wave != 0) return;
  int64_t token = 0;
  if (sstar < 0) {
    fl |= VNX_FLAG_ZERO_RESIDUAL;
  } else {
    float w[VE];
    const double lm = lane_w(sstar, w);
    const double incl = wave_inclusive_scan(lm);
    const double start = L.base + (incl - lm), end = L.base + incl;
    const double tgt = L.target;
    const bool hit = lm > 0.0 && start <= tgt && tgt < end;
    const uint64_t hits = __ballot(hit), pos = __ballot(lm > 0.0);
    int lstar;
    bool edge = false;
    if (hits) {
      lstar = __builtin_ctzll(hits);
    } else {
      lstar = pos ? 63 - __builtin_clzll(pos) : -1;
      edge = true;
    }
    if (lstar < 0) {
      token = (sstar * VNX_WAVE) * VE;
      edge = true;
    } else if (lane == lstar) {
      double run = start, before = start, after = end;
      int pick = -1, lastpos = -1;
#pragma unroll
      for (int i = 0; i < VE; ++i) {
        if (w[i] > 0.0f) {
          lastpos = i;
          if (pick < 0) {
            const double nr = run + (double)w[i];
            if (nr > tgt) { pick = i; before = run; after = nr; }
            run = nr;
          }
        }
      }
      if (pick < 0) { pick = lastpos; edge = true; }
      token = (sstar * VNX_WAVE + lane) * VE + pick;
      const double tol = 1e-12 * L.total;
      if (tgt - before < tol || after - tgt < tol) edge = true;
    }
    if (lstar >= 0) {
      token = __shfl(token, lstar, VNX_WAVE);
      edge = __shfl((int)edge, lstar, VNX_WAVE) != 0;
    }
    if (edge) fl |= VNX_FLAG_CDF_EDGE;
  }
  finish(token, L32, thr, pstar, jstar);
}

// ---------------------------------------------------------------------------
// Logit calibration: out = RN(RN(x / s) * f), s = RN(sqrt(RN(RN32(var) +
// eps))), var = the fp64 population variance of the row (mean first, then
// the squared deviations), one workgroup per row.
// ---------------------------------------------------------------------------
template <typename Tin>
__global__ __launch_bounds__(kST) void k_logit_calibrate(const Tin* __restrict__ x, int64_t V, int64_t ld, float f,
                                                         float eps, float* __restrict__ out, int64_t ldo,
                                                         double* var_out) {
  __shared__ double red[kSW];
  const int64_t b = blockIdx.x;
  const Tin* row = x + b * ld;
  double s = 0.0;
  for_row<Tin>(row, V, [&](int64_t, float v) { s += (double)v; });
  const double mean = block_sum<kST>(s, red) / (double)V;
  double s2 = 0.0;
  for_row<Tin>(row, V, [&](int64_t, float v) {
    const double d = (double)v - mean;
    s2 += d * d;
  });
  const double var = block_sum<kST>(s2, red) / (double)V;
  const float sd = sqrtf((float)var + eps);
  float* o = out + b * ldo;
  for_row<Tin>(row, V, [&](int64_t j, float v) { o[j] = (v / sd) * f; });
  if (threadIdx.x == 0 && var_out) var_out[b] = var;
}

}  // namespace vnx

using namespace vnx;

extern "C" {

int vnx_sampler_sample(const void* logits, int dtype, int64_t B, int64_t V, int64_t ld, float temperature,
                       int64_t top_k, float top_p, int mode, float calib_factor, float calib_eps,
                       const float* uniforms, int64_t* out_ids, uint8_t* flags, float* lse, float* kth,
                       float* p_star, int64_t* j_star, int64_t* k_star, void* stream) {
  if (dtype != VNX_F32 && dtype != VNX_BF16) return VNX_ERR_UNSUPPORTED;
  if (B < 0 || V <= 0 || top_k < 0) return VNX_ERR_INVALID_ARG;
  if (mode & ~(VNX_SAMPLE_EXACT_K | VNX_SAMPLE_CALIBRATE)) return VNX_ERR_INVALID_ARG;
  if ((mode & VNX_SAMPLE_CALIBRATE) && (!__builtin_isfinite(calib_factor) || !(calib_eps >= 0.0f)))
    return VNX_ERR_INVALID_ARG;
  if (!(temperature >= 0.0f) || !__builtin_isfinite(temperature)) return VNX_ERR_INVALID_ARG;
  if (!(top_p > 0.0f && top_p <= 1.0f)) return VNX_ERR_INVALID_ARG;
  if (B == 0) return VNX_OK;
  if (!logits || !out_ids || (temperature > 0.0f && !uniforms)) return VNX_ERR_INVALID_ARG;
  const int ve = dtype == VNX_F32 ? 4 : 8;
  if (ld < V || ld % ve || reinterpret_cast<uintptr_t>(logits) % 16) return VNX_ERR_INVALID_ARG;
  const int64_t nsb = (V + (int64_t)VNX_WAVE * ve - 1) / ((int64_t)VNX_WAVE * ve);
  if (nsb > kSampDraw || B > INT32_MAX) return VNX_ERR_UNSUPPORTED;
  SamplerParams p{};
  p.x = logits; p.B = B; p.V = V; p.ld = ld;
  p.greedy = temperature == 0.0f;
  const int sm = p.greedy ? SM_ID : make_scale(temperature, &p.sc);
  p.top_k = top_k;
  p.exact_k = (mode & VNX_SAMPLE_EXACT_K) != 0;
  p.calib = (mode & VNX_SAMPLE_CALIBRATE) != 0;
  p.cf = calib_factor;
  p.ceps = calib_eps;
  p.use_p = top_p < 1.0f;
  p.p_target = (uint64_t)floor((double)top_p * 1152921504606846976.0);
  p.u = uniforms; p.out = out_ids; p.flags = flags; p.lse = lse; p.kth = kth; p.p_star = p_star; p.j_star = j_star;
  p.k_star = k_star;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t lds = (size_t)nsb * sizeof(double);
  return dispatch_tsm(dtype, sm, false, [&](auto tin, auto smc, auto) {
    using Tin = decltype(tin);
    constexpr int SM = decltype(smc)::value;
    hipLaunchKernelGGL((k_sampler<Tin, SM>), dim3((unsigned)B), dim3(kST), lds, s, p);
    VNX_LAUNCH_CHECK();
    return (int)VNX_OK;
  });
}

int vnx_logit_calibrate(const void* logits, int dtype, int64_t B, int64_t V, int64_t ld, float calib_factor,
                        float eps, float* out, int64_t ld_out, double* var, void* stream) {
  if (dtype != VNX_F32 && dtype != VNX_BF16) return VNX_ERR_UNSUPPORTED;
  if (B < 0 || V <= 0 || !__builtin_isfinite(calib_factor) || !(eps >= 0.0f)) return VNX_ERR_INVALID_ARG;
  if (B == 0) return VNX_OK;
  const int ve = dtype == VNX_F32 ? 4 : 8;
  if (!logits || !out || ld < V || ld % ve || ld_out < V || reinterpret_cast<uintptr_t>(logits) % 16)
    return VNX_ERR_INVALID_ARG;
  if (B > INT32_MAX) return VNX_ERR_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == VNX_F32)
    hipLaunchKernelGGL((k_logit_calibrate<float>), dim3((unsigned)B), dim3(kST), 0, s,
                       static_cast<const float*>(logits), V, ld, calib_factor, eps, out, ld_out, var);
  else
    hipLaunchKernelGGL((k_logit_calibrate<__hip_bfloat16>), dim3((unsigned)B), dim3(kST), 0, s,
                       static_cast<const __hip_bfloat16*>(logits), V, ld, calib_factor, eps, out, ld_out, var);
  VNX_LAUNCH_CHECK();
  return VNX_OK;
}

}  // extern "C"
