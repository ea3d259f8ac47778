// Sampler.sample on the GPU (packages/verse_infra/verse_infra/verse_inference/
// sampler.py:70-138), CometSpark's sampling step (packages/verse_nex/
// verse_nex/cometspark.py:868-910) and the logit calibration of
// VMPC-compressed models (cometspark.py:922-948).
//
// Every row is split into C chunks of whole draw sub-blocks (about four
// workgroups per CU over the batch, at most 8192 elements each), and the
// reference's steps run as a short chain of launches; kernel boundaries carry
// the row state between them (no fences, no grid barrier):
//   init       (without top-k) zero the row's histograms and counters;
//   calib 0,1  (VNX_SAMPLE_CALIBRATE) chunk sums of x, then of (x - mean)^2,
//              in fp64; later launches merge the C partials in chunk order
//              into var, s = RN(sqrt(RN32(var) + eps)), l -> RN(RN(l/s) * f).
// With top-k (0 < k <= 256, V <= 64 * 8192), any rule:
//   local      every chunk is read once into LDS as order-preserving keys of
//              a = RN(l/T) (Sampler: NaN ranks largest; exactly-k: NaN ranks
//              smallest; -0 == +0), takes t = the kth largest of its 256
//              per-thread maxima (at most its own kth largest key) and
//              publishes every key >= t with its id.  Every token the global
//              cut keeps is among them;
//   cand       one 1024-thread workgroup per row, in LDS: the candidates
//              with key >= the largest chunk threshold (a lower bound of the
//              row's kth key), sorted by (key desc, id asc); the global cut
//              (Sampler: a >= kth; exactly-k: argpartition(-a)[:k], ties at
//              the kth value by lower id), max(a) (not finite: numpy.argmax of
//              the row, one more read of it), the fp64 LSE and L32 = RN32(LSE), p =
//              vnx_exp_canon(a - L32), the nucleus (a sort by (p desc, id
//              asc), exact fixed-point cumulative sums floor(p * 2^60), the
//              first cutoff + 1 kept), the kept tokens sorted by id, and the
//              draw (numpy's Generator.choice rule: first j with
//              C_j > u * C_V, fp64 sums); with at most 64 survivors one wave
//              does all of it in registers.
//              A row whose candidates overflow (many ties at a threshold),
//              a larger k or a longer row runs the whole algorithm over the
//              row in the same workgroup instead (single-workgroup form).
// Without top-k:
//   lse        per chunk the max of a (NaN -> +inf), the fp64 sum of
//              2^(a*log2e - mt), and numpy.argmax of the row;
//   ppass 0..3 (top-p) every workgroup merges the C LSE partials (one wave,
//              fixed order) into L32 and radix-selects the nucleus value p*
//              over the keys of p with fixed-point mass histograms (the last
//              pass also counts per chunk, for ranking the ties),
//              one 8-bit digit per launch: per-wave LDS histograms, nonzero
//              bins added to the row's global histogram, the digit derived by
//              the next launch (a block scan) and recorded by its chunk 0;
//   mass       draw weights (p, or p masked by the nucleus: p > p*, or
//              p == p* and id <= j*, j* ranked by the one chunk holding it),
//              fp64 masses per 64-vector sub-block published with agent-scope
//              stores; the workgroup that completes the row walks them to
//              u * total and writes every output.
// T == 0 runs init, an argmax-only lse and the mass launch's final step.
// The CPU checker oracle/sampler.py restates the same rules.  The exactly-k
// draw runs over the kept tokens in id order: argpartition's output order,
// which the reference draws over, is implementation-defined.
#include <algorithm>

#include "rowred.h"
#include "vnx_internal.h"

namespace vnx {

constexpr int kSNT = 256;              // threads per workgroup (chunk kernels)
constexpr int kSNW = kSNT / VNX_WAVE;
constexpr int kST = 1024;              // threads per workgroup (per-row kernels)
constexpr int kSW = kST / VNX_WAVE;
constexpr int kSNB = 4;                // vectors in flight per thread
constexpr int kBins = 256;             // 8-bit digits
constexpr int kSMaxC = 64;             // chunks per row (one wave merges their partials)
constexpr int64_t kChunkMax = 8192;    // elements per chunk (the local kernel's LDS keys)
constexpr int kSampDraw = 4096;        // sub-blocks of 64 vectors per row (the draw walk in LDS)
constexpr int kCandMax = 4096;         // candidates per row (the per-row kernel's LDS)
constexpr int kSegCap = 512;           // candidates per chunk
constexpr int64_t kLocalMaxK = 256;    // top_k of the candidate search (one maximum per thread)
constexpr int kHist = 8;               // per-wave histogram copies of the per-row kernel
constexpr int64_t kLocalMaxV = (int64_t)kSMaxC * kChunkMax;

struct RadixState {
  uint32_t prefix, pmask;
  unsigned long long rem;  // units still to take; after the last pass: ties in the cut chunk
  int done;                // (by mass) fewer units than rem: every token is kept
  int cstar;               // after the last pass: the chunk holding the cut
};

struct SampParams {
  const void* x;
  int64_t B, V, ld;
  TScale sc;
  int greedy, exact, calib, use_k, use_p;
  int single;          // top-k rows too long for the chunked candidate search
  int64_t top_k;
  uint64_t p_target;   // floor(top_p * 2^60)
  float cf, ceps;
  int C;
  int64_t clen, nsb;
  const float* u;      // the rows' uniforms (float), or
  const double* u64;   // ... as doubles (VNX_SAMPLE_UNIFORM_F64; u unused)
  int64_t* out;
  uint8_t* flags;
  float* lse;
  float* kth;
  float* p_star;
  int64_t* j_star;
  int64_t* k_star;
  // workspace
  unsigned long long* phm;    // [B][4][256]
  uint32_t* lp;               // [B][C][256] the last p pass's per-chunk counts
  RadixState* stp;            // [B][5] top-p state before pass i
  double* cs1;                // [B][C] calibration partials
  double* cs2;
  float* pm;                  // [B][C] LSE / argmax partials
  double* ps;
  float* pav;
  int64_t* pai;
  int64_t* jstar;             // [B] the last kept tie of the nucleus (agent-scope)
  double* sbm;                // [B][nsb]
  unsigned* cnt;              // [B]
  unsigned long long* cand;   // [B][C][kSegCap] candidates (key << 32 | ~id)
  unsigned* nct;              // [B][C] candidates per chunk
  uint32_t* tc;               // [B][C] the chunk's threshold key
};

// Row b's uniform in double: a float uniform converts exactly, a double one
// (numpy's Generator.random) is used as drawn.
__device__ __forceinline__ double samp_u(const SampParams& p, int64_t b) {
  return p.u64 ? p.u64[b] : (double)p.u[b];
}


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

// Calls f(j, raw) for every element of [j0, j1) (j0 a multiple of the vector
// width), each thread its vectors tid, tid + NT, ... in batches of kSNB
// loads, all issued before the first use (the last batch predicated), then
// the scalar tail.
template <typename Tin, int NT, typename F>
__device__ __forceinline__ void for_range(const Tin* row, int64_t j0, int64_t j1, F&& f) {
  constexpr int VE = Vec<Tin>::N;
  const int64_t nv = (j1 - j0) / VE;
  const int tid = threadIdx.x;
  // The range's full vectors through a buffer resource: every load is issued
  // (one past the range reads zeros without a memory access, and is not
  // consumed), so no condition or select sits beside a load and the waits
  // count statically; raw bits are converted in the second loop.
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<Tin*>(row + j0), (short)0, (int)(nv * VE * (int64_t)sizeof(Tin)), 0x00020000);
  for (int64_t v0 = 0; v0 < nv; v0 += (int64_t)NT * kSNB) {
    u32x4 raw[kSNB];
#pragma unroll
    for (int q = 0; q < kSNB; ++q) {
      const int64_t v = v0 + tid + (int64_t)NT * q;
      raw[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(v * 16), 0, 2));
    }
#pragma unroll
    for (int q = 0; q < kSNB; ++q) {
      const int64_t v = v0 + tid + (int64_t)NT * q;
      if (v < nv) {
        float x[VE];
        Vec<Tin>::cvt_raw(raw[q], x);
#pragma unroll
        for (int e = 0; e < VE; ++e) f(j0 + v * VE + e, x[e]);
      }
    }
  }
  const int64_t t0 = j0 + nv * VE;
  if (tid < j1 - t0) f(t0 + tid, Vec<Tin>::load1(row + t0 + tid));
}

// Calls f(j, raw) for j in [j0, j1) in increasing order (j0 a multiple of the
// vector width), kSNB vector loads in flight.
template <typename Tin, typename F>
__device__ __forceinline__ void seg_visit(const Tin* row, int64_t j0, int64_t j1, F&& f) {
  constexpr int VE = Vec<Tin>::N;
  constexpr int NB = kSNB;
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

// Inclusive scan of one u64 per thread across a workgroup of NT threads.
template <int NT>
__device__ __forceinline__ unsigned long long block_scan_u64(unsigned long long v, unsigned long long* lds) {
  constexpr int NW = NT / VNX_WAVE;
  const int w = threadIdx.x / VNX_WAVE, l = threadIdx.x % VNX_WAVE;
#pragma unroll
  for (int o = 1; o < VNX_WAVE; o <<= 1) {
    const unsigned long long n = __shfl_up(v, o, VNX_WAVE);
    if (l >= o) v += n;
  }
  __syncthreads();
  if (l == VNX_WAVE - 1) lds[w] = v;
  __syncthreads();
  unsigned long long base = 0;
#pragma unroll
  for (int j = 0; j < NW; ++j)
    if (j < w) base += lds[j];
  return base + v;
}

// The digit whose bin holds the rem-th unit counted from the top of a 256-bin
// histogram h (counts or fixed-point masses): wave 0 scans 4 bins per lane,
// top down; returns kBins when the histogram holds fewer than rem units.
// *above = the units in the bins above it.  Every thread gets the result.
template <typename T>
__device__ __forceinline__ int pick_digit(const T* h, unsigned long long rem, unsigned long long* above, int* sel,
                                          unsigned long long* sabove) {
  if (threadIdx.x < VNX_WAVE) {
    const int lane = threadIdx.x;
    unsigned long long v[4], s = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v[q] = (unsigned long long)h[kBins - 1 - (4 * lane + q)];
      s += v[q];
    }
    unsigned long long incl = s;
#pragma unroll
    for (int o = 1; o < VNX_WAVE; o <<= 1) {
      const unsigned long long n = __shfl_up(incl, o, VNX_WAVE);
      if (lane >= o) incl += n;
    }
    const uint64_t hit = __ballot(incl >= rem && incl - s < rem);
    if (lane == 0) *sel = kBins;
    if (hit && lane == (int)__builtin_ctzll(hit)) {
      unsigned long long run = incl - s;
      int d = kBins;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (d == kBins && v[q] > 0 && run + v[q] >= rem) d = kBins - 1 - (4 * lane + q);
        if (d == kBins) run += v[q];
      }
      *sel = d;
      *sabove = run;
    }
  }
  __syncthreads();
  const int d = *sel;
  *above = *sabove;
  __syncthreads();
  return d;
}

// ===========================================================================
// Chunk kernels (kSNT threads).
// ===========================================================================
struct SampLds {
  unsigned hc[kSNW][kBins];            // per-wave histogram copies
  unsigned long long hm[kSNW][kBins];
  unsigned long long scan[kSW];
  double dd[kSW];
  float f[kSW];
  int64_t i[kSW];
  unsigned long long seg[kSNT];
  int sel, flag;
  unsigned long long rank, above;
  int64_t found;
  // the draw walk
  double T[kSNT], E[kSNT];
  double total, target, base;
  int64_t sb;
  int tstar, tlast;
};

// The id of the m-th element (1-based, id order) of [j0, j1) for which
// pred(j, raw) holds, -1 if there are fewer: contiguous per-thread ranges,
// counts, a scan in thread order, then the owner of the m-th match walks.
template <typename Tin, int NT, typename P>
__device__ __forceinline__ int64_t nth_in_range(const Tin* row, int64_t j0, int64_t j1, unsigned long long m,
                                                SampLds& L, P&& pred) {
  constexpr int VE = Vec<Tin>::N;
  const int tid = threadIdx.x;
  const int64_t seg = ((j1 - j0 + NT - 1) / NT + VE - 1) / VE * VE;
  const int64_t a0 = min(j0 + (int64_t)tid * seg, j1), a1 = min(a0 + seg, j1);
  unsigned long long c = 0;
  seg_visit<Tin>(row, a0, a1, [&](int64_t j, float x) { c += pred(j, x) ? 1ull : 0ull; });
  __syncthreads();
  L.seg[tid] = c;
  __syncthreads();
  if (tid == 0) {
    unsigned long long run = 0;
    int owner = -1;
    for (int t = 0; t < NT; ++t) {
      if (run + L.seg[t] >= m) { owner = t; break; }
      run += L.seg[t];
    }
    L.sel = owner;
    L.rank = m - run;
    L.found = -1;
  }
  __syncthreads();
  if (tid == L.sel) {
    const unsigned long long want = L.rank;
    unsigned long long r = 0;
    int64_t found = -1;
    seg_visit<Tin>(row, a0, a1, [&](int64_t j, float x) {
      if (found < 0 && pred(j, x) && ++r == want) found = j;
    });
    L.found = found;
  }
  __syncthreads();
  const int64_t res = L.found;
  __syncthreads();
  return res;
}

// One step of the nucleus radix select from the state before a pass and
// that pass's global (count, mass) histogram.
__device__ __forceinline__ RadixState p_step(RadixState s, int pass, const unsigned long long* hm, SampLds& L) {
  if (s.done) return s;
  unsigned long long above;
  const int d = pick_digit(hm, s.rem, &above, &L.sel, &L.above);
  RadixState o = s;
  if (d == kBins) {
    o.done = 1;  // the whole mass stays below top_p: every token is kept
  } else {
    const int shift = 24 - 8 * pass;
    o.rem = s.rem - above;
    o.prefix = s.prefix | ((uint32_t)d << shift);
    o.pmask = s.pmask | (0xFFu << shift);
  }
  return o;
}

// After the last pass: the chunk holding the rem-th tie of the cut key (from
// every chunk's count of the last digit's bin) and the rank inside it.
__device__ __forceinline__ RadixState locate_cut(RadixState s, const uint32_t* local, int C, SampLds& L) {
  if (threadIdx.x < VNX_WAVE) {
    const int lane = threadIdx.x;
    const unsigned long long n = lane < C ? (unsigned long long)local[lane * kBins + (s.prefix & 0xFFu)] : 0ull;
    unsigned long long incl = n;
#pragma unroll
    for (int o = 1; o < VNX_WAVE; o <<= 1) {
      const unsigned long long q = __shfl_up(incl, o, VNX_WAVE);
      if (lane >= o) incl += q;
    }
    const uint64_t hits = __ballot(n > 0 && incl >= s.rem && incl - n < s.rem);
    const int cs = hits ? (int)__builtin_ctzll(hits) : C - 1;
    const unsigned long long before = __shfl(incl - n, cs, VNX_WAVE);
    if (lane == 0) {
      L.sel = cs;
      L.rank = s.rem - before;
    }
  }
  __syncthreads();
  s.cstar = L.sel;
  s.rem = L.rank;
  __syncthreads();
  return s;
}

// What every launch after the first rebuilds of a row.
struct RowCtx {
  float sd;
  float M, L32;
  bool fallback;      // max(a) not finite
  int fl;
  float pstar;        // nucleus: keep p > pstar, or p == pstar and id <= jbound (pstar < 0: off)
  int64_t jbound;
};

// CAL: the logit calibration (l -> RN(RN(l/s) * f)) is on.
template <int SM, bool CAL>
struct RowFns {
  const SampParams& p;
  const RowCtx& r;
  __device__ __forceinline__ float val(float x) const {
    if constexpr (CAL) return (x / r.sd) * p.cf;
    return x;
  }
  __device__ __forceinline__ float scaled(float x) const { return tscale<SM>(val(x), p.sc); }
  __device__ __forceinline__ float prob(float x) const { return vnx_exp_canon(scaled(x) - r.L32); }
  __device__ __forceinline__ float weight(int64_t j, float x) const {
    const float pp = prob(x);
    if (r.pstar >= 0.0f && !(pp > r.pstar || (pp == r.pstar && j <= r.jbound))) return 0.0f;
    return pp;
  }
};

__device__ __forceinline__ float calib_sd(const SampParams& p, int64_t b) {
  if (!p.calib) return 1.0f;
  double s = 0.0;
  for (int c = 0; c < p.C; ++c) s += p.cs2[b * p.C + c];
  return sqrtf((float)(s / (double)p.V) + p.ceps);
}

__device__ __forceinline__ void ctx_init(const SampParams& p, int64_t b, RowCtx& r) {
  r.sd = calib_sd(p, b);
  r.M = kNegInf;
  r.L32 = 0.0f;
  r.fallback = false;
  r.fl = 0;
  r.pstar = -1.0f;
  r.jbound = INT64_MAX;
}

// L32 = RN32(row LSE) and the LSE_EDGE flag from the fp64 LSE.
__device__ __forceinline__ void set_l32(RowCtx& r, double Lr) {
  r.L32 = (float)Lr;
  const double up = (double)nextafterf(r.L32, kPosInf), dn = (double)nextafterf(r.L32, kNegInf);
  const double mu = 0.5 * ((double)r.L32 + up), md = 0.5 * ((double)r.L32 + dn);
  if (fabs(Lr - mu) < 1e-7 || fabs(Lr - md) < 1e-7) r.fl |= VNX_FLAG_LSE_EDGE;
}

// The row LSE from the C chunk partials (one wave, fixed order).
__device__ __forceinline__ void ctx_lse(const SampParams& p, int64_t b, RowCtx& r, SampLds& L) {
  if (threadIdx.x < VNX_WAVE) {
    const int lane = threadIdx.x;
    float m = kNegInf;
    double s = 0.0;
    if (lane < p.C) {
      m = p.pm[b * p.C + lane];
      s = p.ps[b * p.C + lane];
    }
    const float M = wave_max(m);
    double t = 0.0;
    if (M > kNegInf && M < kPosInf && m > kNegInf) t = m == M ? s : rescale(s, mt_of(m), mt_of(M));
    const double S = wave_sum(t);
    if (lane == 0) {
      L.f[0] = M;
      L.dd[0] = S;
    }
  }
  __syncthreads();
  r.M = L.f[0];
  const double S = L.dd[0];
  __syncthreads();
  r.fallback = !(r.M > kNegInf && r.M < kPosInf);
  if (!r.fallback) set_l32(r, lse_of(r.M, S));
}

// numpy.argmax of the row from the chunk partials (wave 0).
__device__ __forceinline__ int64_t merged_argmax(const SampParams& p, int64_t b) {
  const int lane = threadIdx.x;
  float v = kNegInf;
  int64_t i = INT64_MAX;
  if (lane < p.C) {
    v = p.pav[b * p.C + lane];
    i = p.pai[b * p.C + lane];
  }
  wave_argmax(v, i);
  return i == INT64_MAX ? 0 : i;
}

__global__ __launch_bounds__(kSNT) void k_samp_init(SampParams p) {
  const int64_t b = blockIdx.x;
  const int t = threadIdx.x;
  for (int i = t; i < 4 * kBins; i += kSNT) p.phm[b * 4 * kBins + i] = 0ull;
  if (t == 0) {
    p.cnt[b] = 0u;
    p.stp[b * 5] = RadixState{0u, 0u, (unsigned long long)p.p_target, 0, 0};
  }
}

template <typename Tin, int PASS>
__global__ __launch_bounds__(kSNT) void k_samp_calib(SampParams p) {
  __shared__ double red[kSNW];
  const int64_t b = blockIdx.x / p.C;
  const int c = blockIdx.x % p.C;
  const Tin* row = static_cast<const Tin*>(p.x) + b * p.ld;
  const int64_t j0 = c * p.clen, j1 = min(j0 + p.clen, p.V);
  double s = 0.0;
  if (PASS == 0) {
    for_range<Tin, kSNT>(row, j0, j1, [&](int64_t, float x) { s += (double)x; });
  } else {
    double t = 0.0;
    for (int q = 0; q < p.C; ++q) t += p.cs1[b * p.C + q];
    const double mean = t / (double)p.V;
    for_range<Tin, kSNT>(row, j0, j1, [&](int64_t, float x) {
      const double d = (double)x - mean;
      s += d * d;
    });
  }
  s = block_sum<kSNT>(s, red);
  if (threadIdx.x == 0) (PASS == 0 ? p.cs1 : p.cs2)[b * p.C + c] = s;
}

struct LocalLds {
  uint32_t keys[kChunkMax];
  uint32_t mx[kSNT];
  uint32_t t;
  unsigned n;
};

__device__ __forceinline__ unsigned lane_rank(uint64_t m) {
  // set bits of m below this lane
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// One chunk of a top-k row: its keys into LDS, a lower bound t of its kth
// largest key, and every key >= t published as a candidate (see the header).
// t is the kth largest of the 256 per-thread maxima: k threads hold a key
// >= t, so the chunk holds at least k keys >= t.  For rows of independent
// logits about k(1 + 1/e) keys pass.
template <typename Tin, int SM, bool CAL>
__global__ __launch_bounds__(kSNT) void k_samp_local(SampParams p) {
  __shared__ LocalLds L;
  const int64_t b = blockIdx.x / p.C;
  const int c = blockIdx.x % p.C;
  const int tid = threadIdx.x, lane = tid % VNX_WAVE;
  const Tin* row = static_cast<const Tin*>(p.x) + b * p.ld;
  const int64_t j0 = c * p.clen, j1 = min(j0 + p.clen, p.V);
  const int n = (int)(j1 - j0);  // <= kChunkMax (host plan)
  RowCtx r;
  ctx_init(p, b, r);
  const RowFns<SM, CAL> fn{p, r};
  const bool ex = p.exact != 0;
  uint32_t mx = 0u;
  for_range<Tin, kSNT>(row, j0, j1, [&](int64_t j, float x) {
    const float a = fn.scaled(x);
    // -0 and +0 one value in both orders (the Sampler rule compares values)
    const uint32_t k = ex ? okey_lo(a) : okey(a + 0.0f);
    L.keys[j - j0] = k;
    mx = max(mx, k);
  });
  L.mx[tid] = mx;
  if (tid == 0) L.n = 0u;
  __syncthreads();
  if (tid < VNX_WAVE) {
    // the kth largest maximum, bit by bit from the top: the largest t with
    // at least k maxima >= t (t stays 0, every key, when fewer than k)
    uint32_t v[kSNT / VNX_WAVE];
#pragma unroll
    for (int q = 0; q < kSNT / VNX_WAVE; ++q) v[q] = L.mx[q * VNX_WAVE + lane];
    const int64_t kk = p.top_k;
    uint32_t t = 0u;
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t cand = t | (1u << bit);
      int cnt = 0;
#pragma unroll
      for (int q = 0; q < kSNT / VNX_WAVE; ++q) cnt += __builtin_popcountll(__ballot(v[q] >= cand));
      if (cnt >= kk) t = cand;
    }
    if (lane == 0) L.t = t;
  }
  __syncthreads();
  const uint32_t t = L.t;
  // candidates (key << 32 | ~id, the per-row kernel's sort key) into this
  // chunk's segment, compacted per wave; the count may exceed the segment
  unsigned long long* seg = p.cand + (b * p.C + c) * kSegCap;
  for (int i0 = 0; i0 < n; i0 += kSNT) {
    const int i = i0 + tid;
    const uint32_t k = i < n ? L.keys[i] : 0u;
    const bool take = i < n && k >= t;
    const uint64_t m = __ballot(take);
    if (m) {
      unsigned base = 0u;
      if (lane == 0) base = atomicAdd(&L.n, (unsigned)__builtin_popcountll(m));
      base = __shfl(base, 0, VNX_WAVE);
      const unsigned pos = base + lane_rank(m);
      if (take && pos < (unsigned)kSegCap)
        seg[pos] = ((unsigned long long)k << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)(j0 + i));
    }
  }
  __syncthreads();
  if (tid == 0) {
    p.nct[b * p.C + c] = L.n;
    p.tc[b * p.C + c] = t;
  }
}

template <typename Tin, int SM, bool CAL>
__global__ __launch_bounds__(kSNT) void k_samp_lse(SampParams p) {
  __shared__ SampLds L;
  const int64_t b = blockIdx.x / p.C;
  const int c = blockIdx.x % p.C;
  const Tin* row = static_cast<const Tin*>(p.x) + b * p.ld;
  const int64_t j0 = c * p.clen, j1 = min(j0 + p.clen, p.V);
  RowCtx r;
  ctx_init(p, b, r);
  const RowFns<SM, CAL> fn{p, r};
  // chunk max (NaN -> +inf) and numpy.argmax of the (calibrated) row
  float M = kNegInf, av = kNegInf;
  bool nan = false;
  int64_t ai = INT64_MAX;
  for_range<Tin, kSNT>(row, j0, j1, [&](int64_t j, float x) {
    const float v = fn.val(x);
    if (ai == INT64_MAX || argmax_better(v, j, av, ai)) { av = v; ai = j; }
    if (!p.greedy) {
      const float a = tscale<SM>(v, p.sc);
      nan |= __builtin_isnan(a);
      M = fmaxf(M, a);
    }
  });
  block_argmax<kSNT>(av, ai, L.f, L.i);
  const float bm = block_max<kSNT>(nan ? kPosInf : M, L.f);
  double s = 0.0;
  if (!p.greedy && bm > kNegInf && bm < kPosInf) {
    const float mt = mt_of(bm);
    for_range<Tin, kSNT>(row, j0, j1, [&](int64_t, float x) {
      const float a = fn.scaled(x);
      if (a > kNegInf) s += (double)exp2_term(a, mt);
    });
  }
  s = block_sum<kSNT>(s, L.dd);
  if (threadIdx.x == 0) {
    p.pm[b * p.C + c] = bm;
    p.ps[b * p.C + c] = s;
    p.pav[b * p.C + c] = av;
    p.pai[b * p.C + c] = ai;
  }
}

template <typename Tin, int SM, bool CAL, int PASS>
__global__ __launch_bounds__(kSNT) void k_samp_ppass(SampParams p) {
  __shared__ SampLds L;
  const int64_t b = blockIdx.x / p.C;
  const int c = blockIdx.x % p.C;
  const int wave = threadIdx.x / VNX_WAVE;
  const Tin* row = static_cast<const Tin*>(p.x) + b * p.ld;
  const int64_t j0 = c * p.clen, j1 = min(j0 + p.clen, p.V);
  RowCtx r;
  ctx_init(p, b, r);
  ctx_lse(p, b, r, L);
  if (r.fallback) return;  // uniform over the workgroup
  const RowFns<SM, CAL> fn{p, r};
  RadixState s = p.stp[b * 5 + (PASS > 0 ? PASS - 1 : 0)];
  if (PASS > 0) {
    s = p_step(s, PASS - 1, p.phm + (b * 4 + PASS - 1) * kBins, L);
    if (c == 0 && threadIdx.x == 0) p.stp[b * 5 + PASS] = s;
  }
  if (s.done) return;  // uniform
  for (int i = threadIdx.x; i < kSNW * kBins; i += kSNT) {
    (&L.hc[0][0])[i] = 0u;
    (&L.hm[0][0])[i] = 0ull;
  }
  __syncthreads();
  const int shift = 24 - 8 * PASS;
  for_range<Tin, kSNT>(row, j0, j1, [&](int64_t, float x) {
    const float pp = fn.prob(x);
    const uint32_t k = __float_as_uint(pp);
    if ((k & s.pmask) == s.prefix) {
      const int d = (k >> shift) & 0xFFu;
      if (PASS == 3) atomicAdd(&L.hc[wave][d], 1u);  // the last digit's ties are ranked by count
      atomicAdd(&L.hm[wave][d], fix60(pp));
    }
  });
  __syncthreads();
  const int t = threadIdx.x;  // kSNT == kBins
  unsigned cn = 0;
  unsigned long long m = 0;
#pragma unroll
  for (int w = 0; w < kSNW; ++w) {
    if (PASS == 3) cn += L.hc[w][t];
    m += L.hm[w][t];
  }
  if (m) atomicAdd(p.phm + (b * 4 + PASS) * kBins + t, m);
  if (PASS == 3) p.lp[(b * p.C + c) * kBins + t] = cn;
}

template <typename Tin, int SM, bool CAL>
__global__ __launch_bounds__(kSNT) void k_samp_mass(SampParams p) {
  __shared__ SampLds L;
  extern __shared__ double sh_m[];  // the draw: the row's sub-block masses
  constexpr int VE = Vec<Tin>::N;
  const int64_t b = blockIdx.x / p.C;
  const int c = blockIdx.x % p.C;
  const int tid = threadIdx.x;
  const int wave = tid / VNX_WAVE, lane = tid % VNX_WAVE;
  const Tin* row = static_cast<const Tin*>(p.x) + b * p.ld;
  const int64_t j0 = c * p.clen, j1 = min(j0 + p.clen, p.V);
  const int64_t sbl = (int64_t)VNX_WAVE * VE;
  RowCtx r;
  ctx_init(p, b, r);
  if (!p.greedy) ctx_lse(p, b, r, L);
  const RowFns<SM, CAL> fn{p, r};
  const bool draw = !p.greedy && !r.fallback;
  if (draw && p.use_p) {
    RadixState s = p_step(p.stp[b * 5 + 3], 3, p.phm + (b * 4 + 3) * kBins, L);
    if (!s.done) {
      r.pstar = __uint_as_float(s.prefix);
      // the nucleus needs m ties of value p* (each adds fix60(p*) > 0: a
      // zero-mass bin is never chosen); the chunk holding the m-th ranks them
      const unsigned long long P = fix60(r.pstar);
      s.rem = (s.rem + P - 1) / P;
      s = locate_cut(s, p.lp + b * p.C * kBins, p.C, L);
      if (c < s.cstar) {
        r.jbound = INT64_MAX;
      } else if (c > s.cstar) {
        r.jbound = -1;
      } else {
        const float ps = r.pstar;
        r.jbound = nth_in_range<Tin, kSNT>(row, j0, j1, s.rem, L, [&](int64_t, float x) { return fn.prob(x) == ps; });
        if (tid == 0) st_agent(p.jstar + b, r.jbound);
      }
    }
  }
  if (draw) {
    // this chunk's sub-blocks (chunks are whole sub-blocks); lane w sums its
    // VE weights in fp64, the wave sums the lanes
    const int64_t s0 = j0 / sbl, s1 = (j1 + sbl - 1) / sbl;
    for (int64_t sbi = s0 + wave; sbi < s1; sbi += kSNW) {
      const int64_t e0 = (sbi * VNX_WAVE + lane) * VE;
      double m = 0.0;
      if (e0 + VE <= p.V) {
        float x[VE];
        Vec<Tin>::load(row + e0, x);
#pragma unroll
        for (int i = 0; i < VE; ++i) m += (double)fn.weight(e0 + i, x[i]);
      } else {
        for (int i = 0; i < VE; ++i)
          if (e0 + i < p.V) m += (double)fn.weight(e0 + i, Vec<Tin>::load1(row + e0 + i));
      }
      m = wave_sum(m);
      if (lane == 0) st_agent(p.sbm + b * p.nsb + sbi, m);
    }
  }
  // every wave's published masses complete before the workgroup arrives
  __builtin_amdgcn_s_waitcnt(0);
  if (!arrive_last(p.cnt + b, (unsigned)p.C, &L.flag)) return;

  // ---- the workgroup that completes the row ----
  auto finish = [&](int64_t token, int fl, float lse, float ps, int64_t js) {
    if (tid == 0) {
      p.out[b] = token;
      if (p.flags) p.flags[b] = (uint8_t)fl;
      if (p.lse) p.lse[b] = lse;
      if (p.kth) p.kth[b] = kNegInf;
      if (p.p_star) p.p_star[b] = ps;
      if (p.j_star) p.j_star[b] = js;
      if (p.k_star) p.k_star[b] = -1;
    }
  };
  if (!draw) {
    int64_t am = 0;
    if (tid < VNX_WAVE) am = merged_argmax(p, b);
    if (tid == 0) L.found = am;
    __syncthreads();
    finish(L.found, r.fl, __builtin_nanf(""), -1.0f, -1);
    return;
  }
  // the nucleus ties of the whole row now hold by id: jbound = j*
  if (r.pstar >= 0.0f) r.jbound = ld_agent(p.jstar + b);
  // thread t owns sub-blocks [t*q, (t+1)*q); the total is sum_t (sum_i) in
  // that nested order, and the walk follows it
  const int64_t nsb = p.nsb;
  const int64_t q = (nsb + kSNT - 1) / kSNT;  // <= kSampDraw / kSNT (host check)
  {
    double t = 0.0;
    for (int64_t i = (int64_t)tid * q; i < min((int64_t)(tid + 1) * q, nsb); ++i) {
      const double m = ld_agent(p.sbm + b * nsb + i);
      sh_m[i] = m;
      t += m;
    }
    const double incl = block_inclusive_scan<kSNT>(t, L.dd);
    L.T[tid] = t;
    L.E[tid] = incl;
    __syncthreads();
    if (tid == kSNT - 1) L.total = incl;
    if (tid == 0) { L.tstar = kSNT; L.tlast = -1; }
    __syncthreads();
  }
  const double total = L.total;
  const double target = samp_u(p, b) * total;
  {
    const double T = L.T[tid], end = L.E[tid];
    const double start = tid ? L.E[tid - 1] : 0.0;
    if (T > 0.0 && start <= target && target < end) atomicMin(&L.tstar, tid);
    if (T > 0.0) atomicMax(&L.tlast, tid);
  }
  __syncthreads();
  if (tid == 0) {
    int ts = L.tstar;
    if (ts == kSNT) ts = L.tlast;
    int64_t sstar = -1;
    double base = 0.0;
    if (ts >= 0) {
      const double b0 = ts ? L.E[ts - 1] : 0.0;
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
  int fl = r.fl;
  int64_t token = 0;
  if (sstar < 0) {
    fl |= VNX_FLAG_ZERO_RESIDUAL;
  } else {
    const int64_t e0 = (sstar * VNX_WAVE + lane) * VE;
    float w[VE];
    double lm = 0.0;
#pragma unroll
    for (int i = 0; i < VE; ++i) {
      w[i] = e0 + i < p.V ? fn.weight(e0 + i, Vec<Tin>::load1(row + e0 + i)) : 0.0f;
      lm += (double)w[i];
    }
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
      token = e0 + pick;
      const double tol = 1e-12 * L.total;
      if (tgt - before < tol || after - tgt < tol) edge = true;
    }
    if (lstar >= 0) {
      token = __shfl(token, lstar, VNX_WAVE);
      edge = __shfl((int)edge, lstar, VNX_WAVE) != 0;
    }
    if (edge) fl |= VNX_FLAG_CDF_EDGE;
  }
  finish(token, fl, r.L32, r.pstar, r.pstar >= 0.0f ? r.jbound : -1);
}

// ===========================================================================
// The per-row kernel of the top-k path (kST threads).
// ===========================================================================

// The single-workgroup form of the whole algorithm, for a row whose
// candidates overflow the list: every pass streams the row.
struct SingleLds {
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
  uint32_t prefix, pmask;
  unsigned long long rem;
  int64_t jstar;
  unsigned long long rank;
  double total, target, base;
  int64_t sb;
  int tstar, tlast;
  int done;
  int sel;
};

// The candidate path's state.
struct CandLds {
  unsigned long long a[kCandMax];  // sort keys
  unsigned long long scan[kSW];
  double dd[kSW];
  float f[kSW];
  int64_t i[kSW];
  int sel;
  unsigned long long above;
  int64_t token;
  double total;
  int hit;
  uint32_t tg;
  unsigned n;
  unsigned hc[kBins];
};

struct RowLds {
  union {
    CandLds c;
    struct {
      SingleLds L;
      double sh_m[kSampDraw];
    } s;
  } u;
};

__device__ __forceinline__ void sr_hist_clear(SingleLds& L) {
  __syncthreads();
  for (int i = threadIdx.x; i < kHist * kBins; i += kST) {
    (&L.u.h.cnt[0][0])[i] = 0u;
    (&L.u.h.mass[0][0])[i] = 0ull;
  }
  __syncthreads();
}

__device__ __forceinline__ void sr_hist_merge(SingleLds& L) {
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

// The m-th match in id order over the whole row (kST threads).
template <typename Tin, typename P>
__device__ __forceinline__ int64_t sr_nth(const Tin* row, int64_t V, unsigned long long m, SingleLds& L, P&& pred) {
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
    L.sel = owner;
    L.rank = m - run;
    L.jstar = -1;
  }
  __syncthreads();
  if (tid == L.sel) {
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

// Outputs of a row (thread 0).
__device__ __forceinline__ void row_finish(const SampParams& p, int64_t b, int64_t token, int fl, float lse,
                                           float kth, float ps, int64_t js, int64_t ks) {
  if (threadIdx.x == 0) {
    p.out[b] = token;
    if (p.flags) p.flags[b] = (uint8_t)fl;
    if (p.lse) p.lse[b] = lse;
    if (p.kth) p.kth[b] = kth;
    if (p.p_star) p.p_star[b] = ps;
    if (p.j_star) p.j_star[b] = js;
    if (p.k_star) p.k_star[b] = ks;
  }
}

// The whole algorithm over row b in one workgroup (the rules of the header;
// sd: the calibration scale of the chunk kernels, 1 without calibration).
template <typename Tin, int SM>
__device__ __forceinline__ void single_row(const SampParams& p, int64_t b, float sd, SingleLds& L, double* sh_m) {
  constexpr int VE = Vec<Tin>::N;
  const int tid = threadIdx.x;
  const int wave = tid / VNX_WAVE, lane = tid % VNX_WAVE;
  const Tin* row = static_cast<const Tin*>(p.x) + b * p.ld;
  const int64_t V = p.V;
  int fl = 0;
  // small lambdas capture by value so every closure stays in registers
  auto val = [calib = p.calib != 0, sd, cf = p.cf](float x) -> float { return calib ? (x / sd) * cf : x; };
  auto scaled = [val, sc = p.sc](float x) -> float { return tscale<SM>(val(x), sc); };
  const bool exact = p.exact != 0;
  auto key = [exact](float a) -> uint32_t { return exact ? okey_lo(a) : okey(a); };
  // ---- top-k: radix select of the kth largest scaled value ----
  if (tid == 0) { L.prefix = 0u; L.pmask = 0u; L.rem = (unsigned long long)p.top_k; }
  for (int pass = 0; pass < 4; ++pass) {
    sr_hist_clear(L);
    const int shift = 24 - 8 * pass;
    const uint32_t prefix = L.prefix, pmask = L.pmask;
    for_range<Tin, kST>(row, 0, V, [&](int64_t, float x) {
      const uint32_t k = key(scaled(x));
      if ((k & pmask) == prefix) atomicAdd(&L.u.h.cnt[wave % kHist][(k >> shift) & 0xFFu], 1u);
    });
    sr_hist_merge(L);
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
  const uint32_t tkey = L.prefix;
  const float thr = okey_value(tkey);
  int64_t kstar = -1;
  if (exact) {
    const unsigned long long m = L.rem;
    kstar = sr_nth<Tin>(row, V, m, L, [key, scaled, tkey](int64_t, float x) { return key(scaled(x)) == tkey; });
  }
  auto masked = [scaled, key, exact, thr, tkey, kstar](int64_t j, float x) -> float {
    const float a = scaled(x);
    if (!exact) return a >= thr ? a : kNegInf;
    const uint32_t k = key(a);
    return (k > tkey || (k == tkey && j <= kstar)) ? a : kNegInf;
  };
  // ---- softmax: max, row LSE (fp64), L32 ----
  float M = kNegInf;
  bool nan = false;
  for_range<Tin, kST>(row, 0, V, [&](int64_t j, float x) {
    const float a = masked(j, x);
    nan |= __builtin_isnan(a);
    M = fmaxf(M, a);
  });
  M = block_max<kST>(nan ? kPosInf : M, L.f);
  if (!(M > kNegInf && M < kPosInf)) {  // np.max not finite: numpy.argmax of the row
    float bv = kNegInf;
    int64_t bi = INT64_MAX;
    for_range<Tin, kST>(row, 0, V, [&](int64_t j, float x) {
      const float v = val(x);
      if (bi == INT64_MAX || argmax_better(v, j, bv, bi)) { bv = v; bi = j; }
    });
    block_argmax<kST>(bv, bi, L.f, L.i);
    row_finish(p, b, bi == INT64_MAX ? 0 : bi, fl, __builtin_nanf(""), thr, -1.0f, -1, exact ? kstar : -1);
    return;
  }
  const float mt = mt_of(M);
  double s = 0.0;
  for_range<Tin, kST>(row, 0, V, [&](int64_t j, float x) {
    const float a = masked(j, x);
    if (a > kNegInf) s += (double)exp2_term(a, mt);
  });
  s = block_sum<kST>(s, L.dd);
  RowCtx rc;
  rc.fl = 0;
  set_l32(rc, lse_of(M, s));
  const float L32 = rc.L32;
  fl |= rc.fl;
  auto prob = [masked, L32](int64_t j, float x) -> float { return vnx_exp_canon(masked(j, x) - L32); };
  // ---- top-p: nucleus value p*, tie count, j* ----
  float pstar = -1.0f;
  int64_t jstar = -1;
  if (p.use_p) {
    if (tid == 0) { L.prefix = 0u; L.pmask = 0u; L.rem = p.p_target; L.done = 0; }
    for (int pass = 0; pass < 4; ++pass) {
      sr_hist_clear(L);
      const int shift = 24 - 8 * pass;
      const uint32_t prefix = L.prefix, pmask = L.pmask;
      for_range<Tin, kST>(row, 0, V, [&](int64_t j, float x) {
        const float pp = prob(j, x);
        const uint32_t k = __float_as_uint(pp);
        if ((k & pmask) == prefix) {
          const int d = (k >> shift) & 0xFFu;
          atomicAdd(&L.u.h.cnt[wave % kHist][d], 1u);
          atomicAdd(&L.u.h.mass[wave % kHist][d], fix60(pp));
        }
      });
      sr_hist_merge(L);
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
      const unsigned long long P = fix60(pstar);  // > 0: a zero-mass bin is never chosen
      const unsigned long long m = (L.rem + P - 1) / P;
      jstar = sr_nth<Tin>(row, V, m, L, [prob, pstar](int64_t j, float x) { return prob(j, x) == pstar; });
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
    double m = 0.0;
#pragma unroll
    for (int i = 0; i < VE; ++i) {
      w[i] = (e0 + i < V) ? weight(e0 + i, Vec<Tin>::load1(row + e0 + i)) : 0.0f;
      m += (double)w[i];
    }
    return m;
  };
  for (int64_t sbi = wave; sbi < nsb; sbi += kSW) {
    float w[VE];
    const double t = wave_sum(lane_w(sbi, w));
    if (lane == 0) sh_m[sbi] = t;
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
  const double target = samp_u(p, b) * total;
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
  row_finish(p, b, token, fl, L32, thr, pstar, jstar, exact ? kstar : -1);
}

// Bitonic sort of a[0, n) (n a power of two, <= kCandMax) in LDS, kST threads;
// descending when desc.
__device__ __forceinline__ void lds_sort(unsigned long long* a, int n, bool desc) {
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n; i += kST) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const unsigned long long x = a[i], y = a[ixj];
          const bool up = ((i & k) == 0) != desc;  // this pair's target order: ascending
          if (up ? (x > y) : (x < y)) {
            a[i] = y;
            a[ixj] = x;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Bitonic sort of one u64 per lane across a wave (ascending, or descending
// when desc): register exchanges only.
__device__ __forceinline__ unsigned long long wave_sort_u64(unsigned long long v, bool desc) {
  const int l = threadIdx.x % VNX_WAVE;
#pragma unroll
  for (int k = 2; k <= VNX_WAVE; k <<= 1)
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      const unsigned long long o = __shfl_xor(v, j, VNX_WAVE);
      const bool up = ((l & k) == 0) != desc;  // this pair's order: ascending
      const bool take_min = ((l & j) == 0) == up;
      v = take_min ? (o < v ? o : v) : (o > v ? o : v);
    }
  return v;
}

__device__ __forceinline__ unsigned long long wave_scan_u64(unsigned long long v) {
  const int l = threadIdx.x % VNX_WAVE;
#pragma unroll
  for (int o = 1; o < VNX_WAVE; o <<= 1) {
    const unsigned long long n = __shfl_up(v, o, VNX_WAVE);
    if (l >= o) v += n;
  }
  return v;
}

// The per-row step after the compaction when at most 64 candidates remain
// (the usual case for small k): the cut, LSE, nucleus and draw of the
// workgroup form, in one wave with register exchanges instead of LDS sorts
// and barriers.  Returns true when max(a) is not finite (the caller then
// takes numpy.argmax of the row; thr and k* are left in L.f[0] / L.i[0]).
__device__ __forceinline__ bool cand_wave(const SampParams& p, int64_t b, int n, CandLds& L) {
  const int lane = threadIdx.x % VNX_WAVE;
  const bool ex = p.exact != 0;
  // (key << 32 | ~id), descending: key descending, id ascending
  unsigned long long e = lane < n ? L.a[lane] : 0ull;
  e = wave_sort_u64(e, true);
  const int kk = (int)p.top_k;  // <= n
  const unsigned long long ek = __shfl(e, kk - 1, VNX_WAVE);
  const uint32_t tkey = (uint32_t)(ek >> 32);
  const float thr = okey_value(tkey);
  const int64_t kstar = ex ? (int64_t)(0xFFFFFFFFu - (uint32_t)ek) : -1;
  const uint32_t id = 0xFFFFFFFFu - (uint32_t)e;
  const float a = okey_value((uint32_t)(e >> 32));  // -0 read as +0: the same value
  const bool keep = lane < n && (ex ? lane < kk : a >= thr);
  const bool anynan = __ballot(keep && __builtin_isnan(a)) != 0;
  const float M = anynan ? kPosInf : wave_max(keep ? a : kNegInf);
  if (!(M > kNegInf && M < kPosInf)) {
    if (lane == 0) {
      L.f[0] = thr;
      L.i[0] = kstar;
    }
    return true;
  }
  double sd = keep ? (double)exp2_term(a, mt_of(M)) : 0.0;
  sd = wave_sum(sd);
  RowCtx rc;
  rc.fl = 0;
  set_l32(rc, lse_of(M, sd));
  const float L32 = rc.L32;
  int fl = rc.fl;
  const float pp = keep ? vnx_exp_canon(a - L32) : 0.0f;
  // kept tokens: a prefix of the sorted order (keys >= the kth, or the first k)
  const int nk = __builtin_popcountll(__ballot(keep));
  int ncut = nk;
  float pstar = -1.0f;
  int64_t jstar = -1;
  unsigned long long d;  // the draw's entries (id << 32 | p bits), ascending
  if (p.use_p) {
    // (p desc, id asc), exact fixed-point prefix sums, the first to reach top_p
    unsigned long long q = keep ? ((unsigned long long)__float_as_uint(pp) << 32) | (0xFFFFFFFFu - id) : 0ull;
    q = wave_sort_u64(q, true);
    const float pq = __uint_as_float((uint32_t)(q >> 32));
    const unsigned long long incl = wave_scan_u64(lane < nk ? fix60(pq) : 0ull);
    const uint64_t reach = __ballot(lane < nk && incl >= p.p_target);
    if (reach) {
      const int cut = __builtin_ctzll(reach);
      ncut = cut + 1;
      const unsigned long long qc = __shfl(q, cut, VNX_WAVE);
      pstar = __uint_as_float((uint32_t)(qc >> 32));
      jstar = (int64_t)(0xFFFFFFFFu - (uint32_t)qc);
    }
    d = lane < ncut ? ((unsigned long long)(0xFFFFFFFFu - (uint32_t)q) << 32) | (q >> 32) : ~0ull;
  } else {
    d = keep ? ((unsigned long long)id << 32) | __float_as_uint(pp) : ~0ull;
  }
  d = wave_sort_u64(d, false);
  const float w = lane < ncut ? __uint_as_float((uint32_t)d) : 0.0f;
  const double incl = wave_inclusive_scan((double)w);
  const double total = __shfl(incl, VNX_WAVE - 1, VNX_WAVE);
  const double target = samp_u(p, b) * total;
  int64_t token = 0;
  if (!(total > 0.0)) {
    fl |= VNX_FLAG_ZERO_RESIDUAL;
  } else {
    const double before = incl - (double)w;
    const uint64_t hits = __ballot(w > 0.0f && before <= target && target < incl);
    int pick;
    if (hits) {
      pick = __builtin_ctzll(hits);
    } else {
      pick = 63 - __builtin_clzll(__ballot(w > 0.0f));  // rounding left the target past every weight
      fl |= VNX_FLAG_CDF_EDGE;
    }
    const double tol = 1e-12 * total;
    const bool edge = (target - before < tol || incl - target < tol);
    if (__shfl((int)edge, pick, VNX_WAVE)) fl |= VNX_FLAG_CDF_EDGE;
    token = (int64_t)(__shfl(d, pick, VNX_WAVE) >> 32);
  }
  row_finish(p, b, token, fl, L32, thr, pstar, jstar, kstar);
  return false;
}

__device__ __forceinline__ int pow2_at_least(int n) {
  int m = 1;
  while (m < n) m <<= 1;
  return m;
}

// The cut, the LSE, the nucleus and the draw of row b over its candidates.
template <typename Tin, int SM>
__global__ __launch_bounds__(kST) void k_samp_cand(SampParams p) {
  __shared__ RowLds R;
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  const float sd = calib_sd(p, b);
  CandLds& L = R.u.c;
  const bool ex = p.exact != 0;
  // the chunks' candidate counts and thresholds: the largest threshold is a
  // lower bound of the row's kth key too (its chunk alone holds k keys above)
  if (tid < VNX_WAVE) {
    unsigned cn = 0u;
    uint32_t t = 0u;
    if (!p.single && tid < p.C) {
      cn = p.nct[b * p.C + tid];
      t = p.tc[b * p.C + tid];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) t = max(t, (uint32_t)__shfl_xor((int)t, o, VNX_WAVE));
    const bool over = __ballot(cn > (unsigned)kSegCap) != 0;
    if (tid == 0) {
      L.tg = t;
      L.hit = over ? 1 : 0;
      L.n = 0u;
    }
  }
  __syncthreads();
  const bool over = p.single || L.hit;
  const uint32_t tg = L.tg;
  if (!over) {
    // every candidate with key >= tg into L.a, compacted per wave
    const int wave = tid / VNX_WAVE, lane = tid % VNX_WAVE;
    for (int c = wave; c < p.C; c += kSW) {
      const unsigned cn = p.nct[b * p.C + c];
      const unsigned long long* seg = p.cand + (b * p.C + c) * kSegCap;
      for (unsigned i0 = 0; i0 < cn; i0 += VNX_WAVE) {
        const unsigned i = i0 + lane;
        const unsigned long long e = i < cn ? seg[i] : 0ull;
        const bool take = i < cn && (uint32_t)(e >> 32) >= tg;
        const uint64_t m = __ballot(take);
        if (m) {
          unsigned base = 0u;
          if (lane == 0) base = atomicAdd(&L.n, (unsigned)__builtin_popcountll(m));
          base = __shfl(base, 0, VNX_WAVE);
          const unsigned pos = base + lane_rank(m);
          if (take && pos < (unsigned)kCandMax) L.a[pos] = e;
        }
      }
    }
  }
  __syncthreads();
  const unsigned nc = L.n;
  __syncthreads();  // every thread has read the LDS state the fallback reuses
  // (fewer than k candidates cannot happen: the chunk of tg holds k of them)
  if (over || nc > (unsigned)kCandMax || (int64_t)nc < p.top_k) {
    single_row<Tin, SM>(p, b, sd, R.u.s.L, R.u.s.sh_m);
    return;
  }
  const int wave = tid / VNX_WAVE, lane = tid % VNX_WAVE;
  constexpr int PER = kCandMax / kST;
  // the row's kth largest key: a radix select over the candidates, on the
  // bits below the common prefix of tg and the largest key (every candidate
  // key lies between the two)
  uint32_t kmax = 0u;
  for (int i = tid; i < (int)nc; i += kST) kmax = max(kmax, (uint32_t)(L.a[i] >> 32));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, o, VNX_WAVE));
  if (lane == 0) L.scan[wave] = kmax;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kSW; ++w) kmax = max(kmax, (uint32_t)L.scan[w]);
  const uint32_t diff = kmax ^ tg;
  int top = diff ? 31 - __builtin_clz(diff) : -1;  // highest undetermined bit
  uint32_t pmask = top < 0 ? 0xFFFFFFFFu : ~((2u << top) - 1u);
  uint32_t prefix = tg & pmask;
  unsigned long long rem = (unsigned long long)p.top_k;
  while (top >= 0) {
    const int width = min(top + 1, 8);
    const int shift = top + 1 - width;
    const uint32_t dm = (1u << width) - 1u;
    __syncthreads();
    for (int i = tid; i < kBins; i += kST) L.hc[i] = 0u;
    __syncthreads();
    for (int i = tid; i < (int)nc; i += kST) {
      const uint32_t k = (uint32_t)(L.a[i] >> 32);
      if ((k & pmask) == prefix) atomicAdd(&L.hc[(k >> shift) & dm], 1u);
    }
    __syncthreads();
    unsigned long long above;
    const int d = pick_digit(L.hc, rem, &above, &L.sel, &L.above);  // the bins hold >= rem
    rem -= above;
    prefix |= (uint32_t)d << shift;
    pmask |= dm << shift;
    top = shift - 1;
  }
  // the candidates at or above the kth key, compacted to the front
  {
    unsigned long long e_r[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int i = tid + q * kST;
      e_r[q] = i < (int)nc ? L.a[i] : 0ull;
    }
    __syncthreads();
    if (tid == 0) L.n = 0u;
    __syncthreads();
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int i = tid + q * kST;
      const bool take = i < (int)nc && (uint32_t)(e_r[q] >> 32) >= prefix;
      const uint64_t m = __ballot(take);
      if (m) {
        unsigned base = 0u;
        if (lane == 0) base = atomicAdd(&L.n, (unsigned)__builtin_popcountll(m));
        base = __shfl(base, 0, VNX_WAVE);
        if (take) L.a[base + lane_rank(m)] = e_r[q];
      }
    }
    __syncthreads();
  }
  const int n = (int)L.n;  // >= k
  if (n <= VNX_WAVE) {
    // one wave finishes the row; the others wait only for the rare argmax
    if (tid < VNX_WAVE) {
      const bool fb = cand_wave(p, b, n, L);
      if (tid == 0) L.hit = fb ? 1 : 0;
    }
    __syncthreads();
    if (!L.hit) return;  // uniform
    const float thr = L.f[0];
    const int64_t kstar = L.i[0];
    __syncthreads();
    const Tin* row = static_cast<const Tin*>(p.x) + b * p.ld;
    const bool cal = p.calib != 0;
    const float cf = p.cf;
    float bv = kNegInf;
    int64_t bi = INT64_MAX;
    for_range<Tin, kST>(row, 0, p.V, [&](int64_t j, float x) {
      const float v = cal ? (x / sd) * cf : x;
      if (bi == INT64_MAX || argmax_better(v, j, bv, bi)) { bv = v; bi = j; }
    });
    block_argmax<kST>(bv, bi, L.f, L.i);
    row_finish(p, b, bi == INT64_MAX ? 0 : bi, 0, __builtin_nanf(""), thr, -1.0f, -1, kstar);
    return;
  }
  const int np = pow2_at_least(n);
  // sort key: (cut key << 32) | ~id, descending = key descending, id ascending
  for (int i = n + tid; i < np; i += kST) L.a[i] = 0ull;
  __syncthreads();
  lds_sort(L.a, np, true);
  // the cut: kth key at position k-1; kept = value >= kth (Sampler) or the
  // first k (exactly-k)
  const int kk = (int)p.top_k;
  const uint32_t tkey = (uint32_t)(L.a[kk - 1] >> 32);
  const float thr = okey_value(tkey);
  const int64_t kstar = ex ? (int64_t)(0xFFFFFFFFu - (uint32_t)L.a[kk - 1]) : -1;
  // kept entries, their max (NaN -> +inf) and count
  float a_r[PER];
  uint32_t j_r[PER];
  bool keep_r[PER];
  float M = kNegInf;
  bool nan = false;
  int nkeep = 0;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
    const int i = tid * PER + q;  // contiguous: thread order is sort order
    keep_r[q] = false;
    a_r[q] = kNegInf;
    j_r[q] = 0u;
    if (i < n) {
      const unsigned long long e = L.a[i];
      const uint32_t k = (uint32_t)(e >> 32);
      j_r[q] = 0xFFFFFFFFu - (uint32_t)e;
      a_r[q] = okey_value(k);  // -0 read as +0: the same value
      keep_r[q] = ex ? i < kk : a_r[q] >= thr;
      if (keep_r[q]) {
        nan |= __builtin_isnan(a_r[q]);
        M = fmaxf(M, a_r[q]);
        ++nkeep;
      }
    }
  }
  M = block_max<kST>(nan ? kPosInf : M, L.f);
  if (!(M > kNegInf && M < kPosInf)) {
    // np.max not finite: numpy.argmax of the (calibrated) row
    const Tin* row = static_cast<const Tin*>(p.x) + b * p.ld;
    const bool cal = p.calib != 0;
    const float cf = p.cf;
    float bv = kNegInf;
    int64_t bi = INT64_MAX;
    for_range<Tin, kST>(row, 0, p.V, [&](int64_t j, float x) {
      const float v = cal ? (x / sd) * cf : x;
      if (bi == INT64_MAX || argmax_better(v, j, bv, bi)) { bv = v; bi = j; }
    });
    block_argmax<kST>(bv, bi, L.f, L.i);
    row_finish(p, b, bi == INT64_MAX ? 0 : bi, 0, __builtin_nanf(""), thr, -1.0f, -1, kstar);
    return;
  }
  const float mt = mt_of(M);
  double s = 0.0;
#pragma unroll
    for (int q = 0; q < PER; ++q)
    if (keep_r[q]) s += (double)exp2_term(a_r[q], mt);
  s = block_sum<kST>(s, L.dd);
  RowCtx rc;
  rc.fl = 0;
  set_l32(rc, lse_of(M, s));
  const float L32 = rc.L32;
  int fl = rc.fl;
  // kept entries compacted to the front as (p bits << 32) | ~id: sorted
  // descending that is (p descending, id ascending)
  const int kin = (int)block_scan_u64<kST>((unsigned long long)nkeep, L.scan);
  if (tid == kST - 1) L.sel = kin;
  __syncthreads();
  const int nk = L.sel;
  const int before = kin - nkeep;
  float p_r[PER];
  {
    int w = before;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
      p_r[q] = 0.0f;
      if (keep_r[q]) p_r[q] = vnx_exp_canon(a_r[q] - L32);
    }
    // every thread's entries are in registers: overwrite the array
#pragma unroll
        for (int q = 0; q < PER; ++q)
      if (keep_r[q]) L.a[w++] = ((unsigned long long)__float_as_uint(p_r[q]) << 32) | (0xFFFFFFFFu - j_r[q]);
  }
  const int nkp = pow2_at_least(nk);
  for (int i = nk + tid; i < nkp; i += kST) L.a[i] = 0ull;
  __syncthreads();
  // ---- the nucleus: the first cutoff + 1 in (p desc, id asc) order ----
  int ncut = nk;  // entries kept by the nucleus (a prefix of the sorted order)
  float pstar = -1.0f;
  int64_t jstar = -1;
  if (p.use_p) {
    lds_sort(L.a, nkp, true);
    unsigned long long fs = 0;
    #pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int i = tid * PER + q;
      if (i < nk) fs += fix60(__uint_as_float((uint32_t)(L.a[i] >> 32)));
    }
    const unsigned long long incl = block_scan_u64<kST>(fs, L.scan);
    if (tid == 0) L.sel = nk;
    __syncthreads();
    if (incl >= p.p_target && incl - fs < p.p_target) {
      // this thread's range holds the first position whose sum reaches top_p
      unsigned long long run = incl - fs;
      #pragma unroll
      for (int q = 0; q < PER; ++q) {
        const int i = tid * PER + q;
        run += fix60(__uint_as_float((uint32_t)(L.a[i] >> 32)));
        if (run >= p.p_target) {
          L.sel = i;
          break;
        }
      }
    }
    __syncthreads();
    const int cut = L.sel;
    __syncthreads();
    if (cut < nk) {
      ncut = cut + 1;
      pstar = __uint_as_float((uint32_t)(L.a[cut] >> 32));
      jstar = (int64_t)(0xFFFFFFFFu - (uint32_t)L.a[cut]);
    }
  }
  // ---- the draw over the kept tokens in id order: (id << 32) | p bits ----
  {
    unsigned long long t[PER];
#pragma unroll
        for (int q = 0; q < PER; ++q) {
      const int i = tid * PER + q;
      t[q] = ~0ull;
      if (i < ncut) {
        const unsigned long long e = L.a[i];
        t[q] = ((unsigned long long)(0xFFFFFFFFu - (uint32_t)e) << 32) | (e >> 32);
      }
    }
    __syncthreads();
#pragma unroll
        for (int q = 0; q < PER; ++q) {
      const int i = tid * PER + q;
      if (i < nkp) L.a[i] = t[q];
    }
    __syncthreads();
  }
  const int ndp = pow2_at_least(ncut);
  lds_sort(L.a, ndp, false);
  double wsum = 0.0;
  float w_r[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
    const int i = tid * PER + q;
    w_r[q] = i < ncut ? __uint_as_float((uint32_t)L.a[i]) : 0.0f;
    wsum += (double)w_r[q];
  }
  const double incl = block_inclusive_scan<kST>(wsum, L.dd);
  if (tid == kST - 1) L.total = incl;
  if (tid == 0) L.hit = kCandMax;  // none yet
  __syncthreads();
  const double total = L.total;
  const double target = samp_u(p, b) * total;
  if (total > 0.0) {
    // first position whose cumulative sum exceeds the target (the last
    // positive one when rounding leaves none)
    double run = incl - wsum;
    #pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int i = tid * PER + q;
      if (w_r[q] > 0.0f) {
        const double nr = run + (double)w_r[q];
        if (run <= target && target < nr) atomicMin(&L.hit, i);
        run = nr;
      }
    }
  }
  __syncthreads();
  int64_t token = 0;
  if (total <= 0.0) {
    fl |= VNX_FLAG_ZERO_RESIDUAL;
  } else {
    int pick = L.hit;
    __syncthreads();
    if (pick == kCandMax) {
      fl |= VNX_FLAG_CDF_EDGE;
      // the last positive weight
      if (tid == 0) L.hit = -1;
      __syncthreads();
      int last = -1;
      #pragma unroll
      for (int q = 0; q < PER; ++q) {
        const int i = tid * PER + q;
        if (w_r[q] > 0.0f) last = i;
      }
      atomicMax(&L.hit, last);
      __syncthreads();
      pick = L.hit;
    }
    token = (int64_t)(L.a[pick] >> 32);
    // CDF_EDGE: the target within 1e-12 of the picked bucket's edges
    if (tid == pick / PER) {
      double run = incl - wsum;
      #pragma unroll
      for (int q = 0; q < PER; ++q) {
        const int i = tid * PER + q;
        const double nr = run + (double)w_r[q];
        if (i == pick) {
          const double tol = 1e-12 * total;
          if (target - run < tol || nr - target < tol) L.sel = 1;
          else L.sel = 0;
        }
        run = nr;
      }
    }
    __syncthreads();
    if (L.sel == 1) fl |= VNX_FLAG_CDF_EDGE;
  }
  row_finish(p, b, token, fl, L32, thr, pstar, jstar, kstar);
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
  for_range<Tin, kST>(row, 0, V, [&](int64_t, float v) { s += (double)v; });
  const double mean = block_sum<kST>(s, red) / (double)V;
  double s2 = 0.0;
  for_range<Tin, kST>(row, 0, V, [&](int64_t, float v) {
    const double d = (double)v - mean;
    s2 += d * d;
  });
  const double var = block_sum<kST>(s2, red) / (double)V;
  const float sd = sqrtf((float)var + eps);
  float* o = out + b * ldo;
  for_range<Tin, kST>(row, 0, V, [&](int64_t j, float v) { o[j] = (v / sd) * f; });
  if (threadIdx.x == 0 && var_out) var_out[b] = var;
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
struct SampPlan {
  int C;
  int64_t clen, nsb;
};

// local: the chunks of the candidate search (at most kChunkMax elements,
// possible for V <= kSMaxC * kChunkMax).
static SampPlan samp_plan(int64_t B, int64_t V, int dtype, bool local) {
  const int ve = dtype == VNX_F32 ? 4 : 8;
  const int64_t sbl = (int64_t)VNX_WAVE * ve;
  SampPlan pl;
  pl.nsb = (V + sbl - 1) / sbl;
  int64_t c = ((int64_t)device_cus() * 4 + B - 1) / B;
  c = std::min<int64_t>(std::min<int64_t>(c, kSMaxC), pl.nsb);
  if (c < 1) c = 1;
  int64_t spc = (pl.nsb + c - 1) / c;  // sub-blocks per chunk
  if (local) spc = std::min<int64_t>(spc, kChunkMax / sbl);
  pl.clen = spc * sbl;
  pl.C = (int)((V + pl.clen - 1) / pl.clen);
  return pl;
}

static size_t samp_carve(void* ws, int64_t B, const SampPlan& pl, SampParams* p) {
  Carve cv(ws);
  const size_t nb = (size_t)B * 4 * kBins, nc = (size_t)B * pl.C;
  unsigned long long* phm = cv.take<unsigned long long>(nb);
  uint32_t* lp = cv.take<uint32_t>(nc * kBins);
  RadixState* stp = cv.take<RadixState>((size_t)B * 5);
  double* cs1 = cv.take<double>(nc);
  double* cs2 = cv.take<double>(nc);
  float* pm = cv.take<float>(nc);
  double* ps = cv.take<double>(nc);
  float* pav = cv.take<float>(nc);
  int64_t* pai = cv.take<int64_t>(nc);
  int64_t* jstar = cv.take<int64_t>((size_t)B);
  double* sbm = cv.take<double>((size_t)B * pl.nsb);
  unsigned* cnt = cv.take<unsigned>((size_t)B);
  unsigned long long* cand = cv.take<unsigned long long>(nc * kSegCap);
  unsigned* nct = cv.take<unsigned>(nc);
  uint32_t* tc = cv.take<uint32_t>(nc);
  if (p) {
    p->phm = phm; p->lp = lp; p->stp = stp;
    p->cs1 = cs1; p->cs2 = cs2; p->pm = pm; p->ps = ps; p->pav = pav; p->pai = pai;
    p->jstar = jstar; p->sbm = sbm; p->cnt = cnt; p->cand = cand; p->nct = nct; p->tc = tc;
  }
  return cv.bytes();
}

}  // namespace vnx

using namespace vnx;

extern "C" {

size_t vnx_sampler_workspace(int64_t B, int64_t V, int dtype) {
  if (B <= 0 || V <= 0 || (dtype != VNX_F32 && dtype != VNX_BF16)) return 256;
  // the candidate search's chunks are the smaller ones: its plan sizes the workspace
  return samp_carve(nullptr, B, samp_plan(B, V, dtype, V <= kLocalMaxV), nullptr);
}

int vnx_sampler_sample(const void* logits, int dtype, int64_t B, int64_t V, int64_t ld, float temperature,
                       int64_t top_k, float top_p, int mode, float calib_factor, float calib_eps,
                       const void* uniforms, int64_t* out_ids, uint8_t* flags, float* lse, float* kth,
                       float* p_star, int64_t* j_star, int64_t* k_star, void* workspace, size_t workspace_bytes,
                       void* stream) {
  if (dtype != VNX_F32 && dtype != VNX_BF16) return VNX_ERR_UNSUPPORTED;
  if (B < 0 || V <= 0 || top_k < 0) return VNX_ERR_INVALID_ARG;
  if (mode & ~(VNX_SAMPLE_EXACT_K | VNX_SAMPLE_CALIBRATE | VNX_SAMPLE_UNIFORM_F64)) return VNX_ERR_INVALID_ARG;
  if ((mode & VNX_SAMPLE_CALIBRATE) && (!__builtin_isfinite(calib_factor) || !(calib_eps >= 0.0f)))
    return VNX_ERR_INVALID_ARG;
  if (!(temperature >= 0.0f) || !__builtin_isfinite(temperature)) return VNX_ERR_INVALID_ARG;
  if (!(top_p > 0.0f && top_p <= 1.0f)) return VNX_ERR_INVALID_ARG;
  if (B == 0) return VNX_OK;
  if (!logits || !out_ids || (temperature > 0.0f && !uniforms)) return VNX_ERR_INVALID_ARG;
  const int ve = dtype == VNX_F32 ? 4 : 8;
  if (ld < V || ld % ve || reinterpret_cast<uintptr_t>(logits) % 16) return VNX_ERR_INVALID_ARG;
  // candidate ids are 32-bit
  if (V >= (int64_t)0xFFFFFFFF) return VNX_ERR_UNSUPPORTED;
  const bool cand = top_k > 0 && top_k < V && temperature > 0.0f;
  const bool local = cand && V <= kLocalMaxV && top_k <= kLocalMaxK;
  const SampPlan pl = samp_plan(B, V, dtype, local);
  if (pl.nsb > kSampDraw || B * (int64_t)pl.C >= INT32_MAX) return VNX_ERR_UNSUPPORTED;
  const size_t need = samp_carve(nullptr, B, pl, nullptr);
  if (!workspace || workspace_bytes < need) return VNX_ERR_WORKSPACE;
  SampParams p{};
  p.x = logits; p.B = B; p.V = V; p.ld = ld;
  p.greedy = temperature == 0.0f;
  const int sm = p.greedy ? SM_ID : make_scale(temperature, &p.sc);
  p.exact = (mode & VNX_SAMPLE_EXACT_K) != 0;
  p.calib = (mode & VNX_SAMPLE_CALIBRATE) != 0;
  p.cf = calib_factor;
  p.ceps = calib_eps;
  p.top_k = top_k;
  p.use_k = top_k > 0 && top_k < V;
  p.use_p = top_p < 1.0f;
  // at least one unit: the first token's sum reaches any top_p > 0
  p.p_target = std::max<uint64_t>(1, (uint64_t)floor((double)top_p * 1152921504606846976.0));
  p.C = pl.C; p.clen = pl.clen; p.nsb = pl.nsb;
  if (mode & VNX_SAMPLE_UNIFORM_F64) p.u64 = static_cast<const double*>(uniforms);
  else p.u = static_cast<const float*>(uniforms);
  p.out = out_ids; p.flags = flags; p.lse = lse; p.kth = kth; p.p_star = p_star;
  p.j_star = j_star; p.k_star = k_star;
  samp_carve(workspace, B, pl, &p);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(B * pl.C)), blk(kSNT);
  if (!cand) {
    hipLaunchKernelGGL(k_samp_init, dim3((unsigned)B), blk, 0, s, p);
    VNX_LAUNCH_CHECK();
  }
  return dispatch_tsm(dtype, sm, false, [&](auto tin, auto smc, auto) {
    using Tin = decltype(tin);
    constexpr int SM = decltype(smc)::value;
    auto run = [&](auto calc) {
      constexpr bool CAL = decltype(calc)::value;
      if (CAL) {
        hipLaunchKernelGGL((k_samp_calib<Tin, 0>), grid, blk, 0, s, p);
        hipLaunchKernelGGL((k_samp_calib<Tin, 1>), grid, blk, 0, s, p);
      }
      if (cand) {
        p.single = !local;
        if (local) hipLaunchKernelGGL((k_samp_local<Tin, SM, CAL>), grid, blk, 0, s, p);
        hipLaunchKernelGGL((k_samp_cand<Tin, SM>), dim3((unsigned)B), dim3(kST), 0, s, p);
      } else {
        hipLaunchKernelGGL((k_samp_lse<Tin, SM, CAL>), grid, blk, 0, s, p);
        if (p.use_p && !p.greedy) {
          hipLaunchKernelGGL((k_samp_ppass<Tin, SM, CAL, 0>), grid, blk, 0, s, p);
          hipLaunchKernelGGL((k_samp_ppass<Tin, SM, CAL, 1>), grid, blk, 0, s, p);
          hipLaunchKernelGGL((k_samp_ppass<Tin, SM, CAL, 2>), grid, blk, 0, s, p);
          hipLaunchKernelGGL((k_samp_ppass<Tin, SM, CAL, 3>), grid, blk, 0, s, p);
        }
        hipLaunchKernelGGL((k_samp_mass<Tin, SM, CAL>), grid, blk, (size_t)pl.nsb * sizeof(double), s, p);
      }
    };
    if (p.calib) run(BoolC<true>{});
    else run(BoolC<false>{});
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
