// Speculative-decoding verification kernels.
//
// vnx_spec_accept (stochastic rule, Leviathan et al. 2023 Alg. 1), two launches:
//   pass 1  grid B*(2k+1)*C: every workgroup streams one chunk of one target or
//           draft row and writes the chunk's (max, sum-exp).  The last
//           workgroup of batch row b merges the 2k+1 row LSEs (fp64), rounds
//           them to fp32, evaluates the k acceptance tests in one wavefront
//           (lane i tests position i; a ballot gives the first rejection n) and
//           writes accept_len, the accepted ids and the pass-2 job.
//   pass 2  grid B*C2: every workgroup streams one chunk of p_n and q_n (or p_k
//           for the bonus draw) and writes the chunk's residual mass
//           sum max(0, p-q) and target mass sum p (fp64).  The last workgroup of
//           b scans the chunk masses, finds the chunk holding u_k * mass and
//           scans that chunk in 1024-element blocks to find the drawn token.
// Probabilities that feed decisions use vnx_exp_canon(a - L32), a = RN(l/T),
// L32 = RN32(row LSE), so the CPU checker reproduces them bit for bit.
//
// vnx_greedy_verify: one launch, grid B*rows_t*C of argmax chunks; the last
// workgroup of b merges the row argmaxes and applies the prefix rule.
#include "rowred.h"
#include "vnx_internal.h"

namespace vnx {

constexpr int kNT = 256;
constexpr int kNB = 8;
constexpr int kMaxK = 64;

struct Job {
  int n;      // first rejected position (k if all accepted)
  int mode;   // 0 = residual draw from max(0, p_n - q_n), 1 = draw from p_k
  float Lp;   // fp32 LSE of the target row drawn from
  float Lq;   // fp32 LSE of draft row n (mode 0)
  float u;    // uniform of the draw
  int pad;
};

struct SpecParams {
  const void* tgt;
  const void* dft;
  int64_t B;
  int k;
  int64_t V, ld_t, ld_d, sb_t, sb_d;
  int chunks;
  int64_t chunk_len;
  int chunks2;
  int64_t chunk_len2;
  Scale sc;
  const float* thr_t;
  const float* thr_d;
  const int64_t* ids;
  const float* u;
  int32_t* accept_len;
  int64_t* out_ids;
  uint8_t* flags;
  float* lse_t;
  float* lse_d;
  float* part_m;
  double* part_s;
  unsigned* cnt1;
  Job* jobs;
  double* part2;
  unsigned* cnt2;
};

// Distance test of an fp64 LSE to the rounding midpoints around its fp32 value.
__device__ __forceinline__ bool near_f32_edge(double L, float L32, double tol) {
  if (!__builtin_isfinite(L)) return false;
  const double up = (double)nextafterf(L32, __builtin_inff());
  const double dn = (double)nextafterf(L32, -__builtin_inff());
  const double mu = 0.5 * ((double)L32 + up), md = 0.5 * ((double)L32 + dn);
  return fabs(L - mu) < tol || fabs(L - md) < tol;
}

template <typename Tin>
__device__ __forceinline__ float scaled_elem(const Tin* row, int64_t j, const Scale& sc, float thr) {
  float a = scale_logit(Vec<Tin>::load1(row + j), sc);
  return (a < thr) ? kNegInf : a;
}

template <typename Tin>
__global__ __launch_bounds__(kNT) void k_spec_pass1(SpecParams p) {
  __shared__ ReduceLds lds;
  __shared__ int last_flag;
  __shared__ float Ls[2 * kMaxK + 1];
  __shared__ int Ledge[2 * kMaxK + 1];
  const int k = p.k;
  const int R = 2 * k + 1;
  const int c = blockIdx.x % p.chunks;
  const int64_t t = blockIdx.x / p.chunks;
  const int64_t b = t % p.B;
  const int s = (int)(t / p.B);
  // Dispatch order: positions k, k-1, ..., 0, so the rows most likely needed
  // by pass 2 (small positions) are the most recently streamed ones.
  const int pos = (s == 0) ? k : k - (s + 1) / 2;
  const bool is_draft = (s != 0) && (s & 1);
  const int ri = is_draft ? (k + 1 + pos) : pos;
  const Tin* row;
  float thr;
  if (is_draft) {
    row = static_cast<const Tin*>(p.dft) + b * p.sb_d + pos * p.ld_d;
    thr = p.thr_d ? p.thr_d[b * k + pos] : kNegInf;
  } else {
    row = static_cast<const Tin*>(p.tgt) + b * p.sb_t + pos * p.ld_t;
    thr = p.thr_t ? p.thr_t[b * (k + 1) + pos] : kNegInf;
  }
  const int64_t c0 = (int64_t)c * p.chunk_len;
  const int64_t c1 = c0 + p.chunk_len < p.V ? c0 + p.chunk_len : p.V;
  ChunkResult cr = reduce_chunk<Tin, kNT, kNB, true, false>(row, c0, c1, p.sc, thr, lds);
  const int64_t slot = (b * R + ri) * p.chunks + c;
  if (threadIdx.x == 0) {
    st_agent(&p.part_m[slot], cr.m);
    st_agent(&p.part_s[slot], cr.s);
  }
  if (!arrive_last(&p.cnt1[b], (unsigned)(R * p.chunks), &last_flag)) return;

  // ---- last workgroup of batch row b: row LSEs, acceptance tests, job ----
  const int tid = threadIdx.x;
  if (tid < R) {
    float M = kNegInf;
    double S = 0.0;
    const int64_t base = (b * R + tid) * p.chunks;
    for (int j = 0; j < p.chunks; ++j) merge_partial(M, S, ld_agent(&p.part_m[base + j]), ld_agent(&p.part_s[base + j]));
    const double L = lse_of(M, S);
    const float L32 = (float)L;
    Ls[tid] = L32;
    Ledge[tid] = near_f32_edge(L, L32, 1e-7) ? 1 : 0;
    if (tid <= k) {
      if (p.lse_t) p.lse_t[b * (k + 1) + tid] = L32;
    } else if (p.lse_d) {
      p.lse_d[b * k + (tid - k - 1)] = L32;
    }
  }
  __syncthreads();
  if (tid >= VNX_WAVE) return;
  const int lane = tid;
  bool acc = true;
  uint8_t fl = 0;
  int64_t x = -1;
  if (lane < k) {
    x = p.ids[b * k + lane];
    const float u = p.u[b * (k + 1) + lane];
    if (x >= 0 && x < p.V) {
      const Tin* trow = static_cast<const Tin*>(p.tgt) + b * p.sb_t + lane * p.ld_t;
      const Tin* drow = static_cast<const Tin*>(p.dft) + b * p.sb_d + lane * p.ld_d;
      const float thr_t = p.thr_t ? p.thr_t[b * (k + 1) + lane] : kNegInf;
      const float thr_d = p.thr_d ? p.thr_d[b * k + lane] : kNegInf;
      const float a = scaled_elem(trow, x, p.sc, thr_t);
      const float bq = scaled_elem(drow, x, p.sc, thr_d);
      const float pp = vnx_exp_canon(a - Ls[lane]);
      const float qq = vnx_exp_canon(bq - Ls[k + 1 + lane]);
      acc = (u < 1.0f) && ((double)u * (double)qq < (double)pp);
      if (qq > 0.0f) {
        double ratio = (double)pp / (double)qq;
        if (ratio > 1.0) ratio = 1.0;
        if (fabs((double)u - ratio) < 1e-6) fl |= VNX_FLAG_NEAR_TIE;
      }
    } else {
      acc = false;
      fl |= VNX_FLAG_BAD_ID;
    }
    if (Ledge[lane] || Ledge[k + 1 + lane]) fl |= VNX_FLAG_LSE_EDGE;
  }
  const uint64_t mask = __ballot(acc);
  const uint64_t rej = ~mask;
  int n = rej ? __builtin_ctzll(rej) : VNX_WAVE;
  if (n > k) n = k;
  int64_t* out = p.out_ids + b * (k + 1);
  if (lane < k) {
    out[lane] = lane < n ? x : -1;
    if (p.flags) p.flags[b * (k + 1) + lane] = fl;
  }
  if (lane == 0) {
    out[k] = -1;
    if (p.flags) p.flags[b * (k + 1) + k] = Ledge[k] ? VNX_FLAG_LSE_EDGE : 0;
    p.accept_len[b] = n;
    Job jb;
    jb.n = n;
    jb.mode = n < k ? 0 : 1;
    jb.Lp = Ls[n];
    jb.Lq = n < k ? Ls[k + 1 + n] : 0.0f;
    jb.u = p.u[b * (k + 1) + k];
    jb.pad = 0;
    p.jobs[b] = jb;
  }
}

// Residual weight of one element: max(0, p - q) (mode 0) or p (mode 1).
template <typename Tin>
__device__ __forceinline__ void resid_weights(const Tin* P, const Tin* Q, int64_t j, const Scale& sc,
                                              float thr_p, float thr_q, const Job& jb, float& w_r,
                                              float& w_p) {
  const float pp = vnx_exp_canon(scaled_elem(P, j, sc, thr_p) - jb.Lp);
  w_p = pp;
  if (jb.mode == 0) {
    const float qq = vnx_exp_canon(scaled_elem(Q, j, sc, thr_q) - jb.Lq);
    const float d = pp - qq;
    w_r = d > 0.0f ? d : 0.0f;
  } else {
    w_r = pp;
  }
}

template <typename Tin>
__global__ __launch_bounds__(kNT) void k_spec_pass2(SpecParams p) {
  constexpr int VE = Vec<Tin>::N;
  __shared__ ReduceLds lds;
  __shared__ int last_flag;
  __shared__ double scan_lds[16];
  __shared__ double sh_incl[kNT];
  __shared__ double sh_base, sh_target, sh_total;
  __shared__ int sh_cstar, sh_use_r;
  __shared__ unsigned long long sh_found, sh_lastpos;
  __shared__ double sh_before, sh_after;
  const int k = p.k;
  const int c = blockIdx.x % p.chunks2;
  const int64_t b = blockIdx.x / p.chunks2;
  const Job jb = p.jobs[b];
  const int prow = jb.mode == 0 ? jb.n : k;
  const Tin* P = static_cast<const Tin*>(p.tgt) + b * p.sb_t + prow * p.ld_t;
  const Tin* Q = static_cast<const Tin*>(p.dft) + b * p.sb_d + (jb.mode == 0 ? jb.n : 0) * p.ld_d;
  const float thr_p = p.thr_t ? p.thr_t[b * (k + 1) + prow] : kNegInf;
  const float thr_q = (p.thr_d && jb.mode == 0) ? p.thr_d[b * k + jb.n] : kNegInf;
  const int64_t c0 = (int64_t)c * p.chunk_len2;
  const int64_t c1 = c0 + p.chunk_len2 < p.V ? c0 + p.chunk_len2 : p.V;

  double sr = 0.0, sp = 0.0;
  {
    const int64_t nvec = (c1 - c0) / VE;
    for (int64_t vi = threadIdx.x; vi < nvec; vi += kNT) {
      float xp[VE], xq[VE];
      Vec<Tin>::load(P + c0 + vi * VE, xp);
      if (jb.mode == 0) Vec<Tin>::load(Q + c0 + vi * VE, xq);
      double dr = 0.0, dp = 0.0;
#pragma unroll
      for (int e = 0; e < VE; ++e) {
        float a = scale_logit(xp[e], p.sc);
        a = (a < thr_p) ? kNegInf : a;
        const float pp = vnx_exp_canon(a - jb.Lp);
        float wr = pp;
        if (jb.mode == 0) {
          float bq = scale_logit(xq[e], p.sc);
          bq = (bq < thr_q) ? kNegInf : bq;
          const float d = pp - vnx_exp_canon(bq - jb.Lq);
          wr = d > 0.0f ? d : 0.0f;
        }
        dr += (double)wr;
        dp += (double)pp;
      }
      sr += dr;
      sp += dp;
    }
    for (int64_t j = c0 + nvec * VE + threadIdx.x; j < c1; j += kNT) {
      float wr, wp;
      resid_weights(P, Q, j, p.sc, thr_p, thr_q, jb, wr, wp);
      sr += (double)wr;
      sp += (double)wp;
    }
  }
  sr = block_sum<kNT>(sr, lds.d);
  sp = block_sum<kNT>(sp, lds.d);
  if (threadIdx.x == 0) {
    st_agent(&p.part2[(b * p.chunks2 + c) * 2 + 0], sr);
    st_agent(&p.part2[(b * p.chunks2 + c) * 2 + 1], sp);
  }
  if (!arrive_last(&p.cnt2[b], (unsigned)p.chunks2, &last_flag)) return;

  // ---- last workgroup of b: locate the chunk, then the token ----
  if (threadIdx.x == 0) {
    double tr = 0.0, tp = 0.0;
    for (int j = 0; j < p.chunks2; ++j) {
      tr += ld_agent(&p.part2[(b * p.chunks2 + j) * 2 + 0]);
      tp += ld_agent(&p.part2[(b * p.chunks2 + j) * 2 + 1]);
    }
    const int use_r = (jb.mode == 1) || (tr > 0.0);
    const double total = use_r ? tr : tp;
    const double target = (double)jb.u * total;
    double run = 0.0;
    int cstar = -1, lastpos = -1;
    double base = 0.0, base_last = 0.0;
    for (int j = 0; j < p.chunks2; ++j) {
      const double m = ld_agent(&p.part2[(b * p.chunks2 + j) * 2 + (use_r ? 0 : 1)]);
      if (m > 0.0) {
        if (cstar < 0 && run + m > target) { cstar = j; base = run; }
        lastpos = j;
        base_last = run;
      }
      run += m;
    }
    if (cstar < 0) { cstar = lastpos; base = base_last; }
    sh_cstar = cstar;
    sh_base = base;
    sh_target = target;
    sh_total = total;
    sh_use_r = use_r;
    sh_found = ~0ull;
    sh_lastpos = 0ull;
    sh_before = 0.0;
    sh_after = 0.0;
  }
  __syncthreads();
  const int cstar = sh_cstar;
  int64_t token = 0;
  uint8_t fl = 0;
  if (cstar >= 0) {
    const int64_t s0 = (int64_t)cstar * p.chunk_len2;
    const int64_t s1 = s0 + p.chunk_len2 < p.V ? s0 + p.chunk_len2 : p.V;
    const double target = sh_target;
    const bool use_r = sh_use_r != 0;
    double base = sh_base;
    for (int64_t sb = s0; sb < s1; sb += (int64_t)kNT * VE) {
      const int64_t e0 = sb + (int64_t)threadIdx.x * VE;
      float w[VE];
      double local = 0.0;
      int lastpos_e = -1;
#pragma unroll
      for (int e = 0; e < VE; ++e) {
        const int64_t j = e0 + e;
        float wr = 0.0f, wp = 0.0f;
        if (j < s1) resid_weights(P, Q, j, p.sc, thr_p, thr_q, jb, wr, wp);
        w[e] = use_r ? wr : wp;
        local += (double)w[e];
        if (w[e] > 0.0f) lastpos_e = e;
      }
      const double incl = block_inclusive_scan<kNT>(local, scan_lds);
      sh_incl[threadIdx.x] = incl;
      __syncthreads();
      const double sb_total = sh_incl[kNT - 1];
      // [start, end) of consecutive threads share endpoints, so the ranges
      // partition [base, base + sb_total) exactly.
      const double start = base + (threadIdx.x ? sh_incl[threadIdx.x - 1] : 0.0);
      const double end = base + incl;
      if (start <= target && target < end) {
        double run = start;
        int pick = -1;
        double before = start, after = end;
#pragma unroll
        for (int e = 0; e < VE; ++e) {
          if (w[e] > 0.0f && pick < 0) {
            const double nr = run + (double)w[e];
            if (nr > target) {
              pick = e;
              before = run;
              after = nr;
            }
            run = nr;
          }
        }
        // Sequential rounding can leave run just below `end`: the target
        // then belongs to this thread's last positive element.
        if (pick < 0) pick = lastpos_e;
        sh_found = (unsigned long long)(e0 + pick);
        sh_before = before;
        sh_after = after;
      }
      if (lastpos_e >= 0) atomicMax(&sh_lastpos, (unsigned long long)(e0 + lastpos_e) + 1ull);
      __syncthreads();
      if (sh_found != ~0ull) break;
      base += sb_total;
      __syncthreads();
    }
    __syncthreads();
    if (sh_found != ~0ull) {
      token = (int64_t)sh_found;
      const double tol = 1e-12 * sh_total;
      if (target - sh_before < tol || sh_after - target < tol) fl |= VNX_FLAG_CDF_EDGE;
    } else {
      token = sh_lastpos ? (int64_t)(sh_lastpos - 1ull) : s0;
      fl |= VNX_FLAG_CDF_EDGE;
    }
  } else {
    fl |= VNX_FLAG_ZERO_RESIDUAL;
  }
  if (threadIdx.x == 0) {
    if (jb.mode == 0 && !sh_use_r) fl |= VNX_FLAG_ZERO_RESIDUAL;
    p.out_ids[b * (k + 1) + jb.n] = token;
    if (p.flags) p.flags[b * (k + 1) + jb.n] |= fl;
  }
}

// ---------------------------------------------------------------------------
// Greedy verify.
// ---------------------------------------------------------------------------
struct GreedyParams {
  const void* tgt;
  int64_t B;
  int k, rows_t;
  int64_t V, ld, sb;
  int chunks;
  int64_t chunk_len;
  const int64_t* ids;
  uint8_t* accepted;
  int64_t* main_pred;
  int32_t* accept_len;
  int64_t* out_ids;
  float* part_v;
  int64_t* part_i;
  unsigned* cnt;
};

template <typename Tin>
__global__ __launch_bounds__(kNT) void k_greedy(GreedyParams p) {
  __shared__ ReduceLds lds;
  __shared__ int last_flag;
  __shared__ int64_t pred[kMaxK + 1];
  const int c = blockIdx.x % p.chunks;
  const int64_t t = blockIdx.x / p.chunks;
  const int64_t b = t % p.B;
  const int i = (int)(t / p.B);
  const Tin* row = static_cast<const Tin*>(p.tgt) + b * p.sb + i * p.ld;
  const int64_t c0 = (int64_t)c * p.chunk_len;
  const int64_t c1 = c0 + p.chunk_len < p.V ? c0 + p.chunk_len : p.V;
  Scale one;
  one.T = 1.0f; one.y = 1.0f; one.mode = 0;
  ChunkResult cr = reduce_chunk<Tin, kNT, kNB, false, true>(row, c0, c1, one, kNegInf, lds);
  const int64_t slot = (b * p.rows_t + i) * p.chunks + c;
  if (threadIdx.x == 0) {
    st_agent(&p.part_v[slot], cr.av);
    st_agent(&p.part_i[slot], cr.ai);
  }
  if (!arrive_last(&p.cnt[b], (unsigned)(p.rows_t * p.chunks), &last_flag)) return;
  const int tid = threadIdx.x;
  if (tid < p.rows_t) {
    float bv = kNegInf;
    int64_t bi = INT64_MAX;
    const int64_t base = (b * p.rows_t + tid) * p.chunks;
    for (int j = 0; j < p.chunks; ++j) {
      const float v = ld_agent(&p.part_v[base + j]);
      const int64_t ix = ld_agent(&p.part_i[base + j]);
      if (argmax_better(v, ix, bv, bi)) { bv = v; bi = ix; }
    }
    pred[tid] = bi;
    if (p.main_pred) p.main_pred[b * p.rows_t + tid] = bi;
  }
  __syncthreads();
  if (tid >= VNX_WAVE) return;
  const int k = p.k;
  bool acc = true;
  int64_t x = -1;
  if (tid < k) {
    x = p.ids[b * k + tid];
    acc = (x == pred[tid]);
    if (p.accepted) p.accepted[b * k + tid] = acc ? 1 : 0;
  }
  const uint64_t rej = ~__ballot(acc);
  int n = rej ? __builtin_ctzll(rej) : VNX_WAVE;
  if (n > k) n = k;
  int64_t* out = p.out_ids + b * (k + 1);
  for (int j = tid; j <= k; j += VNX_WAVE) {
    int64_t v = -1;
    if (j < n) v = p.ids[b * k + j];
    else if (j == n && n < k) v = pred[n];
    else if (j == k && n == k && p.rows_t == k + 1) v = pred[k];
    out[j] = v;
  }
  if (tid == 0) p.accept_len[b] = n;
}

struct SpecPlan {
  int chunks, chunks2;
  int64_t len, len2;
};

static SpecPlan spec_plan(int64_t B, int k, int64_t V, int dtype) {
  const int ve = dtype == VNX_F32 ? 4 : 8;
  SpecPlan pl;
  int c = pick_chunks(B * (2 * k + 1), V, ve, 64);
  int64_t len = ((V + c - 1) / c + ve - 1) / ve * ve;
  pl.len = len;
  pl.chunks = (int)((V + len - 1) / len);
  int c2 = pick_chunks(B, V, ve, 64);
  int64_t len2 = ((V + c2 - 1) / c2 + ve - 1) / ve * ve;
  pl.len2 = len2;
  pl.chunks2 = (int)((V + len2 - 1) / len2);
  return pl;
}

static size_t spec_carve(void* ws, int64_t B, int k, const SpecPlan& pl, SpecParams* p) {
  Carve cv(ws);
  const size_t n1 = (size_t)B * (2 * k + 1) * pl.chunks;
  unsigned* c1 = cv.take<unsigned>(2 * B);  // pass-1 counters, then pass-2 counters
  unsigned* c2 = c1 ? c1 + B : nullptr;
  float* pm = cv.take<float>(n1);
  double* ps = cv.take<double>(n1);
  Job* jobs = cv.take<Job>(B);
  double* p2 = cv.take<double>((size_t)B * pl.chunks2 * 2);
  if (p) {
    p->part_m = pm; p->part_s = ps; p->cnt1 = c1; p->jobs = jobs; p->part2 = p2; p->cnt2 = c2;
  }
  return cv.bytes();
}

// Rows (b, i), i < nrows, at x + b*sb + i*ld must not overlap inside a batch
// row (ld >= V) and batch rows must not overlap (sb >= (nrows-1)*ld + V);
// 16-byte vector loads need x, ld and sb aligned to the vector width.
static int check_rows(const void* x, int dtype, int64_t ld, int64_t sb, int nrows, int64_t V) {
  if (!x) return VNX_ERR_INVALID_ARG;
  if (ld < V || sb < (int64_t)(nrows - 1) * ld + V) return VNX_ERR_INVALID_ARG;
  const int ve = dtype == VNX_F32 ? 4 : 8;
  if (!aligned16(x) || ld % ve != 0 || sb % ve != 0) return VNX_ERR_UNSUPPORTED;
  return VNX_OK;
}

}  // namespace vnx

using namespace vnx;

extern "C" {

size_t vnx_spec_accept_workspace(int64_t B, int k, int64_t V) {
  if (B <= 0 || k <= 0 || V <= 0) return 256;
  return spec_carve(nullptr, B, k, spec_plan(B, k, V, VNX_F32), nullptr);
}

int vnx_spec_accept(const void* target, const void* draft, int dtype, int64_t B, int k, int64_t V,
                    int64_t ld_t, int64_t sb_t, int64_t ld_d, int64_t sb_d,
                    const int64_t* draft_ids, const float* uniforms,
                    float temperature, const float* thr_t, const float* thr_d, int32_t* accept_len,
                    int64_t* out_ids, uint8_t* flags, float* lse_t, float* lse_d, void* workspace,
                    size_t workspace_bytes, void* stream) {
  if (dtype != VNX_F32 && dtype != VNX_BF16) return VNX_ERR_UNSUPPORTED;
  if (B < 0 || k < 1 || k > kMaxK || V <= 0) return VNX_ERR_INVALID_ARG;
  if (!(temperature > 0.0f) || !__builtin_isfinite(temperature)) return VNX_ERR_INVALID_ARG;
  if (B == 0) return VNX_OK;
  if (B > (1 << 20) || V > ((int64_t)1 << 31)) return VNX_ERR_UNSUPPORTED;
  int st = check_rows(target, dtype, ld_t, sb_t, k + 1, V);
  if (st) return st;
  st = check_rows(draft, dtype, ld_d, sb_d, k, V);
  if (st) return st;
  if (!draft_ids || !uniforms || !accept_len || !out_ids) return VNX_ERR_INVALID_ARG;
  SpecPlan pl = spec_plan(B, k, V, dtype);
  if (B * (2 * k + 1) * (int64_t)pl.chunks >= INT32_MAX || B * (int64_t)pl.chunks2 >= INT32_MAX)
    return VNX_ERR_UNSUPPORTED;
  if (!workspace || workspace_bytes < spec_carve(nullptr, B, k, pl, nullptr)) return VNX_ERR_WORKSPACE;
  SpecParams p{};
  p.tgt = target; p.dft = draft; p.B = B; p.k = k; p.V = V;
  p.ld_t = ld_t; p.ld_d = ld_d; p.sb_t = sb_t; p.sb_d = sb_d;
  p.chunks = pl.chunks; p.chunk_len = pl.len; p.chunks2 = pl.chunks2; p.chunk_len2 = pl.len2;
  p.sc = make_scale(temperature);
  p.thr_t = thr_t; p.thr_d = thr_d; p.ids = draft_ids; p.u = uniforms;
  p.accept_len = accept_len; p.out_ids = out_ids; p.flags = flags; p.lse_t = lse_t; p.lse_d = lse_d;
  spec_carve(workspace, B, k, pl, &p);
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 g1((unsigned)(B * (2 * k + 1) * pl.chunks)), g2((unsigned)(B * pl.chunks2));
  st = zero_counters(p.cnt1, 2 * B, s);
  if (st) return st;
  if (dtype == VNX_F32) {
    hipLaunchKernelGGL(k_spec_pass1<float>, g1, dim3(kNT), 0, s, p);
    VNX_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_spec_pass2<float>, g2, dim3(kNT), 0, s, p);
  } else {
    hipLaunchKernelGGL(k_spec_pass1<__hip_bfloat16>, g1, dim3(kNT), 0, s, p);
    VNX_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_spec_pass2<__hip_bfloat16>, g2, dim3(kNT), 0, s, p);
  }
  VNX_LAUNCH_CHECK();
  return VNX_OK;
}

size_t vnx_greedy_verify_workspace(int64_t B, int rows_t, int64_t V) {
  if (B <= 0 || rows_t <= 0 || V <= 0) return 256;
  const int c = pick_chunks(B * rows_t, V, 4, 64);
  Carve cv(nullptr);
  cv.take<unsigned>(B);
  cv.take<float>((size_t)B * rows_t * c);
  cv.take<int64_t>((size_t)B * rows_t * c);
  return cv.bytes();
}

int vnx_greedy_verify(const void* target, int dtype, int64_t B, int k, int rows_t, int64_t V,
                      int64_t ld, int64_t sb, const int64_t* draft_ids, uint8_t* accepted, int64_t* main_pred,
                      int32_t* accept_len, int64_t* out_ids, void* workspace, size_t workspace_bytes,
                      void* stream) {
  if (dtype != VNX_F32 && dtype != VNX_BF16) return VNX_ERR_UNSUPPORTED;
  if (B < 0 || k < 1 || k > kMaxK || V <= 0) return VNX_ERR_INVALID_ARG;
  if (rows_t != k && rows_t != k + 1) return VNX_ERR_INVALID_ARG;
  if (B == 0) return VNX_OK;
  if (B > (1 << 20) || V > ((int64_t)1 << 31)) return VNX_ERR_UNSUPPORTED;
  int st = check_rows(target, dtype, ld, sb, rows_t, V);
  if (st) return st;
  if (!draft_ids || !accept_len || !out_ids) return VNX_ERR_INVALID_ARG;
  const int ve = dtype == VNX_F32 ? 4 : 8;
  int c = pick_chunks(B * rows_t, V, ve, 64);
  const int64_t len = ((V + c - 1) / c + ve - 1) / ve * ve;
  c = (int)((V + len - 1) / len);
  if (B * rows_t * (int64_t)c >= INT32_MAX) return VNX_ERR_UNSUPPORTED;
  Carve cv(workspace);
  GreedyParams p{};
  p.cnt = cv.take<unsigned>(B);
  p.part_v = cv.take<float>((size_t)B * rows_t * c);
  p.part_i = cv.take<int64_t>((size_t)B * rows_t * c);
  if (!workspace || workspace_bytes < cv.bytes()) return VNX_ERR_WORKSPACE;
  p.tgt = target; p.B = B; p.k = k; p.rows_t = rows_t; p.V = V; p.ld = ld; p.sb = sb;
  p.chunks = c; p.chunk_len = len; p.ids = draft_ids; p.accepted = accepted;
  p.main_pred = main_pred; p.accept_len = accept_len; p.out_ids = out_ids;
  hipStream_t s = static_cast<hipStream_t>(stream);
  st = zero_counters(p.cnt, B, s);
  if (st) return st;
  dim3 g((unsigned)(B * rows_t * c));
  if (dtype == VNX_F32)
    hipLaunchKernelGGL(k_greedy<float>, g, dim3(kNT), 0, s, p);
  else
    hipLaunchKernelGGL(k_greedy<__hip_bfloat16>, g, dim3(kNT), 0, s, p);
  VNX_LAUNCH_CHECK();
  return VNX_OK;
}

}  // extern "C"
