// Stochastic speculative acceptance (Leviathan et al. 2023, Alg. 1) on the
// (B, k+1, V) target and (B, k, V) draft logits, in two launches with no
// cross-workgroup waits:
//   A  grid B*(2k+1)*C: every workgroup streams one chunk of one target or
//      draft row and writes the chunk's (max, sum 2^..) partial.  Many short
//      workgroups let the dispatcher balance the CUs.  (The first ones also
//      clear B's arrival counters.)
//   B  grid B*C2: every workgroup of batch row b first merges b's partials
//      into its 2k+1 row LSEs (fp64, staged through LDS, fixed lane order,
//      so all of them get the same bits), rounds them to fp32 and runs the k
//      acceptance tests in one wavefront (lane i tests position i; a ballot
//      gives the first rejection n); the chunk-0 workgroup writes
//      accept_len, the accepted ids, the LSEs and flags.  Then it streams its
//      chunk of p_n and q_n (or p_k for the bonus draw) and publishes the
//      draw mass sum max(0, p-q) (or sum p) of each sub-block of 64 vectors
//      (fp64).  The workgroup completing row b (an arrival counter) sums the
//      sub-block masses in a fixed order, walks them to the sub-block holding
//      u_k * mass and recomputes only that sub-block (one wave, one inclusive
//      scan) to find the token.  Published masses move through agent-scope
//      atomic stores and loads (rowred.h arrive_last); everything else
//      crosses the kernel boundary.
// (Measured and dropped: the acceptance inside launch A by arrival counting
// -- the counter round trip of 17K short workgroups slowed the streaming by
// half; a pipeline of row parts whose accept / mass / draw run beside
// the next part's streaming -- launch B is latency-bound, so a tail part
// costs nearly as much as the whole; and one launch whose mass workgroups
// follow the lse workgroups of a later row in the grid and poll for their
// row's partials (posted as self-validating words, no atomics) -- at
// B = 64, k = 8 it took 205-217 us per call in a graph against 205 us for
// the two launches, because the mass workgroups hold CU slots while the
// rows stream and the merged kernel runs one wave per SIMD fewer.  The mass
// pass is VALU-bound: about 57 instructions per element of max(0, p - q),
// two canonical exps among them.)
// Probabilities that feed decisions use vnx_exp_canon(a - L32), a = RN(l/T),
// L32 = RN32(row LSE), so the CPU checker reproduces them bit for bit.
#include <algorithm>
#include <mutex>

#include "rowred.h"
#include "vnx_internal.h"

namespace vnx {

constexpr int kNT = 256;   // threads per workgroup
constexpr int kNW = kNT / VNX_WAVE;
constexpr int kNB = 8;     // vectors per thread in flight, lse pass
constexpr int kNB2 = 4;    // sub-blocks per wave in flight, mass pass
constexpr int kMaxK = 64;
constexpr int kMaxChunks = 256;
constexpr int kDrawLds = 4096;  // draw: sub-block masses held in LDS (V <= 4096*64*VE)
constexpr int kAccParts = 2048; // accept: (2k+1)*chunks partials staged in LDS

struct Job {
  int n;      // first rejected position (k if all accepted)
  int mode;   // 0 = residual draw from max(0, p_n - q_n), 1 = draw from p_k
  float Lp;   // fp32 LSE of the target row drawn from
  float Lq;   // fp32 LSE of draft row n (mode 0)
  float u;    // uniform of the draw
  int fln;    // the acceptance flags of position n (the draw adds its own)
};

struct SpecParams {
  const void* tgt;
  const void* dft;
  int64_t B;
  int k;
  int64_t V, ld_t, ld_d, sb_t, sb_d;
  int chunks;        // lse pass: chunks per row
  int64_t chunk_len; // lse pass: elements per chunk (multiple of the vector width)
  int64_t nsb;       // sub-blocks (64 vectors) per row
  int spc;           // launch B: sub-blocks per chunk
  int chunks2;       // launch B: chunks per row
  TScale sc;
  const float* thr_t;
  const float* thr_d;
  const int64_t* ids;
  const float* u;
  int32_t* accept_len;
  int64_t* out_ids;
  uint8_t* flags;
  float* lse_t;
  float* lse_d;
  float* part_m;   // [B*(2k+1)][chunks]
  double* part_s;  // [B*(2k+1)][chunks]
  double* sbm;     // [B][nsb] sub-block draw masses
  unsigned* cnt;   // [B] arrival counters of launch B
  float* gath;     // [B][2k] scaled target / draft logits at the draft ids
  // Draft rows' LSEs supplied by the caller (the draws that produced the
  // draft ids computed them): lse_din[i * ld_din + b] = RN32(LSE of q_i / T),
  // fl_din the draws' flags (VNX_FLAG_LSE_EDGE used).  Then launch A streams
  // only the k + 1 target rows (rows_a = k + 1, else 2k + 1) and gathers
  // the draft logits at the draft ids beside the target's.
  const float* lse_din;
  const uint8_t* fl_din;
  int64_t ld_din;
  int rows_a;
};

// Distance test of an fp64 LSE to the rounding midpoints around its fp32 value.
__device__ __forceinline__ bool near_f32_edge(double L, float L32, double tol) {
  if (!__builtin_isfinite(L)) return false;
  const double up = (double)nextafterf(L32, __builtin_inff());
  const double dn = (double)nextafterf(L32, -__builtin_inff());
  const double mu = 0.5 * ((double)L32 + up), md = 0.5 * ((double)L32 + dn);
  return fabs(L - mu) < tol || fabs(L - md) < tol;
}

template <typename Tin, int SM, bool THR>
__device__ __forceinline__ float scaled_at(const Tin* row, int64_t j, const TScale& sc, float thr) {
  return scaled<SM, THR>(Vec<Tin>::load1(row + j), sc, thr);
}

// Row ri of batch row b: target rows 0..k, then draft rows 0..k-1.
template <typename Tin>
__device__ __forceinline__ const Tin* row_ptr(const SpecParams& p, int64_t b, int ri) {
  if (ri <= p.k) return static_cast<const Tin*>(p.tgt) + b * p.sb_t + ri * p.ld_t;
  return static_cast<const Tin*>(p.dft) + b * p.sb_d + (ri - p.k - 1) * p.ld_d;
}

template <bool THR>
__device__ __forceinline__ float row_thr(const SpecParams& p, int64_t b, int ri) {
  if constexpr (!THR) return kNegInf;
  if (ri <= p.k) return p.thr_t ? p.thr_t[b * (p.k + 1) + ri] : kNegInf;
  return p.thr_d ? p.thr_d[b * p.k + (ri - p.k - 1)] : kNegInf;
}

// ---------------------------------------------------------------------------
// lse: chunk c of row r (r = b*(2k+1) + ri) per workgroup.
// ---------------------------------------------------------------------------
template <typename Tin, int SM, bool THR>
__device__ __forceinline__ void lse_work(const SpecParams& p, int64_t r, int c, ReduceLds& lds) {
  const int k = p.k;
  const int R = p.rows_a;
  const int64_t b = r / R;
  const int ri = (int)(r - b * R);
  const int64_t c0 = (int64_t)c * p.chunk_len;
  const int64_t c1 = c0 + p.chunk_len < p.V ? c0 + p.chunk_len : p.V;
  // The chunk holding this row's draft id (target row i < k: x_i; draft row
  // i: x_i) records the scaled logit there for the acceptance test.
  if (ri != k) {
    const int pos = ri < k ? ri : ri - k - 1;
    const int64_t x = p.ids[b * k + pos];
    if (x >= c0 && x < c1 && threadIdx.x == 0) {
      p.gath[b * 2 * k + (ri < k ? pos : k + pos)] =
          scaled_at<Tin, SM, THR>(row_ptr<Tin>(p, b, ri), x, p.sc, row_thr<THR>(p, b, ri));
      // draft rows not streamed here: their value at the id with the target's
      if (p.lse_din && ri < k)
        p.gath[b * 2 * k + k + pos] =
            scaled_at<Tin, SM, THR>(row_ptr<Tin>(p, b, k + 1 + ri), x, p.sc, row_thr<THR>(p, b, k + 1 + ri));
    }
  }
  const ChunkResult cr = reduce_chunk<Tin, SM, THR, true, false, kNT, kNB>(row_ptr<Tin>(p, b, ri), c0, c1,
                                                                           p.sc, row_thr<THR>(p, b, ri), lds);
  if (threadIdx.x == 0) {
    p.part_m[r * p.chunks + c] = cr.m;
    p.part_s[r * p.chunks + c] = cr.s;
  }
}

// ---------------------------------------------------------------------------
// accept: the row LSEs of b from its chunk partials and the k acceptance
// tests.  Every workgroup of b's mass chunks runs it and gets the same job
// (fixed lane order, no atomics); with `write`, the workgroup also stores
// accept_len, out_ids (accepted prefix, -1 after), flags and the LSEs.
// pm_l / ps_l: LDS room for the row's rows_a * chunks partials.
// ---------------------------------------------------------------------------
struct AcceptLds {
  float Ls[2 * kMaxK + 1];
  int Ledge[2 * kMaxK + 1];
  Job job;
};

template <typename Tin, int SM, bool THR>
__device__ __forceinline__ Job accept_row(const SpecParams& p, int64_t b, bool write, AcceptLds& L, float* pm_l,
                                          double* ps_l) {
  const int k = p.k;
  const int R = 2 * k + 1;
  const int tid = threadIdx.x;
  const int lane = tid % VNX_WAVE, wave = tid / VNX_WAVE;
  // Lane i < k of wave 0 first issues the loads that do not depend on the
  // LSEs (draft id, its uniform, the two scaled logits at the id that
  // launch A recorded), so they overlap the partial loads below.
  int64_t x = -1;
  float u = 0.0f, a = 0.0f, bq = 0.0f;
  if (tid < k) {
    x = p.ids[b * k + tid];
    u = p.u[b * (k + 1) + tid];
    a = p.gath[b * 2 * k + tid];
    bq = p.gath[b * 2 * k + k + tid];
  }
  const bool valid = x >= 0 && x < p.V;
  // The row's partials into LDS with every load in flight at once; then
  // segment g of 16 lanes merges rows g, g + 16, ... (every segment of the
  // workgroup at once): the row maximum over the partial maxima, every
  // lane's partials rescaled to it and summed in lane order, then a
  // butterfly sum across the segment.
  const int C = p.chunks;
  const int RA = p.rows_a;   // rows with partials (the draft rows come from lse_din otherwise)
  const int total = RA * C;  // <= kAccParts (host check)
  const int64_t pbase = b * (int64_t)total;
  for (int i = tid; i < total; i += kNT) {
    pm_l[i] = p.part_m[pbase + i];
    ps_l[i] = p.part_s[pbase + i];
  }
  __syncthreads();
  constexpr int SEG = 16;
  const int sl = tid % SEG;
  if (RA < R && tid < k) {
    // the draft rows' LSEs as the draws computed them, with their edge flags
    const float Ld = p.lse_din[tid * p.ld_din + b];
    L.Ls[k + 1 + tid] = Ld;
    L.Ledge[k + 1 + tid] = (p.fl_din && (p.fl_din[tid * p.ld_din + b] & VNX_FLAG_LSE_EDGE)) ? 1 : 0;
    if (write && p.lse_d) p.lse_d[b * k + tid] = Ld;
  }
  for (int r = tid / SEG; r < RA; r += kNT / SEG) {
    const int base = r * C;
    float M = kNegInf;
    for (int c = sl; c < C; c += SEG) M = fmaxf(M, pm_l[base + c]);
#pragma unroll
    for (int o = SEG / 2; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, SEG));
    double S = 0.0;
    if (M < kPosInf) {
      for (int c = sl; c < C; c += SEG) {
        const float m = pm_l[base + c];
        if (m > kNegInf) {
          const double sv = ps_l[base + c];
          S += (m == M) ? sv : rescale(sv, mt_of(m), mt_of(M));
        }
      }
    }
#pragma unroll
    for (int o = SEG / 2; o > 0; o >>= 1) S += __shfl_xor(S, o, SEG);
    if (sl == 0) {
      const double Lr = lse_of(M, S);
      const float L32 = (float)Lr;
      L.Ls[r] = L32;
      L.Ledge[r] = near_f32_edge(Lr, L32, 1e-7) ? 1 : 0;
      if (write) {
        if (r <= k) {
          if (p.lse_t) p.lse_t[b * (k + 1) + r] = L32;
        } else if (p.lse_d) {
          p.lse_d[b * k + (r - k - 1)] = L32;
        }
      }
    }
  }
  __syncthreads();
  if (wave == 0) {
    bool acc = true;
    uint8_t fl = 0;
    if (lane < k) {
      if (valid) {
        const float pp = vnx_exp_canon(a - L.Ls[lane]);
        const float qq = vnx_exp_canon(bq - L.Ls[k + 1 + lane]);
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
      if (L.Ledge[lane] || L.Ledge[k + 1 + lane]) fl |= VNX_FLAG_LSE_EDGE;
    }
    const uint64_t rej = ~__ballot(acc);
    int n = rej ? __builtin_ctzll(rej) : VNX_WAVE;
    if (n > k) n = k;
    const int fl_k = L.Ledge[k] ? VNX_FLAG_LSE_EDGE : 0;
    const int fln = n < k ? __shfl((int)fl, n, VNX_WAVE) : fl_k;
    // Position n (the drawn token and its flags) is written by the workgroup
    // that draws, and only by it.
    if (write) {
      int64_t* out = p.out_ids + b * (k + 1);
      if (lane < k && lane != n) {
        out[lane] = lane < n ? x : -1;
        if (p.flags) p.flags[b * (k + 1) + lane] = fl;
      }
      if (lane == 0) {
        if (n < k) {
          out[k] = -1;
          if (p.flags) p.flags[b * (k + 1) + k] = (uint8_t)fl_k;
        }
        p.accept_len[b] = n;
      }
    }
    if (lane == 0) {
      Job jb;
      jb.n = n;
      jb.mode = n < k ? 0 : 1;
      jb.Lp = L.Ls[n];
      jb.Lq = n < k ? L.Ls[k + 1 + n] : 0.0f;
      jb.u = p.u[b * (k + 1) + k];
      jb.fln = fln;
      L.job = jb;
    }
  }
  __syncthreads();
  return L.job;
}

// ---------------------------------------------------------------------------
// Draw weights.  W_RESID: max(0, p - q); W_P: p.  p = E(a - Lp), q = E(b - Lq),
// E = vnx_exp_canon, a / b the exact scaled logits.
// ---------------------------------------------------------------------------
enum { W_RESID = 0, W_P = 1 };

template <int SM, bool THR>
__device__ __forceinline__ float draw_weight(float lp, float lq, int wsel, const TScale& sc, float thr_p,
                                             float thr_q, float Lp, float Lq) {
  const float pp = vnx_exp_canon(scaled<SM, THR>(lp, sc, thr_p) - Lp);
  if (wsel == W_P) return pp;
  const float d = pp - vnx_exp_canon(scaled<SM, THR>(lq, sc, thr_q) - Lq);
  return d > 0.0f ? d : 0.0f;
}

// Rows drawn from for batch row b (p_n / q_n, or p_k for the bonus draw).
struct DrawRows {
  int64_t poff, qoff;
  float thr_p, thr_q;
};

template <bool THR>
__device__ __forceinline__ DrawRows draw_rows(const SpecParams& p, int64_t b, const Job& jb) {
  DrawRows d;
  const int prow = jb.mode == 0 ? jb.n : p.k;
  d.poff = b * p.sb_t + prow * p.ld_t;
  d.qoff = b * p.sb_d + (jb.mode == 0 ? jb.n : 0) * p.ld_d;
  d.thr_p = kNegInf;
  d.thr_q = kNegInf;
  if constexpr (THR) {
    d.thr_p = p.thr_t ? p.thr_t[b * (p.k + 1) + prow] : kNegInf;
    d.thr_q = (p.thr_d && jb.mode == 0) ? p.thr_d[b * p.k + jb.n] : kNegInf;
  }
  return d;
}

// Raw logits of this lane's vector of sub-block sbi (elements
// sbi*64*VE + lane*VE + [0, VE)); elements past V read as -inf, whose weight is 0.
template <typename Tin>
__device__ __forceinline__ void lane_vec(const Tin* row, int64_t sbi, int64_t V, float (&x)[Vec<Tin>::N]) {
  constexpr int VE = Vec<Tin>::N;
  const int64_t e = (sbi * VNX_WAVE + (threadIdx.x % VNX_WAVE)) * VE;
  if (e + VE <= V) {
    Vec<Tin>::load(row + e, x);
  } else {
#pragma unroll
    for (int i = 0; i < VE; ++i) x[i] = e + i < V ? Vec<Tin>::load1(row + e + i) : kNegInf;
  }
}

// The same vector as raw bits (elements past V carry -inf bits), converted
// later: a conversion beside the load would wait for it there, and with it for
// every load issued before it.
template <typename Tin>
__device__ __forceinline__ u32x4 lane_raw(const Tin* row, int64_t sbi, int64_t V) {
  constexpr int VE = Vec<Tin>::N;
  const int64_t e = (sbi * VNX_WAVE + (threadIdx.x % VNX_WAVE)) * VE;
  if (e + VE <= V) return Vec<Tin>::load_raw(row + e);
  uint32_t w[4];
  if constexpr (VE == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = e + i < V ? __float_as_uint(Vec<Tin>::load1(row + e + i)) : 0xFF800000u;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = e + 2 * i < V ? (__float_as_uint(Vec<Tin>::load1(row + e + 2 * i)) >> 16) : 0xFF80u;
      const uint32_t hi = e + 2 * i + 1 < V ? (__float_as_uint(Vec<Tin>::load1(row + e + 2 * i + 1)) >> 16) : 0xFF80u;
      w[i] = lo | (hi << 16);
    }
  }
  return u32x4{w[0], w[1], w[2], w[3]};
}

// Draw mass of this lane's vector of sub-block sbi (sequential fp64 sum in
// element order), and its weights.
template <typename Tin, int SM, bool THR>
__device__ __forceinline__ double lane_weights(const Tin* P, const Tin* Q, int64_t sbi, int64_t V, int wsel,
                                               const TScale& sc, const DrawRows& d, const Job& jb,
                                               float (&w)[Vec<Tin>::N]) {
  constexpr int VE = Vec<Tin>::N;
  float xp[VE], xq[VE];
  lane_vec<Tin>(P, sbi, V, xp);
  if (wsel == W_RESID) lane_vec<Tin>(Q, sbi, V, xq);
  double m = 0.0;
#pragma unroll
  for (int i = 0; i < VE; ++i) {
    w[i] = draw_weight<SM, THR>(xp[i], wsel == W_RESID ? xq[i] : 0.0f, wsel, sc, d.thr_p, d.thr_q, jb.Lp, jb.Lq);
    m += (double)w[i];
  }
  return m;
}

// ---------------------------------------------------------------------------
// mass: chunk c of batch row b = sub-blocks [c*spc, (c+1)*spc); wave w takes
// sub-blocks c*spc + w + kNW*j, so the workgroup's loads are contiguous.
// ---------------------------------------------------------------------------
template <typename Tin, int SM, bool THR, int WSEL>
__device__ __forceinline__ void mass_chunk(const SpecParams& p, int64_t b, int c, int spc, const Tin* P,
                                           const Tin* Q, const DrawRows& d, const Job& jb) {
  constexpr int VE = Vec<Tin>::N;
  const int wave = threadIdx.x / VNX_WAVE;
  const int64_t s0 = (int64_t)c * spc;
  const int64_t s1 = min(s0 + spc, p.nsb);
  for (int64_t sb = s0 + wave; sb < s1; sb += (int64_t)kNW * kNB2) {
    // every load of the batch in flight first (raw bits), then the weights
    u32x4 rp[kNB2], rq[kNB2];
#pragma unroll
    for (int j = 0; j < kNB2; ++j) {
      const int64_t sbi = sb + (int64_t)kNW * j;
      rp[j] = rq[j] = u32x4{0u, 0u, 0u, 0u};
      if (sbi < s1) {
        rp[j] = lane_raw<Tin>(P, sbi, p.V);
        if constexpr (WSEL == W_RESID) rq[j] = lane_raw<Tin>(Q, sbi, p.V);
      }
    }
#pragma unroll
    for (int j = 0; j < kNB2; ++j) {
      const int64_t sbi = sb + (int64_t)kNW * j;
      if (sbi < s1) {
        float xp[VE], xq[VE];
        Vec<Tin>::cvt_raw(rp[j], xp);
        if constexpr (WSEL == W_RESID) Vec<Tin>::cvt_raw(rq[j], xq);
        double m = 0.0;
#pragma unroll
        for (int i = 0; i < VE; ++i)
          m += (double)draw_weight<SM, THR>(xp[i], WSEL == W_RESID ? xq[i] : 0.0f, WSEL, p.sc, d.thr_p,
                                            d.thr_q, jb.Lp, jb.Lq);
        m = wave_sum(m);
        if (threadIdx.x % VNX_WAVE == 0) st_agent(&p.sbm[b * p.nsb + sbi], m);
      }
    }
  }
  // every wave's published masses complete before the workgroup arrives
  __builtin_amdgcn_s_waitcnt(0);
}

// ---------------------------------------------------------------------------
// draw: thread t owns sub-blocks [t*q, (t+1)*q) (q = ceil(nsb/kNT)); the
// total is sum_t (sum_i sbm[t*q+i]) in that nested sequential order, and the
// walk to the target follows the same order: thread, then sub-block, then
// (one wave, lane-order inclusive scan) lane, then element.  sh_m holds the
// row's nsb sub-block masses (dynamic LDS), published by the other
// workgroups of launch B (coherent loads).
// ---------------------------------------------------------------------------
struct DrawLds {
  double T[kNT], E[kNT];
  double scan[kNW];
  double total, target, base;
  int64_t sb;
  int tstar, tlast;
};

template <typename Tin, int SM, bool THR>
__device__ __forceinline__ void draw_work(const SpecParams& p, int64_t b, const Job& jb, DrawLds& L, double* sh_m) {
  constexpr int VE = Vec<Tin>::N;
  const int k = p.k;
  const int tid = threadIdx.x;
  const DrawRows d = draw_rows<THR>(p, b, jb);
  const Tin* P = static_cast<const Tin*>(p.tgt) + d.poff;
  const Tin* Q = static_cast<const Tin*>(p.dft) + d.qoff;
  double* sbm = p.sbm + b * p.nsb;
  const int64_t q = (p.nsb + kNT - 1) / kNT;  // <= kDrawLds / kNT (host check)
  int wsel = jb.mode == 0 ? W_RESID : W_P;
  uint8_t fl = 0;

  // All sub-block masses into LDS (one load per element, all in flight);
  // thread t sums its q consecutive sub-blocks in order (T_t); an inclusive
  // block scan of T_t in thread order gives every thread its range
  // [start_t, end_t), and the total is the scan's last value, so the total
  // and the ranges come from the same sums.
  auto scan_totals = [&]() {
    __syncthreads();
    double t = 0.0;
    for (int64_t i = (int64_t)tid * q; i < min((int64_t)(tid + 1) * q, p.nsb); ++i) t += sh_m[i];
    const double incl = block_inclusive_scan<kNT>(t, L.scan);
    L.T[tid] = t;
    L.E[tid] = incl;
    __syncthreads();
    if (tid == kNT - 1) L.total = incl;
    __syncthreads();
  };
  {
    // every load in flight first (at most kDrawLds / kNT per thread), then
    // the LDS stores
    double v[kDrawLds / kNT];
#pragma unroll
    for (int j = 0; j < kDrawLds / kNT; ++j) {
      const int64_t i = tid + (int64_t)j * kNT;
      v[j] = i < p.nsb ? ld_agent(&sbm[i]) : 0.0;
    }
#pragma unroll
    for (int j = 0; j < kDrawLds / kNT; ++j) {
      const int64_t i = tid + (int64_t)j * kNT;
      if (i < p.nsb) sh_m[i] = v[j];
    }
  }
  scan_totals();
  if (!(L.total > 0.0) && wsel == W_RESID) {
    // max(0, p_n - q_n) has no mass (p_n == q_n after rounding): draw from
    // p_n.  This workgroup recomputes the sub-block masses of p_n (rare path).
    fl |= VNX_FLAG_ZERO_RESIDUAL;
    wsel = W_P;
    for (int64_t sbi = tid / VNX_WAVE; sbi < p.nsb; sbi += kNW) {
      float w[VE];
      const double m = wave_sum(lane_weights<Tin, SM, THR>(P, Q, sbi, p.V, wsel, p.sc, d, jb, w));
      if (tid % VNX_WAVE == 0) sh_m[sbi] = m;
    }
    scan_totals();
  }
  // The thread whose range holds target = u * total (ranges of zero mass are
  // empty); if rounding leaves none, the last thread with positive mass.
  if (tid == 0) {
    L.tstar = kNT;  // atomicMin sentinel: no thread
    L.tlast = -1;
  }
  __syncthreads();
  const double total = L.total;
  const double target = (double)jb.u * total;
  {
    const double T = L.T[tid], end = L.E[tid];
    const double start = tid ? L.E[tid - 1] : 0.0;
    if (T > 0.0 && start <= target && target < end) atomicMin(&L.tstar, tid);
    if (T > 0.0) atomicMax(&L.tlast, tid);
  }
  __syncthreads();
  if (tid == 0) {
    int tstar = L.tstar;
    if (tstar == kNT) tstar = L.tlast;
    int64_t sstar = -1;
    double base = 0.0;
    if (tstar >= 0) {
      // Sub-blocks of that thread, in order, from the thread's start.
      const double b0 = tstar ? L.E[tstar - 1] : 0.0;
      double r2 = b0, b_last = b0;
      int64_t slast = -1;
      for (int64_t i = (int64_t)tstar * q; i < min((int64_t)(tstar + 1) * q, p.nsb); ++i) {
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
  if (tid >= VNX_WAVE) return;
  // Wave 0: the sub-block's weights, lane-order inclusive scan, element walk.
  int64_t token = 0;
  if (sstar < 0) {
    fl |= VNX_FLAG_ZERO_RESIDUAL;
  } else {
    float w[VE];
    const double lm = lane_weights<Tin, SM, THR>(P, Q, sstar, p.V, wsel, p.sc, d, jb, w);
    const double incl = wave_inclusive_scan(lm);
    const double start = L.base + (incl - lm);
    const double end = L.base + incl;
    const double tgt = L.target;
    // The lane whose [start, end) holds the target; if rounding leaves the
    // target past every lane, the last lane with positive mass.
    const bool hit = lm > 0.0 && start <= tgt && tgt < end;
    const uint64_t hits = __ballot(hit);
    const uint64_t pos = __ballot(lm > 0.0);
    const int lane = tid;
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
  if (tid == 0) {
    p.out_ids[b * (k + 1) + jb.n] = token;
    if (p.flags) p.flags[b * (k + 1) + jb.n] = (uint8_t)(jb.fln | fl);
  }
}

// ---------------------------------------------------------------------------
// Launch A: chunk partials of every row; the first workgroups also clear the
// arrival counters of launch B.
// ---------------------------------------------------------------------------
template <typename Tin, int SM, bool THR>
__global__ __launch_bounds__(kNT) void k_spec_lse(SpecParams p) {
  __shared__ ReduceLds lds;
  const int64_t zc = (int64_t)blockIdx.x * kNT + threadIdx.x;
  if (zc < p.B) p.cnt[zc] = 0u;
  const int64_t w = blockIdx.x;
  if (w < p.B * p.rows_a * p.chunks) lse_work<Tin, SM, THR>(p, w / p.chunks, (int)(w % p.chunks), lds);
}

// ---------------------------------------------------------------------------
// Launch B: accept of the row, draw masses of one chunk; the workgroup
// completing batch row b draws its token.  Dynamic LDS: the row's partials
// during the accept, then its sub-block masses if it draws.
// ---------------------------------------------------------------------------
union MassDrawLds {
  AcceptLds acc;
  DrawLds draw;
};

template <typename Tin, int SM, bool THR>
__global__ __launch_bounds__(kNT) void k_spec_mass_draw(SpecParams p) {
  __shared__ MassDrawLds lds;
  __shared__ int last_flag;
  extern __shared__ double dyn[];
  const int c = blockIdx.x % p.chunks2;
  const int64_t b = blockIdx.x / p.chunks2;
  const int total = p.rows_a * p.chunks;  // the partials' LDS, sized by the host for rows_a rows
  const Job jb = accept_row<Tin, SM, THR>(p, b, c == 0, lds.acc, reinterpret_cast<float*>(dyn + total), dyn);
  const DrawRows d = draw_rows<THR>(p, b, jb);
  const Tin* P = static_cast<const Tin*>(p.tgt) + d.poff;
  const Tin* Q = static_cast<const Tin*>(p.dft) + d.qoff;
  if (jb.mode == 0)
    mass_chunk<Tin, SM, THR, W_RESID>(p, b, c, p.spc, P, Q, d, jb);
  else
    mass_chunk<Tin, SM, THR, W_P>(p, b, c, p.spc, P, Q, d, jb);
  if (!arrive_last(&p.cnt[b], (unsigned)p.chunks2, &last_flag)) return;
  draw_work<Tin, SM, THR>(p, b, jb, lds.draw, dyn);
}

struct SpecPlan {
  int chunks;
  int64_t len;
  int64_t nsb;
  int spc, chunks2;
};

// A: chunks per row for about kLseWgs workgroups (many short workgroups; the
// dispatcher balances them over the CUs).  B: chunks of whole sub-blocks,
// about kMassPerCu workgroups per CU.
constexpr int64_t kLseWgs = 16384;
constexpr int64_t kMassPerCu = 4;
// k = 0 (a plain draw from p_0) streams one row per batch row, not p_n and
// q_n: half the bytes per workgroup, so half the workgroups (32 rows of
// 248,320: a 10 us shorter config-5 round; the acceptance at B = 64, k = 8
// ran its launch B 8 us slower with 2 per CU)
constexpr int64_t kMassPerCuDraw = 2;

static SpecPlan spec_plan(int64_t B, int k, int64_t V, int dtype, int rows_a = -1) {
  const int ve = dtype == VNX_F32 ? 4 : 8;
  SpecPlan pl;
  if (rows_a < 0) rows_a = 2 * k + 1;
  const int64_t rows = B * rows_a;
  // chunks of at least kNB / 2 vectors per thread: few rows (a decode batch)
  // get fewer, longer workgroups instead of thousands of one-load ones.  A
  // k = 0 draw (one row per batch row) takes about two workgroups per CU:
  // at 32 rows of 248,320, 16 chunks per row gave a 20 us shorter config-5
  // round than 60 (and 8 or 4 chunks were slower again)
  // An acceptance (k > 0) takes chunks of at least one full batch (kNB
  // vectors per thread): at B = 32, k = 6 in bf16, 30 chunks of 4 vectors per
  // thread ran the 224-row LSE launch in 51 us, mostly per-workgroup cost.
  const int64_t wgs = k == 0 ? 2 * (int64_t)device_cus() : kLseWgs;
  int c = pick_chunks(rows, V, ve * (k == 0 ? kNB / 2 : kNB), std::min(kMaxChunks, kAccParts / rows_a), wgs);
  const int64_t len = ((V + c - 1) / c + ve - 1) / ve * ve;
  pl.len = len;
  pl.chunks = (int)((V + len - 1) / len);
  const int64_t sbl = (int64_t)VNX_WAVE * ve;
  pl.nsb = (V + sbl - 1) / sbl;
  int64_t c2 = ((int64_t)device_cus() * (k == 0 ? kMassPerCuDraw : kMassPerCu) + B - 1) / B;
  const int64_t max_c2 = (pl.nsb + kNW - 1) / kNW;  // at least one sub-block per wave
  if (c2 > max_c2) c2 = max_c2;
  if (c2 < 1) c2 = 1;
  pl.spc = (int)((pl.nsb + c2 - 1) / c2);
  pl.chunks2 = (int)((pl.nsb + pl.spc - 1) / pl.spc);
  return pl;
}

static size_t spec_carve(void* ws, int64_t B, int k, const SpecPlan& pl, SpecParams* p) {
  Carve cv(ws);
  const size_t n1 = (size_t)B * (2 * k + 1) * pl.chunks;
  float* pm = cv.take<float>(n1);
  double* ps = cv.take<double>(n1);
  double* sbm = cv.take<double>((size_t)B * pl.nsb);
  unsigned* cnt = cv.take<unsigned>((size_t)B);
  float* gath = cv.take<float>((size_t)B * 2 * k);
  if (p) {
    p->part_m = pm; p->part_s = ps; p->sbm = sbm; p->cnt = cnt; p->gath = gath;
  }
  return cv.bytes();
}

// Workspace bound over both dtypes, with and without caller-supplied draft
// LSEs (whose plan may cut the rows into more chunks).
static size_t spec_ws_bytes(int64_t B, int k, int64_t V) {
  size_t m = 0;
  for (int dt : {VNX_F32, VNX_BF16})
    for (int ra : {2 * k + 1, k + 1}) m = std::max(m, spec_carve(nullptr, B, k, spec_plan(B, k, V, dt, ra), nullptr));
  return m;
}

// Commit of one speculative round for every sequence (one workgroup, one
// thread per sequence): the accepted drafts and the drawn / bonus token
// ids[b, 0 .. n_b] go to out[b, count_b ...] (positions at or past n_cap are
// dropped), count, lens_t and lens_d advance by n_b + 1 (the rejected suffix
// of both caches is rolled back by not advancing), c[b] = ids[b, n_b], and
// info = (min count, max lens_t, max lens_d, sum n_b) for the host's loop.
constexpr int kCommitMaxB = 1024;

__global__ __launch_bounds__(kCommitMaxB) void k_spec_commit(const int32_t* alen, const int64_t* ids, int64_t ldi,
                                                             int B, int k, int64_t* out, int64_t ldo, int64_t n_cap,
                                                             int64_t* count, int64_t* c, int32_t* lens_t,
                                                             int32_t* lens_d, int64_t* info) {
  __shared__ int64_t red[4][kCommitMaxB / VNX_WAVE];
  const int b = threadIdx.x;
  int64_t cnt = INT64_MAX, lt = INT64_MIN, ld_ = INT64_MIN, acc = 0;
  if (b < B) {
    const int n = min(max(alen[b], 0), k);  // accepted drafts
    const int64_t c0 = count[b];
    for (int j = 0; j <= n; ++j) {
      const int64_t pos = c0 + j;
      if (pos < n_cap) out[b * ldo + pos] = ids[b * ldi + j];
    }
    cnt = c0 + n + 1;
    count[b] = cnt;
    c[b] = ids[b * ldi + n];
    lt = lens_t[b] + n + 1;
    ld_ = lens_d[b] + n + 1;
    lens_t[b] = (int32_t)lt;
    lens_d[b] = (int32_t)ld_;
    acc = n;
  }
  // workgroup min / max / max / sum (fixed order)
  for (int o = 32; o > 0; o >>= 1) {
    cnt = min(cnt, (int64_t)__shfl_xor(cnt, o));
    lt = max(lt, (int64_t)__shfl_xor(lt, o));
    ld_ = max(ld_, (int64_t)__shfl_xor(ld_, o));
    acc += (int64_t)__shfl_xor(acc, o);
  }
  const int w = b / VNX_WAVE;
  if ((b % VNX_WAVE) == 0) {
    red[0][w] = cnt;
    red[1][w] = lt;
    red[2][w] = ld_;
    red[3][w] = acc;
  }
  __syncthreads();
  if (b == 0) {
    const int nw = (int)((blockDim.x + VNX_WAVE - 1) / VNX_WAVE);
    int64_t r0 = red[0][0], r1 = red[1][0], r2 = red[2][0], r3 = red[3][0];
    for (int i = 1; i < nw; ++i) {
      r0 = min(r0, red[0][i]);
      r1 = max(r1, red[1][i]);
      r2 = max(r2, red[2][i]);
      r3 += red[3][i];
    }
    info[0] = r0;
    info[1] = r1;
    info[2] = r2;
    info[3] = r3;
  }
}

// ---------------------------------------------------------------------------
// Fixed scratch of vnx_spec_accept_noalloc (callers that cannot allocate):
// one copy of `scratch` per GPU, held until the process ends.  Host code
// never passes the array's name to a kernel (on the host it is a stand-in,
// not a device address): spec_scratch_init() resolves each device's own
// address once, with that device current, and kernels receive that pointer.
// ---------------------------------------------------------------------------
constexpr size_t kSpecScratchBytes = size_t(8) << 20;
static __device__ __align__(256) unsigned char scratch[kSpecScratchBytes];

constexpr int kMaxScratchDevices = 64;
static void* g_scratch_ptr[kMaxScratchDevices];
static std::mutex g_scratch_mu;

int spec_scratch_init(int device) {
  if (device < 0 || device >= kMaxScratchDevices) return VNX_ERR_NO_DEVICE;
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (g_scratch_ptr[device]) return VNX_OK;
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return hip_fail(e);
  if (!ptr) return VNX_ERR_HIP;
  g_scratch_ptr[device] = ptr;
  return VNX_OK;
}

}  // namespace vnx

using namespace vnx;

extern "C" {

size_t vnx_spec_accept_workspace(int64_t B, int k, int64_t V) {
  if (B <= 0 || k <= 0 || V <= 0) return 256;
  return spec_ws_bytes(B, k, V);
}

// The two launches for k >= 0 draft positions (k = 0: the draw from p_0
// alone, which is sampling from softmax(target / T)).
static int spec_run(const void* target, const void* draft, int dtype, int64_t B, int k, int64_t V,
                    int64_t ld_t, int64_t sb_t, int64_t ld_d, int64_t sb_d,
                    const int64_t* draft_ids, const float* uniforms,
                    float temperature, const float* thr_t, const float* thr_d, int32_t* accept_len,
                    int64_t* out_ids, uint8_t* flags, float* lse_t, float* lse_d, void* workspace,
                    size_t workspace_bytes, void* stream, const float* lse_din = nullptr,
                    const uint8_t* fl_din = nullptr, int64_t ld_din = 0) {
  if (dtype != VNX_F32 && dtype != VNX_BF16) return VNX_ERR_UNSUPPORTED;
  if (B < 0 || k < 0 || k > kMaxK || V <= 0) return VNX_ERR_INVALID_ARG;
  if (!(temperature > 0.0f) || !__builtin_isfinite(temperature)) return VNX_ERR_INVALID_ARG;
  if (B == 0) return VNX_OK;
  if (B > (1 << 20)) return VNX_ERR_UNSUPPORTED;
  int st = check_rows(target, dtype, ld_t, sb_t, k + 1, V);
  if (st) return st;
  if (k > 0) {
    st = check_rows(draft, dtype, ld_d, sb_d, k, V);
    if (st) return st;
    if (!draft_ids) return VNX_ERR_INVALID_ARG;
  }
  if (!uniforms || !accept_len || !out_ids) return VNX_ERR_INVALID_ARG;
  const int rows_a = lse_din ? k + 1 : 2 * k + 1;
  const SpecPlan pl = spec_plan(B, k, V, dtype, rows_a);
  if (B * rows_a * (int64_t)pl.chunks >= INT32_MAX || B * (int64_t)pl.chunks2 >= INT32_MAX ||
      pl.nsb > kDrawLds || rows_a * pl.chunks > kAccParts)
    return VNX_ERR_UNSUPPORTED;
  // (the partials are carved for 2k + 1 rows of this plan's chunks: enough)
  if (!workspace || workspace_bytes < spec_carve(nullptr, B, k, pl, nullptr)) return VNX_ERR_WORKSPACE;
  SpecParams p{};
  p.tgt = target; p.dft = draft; p.B = B; p.k = k; p.V = V;
  p.ld_t = ld_t; p.ld_d = ld_d; p.sb_t = sb_t; p.sb_d = sb_d;
  p.chunks = pl.chunks; p.chunk_len = pl.len; p.nsb = pl.nsb; p.spc = pl.spc; p.chunks2 = pl.chunks2;
  const int sm = make_scale(temperature, &p.sc);
  p.thr_t = thr_t; p.thr_d = thr_d; p.ids = draft_ids; p.u = uniforms;
  p.accept_len = accept_len; p.out_ids = out_ids; p.flags = flags; p.lse_t = lse_t; p.lse_d = lse_d;
  p.lse_din = lse_din; p.fl_din = fl_din; p.ld_din = ld_din; p.rows_a = rows_a;
  spec_carve(workspace, B, k, pl, &p);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t na = B * rows_a * pl.chunks;
  const dim3 ga((unsigned)std::max<int64_t>(na, (B + kNT - 1) / kNT)), gb((unsigned)(B * pl.chunks2));
  const size_t lds_b = std::max((size_t)pl.nsb * sizeof(double), (size_t)rows_a * pl.chunks * 12);
  hipEvent_t* ev = profile_slot(2);
  auto mark = [&](int j) -> int {
    if (ev) VNX_HIP_CHECK(hipEventRecord(ev[j], s));
    return VNX_OK;
  };
  return dispatch_tsm(dtype, sm, thr_t || thr_d, [&](auto tin, auto smc, auto thrc) {
    using Tin = decltype(tin);
    constexpr int SM = decltype(smc)::value;
    constexpr bool THR = decltype(thrc)::value;
    int e = mark(0);
    if (e) return e;
    hipLaunchKernelGGL((k_spec_lse<Tin, SM, THR>), ga, dim3(kNT), 0, s, p);
    VNX_LAUNCH_CHECK();
    if ((e = mark(1))) return e;
    hipLaunchKernelGGL((k_spec_mass_draw<Tin, SM, THR>), gb, dim3(kNT), lds_b, s, p);
    VNX_LAUNCH_CHECK();
    return mark(2);
  });
}

int vnx_spec_accept(const void* target, const void* draft, int dtype, int64_t B, int k, int64_t V,
                    int64_t ld_t, int64_t sb_t, int64_t ld_d, int64_t sb_d,
                    const int64_t* draft_ids, const float* uniforms,
                    float temperature, const float* thr_t, const float* thr_d, int32_t* accept_len,
                    int64_t* out_ids, uint8_t* flags, float* lse_t, float* lse_d, void* workspace,
                    size_t workspace_bytes, void* stream) {
  if (k < 1) return VNX_ERR_INVALID_ARG;
  return spec_run(target, draft, dtype, B, k, V, ld_t, sb_t, ld_d, sb_d, draft_ids, uniforms, temperature,
                  thr_t, thr_d, accept_len, out_ids, flags, lse_t, lse_d, workspace, workspace_bytes, stream);
}

int vnx_spec_accept_draft_lse(const void* target, const void* draft, int dtype, int64_t B, int k, int64_t V,
                              int64_t ld_t, int64_t sb_t, int64_t ld_d, int64_t sb_d,
                              const int64_t* draft_ids, const float* uniforms, float temperature,
                              const float* lse_d_in, const uint8_t* flags_d_in, int64_t ld_in,
                              int32_t* accept_len, int64_t* out_ids, uint8_t* flags, float* lse_t, void* workspace,
                              size_t workspace_bytes, void* stream) {
  if (k < 1 || !lse_d_in || ld_in < B) return VNX_ERR_INVALID_ARG;
  return spec_run(target, draft, dtype, B, k, V, ld_t, sb_t, ld_d, sb_d, draft_ids, uniforms, temperature,
                  nullptr, nullptr, accept_len, out_ids, flags, lse_t, nullptr, workspace, workspace_bytes, stream,
                  lse_d_in, flags_d_in, ld_in);
}

size_t vnx_spec_accept_noalloc_max_bytes(void) { return kSpecScratchBytes; }

int vnx_spec_accept_noalloc(const void* target, const void* draft, int dtype, int64_t B, int k, int64_t V,
                            int64_t ld_t, int64_t sb_t, int64_t ld_d, int64_t sb_d,
                            const int64_t* draft_ids, const float* uniforms,
                            float temperature, const float* thr_t, const float* thr_d, int32_t* accept_len,
                            int64_t* out_ids, uint8_t* flags, float* lse_t, float* lse_d, void* stream) {
  if (k < 1) return VNX_ERR_INVALID_ARG;
  if (B < 0 || k > kMaxK || V <= 0) return VNX_ERR_INVALID_ARG;
  if (B > 0 && spec_ws_bytes(B, k, V) > kSpecScratchBytes) return VNX_ERR_TOO_LARGE;
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e);
  const int st = spec_scratch_init(dev);  // a no-op after the first call on this device
  if (st) return st;
  return spec_run(target, draft, dtype, B, k, V, ld_t, sb_t, ld_d, sb_d, draft_ids, uniforms, temperature,
                  thr_t, thr_d, accept_len, out_ids, flags, lse_t, lse_d, g_scratch_ptr[dev], kSpecScratchBytes,
                  stream);
}

size_t vnx_sample_workspace(int64_t B, int64_t V) {
  if (B <= 0 || V <= 0) return 256;
  return spec_ws_bytes(B, 0, V) + (((size_t)B * 4 + 255) & ~(size_t)255);
}

int vnx_sample(const void* logits, int dtype, int64_t B, int64_t V, int64_t ld, const float* uniforms,
               float temperature, const float* thresholds, int64_t* out_ids, uint8_t* flags, float* lse,
               void* workspace, size_t workspace_bytes, void* stream) {
  if (B < 0 || V <= 0) return VNX_ERR_INVALID_ARG;
  if (B == 0) return VNX_OK;
  const size_t need = vnx_sample_workspace(B, V);
  if (!workspace || workspace_bytes < need) return VNX_ERR_WORKSPACE;
  // accept_len (always 0 here) lives at the end of the workspace.
  const size_t head = need - (((size_t)B * 4 + 255) & ~(size_t)255);
  int32_t* alen = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + head);
  return spec_run(logits, logits, dtype, B, 0, V, ld, ld, ld, ld, nullptr, uniforms, temperature, thresholds,
                  nullptr, alen, out_ids, flags, lse, nullptr, workspace, head, stream);
}

int vnx_spec_commit(const int32_t* accept_len, const int64_t* out_ids, int64_t ld_ids, int B, int k, int64_t* out,
                    int64_t ld_out, int64_t n_cap, int64_t* count, int64_t* c, int32_t* lens_t, int32_t* lens_d,
                    int64_t* info, void* stream) {
  if (!accept_len || !out_ids || !out || !count || !c || !lens_t || !lens_d || !info) return VNX_ERR_INVALID_ARG;
  if (B < 0 || k < 0 || ld_ids < k + 1 || n_cap < 0 || ld_out < n_cap) return VNX_ERR_INVALID_ARG;
  if (B > kCommitMaxB) return VNX_ERR_UNSUPPORTED;
  if (B == 0) return VNX_OK;
  const unsigned threads = (unsigned)((B + VNX_WAVE - 1) / VNX_WAVE * VNX_WAVE);
  hipLaunchKernelGGL(k_spec_commit, dim3(1), dim3(threads), 0, static_cast<hipStream_t>(stream), accept_len,
                     out_ids, ld_ids, B, k, out, ld_out, n_cap, count, c, lens_t, lens_d, info);
  VNX_LAUNCH_CHECK();
  return VNX_OK;
}

}  // extern "C"
