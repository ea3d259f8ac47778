/*
 * CPU checker for the vnx kernels — TEST INFRASTRUCTURE ONLY.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker, never as the measured path.
 *
 * Restates, in plain C with IEEE-754 fp32/fp64 arithmetic, the arithmetic the
 * kernels are specified to perform:
 *   - RN(l / T) temperature scaling: numpy's float32 `logits / temperature`
 *     (packages/verse_infra/verse_infra/verse_inference/sampler.py:95);
 *   - the canonical exp (Cody-Waite reduction by ln2, degree-7 Taylor, fp32,
 *     every step one rounded IEEE operation) used for probabilities that
 *     feed discrete decisions;
 *   - the inverse-CDF draw j* = min{j : C_j > u * C_V} over a sequential fp64
 *     cumulative sum, which is numpy's Generator.choice(p=...) rule
 *     (searchsorted(cdf / cdf[-1], u, side="right"), sampler.py:135-137)
 *     with the normalisation folded into the target.
 * Build: see oracle/Makefile (gcc -ffp-contract=off, no fast-math).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

float vnx_ref_exp_canon(float t) {
  const float kLog2e = 0x1.715476p+0f;
  const float kLn2Hi = 0x1.62e430p-1f;
  const float kLn2Lo = -0x1.05c610p-29f;
  const float c7 = 0x1.a01a02p-13f;
  const float c6 = 0x1.6c16c2p-10f;
  const float c5 = 0x1.111112p-7f;
  const float c4 = 0x1.555556p-5f;
  const float c3 = 0x1.555556p-3f;
  const float c2 = 0x1p-1f;
  if (!(t >= -86.5f)) return 0.0f;
  if (t > 88.0f) t = 88.0f;
  float kf = rintf(t * kLog2e);
  float r = fmaf(-kf, kLn2Hi, t);
  r = fmaf(-kf, kLn2Lo, r);
  float p = c7;
  p = fmaf(p, r, c6);
  p = fmaf(p, r, c5);
  p = fmaf(p, r, c4);
  p = fmaf(p, r, c3);
  p = fmaf(p, r, c2);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int k = (int)kf;
  uint32_t bits = (uint32_t)(k + 127) << 23;
  float two_k;
  memcpy(&two_k, &bits, 4);
  return p * two_k;
}

void vnx_ref_exp_canon_arr(const float* t, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = vnx_ref_exp_canon(t[i]);
}

/* RN(l / T) for T != 1; identity for T == 1; -inf below thr. */
static inline float scale_mask(float l, float T, float thr) {
  float a = (T == 1.0f) ? l : l / T;
  return (a < thr) ? -INFINITY : a;
}

/* Markstein one-step division q1 = RN(q0 + r*y), q0 = RN(l*y), r = l - q0*T,
 * y = RN(1/T): the kernels' fast path, compared against l / T by the tests. */
float vnx_ref_div_markstein(float l, float T) {
  float y = 1.0f / T;
  float q0 = l * y;
  float r = fmaf(-q0, T, l);
  float q1 = fmaf(r, y, q0);
  return isfinite(q0) ? q1 : q0;
}

/* Number of significands of a in [1,2) where the Markstein step differs from
 * a / T (0 means the fast path is exact for this T). */
int64_t vnx_ref_markstein_mismatches(float T) {
  int64_t bad = 0;
  for (uint32_t m = 0; m < (1u << 23); ++m) {
    uint32_t bits = (127u << 23) | m;
    float a;
    memcpy(&a, &bits, 4);
    if (vnx_ref_div_markstein(a, T) != a / T) ++bad;
  }
  return bad;
}

/* Residual / bonus weights of one row pair, exactly as the kernels form them:
 * w_p[j] = E(a_j - Lp), w_r[j] = max(0, w_p[j] - E(b_j - Lq)) (Q != NULL) or
 * w_p[j] (Q == NULL). */
void vnx_ref_resid_weights(const float* P, const float* Q, int64_t V, float T, float thr_p,
                           float thr_q, float Lp, float Lq, float* w_r, float* w_p) {
  for (int64_t j = 0; j < V; ++j) {
    float pp = vnx_ref_exp_canon(scale_mask(P[j], T, thr_p) - Lp);
    if (w_p) w_p[j] = pp;
    if (Q) {
      float d = pp - vnx_ref_exp_canon(scale_mask(Q[j], T, thr_q) - Lq);
      w_r[j] = d > 0.0f ? d : 0.0f;
    } else {
      w_r[j] = pp;
    }
  }
}

/* Inverse-CDF draw over weights w (length V): the first j with
 * C_j > u * C_{V-1}, C sequential fp64 partial sums; returns -1 if the total
 * is zero.  before/after receive C_{j-1}, C_j; total the full sum. */
int64_t vnx_ref_icdf(const float* w, int64_t V, double u, double* before, double* after,
                     double* total) {
  double tot = 0.0;
  for (int64_t j = 0; j < V; ++j) tot += (double)w[j];
  if (total) *total = tot;
  if (!(tot > 0.0)) return -1;
  const double target = u * tot;
  double run = 0.0;
  int64_t last = -1;
  for (int64_t j = 0; j < V; ++j) {
    if (w[j] > 0.0f) {
      double nr = run + (double)w[j];
      if (nr > target) {
        if (before) *before = run;
        if (after) *after = nr;
        return j;
      }
      run = nr;
      last = j;
    }
  }
  if (before) *before = run;
  if (after) *after = run;
  return last;
}
