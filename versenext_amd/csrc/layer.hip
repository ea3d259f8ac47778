// Per-layer elementwise work of the CometSpark forward, fused so that a
// verify or draft step launches a handful of kernels per layer instead of
// dozens of small PyTorch ones:
//   vnx_rmsnorm   x += r (optional residual), y = x / sqrt(mean(x^2) + eps) * w
//                 (RMSNorm, packages/verse_torch/verse_torch/vnnn.py:593-615;
//                 the residual adds of VerseNexBlock.forward, cometspark.py:236-247);
//   vnx_rope_kv   RoPE of q and k at each sequence's positions lens[b] + i
//                 (TriSparseAttention._apply_rope, tri_sparse_attn.py:182-221),
//                 q to the attention layout, k / v written into the KV cache;
//   vnx_swiglu    silu(g) * u of the fused gate|up product (SwiGLUMLP,
//                 vnnn.py:779-807);
//   vnx_axpby     c0 * a + c1 * b with device coefficients (the sigmoid-gated
//                 sum of the TriSparse paths, tri_sparse_attn.py:585-608);
//   vnx_mod_route / vnx_mod_swiglu  MoD routing weights and the weighted
//                 expert activations (mod.py:142-213, :337-440, :779-803).
// Activations are fp32, bf16 or fp16 (dtype codes of vnx.h); every kernel
// reads its inputs once and writes its outputs once.
#include "vnx_internal.h"

namespace vnx {
namespace {

template <typename T>
struct Elt;
template <>
struct Elt<float> {
  __device__ __forceinline__ static float ld(const float* p) { return *p; }
  __device__ __forceinline__ static void st(float* p, float v) { *p = v; }
};
template <>
struct Elt<__hip_bfloat16> {
  __device__ __forceinline__ static float ld(const __hip_bfloat16* p) {
    return __uint_as_float((uint32_t)(*reinterpret_cast<const uint16_t*>(p)) << 16);
  }
  __device__ __forceinline__ static void st(__hip_bfloat16* p, float v) {
    const uint32_t u = __float_as_uint(v);
    uint16_t b;
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) b = (uint16_t)((u >> 16) | 0x40u);
    else b = (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);  // round to nearest even
    *reinterpret_cast<uint16_t*>(p) = b;
  }
};
template <>
struct Elt<_Float16> {
  __device__ __forceinline__ static float ld(const _Float16* p) { return (float)*p; }
  __device__ __forceinline__ static void st(_Float16* p, float v) { *p = (_Float16)v; }
};

// Four consecutive elements as fp32 (16-byte loads for fp32, 8-byte for the
// 16-bit types; the caller checks the alignment).
template <typename T>
__device__ __forceinline__ void ld4(const T* p, float (&v)[4]) {
  if constexpr (sizeof(T) == 4) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  } else {
    const uint2 a = *reinterpret_cast<const uint2*>(p);
    const T* e = reinterpret_cast<const T*>(&a);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = Elt<T>::ld(e + i);
  }
}
template <typename T>
__device__ __forceinline__ void st4(T* p, const float (&v)[4]) {
  if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    uint2 a;
    T* e = reinterpret_cast<T*>(&a);
#pragma unroll
    for (int i = 0; i < 4; ++i) Elt<T>::st(e + i, v[i]);
    *reinterpret_cast<uint2*>(p) = a;
  }
}

// The 4-wide kernels need every row start at a multiple of 4 elements.
inline bool vec4_ok(const void* p, int elt_bytes) {
  return (reinterpret_cast<uintptr_t>(p) % (4u * (unsigned)elt_bytes)) == 0;
}
inline int dtype_bytes(int dt) { return dt == VNX_F32 ? 4 : 2; }

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

template <typename F>
int by_dtype(int dt, F&& f) {
  switch (dt) {
    case VNX_F32: return f(float{});
    case VNX_BF16: return f(__hip_bfloat16{});
    case VNX_F16: return f(_Float16{});
    default: return (int)VNX_ERR_UNSUPPORTED;
  }
}

// ---------------------------------------------------------------------------
// RMSNorm: one workgroup per row, the row held in registers (D <= 16 * 256).
// ---------------------------------------------------------------------------
constexpr int kRnThreads = 256;
constexpr int kRnPer = 16;

template <typename TY>
__device__ __forceinline__ void rms_tail(const float (&v)[kRnPer], const float (&wv)[kRnPer], float ss,
                                         float* red, float eps, int64_t D, int64_t row, float* xo, int64_t ldxo,
                                         TY* y, int64_t ldy);

template <typename TR, typename TY>
__global__ __launch_bounds__(kRnThreads) void k_rmsnorm(const float* x, int64_t ldx, const TR* r, int64_t ldr,
                                                        const float* w, float eps, int64_t D, float* xo,
                                                        int64_t ldxo, TY* y, int64_t ldy) {
  __shared__ float red[kRnThreads / VNX_WAVE];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  float v[kRnPer], wv[kRnPer], rv[kRnPer];
  float ss = 0.0f;
  // Every load (x, residual, weight) is issued before any value is used, with
  // no per-lane condition between them (columns past D re-read column D - 1
  // and count as 0 below): a use or a select beside a conditional load would
  // wait there for every load in flight.  nb (wave-uniform) bounds the blocks.
  const int nb = (int)min((int64_t)kRnPer, (D + kRnThreads - 1) / kRnThreads);
#pragma unroll
  for (int j = 0; j < kRnPer; ++j) {
    if (j < nb) {
      const int64_t c = min((int64_t)(tid + j * kRnThreads), D - 1);
      v[j] = x[row * ldx + c];
      wv[j] = w[c];
      if (r) rv[j] = Elt<TR>::ld(r + row * ldr + c);
    }
  }
#pragma unroll
  for (int j = 0; j < kRnPer; ++j) {
    const bool in = j < nb && tid + j * kRnThreads < D;
    float a = 0.0f;
    if (j < nb) {
      a = v[j];
      if (r) a += rv[j];
      a = in ? a : 0.0f;
      wv[j] = in ? wv[j] : 0.0f;
    }
    v[j] = a;
    ss = __builtin_fmaf(a, a, ss);
  }
  rms_tail<TY>(v, wv, ss, red, eps, D, row, xo, ldxo, y, ldy);
}

// x_out[row] = x (the residual stream), y[row] = x / sqrt(mean(x^2) + eps) * w
// from a workgroup's values v (kRnPer per thread, column tid + j*256) and
// their per-thread sum of squares ss.
template <typename TY>
__device__ __forceinline__ void rms_tail(const float (&v)[kRnPer], const float (&wv)[kRnPer], float ss,
                                         float* red, float eps, int64_t D, int64_t row, float* xo, int64_t ldxo,
                                         TY* y, int64_t ldy) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, VNX_WAVE);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int i = 0; i < kRnThreads / VNX_WAVE; ++i) tot += red[i];
  const float inv = 1.0f / __builtin_sqrtf(tot / (float)D + eps);
#pragma unroll
  for (int j = 0; j < kRnPer; ++j) {
    const int c = tid + j * kRnThreads;
    if (c < D) {
      if (xo) xo[row * ldxo + c] = v[j];
      Elt<TY>::st(y + row * ldy + c, v[j] * inv * wv[j]);
    }
  }
}

// The first layer's norm with the embedding lookup folded in: x[row] =
// emb[tokens[row]] * scale (fp32), written to x_out as the residual stream.
template <typename TE, typename TY>
__global__ __launch_bounds__(kRnThreads) void k_embed_rmsnorm(const int64_t* tokens, const TE* emb, int64_t lde,
                                                              int64_t vocab, float scale, const float* w, float eps,
                                                              int64_t D, float* xo, int64_t ldxo, TY* y,
                                                              int64_t ldy) {
  __shared__ float red[kRnThreads / VNX_WAVE];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  int64_t tok = tokens[row];
  tok = tok < 0 ? 0 : (tok >= vocab ? vocab - 1 : tok);  // never outside the table
  const TE* e = emb + tok * lde;
  float v[kRnPer], wv[kRnPer];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < kRnPer; ++j) {
    const int c = tid + j * kRnThreads;
    float a = 0.0f;
    wv[j] = 0.0f;
    if (c < D) {
      a = Elt<TE>::ld(e + c) * scale;
      wv[j] = w[c];
    }
    v[j] = a;
    ss = __builtin_fmaf(a, a, ss);
  }
  rms_tail<TY>(v, wv, ss, red, eps, D, row, xo, ldxo, y, ldy);
}

// ---------------------------------------------------------------------------
// RoPE + KV-cache write.  qkv rows (b, i) hold [q heads | k heads | v heads]
// of head_dim d; position p = lens[b] + i.  One thread per (row, head, pair
// (j, j + d/2)) of the rotate-half form x*cos + rotate_half(x)*sin.
// ---------------------------------------------------------------------------
struct RopeParams {
  const void* qkv;
  int64_t ldq;
  int64_t B;
  int n, H, Hkv, d;
  const int32_t* lens;
  const float* cos;
  const float* sin;
  int rope;
  void* q;                  // (B, H, n, d) contiguous, cache dtype
  void* kc;
  void* vc;
  int64_t c_sb, c_sh, c_sr;  // cache strides (elements)
  int64_t cap;               // rows of the cache (and at most the table length)
};

template <typename TQ, typename TO>
__global__ __launch_bounds__(256) void k_rope_kv(RopeParams p) {
  // one workgroup per token row (b, i); threads over (head, pair j)
  const int half = p.d / 2;
  const int heads = p.H + 2 * p.Hkv;
  const int64_t row = blockIdx.x;
  const int64_t b = row / p.n;
  const int i = (int)(row - b * p.n);
  const int64_t pos = (int64_t)p.lens[b] + i;
  if (pos < 0 || pos >= p.cap) return;  // never past the cache or the RoPE table
  const TQ* src_row = static_cast<const TQ*>(p.qkv) + row * p.ldq;
  for (int t = threadIdx.x; t < heads * half; t += blockDim.x) {
    const int hh = t / half, j = t - hh * half;
    const TQ* src = src_row + (int64_t)hh * p.d;
    float x0 = Elt<TQ>::ld(src + j), x1 = Elt<TQ>::ld(src + j + half);
    if (p.rope && hh < p.H + p.Hkv) {
      const float c0 = p.cos[pos * p.d + j], c1 = p.cos[pos * p.d + j + half];
      const float s0 = p.sin[pos * p.d + j], s1 = p.sin[pos * p.d + j + half];
      const float y0 = x0 * c0 - x1 * s0;   // rotate_half(x)[j] = -x[j + half]
      const float y1 = x1 * c1 + x0 * s1;   // rotate_half(x)[j + half] = x[j]
      x0 = y0;
      x1 = y1;
    }
    TO* dst;
    if (hh < p.H) {
      dst = static_cast<TO*>(p.q) + ((b * p.H + hh) * p.n + i) * (int64_t)p.d;
    } else if (hh < p.H + p.Hkv) {
      dst = static_cast<TO*>(p.kc) + b * p.c_sb + (int64_t)(hh - p.H) * p.c_sh + pos * p.c_sr;
    } else {
      dst = static_cast<TO*>(p.vc) + b * p.c_sb + (int64_t)(hh - p.H - p.Hkv) * p.c_sh + pos * p.c_sr;
    }
    Elt<TO>::st(dst + j, x0);
    Elt<TO>::st(dst + j + half, x1);
  }
}

// ---------------------------------------------------------------------------
// SwiGLU activation: out[m, c] = silu(gu[m, c]) * gu[m, Hf + c].
// ---------------------------------------------------------------------------
// Grid: x = rows, y = column blocks of 256 * VW; VW = 4 reads and writes 4
// consecutive columns per thread.
template <typename TI, typename TO, int VW>
__global__ __launch_bounds__(256) void k_swiglu(const TI* gu, int64_t ldg, int64_t Hf, TO* out, int64_t ldo) {
  const int64_t m = blockIdx.x;
  const int64_t c = ((int64_t)blockIdx.y * 256 + threadIdx.x) * VW;
  if (c >= Hf) return;
  const TI* g = gu + m * ldg + c;
  TO* o = out + m * ldo + c;
  if constexpr (VW == 4) {
    float a[4], u[4], r[4];
    ld4(g, a);
    ld4(g + Hf, u);
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = silu(a[e]) * u[e];
    st4(o, r);
  } else {
    Elt<TO>::st(o, silu(Elt<TI>::ld(g)) * Elt<TI>::ld(g + Hf));
  }
}

// out = coef[0] * a + coef[1] * b (coef on the device, so captured graphs
// keep reading the current gate values).
template <typename TO>
__global__ __launch_bounds__(256) void k_axpby(const float* a, const float* b, const float* coef, int64_t n,
                                               TO* out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n) return;
  Elt<TO>::st(out + t, coef[0] * a[t] + coef[1] * b[t]);
}

// ---------------------------------------------------------------------------
// MoD routing (Router.forward, packages/verse_nex/verse_nex/mod.py:337-440,
// MoDLayer.forward :779-803): per row, the part weights are the softmax of
// the P part-router logits (top_k = P, all parts); inside part p the top-k
// of its E expert logits (larger first, ties to the lower index) are weighted
// by the softmax over the selected logits.  comb[m, p*E + e] = part weight x
// expert weight, 0 for unselected experts.  One wave per row.
// ---------------------------------------------------------------------------
constexpr int kModMaxP = 8;
constexpr int kModMaxE = 16;

// One row's routing weights, computed by one wave: lane j < P + P*E holds
// logit j (the P part logits, then the E expert logits of each part).  Part
// weights are the softmax of the part logits; inside part p, lane j's rank
// is the number of its segment's logits that beat it (larger, or equal at a
// lower index), it is selected when rank < topk, and the selected logits are
// re-softmaxed with the sum taken in rank order (largest first).  Lane
// P + p*E + e writes c[p*E + e].  All exchanges are wave shuffles.
__device__ void route_wave(float lj, int P, int E, int topk, float* c) {
  const int lane = threadIdx.x & 63;
  const int R = P + P * E;
  // part softmax
  float mx = -__builtin_inff();
  for (int q = 0; q < P; ++q) mx = fmaxf(mx, __shfl(lj, q));
  float sp = 0.0f;
  for (int q = 0; q < P; ++q) sp += expf(__shfl(lj, q) - mx);
  // this lane's part (every lane shuffles here, before the part lanes leave)
  const int pl = lane >= P && lane < R ? (lane - P) / E : 0;
  const float pw = expf(__shfl(lj, pl) - mx) / sp;
  if (lane < P || lane >= R) return;  // (no shuffle below reads these lanes)
  const int p = pl, e = lane - P - p * E, base = P + p * E;
  // rank inside the segment, and the segment's largest logit
  int rank = 0;
  float ms = -__builtin_inff();
  for (int e2 = 0; e2 < E; ++e2) {
    const float v = __shfl(lj, base + e2);
    rank += (v > lj || (v == lj && e2 < e)) ? 1 : 0;
    ms = fmaxf(ms, v);
  }
  // sum of the selected terms in rank order
  float ss = 0.0f;
  for (int i = 0; i < topk; ++i) {
    float vi = 0.0f;
    for (int e2 = 0; e2 < E; ++e2) {
      const float v = __shfl(lj, base + e2);
      int r2 = 0;
      for (int e3 = 0; e3 < E; ++e3) {
        const float w = __shfl(lj, base + e3);
        r2 += (w > v || (w == v && e3 < e2)) ? 1 : 0;
      }
      if (r2 == i) vi = v;
    }
    ss += expf(vi - ms);
  }
  c[p * E + e] = rank < topk ? pw * (expf(lj - ms) / ss) : 0.0f;
}

__global__ __launch_bounds__(64) void k_mod_route(const float* logits, int64_t ld, int64_t M, int P, int E,
                                                  int topk, float* comb, int64_t ldc) {
  // one wave per row
  const int64_t m = blockIdx.x;
  const int lane = threadIdx.x;
  const int R = P + P * E;
  const float lj = lane < R ? logits[m * ld + lane] : 0.0f;
  route_wave(lj, P, E, topk, comb + m * ldc);
}

// The router products folded in: one workgroup per row computes its
// R = P + P*E logits (fp32 dot products: per-thread partial sums over
// columns tid, tid + 256, ..., then the wave and workgroup sums in a fixed
// order) and routes them.
constexpr int kRouteMaxR = 32;

template <int VW, int RM>
__global__ __launch_bounds__(256) void k_mod_route_x(const float* h, int64_t ldh, const float* nw, float eps,
                                                     const float* wr, int64_t ldw, int64_t D, int P, int E, int topk,
                                                     float* comb, int64_t ldc, __hip_bfloat16* xo, int64_t ldxo,
                                                     int64_t sxo, int copies) {
  __shared__ float red[4][RM];
  __shared__ float lg[RM];
  __shared__ float ssr[4];
  const int64_t m = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int R = P + P * E;
  float acc[RM];
#pragma unroll
  for (int r = 0; r < RM; ++r) acc[r] = 0.0f;
  float ss = 0.0f;  // nw: sum of squares of the raw row
  // A row of at most 256 * VW columns (one block per thread) stays in
  // registers for the experts' bf16 copies below.
  const bool one_block = D <= 256 * VW;
  float x1[VW], w1[VW];
  // thread tid takes columns tid*VW .. +VW of every 256*VW block
  for (int64_t c = (int64_t)tid * VW; c < D; c += 256 * VW) {
    // every row's load issued unconditionally (rows past R re-read row R-1
    // and are not accumulated): no branches between the loads
    // every load of the block first (row, norm weight, router rows), the
    // math after them: a use beside a load would wait there for all loads
    float x[VW], w[VW];
    if constexpr (VW == 4) {
      ld4(h + m * ldh + c, x);
    } else {
      x[0] = h[m * ldh + c];
    }
    if (nw) {
      if constexpr (VW == 4) ld4(nw + c, w);
      else w[0] = nw[c];
    }
    float wv[RM][VW];
#pragma unroll
    for (int r = 0; r < RM; ++r) {
      const float* wrow = wr + (int64_t)(r < R ? r : R - 1) * ldw + c;
      if constexpr (VW == 4) ld4(wrow, wv[r]);
      else wv[r][0] = wrow[0];
    }
    if (nw) {
      // RMSNorm input: the products use x * w; the per-row factor is applied
      // to the reduced logits
#pragma unroll
      for (int e = 0; e < VW; ++e) {
        x1[e] = x[e];
        w1[e] = w[e];
        ss = __builtin_fmaf(x[e], x[e], ss);
        x[e] *= w[e];
      }
    } else if (xo) {  // the experts' bf16 input rows, one copy per expert batch
      __hip_bfloat16* dst = xo + m * ldxo + c;
      for (int q = 0; q < copies; ++q) {
        if constexpr (VW == 4) st4(dst + q * sxo, x);
        else Elt<__hip_bfloat16>::st(dst + q * sxo, x[0]);
      }
    }
#pragma unroll
    for (int r = 0; r < RM; ++r)
#pragma unroll
      for (int e = 0; e < VW; ++e) acc[r] = __builtin_fmaf(x[e], r < R ? wv[r][e] : 0.0f, acc[r]);
  }
#pragma unroll
  for (int r = 0; r < RM; ++r) {
    if (r < R) {
      float v = acc[r];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, VNX_WAVE);
      if (lane == 0) red[wave][r] = v;
    }
  }
  if (nw) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, VNX_WAVE);
    if (lane == 0) ssr[wave] = ss;
  }
  __syncthreads();
  float rstd = 1.0f;
  if (nw) rstd = 1.0f / __builtin_sqrtf((((ssr[0] + ssr[1]) + ssr[2]) + ssr[3]) / (float)D + eps);
  if (tid < R) {
    const float v = ((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid];
    lg[tid] = nw ? v * rstd : v;
  }
  __syncthreads();
  if (nw && xo) {
    // the experts' bf16 input rows: bf16(x * rstd * w), as RMSNorm rounds them
    // (stored before wave 0 routes, so the stores drain under the routing)
    for (int64_t c = (int64_t)tid * VW; c < D; c += 256 * VW) {
      float x[VW], w[VW];
      if (one_block) {
#pragma unroll
        for (int e = 0; e < VW; ++e) {
          x[e] = x1[e];
          w[e] = w1[e];
        }
      } else if constexpr (VW == 4) {
        ld4(h + m * ldh + c, x);
        ld4(nw + c, w);
      } else {
        x[0] = h[m * ldh + c];
        w[0] = nw[c];
      }
#pragma unroll
      for (int e = 0; e < VW; ++e) x[e] = x[e] * rstd * w[e];
      __hip_bfloat16* dst = xo + m * ldxo + c;
      for (int q = 0; q < copies; ++q) {
        if constexpr (VW == 4) st4(dst + q * sxo, x);
        else Elt<__hip_bfloat16>::st(dst + q * sxo, x[0]);
      }
    }
  }
  if (wave == 0) route_wave(lane < R ? lg[lane] : 0.0f, P, E, topk, comb + m * ldc);
}

// Expert activations of all PE experts for every row, scaled by the routing
// weights: out[m, x*He + j] = comb[m, x] * silu(gu[m, x*2He + j]) *
// gu[m, x*2He + He + j] (gu = the fused gate|up product of every expert), so
// one product with the concatenated down projections sums the experts.
// gu row (m, x) at gu + m*ldg + x*sxg (gate in [0, He), up in [He, 2He));
// out row (m, x) at out + m*ldo + x*sxo: the row-major (M, PE*2He) form of
// one product over the concatenated experts (sxg = 2He, sxo = He) and the
// expert-major (PE, M, 2He) form of a batched product (ldg = 2He,
// sxg = M*2He) are both strides of this.
// Grid: x = (row, expert) pairs m*PE + x, y = column blocks of 256 * VW.
// The routing weight is uniform over a workgroup: an unselected expert's
// block writes zeros without reading gu.
template <typename TI, typename TO, int VW>
__global__ __launch_bounds__(256) void k_mod_swiglu(const TI* gu, int64_t ldg, int64_t sxg, const float* comb,
                                                    int64_t ldc, int PE, int64_t He, TO* out, int64_t ldo,
                                                    int64_t sxo) {
  const int pair = blockIdx.x;
  const int m = pair / PE, x = pair - m * PE;
  const int64_t j = ((int64_t)blockIdx.y * 256 + threadIdx.x) * VW;
  if (j >= He) return;
  const float w = comb[(int64_t)m * ldc + x];
  const TI* g = gu + m * ldg + (int64_t)x * sxg + j;
  TO* o = out + m * ldo + (int64_t)x * sxo + j;
  if constexpr (VW == 4) {
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f}, u[4] = {0.0f, 0.0f, 0.0f, 0.0f}, r[4];
    if (w != 0.0f) {
      ld4(g, a);
      ld4(g + He, u);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = w != 0.0f ? w * silu(a[e]) * u[e] : 0.0f;
    st4(o, r);
  } else {
    float v = 0.0f;
    if (w != 0.0f) v = w * silu(Elt<TI>::ld(g)) * Elt<TI>::ld(g + He);
    Elt<TO>::st(o, v);
  }
}

// out[m, c] = sum over x < PE of y[x, m, c] (fp32 accumulation in x order):
// the sum of the routed experts' down projections (already weighted).
// VW consecutive elements per thread.
template <typename TY, int VW>
__global__ __launch_bounds__(256) void k_sum_experts(const TY* y, int64_t MD, int PE, float* out) {
  const int64_t t = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * VW;
  if (t >= MD) return;
  if constexpr (VW == 4) {
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, v[4];
    for (int x = 0; x < PE; ++x) {
      ld4(y + (int64_t)x * MD + t, v);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] += v[e];
    }
    st4(out + t, acc);
  } else {
    float acc = 0.0f;
    for (int x = 0; x < PE; ++x) acc += Elt<TY>::ld(y + (int64_t)x * MD + t);
    out[t] = acc;
  }
}

// out[m] = the sum, in expert order, of the rows y[z][slots[m*E + z]] of the
// experts that row m was routed to (slot >= 0): k_sum_experts over the
// compact per-expert outputs.  Grid (column blocks, rows).
template <typename TY, int VW>
__global__ __launch_bounds__(256) void k_sum_expert_rows(const TY* y, int64_t ldy, int64_t syb,
                                                         const int32_t* slots, int E, int64_t D, float* out,
                                                         int64_t ldo, int accumulate) {
  constexpr int ZB = 8;  // experts whose loads are in flight together
  const int64_t m = blockIdx.y;
  const int64_t c = ((int64_t)blockIdx.x * 256 + threadIdx.x) * VW;
  if (c >= D) return;
  float acc[VW];
#pragma unroll
  for (int e = 0; e < VW; ++e) acc[e] = 0.0f;
  // the residual values (accumulate) load first, under the expert loads
  float o[VW];
  if (accumulate) {
    if constexpr (VW == 4) ld4(out + m * ldo + c, o);
    else o[0] = out[m * ldo + c];
  }
  for (int z0 = 0; z0 < E; z0 += ZB) {
    // every load of the batch issued before any is used: unrouted experts
    // read row 0 and add +0.0, as their zero rows do in the dense sum
    int sl[ZB];
    float v[ZB][VW];
#pragma unroll
    for (int q = 0; q < ZB; ++q) sl[q] = z0 + q < E ? slots[m * E + z0 + q] : -1;
#pragma unroll
    for (int q = 0; q < ZB; ++q) {
      const int zq = min(z0 + q, E - 1);
      const TY* src = y + zq * syb + (int64_t)max(sl[q], 0) * ldy + c;
      if constexpr (VW == 4) ld4(src, v[q]);
      else v[q][0] = Elt<TY>::ld(src);
    }
#pragma unroll
    for (int q = 0; q < ZB; ++q)
#pragma unroll
      for (int e = 0; e < VW; ++e) acc[e] += sl[q] >= 0 ? v[q][e] : 0.0f;
  }
  if (accumulate) {  // out += the expert sum (the block's residual add)
#pragma unroll
    for (int e = 0; e < VW; ++e) acc[e] = o[e] + acc[e];
  }
  if constexpr (VW == 4) st4(out + m * ldo + c, acc);
  else out[m * ldo + c] = acc[0];
}

inline unsigned blocks_for(int64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

int rope_out_from(const vnx_rope_kv_args* a, int64_t N, RopeOut* out) {
  if (!a || !a->lens || !a->q_out || !a->k_cache || !a->v_cache) return VNX_ERR_INVALID_ARG;
  if (a->n < 1 || a->H < 1 || a->Hkv < 1 || a->d < 2) return VNX_ERR_INVALID_ARG;
  if (a->d % 16) return VNX_ERR_UNSUPPORTED;  // whole 16-row tiles of rotate-half pairs per head
  if ((int64_t)(a->H + 2 * a->Hkv) * a->d != N) return VNX_ERR_INVALID_ARG;
  if (a->c_sb < 0 || a->c_sh < 0 || a->c_sr < a->d || a->cap < 1) return VNX_ERR_INVALID_ARG;
  if (a->rope && (!a->cos_table || !a->sin_table || a->table_rows < 1)) return VNX_ERR_INVALID_ARG;
  RopeOut r{};
  r.lens = a->lens; r.cos = a->cos_table; r.sin = a->sin_table;
  r.q = static_cast<uint16_t*>(a->q_out); r.kc = static_cast<uint16_t*>(a->k_cache);
  r.vc = static_cast<uint16_t*>(a->v_cache);
  r.c_sb = a->c_sb; r.c_sh = a->c_sh; r.c_sr = a->c_sr;
  r.cap = a->rope ? (a->cap < a->table_rows ? a->cap : a->table_rows) : a->cap;
  r.n = a->n; r.H = a->H; r.Hkv = a->Hkv; r.d = a->d; r.rope = a->rope ? 1 : 0;
  *out = r;
  return VNX_OK;
}
}  // namespace vnx

using namespace vnx;

extern "C" {

int vnx_rmsnorm(const float* x, int64_t ldx, const void* res, int res_dtype, int64_t ldr, const float* w,
                float eps, int64_t M, int64_t D, float* x_out, int64_t ldxo, void* y, int y_dtype, int64_t ldy,
                void* stream) {
  if (!x || !w || !y || M < 0 || D <= 0 || ldx < D || ldy < D || (res && ldr < D) || (x_out && ldxo < D))
    return VNX_ERR_INVALID_ARG;
  if (D > (int64_t)kRnThreads * kRnPer || !(eps >= 0.0f)) return VNX_ERR_UNSUPPORTED;
  if (M == 0) return VNX_OK;
  if (M >= INT32_MAX) return VNX_ERR_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int rdt = res ? res_dtype : VNX_F32;
  return by_dtype(rdt, [&](auto tr) {
    using TR = decltype(tr);
    return by_dtype(y_dtype, [&](auto ty) {
      using TY = decltype(ty);
      hipLaunchKernelGGL((k_rmsnorm<TR, TY>), dim3((unsigned)M), dim3(kRnThreads), 0, s, x, ldx,
                         static_cast<const TR*>(res), ldr, w, eps, D, x_out, ldxo, static_cast<TY*>(y), ldy);
      VNX_LAUNCH_CHECK();
      return (int)VNX_OK;
    });
  });
}

int vnx_embed_rmsnorm(const int64_t* tokens, const void* emb, int emb_dtype, int64_t lde, int64_t vocab,
                      float scale, const float* w, float eps, int64_t M, int64_t D, float* x_out, int64_t ldxo,
                      void* y, int y_dtype, int64_t ldy, void* stream) {
  if (!tokens || !emb || !w || !x_out || !y || M < 0 || D <= 0 || vocab <= 0 || lde < D || ldxo < D || ldy < D)
    return VNX_ERR_INVALID_ARG;
  if (D > (int64_t)kRnThreads * kRnPer || !(eps >= 0.0f)) return VNX_ERR_UNSUPPORTED;
  if (M == 0) return VNX_OK;
  if (M >= INT32_MAX) return VNX_ERR_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return by_dtype(emb_dtype, [&](auto te) {
    using TE = decltype(te);
    return by_dtype(y_dtype, [&](auto ty) {
      using TY = decltype(ty);
      hipLaunchKernelGGL((k_embed_rmsnorm<TE, TY>), dim3((unsigned)M), dim3(kRnThreads), 0, s, tokens,
                         static_cast<const TE*>(emb), lde, vocab, scale, w, eps, D, x_out, ldxo, static_cast<TY*>(y),
                         ldy);
      VNX_LAUNCH_CHECK();
      return (int)VNX_OK;
    });
  });
}

int vnx_rope_kv(const void* qkv, int dtype, int64_t ldq, int64_t B, int n, int H, int Hkv, int d,
                const int32_t* lens, const float* cos_table, const float* sin_table, int64_t table_rows, int rope,
                void* q_out, void* k_cache, void* v_cache, int out_dtype, int64_t c_sb, int64_t c_sh,
                int64_t c_sr, int64_t cap, void* stream) {
  if (!qkv || !lens || !q_out || !k_cache || !v_cache || B < 0 || n < 1 || H < 1 || Hkv < 1 || d < 2 || d % 2)
    return VNX_ERR_INVALID_ARG;
  if (ldq < (int64_t)(H + 2 * Hkv) * d || c_sb < 0 || c_sh < 0 || c_sr < d) return VNX_ERR_INVALID_ARG;
  if (rope && (!cos_table || !sin_table || table_rows < 1)) return VNX_ERR_INVALID_ARG;
  if (cap < 1 || (out_dtype != VNX_F32 && out_dtype != VNX_BF16)) return VNX_ERR_INVALID_ARG;
  if (B == 0) return VNX_OK;
  // Positions lens[b] + i are read on the device; rows at or past the cache
  // capacity (or the RoPE table) are skipped there, so a bad length cannot
  // write out of bounds.
  RopeParams p{};
  p.qkv = qkv; p.ldq = ldq; p.B = B; p.n = n; p.H = H; p.Hkv = Hkv; p.d = d;
  p.lens = lens; p.cos = cos_table; p.sin = sin_table; p.rope = rope ? 1 : 0;
  p.q = q_out; p.kc = k_cache; p.vc = v_cache;
  p.c_sb = c_sb; p.c_sh = c_sh; p.c_sr = c_sr;
  p.cap = rope ? (cap < table_rows ? cap : table_rows) : cap;
  const int64_t rows = B * (int64_t)n;
  if (rows >= INT32_MAX || (int64_t)(H + 2 * Hkv) * (d / 2) >= INT32_MAX) return VNX_ERR_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return by_dtype(dtype, [&](auto tq) {
    using TQ = decltype(tq);
    if (out_dtype == VNX_F32)
      hipLaunchKernelGGL((k_rope_kv<TQ, float>), dim3((unsigned)rows), dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL((k_rope_kv<TQ, __hip_bfloat16>), dim3((unsigned)rows), dim3(256), 0, s, p);
    VNX_LAUNCH_CHECK();
    return (int)VNX_OK;
  });
}

int vnx_swiglu(const void* gu, int dtype, int64_t ldg, int64_t M, int64_t Hf, void* out, int out_dtype,
               int64_t ldo, void* stream) {
  if (!gu || !out || M < 0 || Hf <= 0 || ldg < 2 * Hf || ldo < Hf) return VNX_ERR_INVALID_ARG;
  if (M == 0) return VNX_OK;
  if (M >= INT32_MAX || Hf > (int64_t)65535 * 256) return VNX_ERR_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool v4 = Hf % 4 == 0 && ldg % 4 == 0 && ldo % 4 == 0 && vec4_ok(gu, dtype_bytes(dtype)) &&
                  vec4_ok(out, dtype_bytes(out_dtype));
  return by_dtype(dtype, [&](auto ti) {
    using TI = decltype(ti);
    return by_dtype(out_dtype, [&](auto to) {
      using TO = decltype(to);
      if (v4)
        hipLaunchKernelGGL((k_swiglu<TI, TO, 4>), dim3((unsigned)M, (unsigned)((Hf + 1023) / 1024)), dim3(256), 0,
                           s, static_cast<const TI*>(gu), ldg, Hf, static_cast<TO*>(out), ldo);
      else
        hipLaunchKernelGGL((k_swiglu<TI, TO, 1>), dim3((unsigned)M, (unsigned)((Hf + 255) / 256)), dim3(256), 0,
                           s, static_cast<const TI*>(gu), ldg, Hf, static_cast<TO*>(out), ldo);
      VNX_LAUNCH_CHECK();
      return (int)VNX_OK;
    });
  });
}

int vnx_axpby(const float* a, const float* b, const float* coef, int64_t n, void* out, int out_dtype,
              void* stream) {
  if (!a || !b || !coef || !out || n < 0) return VNX_ERR_INVALID_ARG;
  if (n == 0) return VNX_OK;
  if (n >= ((int64_t)1 << 40)) return VNX_ERR_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return by_dtype(out_dtype, [&](auto to) {
    using TO = decltype(to);
    hipLaunchKernelGGL((k_axpby<TO>), dim3(blocks_for(n)), dim3(256), 0, s, a, b, coef, n, static_cast<TO*>(out));
    VNX_LAUNCH_CHECK();
    return (int)VNX_OK;
  });
}

int vnx_mod_route(const float* logits, int64_t ld, int64_t M, int P, int E, int topk, float* comb, int64_t ldc,
                  void* stream) {
  if (!logits || !comb || M < 0 || P < 1 || E < 1 || topk < 1 || topk > E) return VNX_ERR_INVALID_ARG;
  if (P > kModMaxP || E > kModMaxE || P + P * E > VNX_WAVE) return VNX_ERR_UNSUPPORTED;
  if (ld < P + (int64_t)P * E || ldc < (int64_t)P * E) return VNX_ERR_INVALID_ARG;
  if (M == 0) return VNX_OK;
  if (M >= INT32_MAX) return VNX_ERR_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_mod_route, dim3((unsigned)M), dim3(64), 0, s, logits, ld, M, P, E, topk, comb, ldc);
  VNX_LAUNCH_CHECK();
  return VNX_OK;
}

int vnx_mod_route_x(const float* h, int64_t ldh, const float* norm_w, float eps, const float* wr, int64_t ldw,
                    int64_t M, int64_t D, int P, int E, int topk, float* comb, int64_t ldc, void* x_out, int64_t ldxo,
                    int64_t sxo, int copies, void* stream) {
  if (!h || !wr || !comb || M < 0 || D < 1 || P < 1 || E < 1 || topk < 1 || topk > E) return VNX_ERR_INVALID_ARG;
  if (norm_w && !(eps >= 0.0f)) return VNX_ERR_INVALID_ARG;
  if (x_out && (ldxo < D || copies < 1 || (copies > 1 && sxo < M * ldxo))) return VNX_ERR_INVALID_ARG;
  if (P > kModMaxP || E > kModMaxE || P + P * E > kRouteMaxR) return VNX_ERR_UNSUPPORTED;
  if (ldh < D || ldw < D || ldc < (int64_t)P * E) return VNX_ERR_INVALID_ARG;
  if (M == 0) return VNX_OK;
  if (M >= INT32_MAX) return VNX_ERR_UNSUPPORTED;
  const bool v4 = D % 4 == 0 && ldh % 4 == 0 && ldw % 4 == 0 && vec4_ok(h, 4) && vec4_ok(wr, 4) &&
                  (!norm_w || vec4_ok(norm_w, 4)) && (!x_out || (ldxo % 4 == 0 && sxo % 4 == 0 && vec4_ok(x_out, 2)));
  // router rows held per thread: P + P*E rounded up to 8 (rows past it are not loaded)
  const int R = P + P * E;
  auto go = [&](auto vw, auto rm) {
    constexpr int VW = decltype(vw)::value, RM = decltype(rm)::value;
    hipLaunchKernelGGL((k_mod_route_x<VW, RM>), dim3((unsigned)M), dim3(256), 0, static_cast<hipStream_t>(stream),
                       h, ldh, norm_w, eps, wr, ldw, D, P, E, topk, comb, ldc, static_cast<__hip_bfloat16*>(x_out),
                       ldxo, sxo, x_out ? copies : 0);
  };
  auto by_r = [&](auto vw) {
    if (R <= 8) go(vw, IntC<8>{});
    else if (R <= 16) go(vw, IntC<16>{});
    else if (R <= 24) go(vw, IntC<24>{});
    else go(vw, IntC<32>{});
  };
  if (v4) by_r(IntC<4>{});
  else by_r(IntC<1>{});
  VNX_LAUNCH_CHECK();
  return VNX_OK;
}

int vnx_mod_swiglu(const void* gu, int dtype, int64_t ldg, int64_t sxg, const float* comb, int64_t ldc, int64_t M,
                   int PE, int64_t He, void* out, int out_dtype, int64_t ldo, int64_t sxo, void* stream) {
  if (!gu || !comb || !out || M < 0 || PE < 1 || He < 1) return VNX_ERR_INVALID_ARG;
  if (ldg < 0 || sxg < 0 || ldo < 0 || sxo < 0 || ldc < PE) return VNX_ERR_INVALID_ARG;
  // rows and experts must not overlap: either layout of the two products
  const bool g_rowmajor = sxg >= 2 * He && ldg >= sxg * PE;
  const bool g_expmajor = ldg >= 2 * He && sxg >= ldg * M;
  const bool o_rowmajor = sxo >= He && ldo >= sxo * PE;
  const bool o_expmajor = ldo >= He && sxo >= ldo * M;
  if (!(g_rowmajor || g_expmajor) || !(o_rowmajor || o_expmajor)) return VNX_ERR_INVALID_ARG;
  if (M == 0) return VNX_OK;
  if (M * PE >= INT32_MAX || He > (int64_t)65535 * 256) return VNX_ERR_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool v4 = He % 4 == 0 && ldg % 4 == 0 && sxg % 4 == 0 && ldo % 4 == 0 && sxo % 4 == 0 &&
                  vec4_ok(gu, dtype_bytes(dtype)) && vec4_ok(out, dtype_bytes(out_dtype));
  const unsigned pairs = (unsigned)(M * PE);
  return by_dtype(dtype, [&](auto ti) {
    using TI = decltype(ti);
    return by_dtype(out_dtype, [&](auto to) {
      using TO = decltype(to);
      if (v4)
        hipLaunchKernelGGL((k_mod_swiglu<TI, TO, 4>), dim3(pairs, (unsigned)((He + 1023) / 1024)), dim3(256), 0, s,
                           static_cast<const TI*>(gu), ldg, sxg, comb, ldc, PE, He, static_cast<TO*>(out), ldo,
                           sxo);
      else
        hipLaunchKernelGGL((k_mod_swiglu<TI, TO, 1>), dim3(pairs, (unsigned)((He + 255) / 256)), dim3(256), 0, s,
                           static_cast<const TI*>(gu), ldg, sxg, comb, ldc, PE, He, static_cast<TO*>(out), ldo,
                           sxo);
      VNX_LAUNCH_CHECK();
      return (int)VNX_OK;
    });
  });
}

int vnx_sum_experts(const void* y, int dtype, int64_t M, int PE, int64_t D, float* out, void* stream) {
  if (!y || !out || M < 0 || PE < 1 || D < 1) return VNX_ERR_INVALID_ARG;
  if (M == 0) return VNX_OK;
  if (M * D >= ((int64_t)1 << 40)) return VNX_ERR_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t MD = M * D;
  const bool v4 = MD % 4 == 0 && vec4_ok(y, dtype_bytes(dtype)) && vec4_ok(out, 4);
  return by_dtype(dtype, [&](auto ty) {
    using TY = decltype(ty);
    if (v4)
      hipLaunchKernelGGL((k_sum_experts<TY, 4>), dim3(blocks_for(MD / 4)), dim3(256), 0, s,
                         static_cast<const TY*>(y), MD, PE, out);
    else
      hipLaunchKernelGGL((k_sum_experts<TY, 1>), dim3(blocks_for(MD)), dim3(256), 0, s, static_cast<const TY*>(y),
                         MD, PE, out);
    VNX_LAUNCH_CHECK();
    return (int)VNX_OK;
  });
}

int vnx_sum_expert_rows(const void* y, int dtype, int64_t ldy, int64_t syb, const int32_t* slots, int64_t M,
                        int E, int64_t D, float* out, int64_t ldo, int accumulate, void* stream) {
  if (!y || !slots || !out || M < 0 || E < 1 || D < 1 || ldy < D || syb < 0 || ldo < D) return VNX_ERR_INVALID_ARG;
  if (M == 0) return VNX_OK;
  if (M > 65535) return VNX_ERR_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool v4 = D % 4 == 0 && ldy % 4 == 0 && syb % 4 == 0 && ldo % 4 == 0 && vec4_ok(y, dtype_bytes(dtype)) &&
                  vec4_ok(out, 4);
  return by_dtype(dtype, [&](auto ty) {
    using TY = decltype(ty);
    if (v4)
      hipLaunchKernelGGL((k_sum_expert_rows<TY, 4>), dim3(blocks_for(D / 4), (unsigned)M), dim3(256), 0, s,
                         static_cast<const TY*>(y), ldy, syb, slots, E, D, out, ldo, accumulate);
    else
      hipLaunchKernelGGL((k_sum_expert_rows<TY, 1>), dim3(blocks_for(D), (unsigned)M), dim3(256), 0, s,
                         static_cast<const TY*>(y), ldy, syb, slots, E, D, out, ldo, accumulate);
    VNX_LAUNCH_CHECK();
    return (int)VNX_OK;
  });
}

}  // extern "C"
