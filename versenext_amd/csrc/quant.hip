// Weight-only quantized GEMV / skinny GEMM for draft decode and the tied LM
// head: y (B, N) fp32 = x (B, K) fp16 . dequant(W)^T.
//   W4: int4 packed two per byte along K, low nibble = even k (the layout of
//       quantize.py:36-68), one scale per (row, group of G columns), scales
//       fp16 or fp32.  G = 128 with fp16 scales is the group-128 format;
//       G = K with fp32 scales is the reference's per-channel INT4
//       (quantize.py:231-258).
//   W8: int8 (N, K), one fp32 scale per row (quantize.py:187-214).
// The dequantized weight is q * s, so y = sum_g s_g * sum_{k in g} x_k q_k.
//
// Matrix cores: v_mfma_f32_16x16x32_f16 with A = 16 weight rows x 32 k (the
// integers, converted exactly to fp16 in registers), B = 32 k x 16 batch
// columns (x, staged in LDS) and a 16x16 fp32 accumulator per 128-k group.
// The integers are read in offset form, u = q ^ 8 (0..15) or q ^ 0x80
// (0..255); one v_perm_b32 per pair places two of them under 0x64 exponent
// bytes (the fp16 values 1024 + u) and one packed fp16 subtract restores q
// (exact: small integers).  A group's MFMA result is scaled by s_g and added
// to the fp32 output.
//
// Work split (large N): a workgroup (4 waves) owns 64*TPW consecutive rows
// (tiles of 16 rows; wave w takes tiles w, w+4, ...) and all of K; it streams
// K in slices, staging each slice of x (up to 32 batch columns) once in LDS
// for all of its tiles.  Small N: k_qgemv_tile (one tile per workgroup, K
// split over its waves and summed in wave order, so the result does not
// depend on scheduling).  Within a 128-k group, lane (m = lane % 16, kq = lane / 16)
// holds k = kq*32 + [0, 32) of row m (16 bytes of W4, 32 of W8), used as
// four MFMA k-steps; the B operand takes x at the same k (the k order inside
// a group is a permutation shared by A and B, so the dot product is unchanged).
#include <stdlib.h>

#include <type_traits>

#include "vnx_internal.h"

namespace vnx {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __fp16 fp16x2 __attribute__((ext_vector_type(2)));

constexpr int kQNT = 256;        // threads per workgroup
constexpr int kQTiles = 4;       // tiles per wave
constexpr int kQRows = 16 * 4 * kQTiles;  // rows per workgroup (256)
constexpr int kGK = 128;         // k per accumulation group
constexpr int kXPad = 8;         // fp16 padding per LDS row of x (16 bytes)

struct QGemvParams {
  const uint16_t* x;   // fp16 bits, (B, K), row pitch ldx
  int64_t ldx;
  const uint8_t* w;    // W4: (N, K/2) bytes; W8: (N, K) bytes; row pitch ldw bytes
  int64_t ldw;
  const void* sc;      // scales, row pitch lds elements
  int64_t lds;
  int sc_f16;          // 1: fp16 scales, 0: fp32
  int64_t B, N, K;
  int G;               // columns per scale (W4); W8 uses one scale per row
  int gpg;             // 128-column groups per scale: G / 128
  float* y;            // (B, N), row pitch ldy
  int64_t ldy;
  uint16_t* yb;        // k_qgemv_tiles with OB: bf16 bits (B, N), row pitch ldy (then y is unused)
  uint16_t* yh;        // SwiGLU output: fp16 bits (B, N/2), row pitch ldy (then y is unused)
  int rope_on;         // RoPE + cache store epilogue (ro; y and yh unused)
  int resid;           // residual epilogue: y += the product (fp32)
  const float* xf;     // NX: fp32 rows to normalize (x unused), row pitch ldx
  const float* nw;     // NX: RMSNorm weight (K)
  float eps;
  int64_t row_off;     // batch row of x's first row (the launch's 32-row chunks)
  // NX 2: x rows are the token embedding, xf unused: row b is
  // emb[ids[b]] * emb_scale (bf16 table, ids clamped to [0, vocab)), and the
  // workgroups write those fp32 rows to xout (pitch ldx)
  const int64_t* ids;
  const uint16_t* emb;
  int64_t lde, vocab;
  float emb_scale;
  float* xout;
  RopeOut ro;
  int64_t ksplit_len;  // K per grid.y split (multiple of kGK; the launches use K)
};

// The same with the format fixed at compile time: no branch between a scale
// load and its conversion, so the conversion waits at the scale's use, not
// at the load (a converting branch right after the load waits for every load
// issued before it, weights and x included).
template <bool SF16>
__device__ __forceinline__ float load_scale_t(const QGemvParams& p, int64_t row, unsigned g) {
  if constexpr (SF16) {
    const uint16_t h = static_cast<const uint16_t*>(p.sc)[row * p.lds + g];
    return (float)__builtin_bit_cast(_Float16, h);
  } else {
    return static_cast<const float*>(p.sc)[row * p.lds + g];
  }
}

__device__ __forceinline__ float load_scale(const QGemvParams& p, int64_t row, unsigned g) {
  if (p.sc_f16) {
    const uint16_t h = static_cast<const uint16_t*>(p.sc)[row * p.lds + g];
    return (float)__builtin_bit_cast(_Float16, h);
  }
  return static_cast<const float*>(p.sc)[row * p.lds + g];
}

// Integers -> fp16 with one v_perm_b32 per pair: the fp16 bits 0x64vv are
// 1024 + vv for a byte vv, so selecting two offset-form bytes of u and two
// 0x64 bytes of a constant gives the pair (1024 + u_a, 1024 + u_b); one packed
// fp16 subtract then leaves the signed integers (exact: |q| <= 128).
__device__ __forceinline__ fp16x2 pair_from(uint32_t u, uint32_t sel, fp16x2 off) {
  const uint32_t bits = __builtin_amdgcn_perm(0x64646464u, u, sel);
  return __builtin_bit_cast(fp16x2, bits) - off;
}

// Selectors: D = {u.b_lo, 0x64, u.b_hi, 0x64} (codes 0-3 pick u, 4 picks 0x64).
constexpr uint32_t kSel01 = 0x04010400u;  // bytes 0, 1
constexpr uint32_t kSel23 = 0x04030402u;  // bytes 2, 3

__device__ __forceinline__ half8 pack_half8(fp16x2 p0, fp16x2 p1, fp16x2 p2, fp16x2 p3) {
  half8 a;
  a[0] = (_Float16)p0.x; a[1] = (_Float16)p0.y; a[2] = (_Float16)p1.x; a[3] = (_Float16)p1.y;
  a[4] = (_Float16)p2.x; a[5] = (_Float16)p2.y; a[6] = (_Float16)p3.x; a[7] = (_Float16)p3.y;
  return a;
}

// A operand of one MFMA k-step from one W4 dword (8 nibbles, nibble i = k i;
// low nibble of byte j is k 2j).  Element order: k = 0, 2, 4, 6, 1, 3, 5, 7
// (the low nibbles, then the high nibbles); x is staged in LDS in the same
// order (stage_perm_w4).
__device__ __forceinline__ half8 a_w4(uint32_t d) {
  const uint32_t lo = (d ^ 0x88888888u) & 0x0F0F0F0Fu;         // q + 8 of k 0, 2, 4, 6
  const uint32_t hi = ((d >> 4) ^ 0x08888888u) & 0x0F0F0F0Fu;  // q + 8 of k 1, 3, 5, 7
  const fp16x2 off = {(__fp16)1032.0f, (__fp16)1032.0f};
  return pack_half8(pair_from(lo, kSel01, off), pair_from(lo, kSel23, off), pair_from(hi, kSel01, off),
                    pair_from(hi, kSel23, off));
}

// W8: two dwords = 8 int8 in k order (natural order, x staged unpermuted).
__device__ __forceinline__ half8 a_w8(uint32_t d0, uint32_t d1) {
  const uint32_t u0 = d0 ^ 0x80808080u, u1 = d1 ^ 0x80808080u;  // q + 128
  const fp16x2 off = {(__fp16)1152.0f, (__fp16)1152.0f};
  return pack_half8(pair_from(u0, kSel01, off), pair_from(u0, kSel23, off), pair_from(u1, kSel01, off),
                    pair_from(u1, kSel23, off));
}

// Orders one wave's LDS writes before its later LDS reads (and reads before
// later writes): the LDS runs a wave's instructions in order, so only the
// compiler's ordering needs pinning.
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// W4 staging order of 8 consecutive fp16 (4 dwords w0..w3 = (h0,h1)..(h6,h7)):
// h0, h2, h4, h6, h1, h3, h5, h7.
__device__ __forceinline__ u32x4 stage_perm_w4(u32x4 v) {
  u32x4 o;
  o.x = __builtin_amdgcn_perm(v.y, v.x, 0x05040100u);  // h0, h2
  o.y = __builtin_amdgcn_perm(v.w, v.z, 0x05040100u);  // h4, h6
  o.z = __builtin_amdgcn_perm(v.y, v.x, 0x07060302u);  // h1, h3
  o.w = __builtin_amdgcn_perm(v.w, v.z, 0x07060302u);  // h5, h7
  return o;
}

template <int BITS, int NC, int TPW>
__global__ __launch_bounds__(kQNT) void k_qgemv(QGemvParams p) {
  constexpr int KS = 1024 / NC;                 // k per slice
  constexpr int XS = KS + kXPad;                // LDS row pitch of x (fp16)
  constexpr int NG = KS / kGK;                  // groups per slice
  constexpr int WBYTES = BITS == 4 ? 16 : 32;   // weight bytes per lane per group
  __shared__ __attribute__((aligned(16))) uint16_t xs[NC * 16 * XS];

  const int tid = threadIdx.x;
  const int wave = tid / VNX_WAVE, lane = tid % VNX_WAVE;
  const int m = lane % 16, kq = lane / 16;
  const int64_t row_base = (int64_t)blockIdx.x * (64 * TPW);
  const int64_t kb = (int64_t)blockIdx.y * p.ksplit_len;
  const int64_t ke = min(p.K, kb + p.ksplit_len);
  // fp16 group scales can be read 16 bytes per row when a group is 128 wide.
  const bool vec_sc = BITS == 4 && p.sc_f16 && p.G == kGK && (p.lds % 8) == 0 &&
                      (reinterpret_cast<uintptr_t>(p.sc) & 15) == 0;

  f32x4 yacc[TPW][NC];
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int c = 0; c < NC; ++c) yacc[t][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int64_t k0 = kb; k0 < ke; k0 += KS) {
    const int ks = (int)min((int64_t)KS, ke - k0);  // multiple of kGK
    // ---- stage x[:, k0 : k0+ks) (zero rows past B, zero columns past ks) ----
    __syncthreads();
    // Batch rows past B are zero; they are written once (first slice) and
    // never read from global memory.
    const int brows = k0 == kb ? NC * 16 : (int)min((int64_t)NC * 16, p.B);
    for (int idx = tid; idx < brows * (KS / 8); idx += kQNT) {
      const int b = idx / (KS / 8), c8 = idx % (KS / 8);
      u32x4 v = {0u, 0u, 0u, 0u};
      if (b < p.B && c8 * 8 < ks) v = *reinterpret_cast<const u32x4*>(p.x + b * p.ldx + k0 + c8 * 8);
      if constexpr (BITS == 4) v = stage_perm_w4(v);
      *reinterpret_cast<u32x4*>(&xs[b * XS + c8 * 8]) = v;
    }
    __syncthreads();

#pragma unroll 1
    for (int t = 0; t < TPW; ++t) {
      const int64_t row0 = row_base + (int64_t)(wave + 4 * t) * 16;
      if (row0 >= p.N) break;
      // A rows: m; D rows: 4*kq + j.  Rows past N read row N-1 (not stored).
      const int64_t ra = min(row0 + m, p.N - 1);
      const uint8_t* wr = p.w + ra * p.ldw + (BITS == 4 ? k0 / 2 : k0);
      // All of the slice's weight loads first.
      uint32_t wv[NG][WBYTES / 4];
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        if (g * kGK < ks) {
          const uint8_t* src = wr + (BITS == 4 ? g * 64 + kq * 16 : g * 128 + kq * 32);
          const u32x4 v0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
          wv[g][0] = v0.x; wv[g][1] = v0.y; wv[g][2] = v0.z; wv[g][3] = v0.w;
          if constexpr (BITS == 8) {
            const u32x4 v1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + 16));
            wv[g][4] = v1.x; wv[g][5] = v1.y; wv[g][6] = v1.z; wv[g][7] = v1.w;
          }
        }
      }
      // Scales of the lane's four D rows for the slice's groups (W4).
      float sc[NG][4];
      if constexpr (BITS == 4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t rd = min(row0 + 4 * kq + j, p.N - 1);
          if (vec_sc && ks == KS && (k0 / kGK) % NG == 0) {
            // The slice's NG scales of row rd: exactly NG halves (16 or 8
            // bytes), aligned because lds % 8 == 0 and k0 / kGK % NG == 0.
            const uint16_t* srow = static_cast<const uint16_t*>(p.sc) + rd * p.lds + k0 / kGK;
            uint32_t wds[NG / 2];
            if constexpr (NG == 8) {
              const u32x4 v = *reinterpret_cast<const u32x4*>(srow);
              wds[0] = v.x; wds[1] = v.y; wds[2] = v.z; wds[3] = v.w;
            } else {
              static_assert(NG == 4, "slices hold 4 or 8 groups");
              const uint2 v = *reinterpret_cast<const uint2*>(srow);
              wds[0] = v.x; wds[1] = v.y;
            }
#pragma unroll
            for (int e = 0; e < NG; ++e)
              sc[e][j] = (float)__builtin_bit_cast(_Float16, (uint16_t)(wds[e / 2] >> (16 * (e % 2))));
          } else {
            // Scale column of group g: (k0/128 + g) / gpg, in 32-bit
            // arithmetic (gpg = 1 for group-128, K/128 for one scale per row).
            const unsigned g0 = (unsigned)(k0 / kGK);
#pragma unroll
            for (int g = 0; g < NG; ++g)
              if (g * kGK < ks) {
                const unsigned col = p.gpg == 1 ? g0 + g : (g0 + (unsigned)g) / (unsigned)p.gpg;
                sc[g][j] = load_scale(p, rd, col);
              }
          }
        }
      }
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        if (g * kGK >= ks) break;
        f32x4 acc[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const half8 a = BITS == 4 ? a_w4(wv[g][s]) : a_w8(wv[g][2 * s], wv[g][2 * s + 1]);
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const int b = c * 16 + m;
            const half8 bx = *reinterpret_cast<const half8*>(&xs[b * XS + g * kGK + kq * 32 + s * 8]);
            acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bx, acc[c], 0, 0, 0);
          }
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if constexpr (BITS == 4) yacc[t][c][j] = __builtin_fmaf(sc[g][j], acc[c][j], yacc[t][c][j]);
            else yacc[t][c][j] += acc[c][j];
          }
        }
      }
    }
  }

  // ---- store: lane holds D[row 4*kq + j][column m] ----
  float* out = p.y;
  const int64_t ldo = p.ldy;
#pragma unroll 1
  for (int t = 0; t < TPW; ++t) {
    const int64_t row0 = row_base + (int64_t)(wave + 4 * t) * 16;
    if (row0 >= p.N) break;
    const int64_t n0 = row0 + 4 * kq;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int64_t b = c * 16 + m;
      if (b >= p.B) continue;
      f32x4 v = yacc[t][c];
      if constexpr (BITS == 8) {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] *= load_scale(p, min(n0 + j, p.N - 1), 0);
      }
      float* dst = out + b * ldo + n0;
      if (n0 + 4 <= p.N && (reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
        *reinterpret_cast<f32x4*>(dst) = v;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (n0 + j < p.N) dst[j] = v[j];
      }
    }
  }
}

// Small N (fewer than kQTileMaxN rows): one 16-row tile per workgroup and
// the whole K inside it, split over its NW waves by 128-k group (wave w takes
// groups w, w + NW, ..., two at a time so both groups' loads are in flight);
// the waves' partial tiles are summed through LDS in wave order, so the
// result does not depend on scheduling and no second launch is needed.  A
// wave stages its group's x block (up to 32 batch rows x 128 k) through its
// own LDS tile: coalesced 256-byte row reads in, the MFMA B-operand layout
// out.
// QE: 0 plain fp32 output, 1 SwiGLU (fp16), 2 RoPE + KV-cache store,
// 3 residual (y += the product, fp32).  NX (W4): x is RMSNorm(xf) * nw: the
// staged operand is fp16(xf * nw), each wave sums the squares of its groups'
// values per row, and the epilogue scales row b by rstd_b = 1/sqrt(mean
// xf^2 + eps) (vnnn.py:593-615, the per-row factor on the fp32 sums).
// NX 2: the same with the rows gathered from the token embedding (the first
// block's norm of CometSparkV05LM.forward, spark/src/base_model.py:170-208);
// group g's values of every row go to xout from workgroup g % gridDim.x, so
// the fp32 residual stream starts without a launch of its own.
// TP: 16-row tiles per workgroup (2 for grids of more tiles than CUs: each
// wave's x block is loaded and staged once for both tiles).  GP: groups per
// pass of a wave (1 where K has at most one group per wave, or TP 2).
template <int BITS, int NC, int NW, int QE, int NX, int TP, int GP, bool SF16>
__device__ __forceinline__ void qgemv_tile_body(const QGemvParams& p, char* smem, float* ssp_flat) {
  constexpr int WBYTES = BITS == 4 ? 16 : 32;
  constexpr int XR = NC * 16;            // staged batch rows
  constexpr int XP = kGK + kXPad;        // LDS row pitch (fp16)
  constexpr int XL = XR * (kGK / 8) / 64;  // 16-byte x loads per lane per group
  // the per-wave x tiles, reused for the partial tiles after the K loop
  constexpr size_t kXBytes = size_t(NW) * XR * XP * 2, kRBytes = size_t(NW) * TP * NC * 64 * 16;
  auto xs_all = reinterpret_cast<uint16_t(*)[XR * XP]>(smem);
  auto red = reinterpret_cast<f32x4(*)[TP][NC][64]>(smem);
  auto ssp = reinterpret_cast<float(*)[NX ? XR : 1]>(ssp_flat);  // NX: per-wave sums of squares per row
  const int tid = threadIdx.x;
  const int wave = tid / VNX_WAVE, lane = tid % VNX_WAVE;
  const int m = lane % 16, kq = lane / 16;
  uint16_t* xs = xs_all[wave];
  const int64_t tile0 = (int64_t)blockIdx.x * TP;
  const uint8_t* wr[TP];
#pragma unroll
  for (int t = 0; t < TP; ++t) {
    const int64_t ra = min((tile0 + t) * 16 + m, p.N - 1);  // A row (rows past N read row N-1, not stored)
    wr[t] = p.w + ra * p.ldw;
  }
  const int ngroups = (int)(p.K / kGK);

  f32x4 yacc[TP][NC];
#pragma unroll
  for (int t = 0; t < TP; ++t)
#pragma unroll
    for (int c = 0; c < NC; ++c) yacc[t][c] = f32x4{0.f, 0.f, 0.f, 0.f};
  // QE 3: the residual values wave t*NC + c adds to (row c*16 + m, columns
  // (tile0 + t)*16 + 4*kq .. +4) load now, under the K loop
  f32x4 rold = {0.f, 0.f, 0.f, 0.f};
  if constexpr (QE == 3) {
    if (wave < NC * TP) {
      const int64_t rb = (wave % NC) * 16 + m, rn = (tile0 + wave / NC) * 16 + 4 * kq;
      if (rb < p.B && rn < p.N) {
        const float* src = p.y + rb * p.ldy + rn;
        if (rn + 4 <= p.N && (reinterpret_cast<uintptr_t>(src) & 15) == 0) {
          rold = *reinterpret_cast<const f32x4*>(src);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) rold[j] = rn + j < p.N ? src[j] : 0.0f;
        }
      }
    }
  }
  float ss[NX ? XL : 1];  // NX: this lane's sums of squares, row (i*64 + lane) / 16
#pragma unroll
  for (int i = 0; i < (NX ? XL : 1); ++i) ss[i] = 0.0f;
  const uint16_t* erow[NX == 2 ? XL : 1];  // NX 2: embedding row of row (i*64 + lane) / 16
  if constexpr (NX == 2) {
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      int64_t tok = p.ids[min((i * 64 + lane) / 16, (int)p.B - 1)];
      tok = tok < 0 ? 0 : (tok >= p.vocab ? p.vocab - 1 : tok);  // never outside the table
      erow[i] = p.emb + tok * p.lde;
    }
  }

  static_assert(GP == 1 || GP == 2, "one or two groups per pass");
  for (int g0 = wave; g0 < ngroups; g0 += GP * NW) {
    // GP 2: groups g0 and g0 + NW (the second weighted 0 when past K)
    const int gg[2] = {g0, g0 + NW < ngroups ? g0 + NW : g0};
    const bool second = g0 + NW < ngroups;
    uint32_t wv[GP][TP][WBYTES / 4];
    u32x4 xv[GP][XL][NX ? 2 : 1];
    u32x4 nwv[GP][NX ? 2 : 1];
    float sc[GP][TP][4];
#pragma unroll
    for (int u = 0; u < GP; ++u) {
      const int64_t k0 = (int64_t)gg[u] * kGK;
#pragma unroll
      for (int t = 0; t < TP; ++t) {
        const uint8_t* src = wr[t] + (BITS == 4 ? k0 / 2 + kq * 16 : k0 + kq * 32);
        const u32x4 v0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
        wv[u][t][0] = v0.x; wv[u][t][1] = v0.y; wv[u][t][2] = v0.z; wv[u][t][3] = v0.w;
        if constexpr (BITS == 8) {
          const u32x4 v1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + 16));
          wv[u][t][4] = v1.x; wv[u][t][5] = v1.y; wv[u][t][6] = v1.z; wv[u][t][7] = v1.w;
        }
      }
      // x block: load i covers batch row (i*64 + lane) / 16, chunk lane % 16
#pragma unroll
      for (int i = 0; i < XL; ++i) {
        const int b = (i * 64 + lane) / 16;
        if constexpr (NX == 2) {
          xv[u][i][0] = *reinterpret_cast<const u32x4*>(erow[i] + k0 + m * 8);
        } else if constexpr (NX) {
          const float* src = p.xf + (int64_t)min(b, (int)p.B - 1) * p.ldx + k0 + m * 8;
          xv[u][i][0] = *reinterpret_cast<const u32x4*>(src);
          xv[u][i][1] = *reinterpret_cast<const u32x4*>(src + 4);
        } else {
          xv[u][i][0] = *reinterpret_cast<const u32x4*>(p.x + (int64_t)min(b, (int)p.B - 1) * p.ldx + k0 + m * 8);
        }
      }
      if constexpr (NX) {
        nwv[u][0] = *reinterpret_cast<const u32x4*>(p.nw + k0 + m * 8);
        nwv[u][1] = *reinterpret_cast<const u32x4*>(p.nw + k0 + m * 8 + 4);
      }
      if constexpr (BITS == 4) {
        const unsigned col = p.gpg == 1 ? (unsigned)gg[u] : (unsigned)gg[u] / (unsigned)p.gpg;
#pragma unroll
        for (int t = 0; t < TP; ++t)
#pragma unroll
          for (int j = 0; j < 4; ++j) sc[u][t][j] = load_scale_t<SF16>(p, min((tile0 + t) * 16 + 4 * kq + j, p.N - 1), col);
      }
    }
#pragma unroll
    for (int u = 0; u < GP; ++u) {
      wave_lds_fence();  // the previous group's B-operand reads are done
      const bool use = u == 0 || second;
#pragma unroll
      for (int i = 0; i < XL; ++i) {
        const int b = (i * 64 + lane) / 16;
        u32x4 v;
        if constexpr (NX) {
          // fp16(x * w) of 8 columns; their squares into ss (counted once)
          f32x4 xa, xb;
          if constexpr (NX == 2) {
            // bf16 -> fp32 is exact; one rounding for the scale, as the
            // residual stream's first value
            const u32x4 e = xv[u][i][0];
            const float sc_e = p.emb_scale;
            xa = f32x4{__builtin_bit_cast(float, e.x << 16) * sc_e, __builtin_bit_cast(float, e.x & 0xFFFF0000u) * sc_e,
                       __builtin_bit_cast(float, e.y << 16) * sc_e, __builtin_bit_cast(float, e.y & 0xFFFF0000u) * sc_e};
            xb = f32x4{__builtin_bit_cast(float, e.z << 16) * sc_e, __builtin_bit_cast(float, e.z & 0xFFFF0000u) * sc_e,
                       __builtin_bit_cast(float, e.w << 16) * sc_e, __builtin_bit_cast(float, e.w & 0xFFFF0000u) * sc_e};
            if (use && b < p.B && gg[u] % (int)gridDim.x == (int)blockIdx.x) {
              float* dst = p.xout + (int64_t)b * p.ldx + (int64_t)gg[u] * kGK + m * 8;
              *reinterpret_cast<f32x4*>(dst) = xa;
              *reinterpret_cast<f32x4*>(dst + 4) = xb;
            }
          } else {
            xa = __builtin_bit_cast(f32x4, xv[u][i][0]);
            xb = __builtin_bit_cast(f32x4, xv[u][i][1]);
          }
          const f32x4 wa = __builtin_bit_cast(f32x4, nwv[u][0]), wb = __builtin_bit_cast(f32x4, nwv[u][1]);
          float t = 0.0f;
#pragma unroll
          for (int e = 0; e < 4; ++e) t = __builtin_fmaf(xa[e], xa[e], t);
#pragma unroll
          for (int e = 0; e < 4; ++e) t = __builtin_fmaf(xb[e], xb[e], t);
          ss[i] += use ? t : 0.0f;
          half8 hv;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            hv[e] = (_Float16)(xa[e] * wa[e]);
            hv[4 + e] = (_Float16)(xb[e] * wb[e]);
          }
          v = __builtin_bit_cast(u32x4, hv);
        } else {
          v = xv[u][i][0];
        }
        if (b >= p.B) v = u32x4{0u, 0u, 0u, 0u};
        if constexpr (BITS == 4) v = stage_perm_w4(v);
        *reinterpret_cast<u32x4*>(&xs[b * XP + m * 8]) = v;
      }
      wave_lds_fence();
      f32x4 acc[TP][NC];
#pragma unroll
      for (int t = 0; t < TP; ++t)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[t][c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        half8 a[TP];
#pragma unroll
        for (int t = 0; t < TP; ++t)
          a[t] = BITS == 4 ? a_w4(wv[u][t][s4]) : a_w8(wv[u][t][2 * s4], wv[u][t][2 * s4 + 1]);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const half8 bx = *reinterpret_cast<const half8*>(&xs[(c * 16 + m) * XP + kq * 32 + s4 * 8]);
#pragma unroll
          for (int t = 0; t < TP; ++t) acc[t][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[t], bx, acc[t][c], 0, 0, 0);
        }
      }
#pragma unroll
      for (int t = 0; t < TP; ++t)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if constexpr (BITS == 4) yacc[t][c][j] = __builtin_fmaf(use ? sc[u][t][j] : 0.0f, acc[t][c][j], yacc[t][c][j]);
            else yacc[t][c][j] += use ? acc[t][c][j] : 0.0f;
          }
        }
    }
  }

  if constexpr (NX) {
    // each row's sum over its 16 lanes (consecutive), one partial per wave
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      float t = ss[i];
      t += __shfl_xor(t, 1);
      t += __shfl_xor(t, 2);
      t += __shfl_xor(t, 4);
      t += __shfl_xor(t, 8);
      if (m == 0) ssp[wave][(i * 64 + lane) / 16] = t;
    }
  }
  __syncthreads();  // every wave is done with its x tile
#pragma unroll
  for (int t = 0; t < TP; ++t)
#pragma unroll
    for (int c = 0; c < NC; ++c) red[wave][t][c][lane] = yacc[t][c];
  __syncthreads();
  // wave t*NC + c sums column block c of tile t over the waves, in wave
  // order, and stores it: lane holds D[row 4*kq + j][column m]
  if (wave >= NC * TP) return;
  const int c = wave % NC;
  const int64_t tile = tile0 + wave / NC;
  const int64_t row0 = tile * 16;
  const int64_t b = c * 16 + m;
  if (b >= p.B) return;
  f32x4 v = red[0][wave / NC][c][lane];
#pragma unroll
  for (int w = 1; w < NW; ++w) v += red[w][wave / NC][c][lane];
  const int64_t n0 = row0 + 4 * kq;
  if (n0 >= p.N) return;
  if constexpr (BITS == 8) {
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] *= load_scale_t<SF16>(p, min(n0 + j, p.N - 1), 0);
  }
  if constexpr (NX) {
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) t += ssp[w][b];
    const float rstd = 1.0f / __builtin_sqrtf(t / (float)p.K + p.eps);
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] *= rstd;
  }
  if constexpr (QE == 3) {
    float* dr = p.y + b * p.ldy + n0;
    if (n0 + 4 <= p.N && (reinterpret_cast<uintptr_t>(dr) & 15) == 0) {
      *reinterpret_cast<f32x4*>(dr) = rold + v;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (n0 + j < p.N) dr[j] = rold[j] + v[j];
    }
    return;
  }
  if constexpr (QE == 2) {
    // tile t of head hh holds dims qb*8 + 0..7 (rows 0-7) and d/2 + qb*8 +
    // 0..7 (rows 8-15): lane (m, kq) and lane (m, kq ^ 2) are partners
    float part[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) part[j] = __shfl_xor(v[j], 32);
    const int t = (int)tile;
    const int hh = t * 16 / p.ro.d;
    const int qb = (t * 16 - hh * p.ro.d) / 16;
    // one token row, four consecutive dims (all loads before any use)
    const RopeOut& ro = p.ro;
    const int m = (int)(p.row_off + b);  // rows < 2^31: 32-bit division
    const int64_t bs = m / ro.n;
    const int ti = m - (int)bs * ro.n;
    const int64_t pos = (int64_t)ro.lens[bs] + ti;
    if (pos < 0 || pos >= ro.cap) return;
    const int dim0 = kq < 2 ? qb * 8 + 4 * kq : ro.d / 2 + qb * 8 + 4 * (kq - 2);
    float y[4] = {v[0], v[1], v[2], v[3]};
    if (ro.rope && hh < ro.H + ro.Hkv) {
      float c[4], sn[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c[j] = ro.cos[pos * ro.d + dim0 + j];
        sn[j] = ro.sin[pos * ro.d + dim0 + j];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // y[j] = x[j] cos[j] - x[j + d/2] sin[j];  y[j + d/2] = x[j + d/2] cos + x[j] sin
        const float sp = kq < 2 ? -part[j] : part[j];
        y[j] = v[j] * c[j] + sp * sn[j];
      }
    }
    uint16_t* dst;
    if (hh < ro.H) dst = ro.q + ((bs * ro.H + hh) * ro.n + ti) * (int64_t)ro.d;
    else if (hh < ro.H + ro.Hkv) dst = ro.kc + bs * ro.c_sb + (int64_t)(hh - ro.H) * ro.c_sh + pos * ro.c_sr;
    else dst = ro.vc + bs * ro.c_sb + (int64_t)(hh - ro.H - ro.Hkv) * ro.c_sh + pos * ro.c_sr;
#pragma unroll
    for (int j = 0; j < 4; ++j) dst[dim0 + j] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(y[j]));
    return;
  }
  if constexpr (QE == 1) {
    // rows 0-7 of the tile are the gate rows of hidden units tile*8 + 0..7,
    // rows 8-15 their up rows: lane (m, kq) with kq < 2 holds gates 4kq + j,
    // lane (m, kq + 2) the matching ups (same batch row m: N % 16 == 0, so
    // both lanes are live or both returned above)
    float u[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) u[j] = __shfl_xor(v[j], 32);
    if (kq >= 2) return;
    uint16_t* dh = p.yh + b * p.ldy + tile * 8 + 4 * kq;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float g = v[j];
      dh[j] = __builtin_bit_cast(uint16_t, (_Float16)(g / (1.0f + __expf(-g)) * u[j]));
    }
    return;
  }
  float* dst = p.y + b * p.ldy + n0;
  if (n0 + 4 <= p.N && (reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
    *reinterpret_cast<f32x4*>(dst) = v;
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (n0 + j < p.N) dst[j] = v[j];
  }
}

// The kernel: the scale format picks one of two bodies once, at entry.
template <int BITS, int NC, int NW, int QE = 0, int NX = 0, int TP = 1, int GP = 2>
__global__ __launch_bounds__(NW * 64) void k_qgemv_tile(QGemvParams p) {
  constexpr int XR = NC * 16;
  constexpr int XP = kGK + kXPad;
  constexpr size_t kXBytes = size_t(NW) * XR * XP * 2, kRBytes = size_t(NW) * TP * NC * 64 * 16;
  __shared__ __attribute__((aligned(16))) char smem[kXBytes > kRBytes ? kXBytes : kRBytes];
  __shared__ float ssp[NX ? NW : 1][NX ? XR : 1];
  if (p.sc_f16) qgemv_tile_body<BITS, NC, NW, QE, NX, TP, GP, true>(p, smem, &ssp[0][0]);
  else qgemv_tile_body<BITS, NC, NW, QE, NX, TP, GP, false>(p, smem, &ssp[0][0]);
}

// Large N, W4 with group-128 fp16 scales (the tied LM head of a draft):
// x (up to 32 batch rows x K) is staged in LDS once per workgroup, and each
// wave streams 16-row tiles (tiles w, w + 4, ... of the workgroup's range)
// through a ring of RS tiles in flight.  KG = K / 128 groups.  The MFMA takes
// x as its A operand and the weights as B, so a lane's four outputs belong to
// the one weight row it loads (batch rows 4kq .. 4kq + 3): each lane needs
// only its own row's scales.
template <int NC, int KG, int RS>
__global__ __launch_bounds__(kQNT) void k_qgemv_stream(QGemvParams p, int tiles_per_wg) {
  static_assert(KG == 4 || KG == 8, "K of 512 or 1024");
  using SV = std::conditional_t<KG == 8, u32x4, uint2>;  // one row's KG fp16 scales
  constexpr int XS = KG * kGK + kXPad;  // LDS row pitch of x (fp16)
  extern __shared__ __attribute__((aligned(16))) uint16_t xs_dyn[];
  uint16_t* xs = xs_dyn;
  const int tid = threadIdx.x;
  const int wave = tid / VNX_WAVE, lane = tid % VNX_WAVE;
  const int m = lane % 16, kq = lane / 16;
  for (int idx = tid; idx < NC * 16 * KG * 16; idx += kQNT) {
    const int b = idx / (KG * 16), c8 = idx % (KG * 16);
    u32x4 v = {0u, 0u, 0u, 0u};
    if (b < p.B) v = *reinterpret_cast<const u32x4*>(p.x + b * p.ldx + c8 * 8);
    *reinterpret_cast<u32x4*>(&xs[b * XS + c8 * 8]) = stage_perm_w4(v);
  }
  __syncthreads();

  const int64_t tiles = (p.N + 15) / 16;
  const int64_t t_lo = (int64_t)blockIdx.x * tiles_per_wg;
  const int64_t t_hi = min(tiles, t_lo + tiles_per_wg);
  // the workgroup's weight rows as a buffer resource: the ring's loads past
  // t_hi (issued unconditionally, so the waits count statically) read zeros
  // without a memory access instead of the next workgroup's rows
  const int64_t r_lo = t_lo * 16, r_hi = min(p.N, t_hi * 16);
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(p.w) + r_lo * p.ldw, (short)0, (int)((r_hi - r_lo) * p.ldw), 0x00020000);
  // one tile's loads: the lane's weight row (KG x 16 bytes) and its scales
  auto load = [&](int64_t tile, u32x4 (&wv)[KG], SV& sv) {
    const int64_t t = min(tile, tiles - 1);
    const int64_t rw = min(t * 16 + m, p.N - 1);
    const int64_t ra = min(rw, r_hi - 1);             // scale rows stay in the range (a cache hit past it)
    const int off = (int)(min(t * 16 + m, r_lo + 2 * tiles_per_wg * 16) - r_lo) * (int)p.ldw + kq * 16;
#pragma unroll
    for (int g = 0; g < KG; ++g)
      wv[g] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wres, off + g * 64, 0, 2));
    (void)rw;
    sv = *reinterpret_cast<const SV*>(static_cast<const uint16_t*>(p.sc) + ra * p.lds);
  };
  auto scale = [&](const SV& sv, int g) {
    uint32_t wd;
    if constexpr (KG == 8) {
      const int e = g / 2;
      wd = e == 0 ? sv.x : e == 1 ? sv.y : e == 2 ? sv.z : sv.w;
    } else {
      wd = (g / 2) == 0 ? sv.x : sv.y;
    }
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(wd >> (16 * (g % 2))));
  };
  auto compute_store = [&](int64_t tile, const u32x4 (&wv)[KG], const SV& sv) {
    f32x4 yacc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) yacc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < KG; ++g) {
      f32x4 acc[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
      const uint32_t wd[4] = {wv[g].x, wv[g].y, wv[g].z, wv[g].w};
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const half8 bw = a_w4(wd[s4]);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const half8 ax = *reinterpret_cast<const half8*>(&xs[(c * 16 + m) * XS + g * kGK + kq * 32 + s4 * 8]);
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax, bw, acc[c], 0, 0, 0);
        }
      }
      const float sg = scale(sv, g);
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j) yacc[c][j] = __builtin_fmaf(sg, acc[c][j], yacc[c][j]);
      // one group's conversions live at a time (the scheduler would otherwise
      // hoist all of them, and the registers would cap the occupancy at one wave)
      __builtin_amdgcn_sched_barrier(0);
    }
    if (tile >= t_hi) return;
    const int64_t n = tile * 16 + m;
    if (n >= p.N) return;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t b = c * 16 + 4 * kq + j;
        if (b < p.B) p.y[b * p.ldy + n] = yacc[c][j];
      }
  };
  // RS slots: slot j holds tile ta + 4j; each slot is reloaded (tiles past
  // the range load the last tile again) as soon as its math is issued
  u32x4 wr[RS][KG];
  SV sr[RS];
  const int64_t t0 = t_lo + wave;
#pragma unroll
  for (int j = 0; j < RS; ++j) load(t0 + 4 * j, wr[j], sr[j]);
  for (int64_t ta = t0; ta < t_hi; ta += 4 * RS) {
#pragma unroll
    for (int j = 0; j < RS; ++j) {
      compute_store(ta + 4 * j, wr[j], sr[j]);
      load(ta + 4 * (j + RS), wr[j], sr[j]);
    }
  }
}

// A operand of one MFMA k-step from one dword of the tiled layout, whose
// nibbles are in offset form (u = q + 8; nibble i = k i).  Two fp16 values
// per v_and_or_b32 under the 0x64 exponent bytes (1024 + u for the nibbles
// at bits 0 and 16, 1024 + 16u for those at bits 4 and 20), then one packed
// fp16 subtract (u - 8) or fused multiply-add ((1024 + 16u) / 16 - 72 =
// u - 8), all exact: 9 VALU ops per 8 weights.  Element order k = 0, 4, 1,
// 5, 2, 6, 3, 7 (stage_perm_w4o stages x the same way).  mlo / mhi / mag are
// the masks and exponent bytes, held in VGPRs so each pair is one
// v_and_or_b32 (a VOP3 instruction takes no literal here).
__device__ __forceinline__ half8 a_w4o(uint32_t u, uint32_t mlo, uint32_t mhi, uint32_t mag) {
  const uint32_t u8 = u >> 8;
  const fp16x2 off = {(__fp16)1032.0f, (__fp16)1032.0f};
  const fp16x2 sixteenth = {(__fp16)0.0625f, (__fp16)0.0625f};
  const fp16x2 m72 = {(__fp16)-72.0f, (__fp16)-72.0f};
  const fp16x2 h0 = __builtin_bit_cast(fp16x2, (u & mlo) | mag) - off;
  const fp16x2 h1 = __builtin_elementwise_fma(__builtin_bit_cast(fp16x2, (u & mhi) | mag), sixteenth, m72);
  const fp16x2 h2 = __builtin_bit_cast(fp16x2, (u8 & mlo) | mag) - off;
  const fp16x2 h3 = __builtin_elementwise_fma(__builtin_bit_cast(fp16x2, (u8 & mhi) | mag), sixteenth, m72);
  return pack_half8(h0, h1, h2, h3);
}

// x staging order of a_w4o: 8 consecutive fp16 (dwords (h0,h1) .. (h6,h7))
// as h0, h4, h1, h5, h2, h6, h3, h7.
__device__ __forceinline__ u32x4 stage_perm_w4o(u32x4 v) {
  u32x4 o;
  o.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);  // h0, h4
  o.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);  // h1, h5
  o.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);  // h2, h6
  o.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);  // h3, h7
  return o;
}

// The same product on the tiled weight layout (vnx_pack_w4_tiles): 16-row
// tile t holds KG loads of 1 KB, load g of lane l = (kq, m) being the 16
// bytes W[16t + m][64g + 16kq .. +16] (the lane's slice of row m, group g)
// with every nibble in offset form (q + 8), so every weight load of a wave
// reads one contiguous KB and converts with a_w4o.  Each wave takes
// steps s0, s0 + 4, ... of its workgroup's range (a step = TP adjacent
// tiles, whose MFMAs share each x fragment read from LDS) through a ring of
// RS steps; the ring's first loads are issued before x is staged, and no
// load reaches past the workgroup's range (a streaming read measured 6.2-6.5
// TB/s this way, against 4.7 with 64-byte row pieces and the ring's
// overshoot into the next workgroup's tiles).
template <int NC, int KG, int TP, int RS, int NW, int OCC, bool OB = false>
__global__ __launch_bounds__(NW * 64, OCC) void k_qgemv_tiles(QGemvParams p, int steps_per_wg) {
  static_assert(KG == 4 || KG == 8, "K of 512 or 1024");
  using SV = std::conditional_t<KG == 8, u32x4, uint2>;  // one row's KG fp16 scales
  constexpr int XS = KG * kGK + kXPad;                    // LDS row pitch of x (fp16)
  extern __shared__ __attribute__((aligned(16))) uint16_t xs_dyn[];
  uint16_t* xs = xs_dyn;
  const int tid = threadIdx.x;
  const int wave = tid / VNX_WAVE, lane = tid % VNX_WAVE;
  const int m = lane % 16, kq = lane / 16;
  const int64_t tiles = (p.N + 15) / 16;
  const int64_t steps = (tiles + TP - 1) / TP;
  const int64_t s_lo = (int64_t)blockIdx.x * steps_per_wg;
  const int64_t s_hi = min(steps, s_lo + steps_per_wg);
  // the workgroup's tiles as a buffer resource: every load below is issued
  // (so the waits count statically), and one past the range reads zeros
  // without a memory access
  constexpr int64_t kTileB = KG * 1024;
  const int64_t range_b = max((int64_t)0, s_hi - s_lo) * TP * kTileB;
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(p.w) + s_lo * TP * kTileB, (short)0, (int)range_b, 0x00020000);
  const int64_t last_row = min(p.N, (s_hi * TP) * 16) - 1;  // the range's last real weight row
  uint32_t mlo = 0x000F000Fu, mhi = 0x00F000F0u, mag = 0x64006400u;
  asm volatile("" : "+v"(mlo), "+v"(mhi), "+v"(mag));  // in VGPRs (see a_w4o)
  auto load = [&](int64_t st, u32x4 (&wv)[TP][KG], SV (&sv)[TP]) {
#pragma unroll
    for (int tp = 0; tp < TP; ++tp) {
      const int64_t rel = min(st - s_lo, (int64_t)steps_per_wg + 2 * NW * RS) * TP + tp;  // tiles from the range start
      const int off = (int)(rel * kTileB) + lane * 16;
#pragma unroll
      for (int g = 0; g < KG; ++g)
        wv[tp][g] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wres, off + g * 1024, 0, 2));
      const int64_t ra = min((s_lo * TP + rel) * 16 + m, last_row);
      sv[tp] = *reinterpret_cast<const SV*>(static_cast<const uint16_t*>(p.sc) + ra * p.lds);
    }
  };
  auto scale = [&](const SV& sv, int g) {
    uint32_t wd;
    if constexpr (KG == 8) {
      const int e = g / 2;
      wd = e == 0 ? sv.x : e == 1 ? sv.y : e == 2 ? sv.z : sv.w;
    } else {
      wd = (g / 2) == 0 ? sv.x : sv.y;
    }
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(wd >> (16 * (g % 2))));
  };
  auto compute_store = [&](int64_t st, const u32x4 (&wv)[TP][KG], const SV (&sv)[TP]) {
    f32x4 yacc[TP][NC];
#pragma unroll
    for (int tp = 0; tp < TP; ++tp)
#pragma unroll
      for (int c = 0; c < NC; ++c) yacc[tp][c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < KG; ++g) {
      f32x4 acc[TP][NC];
#pragma unroll
      for (int tp = 0; tp < TP; ++tp)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[tp][c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        half8 bw[TP];
#pragma unroll
        for (int tp = 0; tp < TP; ++tp) {
          const u32x4 v = wv[tp][g];
          bw[tp] = a_w4o(s4 == 0 ? v.x : s4 == 1 ? v.y : s4 == 2 ? v.z : v.w, mlo, mhi, mag);
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const half8 ax = *reinterpret_cast<const half8*>(&xs[(c * 16 + m) * XS + g * kGK + kq * 32 + s4 * 8]);
#pragma unroll
          for (int tp = 0; tp < TP; ++tp)
            acc[tp][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax, bw[tp], acc[tp][c], 0, 0, 0);
        }
      }
#pragma unroll
      for (int tp = 0; tp < TP; ++tp) {
        const float sg = scale(sv[tp], g);
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int j = 0; j < 4; ++j) yacc[tp][c][j] = __builtin_fmaf(sg, acc[tp][c][j], yacc[tp][c][j]);
      }
      // one group's conversions live at a time (keeps the register count,
      // and so two waves per SIMD)
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int tp = 0; tp < TP; ++tp) {
      const int64_t tile = st * TP + tp;
      const int64_t n = tile * 16 + m;
      if (tile >= tiles || n >= p.N) continue;
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t b = c * 16 + 4 * kq + j;
          if (b < p.B) {
            if constexpr (OB) p.yb[b * p.ldy + n] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(yacc[tp][c][j]));
            else p.y[b * p.ldy + n] = yacc[tp][c][j];
          }
        }
    }
  };
  u32x4 wr[RS][TP][KG];
  SV sr[RS][TP];
  const int64_t s0 = s_lo + wave;
#pragma unroll
  for (int j = 0; j < RS; ++j) load(s0 + NW * j, wr[j], sr[j]);
  // x (up to NC*16 batch rows) into LDS, in the A operand's k order; rows
  // past B are zeros
  for (int idx = tid; idx < NC * 16 * KG * 16; idx += NW * 64) {
    const int b = idx / (KG * 16), c8 = idx % (KG * 16);
    u32x4 v = {0u, 0u, 0u, 0u};
    if (b < p.B) v = *reinterpret_cast<const u32x4*>(p.x + b * p.ldx + c8 * 8);
    *reinterpret_cast<u32x4*>(&xs[b * XS + c8 * 8]) = stage_perm_w4o(v);
  }
  __syncthreads();
  for (int64_t sa = s0; sa < s_hi; sa += NW * RS) {
#pragma unroll
    for (int j = 0; j < RS; ++j) {
      const int64_t st = sa + NW * j;
      if (st < s_hi) compute_store(st, wr[j], sr[j]);  // uniform per wave
      load(st + NW * RS, wr[j], sr[j]);
    }
  }
}

// The tiled layout from the row-major packing: one thread per 16-byte piece
// of the output, every nibble flipped to offset form (q ^ 8 = q + 8 in 0..15);
// rows past N (the last tile's padding) hold q = 0.
__global__ void k_pack_w4_tiles(const uint8_t* __restrict__ wq, int64_t ldw, int64_t N, int kg, int64_t pieces,
                                uint8_t* __restrict__ out) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= pieces) return;
  const int l = (int)(q % 64);
  const int64_t tg = q / 64;  // tile * kg + g
  const int g = (int)(tg % kg);
  const int64_t t = tg / kg;
  const int64_t row = t * 16 + (l % 16);
  u32x4 v = {0u, 0u, 0u, 0u};
  if (row < N) v = *reinterpret_cast<const u32x4*>(wq + row * ldw + g * 64 + (l / 16) * 16);
  const uint32_t f = 0x88888888u;
  *reinterpret_cast<u32x4*>(out + q * 16) = u32x4{v.x ^ f, v.y ^ f, v.z ^ f, v.w ^ f};
}

// Dequantization (bit-exact reference for the kernels' weights):
// out[n][k] = q[n][k] * s[n][k / G] in fp32 (one rounded multiply).
__global__ void k_dequant(QGemvParams p, int bits, float* out, int64_t ldo) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t n = i / p.K, k = i % p.K;
  if (n >= p.N) return;
  int q;
  if (bits == 4) {
    const uint8_t byte = p.w[n * p.ldw + k / 2];
    const int nib = (k & 1) ? (byte >> 4) : (byte & 0xF);
    q = nib >= 8 ? nib - 16 : nib;
  } else {
    q = (int)static_cast<const int8_t*>(static_cast<const void*>(p.w))[n * p.ldw + k];
  }
  const float s = bits == 4 ? load_scale(p, n, k / p.G) : load_scale(p, n, 0);
  out[n * ldo + k] = (float)q * s;
}

constexpr int64_t kQTargetWgs = 512;
constexpr int64_t kQTileMaxN = 64 * kQTargetWgs;

static int qgemv_check(const QGemvParams& p, int bits) {
  if (!p.x || !p.w || !p.sc || (!p.y && !p.yh && !p.rope_on)) return VNX_ERR_INVALID_ARG;
  if (p.B < 0 || p.N < 0 || p.K <= 0) return VNX_ERR_INVALID_ARG;
  if (p.K % kGK) return VNX_ERR_UNSUPPORTED;
  if (bits == 4 && (p.G <= 0 || p.G % kGK || p.K % p.G)) return VNX_ERR_UNSUPPORTED;
  if (p.K > ((int64_t)1 << 30)) return VNX_ERR_UNSUPPORTED;
  if (p.ldx < p.K || (!p.rope_on && p.ldy < (p.yh ? p.N / 2 : p.N))) return VNX_ERR_INVALID_ARG;
  if (p.rope_on && (bits != 4 || p.N >= kQTileMaxN)) return VNX_ERR_UNSUPPORTED;
  // SwiGLU: blocks of 8 gate + 8 up rows, one 16-row tile each (tile kernel)
  if (p.yh && (p.N % 16 || p.N >= kQTileMaxN)) return VNX_ERR_UNSUPPORTED;
  // residual and normalized-input forms run the tile kernel only (W4)
  if ((p.resid || p.xf) && (bits != 4 || p.N >= kQTileMaxN)) return VNX_ERR_UNSUPPORTED;
  if (p.xf && (!p.nw || !(p.eps >= 0.0f))) return VNX_ERR_INVALID_ARG;
  if (p.ldw < (bits == 4 ? p.K / 2 : p.K)) return VNX_ERR_INVALID_ARG;
  if (p.lds < (bits == 4 ? p.K / p.G : 1)) return VNX_ERR_INVALID_ARG;
  // 16-byte vector loads of x (fp16, or fp32 rows to normalize) and of every row's weights.
  if (!aligned16(p.x) || p.ldx % (p.xf ? 4 : 8) || !aligned16(p.w) || p.ldw % 16) return VNX_ERR_UNSUPPORTED;
  if (p.xf && !aligned16(p.nw)) return VNX_ERR_UNSUPPORTED;
  return VNX_OK;
}

// Launch shape.  N >= kQTileMaxN: the LDS-staged kernel, 64*TPW rows per
// workgroup (TPW = 4 when the staged x slice is large, more than 16 batch
// columns, and N fills the GPU anyway, else 1), whole K.  Smaller N: the
// tile kernel, one 16-row tile per workgroup with K split over its waves.

static int qgemv_launch(QGemvParams p, int bits, hipStream_t s) {
  if (p.B == 0 || p.N == 0) return VNX_OK;
  // Batch columns in chunks of 32 (two MFMA column blocks) or one of 16.
  for (int64_t b0 = 0; b0 < p.B; b0 += 32) {
    QGemvParams c = p;
    c.x = p.x + b0 * p.ldx;
    if (p.xf) c.xf = p.xf + b0 * p.ldx;
    if (p.emb) {
      c.ids = p.ids + b0;
      c.xout = p.xout + b0 * p.ldx;
    }
    if (p.y) c.y = p.y + b0 * p.ldy;
    if (p.yh) c.yh = p.yh + b0 * p.ldy;
    c.row_off = b0;
    c.B = min((int64_t)32, p.B - b0);
    c.ksplit_len = c.K;
    const bool two = c.B > 16;
    if (c.N < kQTileMaxN) {
      // 8 waves per tile while the tiles leave CUs idle, 4 beyond
      const int64_t tiles = (c.N + 15) / 16;
      const bool wide = tiles <= device_cus();
      const dim3 grid((unsigned)tiles);
#define VNX_QTILE(BITS, NC, NW) \
  hipLaunchKernelGGL((k_qgemv_tile<BITS, NC, NW>), grid, dim3(NW * 64), 0, s, c)
#define VNX_QTILE_E(NC, NW, QE, NX) \
  hipLaunchKernelGGL((k_qgemv_tile<4, NC, NW, QE, NX>), grid, dim3(NW * 64), 0, s, c)
#define VNX_QTILE_E1(NC, QE, NX) \
  hipLaunchKernelGGL((k_qgemv_tile<4, NC, 8, QE, NX, 1, 1>), grid, dim3(8 * 64), 0, s, c)
#define VNX_QTILE_E2(NC, QE, NX) \
  hipLaunchKernelGGL((k_qgemv_tile<4, NC, 8, QE, NX, 2, 1>), grid2, dim3(8 * 64), 0, s, c)
      // epilogue variants: beyond one tile per CU, 2 tiles per 8-wave
      // workgroup (x loaded once for both; 2.4% of the config-5 round); one
      // group per wave where K has at most 8 groups (no second, zero-weighted
      // group)
      const bool g1 = c.K <= 8 * kGK;
      const dim3 grid2((unsigned)((tiles + 1) / 2));
#define VNX_QTILE_W(NC, QE, NX) \
  do { \
    if (wide) { if (g1) VNX_QTILE_E1(NC, QE, NX); else VNX_QTILE_E(NC, 8, QE, NX); } \
    else VNX_QTILE_E2(NC, QE, NX); \
  } while (0)
#define VNX_QTILE_Q(QE, NX) \
  do { \
    if (two) VNX_QTILE_W(2, QE, NX); else VNX_QTILE_W(1, QE, NX); \
  } while (0)
      if (c.rope_on) {
        if (c.emb) VNX_QTILE_Q(2, 2); else if (c.xf) VNX_QTILE_Q(2, 1); else VNX_QTILE_Q(2, 0);
      } else if (c.yh) {
        if (c.xf) VNX_QTILE_Q(1, 1); else VNX_QTILE_Q(1, 0);
      } else if (c.resid) {
        VNX_QTILE_Q(3, 0);
      } else if (bits == 4) {
        if (two) { if (wide) VNX_QTILE(4, 2, 8); else VNX_QTILE(4, 2, 4); }
        else { if (wide) VNX_QTILE(4, 1, 8); else VNX_QTILE(4, 1, 4); }
      } else {
        if (two) { if (wide) VNX_QTILE(8, 2, 8); else VNX_QTILE(8, 2, 4); }
        else { if (wide) VNX_QTILE(8, 1, 8); else VNX_QTILE(8, 1, 4); }
      }
#undef VNX_QTILE
#undef VNX_QTILE_E
#undef VNX_QTILE_E1
#undef VNX_QTILE_E2
#undef VNX_QTILE_W
#undef VNX_QTILE_Q
    } else if (bits == 4 && c.G == kGK && c.sc_f16 && c.lds % 8 == 0 && aligned16(c.sc) &&
               (c.K == 512 || c.K == 1024)) {
      // two workgroups per CU (x staged once each), tiles split evenly
      const int64_t tiles = (c.N + 15) / 16;
      const int64_t wgs_target = 2 * device_cus();
      int64_t tpw = (tiles + wgs_target - 1) / wgs_target;
      tpw = (tpw + 7) / 8 * 8;
      // a workgroup's row range (and the ring's overshoot) stays inside the
      // 32-bit buffer offsets
      tpw = min(tpw, ((int64_t)1 << 30) / (3 * 16 * c.ldw) / 8 * 8);
      const dim3 grid((unsigned)((tiles + tpw - 1) / tpw));
      const int nc = two ? 2 : 1;
      const size_t lds = (size_t)nc * 16 * (c.K + kXPad) * 2;
      // (a ring of 4 tiles measured 1.2x slower at B = 32: 199 VGPRs)
#define VNX_QSTREAM(NC, KG) \
  hipLaunchKernelGGL((k_qgemv_stream<NC, KG, 2>), grid, dim3(kQNT), lds, s, c, (int)tpw)
      if (c.K == 512) { if (two) VNX_QSTREAM(2, 4); else VNX_QSTREAM(1, 4); }
      else { if (two) VNX_QSTREAM(2, 8); else VNX_QSTREAM(1, 8); }
#undef VNX_QSTREAM
    } else {
      const int tpw = c.B > 16 && c.N >= 256 * kQTargetWgs ? 4 : 1;
      const dim3 grid((unsigned)((c.N + 64 * tpw - 1) / (64 * tpw)));
#define VNX_QLAUNCH(BITS, NC, TPW) hipLaunchKernelGGL((k_qgemv<BITS, NC, TPW>), grid, dim3(kQNT), 0, s, c)
      if (bits == 4) {
        if (two) { if (tpw == 4) VNX_QLAUNCH(4, 2, 4); else VNX_QLAUNCH(4, 2, 1); }
        else { if (tpw == 4) VNX_QLAUNCH(4, 1, 4); else VNX_QLAUNCH(4, 1, 1); }
      } else {
        if (two) { if (tpw == 4) VNX_QLAUNCH(8, 2, 4); else VNX_QLAUNCH(8, 2, 1); }
        else { if (tpw == 4) VNX_QLAUNCH(8, 1, 4); else VNX_QLAUNCH(8, 1, 1); }
      }
#undef VNX_QLAUNCH
    }
    VNX_LAUNCH_CHECK();
  }
  return VNX_OK;
}

// ---------------------------------------------------------------------------
// INT4 group-128 quantization on the device: the writer of the format the
// GEMVs read (quantize_int4_g: per group of 128 columns s = RN16(RN32(max|w|
// / 7)), 1/7 for an all-zero group; q = clamp(rint(w / f32(s)), -8, 7); two q
// per byte, the even column in the low nibble).  One wave per group, lane l
// holding columns 2l and 2l + 1: a wave max, then one packed byte per lane.
// A group with a non-finite weight or a scale that underflows fp16 is
// counted in *bad (the host turns it into an error).
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ float qw_load(const T* p) {
  if constexpr (std::is_same<T, float>::value) {
    return *p;
  } else if constexpr (std::is_same<T, __half>::value) {
    return __half2float(*p);
  } else {
    return __uint_as_float((uint32_t)(*reinterpret_cast<const uint16_t*>(p)) << 16);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void k_quantize_w4_g(const T* __restrict__ w, int64_t N, int64_t K, int64_t ldw,
                                                       uint8_t* __restrict__ out, int64_t ldo,
                                                       __half* __restrict__ sc, int64_t lds, int* bad) {
  const int lane = threadIdx.x & 63;
  const int64_t groups = K / kGK;
  const int64_t gid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (gid >= N * groups) return;  // uniform over the wave
  const int64_t row = gid / groups, g = gid - row * groups;
  const T* src = w + row * ldw + g * kGK + 2 * lane;
  const float a0 = qw_load(src), a1 = qw_load(src + 1);
  const bool nonfinite = !__builtin_isfinite(a0) || !__builtin_isfinite(a1);
  const float m = wave_max(fmaxf(fabsf(a0), fabsf(a1)));
  const float safe = m > 0.0f ? m : 1.0f;
  const __half s16 = __float2half_rn(safe / 7.0f);
  const float s = __half2float(s16);
  const int q0 = (int)fminf(fmaxf(rintf(a0 / s), -8.0f), 7.0f);
  const int q1 = (int)fminf(fmaxf(rintf(a1 / s), -8.0f), 7.0f);
  out[row * ldo + g * (kGK / 2) + lane] = (uint8_t)((q0 & 15) | ((q1 & 15) << 4));
  const bool flag = __ballot(nonfinite) != 0 || s == 0.0f;
  if (lane == 0) {
    sc[row * lds + g] = s16;
    if (flag && bad) atomicAdd(bad, 1);
  }
}

}  // namespace vnx

using namespace vnx;

extern "C" {

size_t vnx_gemv_workspace(int64_t B, int64_t N, int64_t K) {
  (void)B; (void)N; (void)K;
  return 256;  // no kernel needs it: the small-N kernel sums its K split inside a workgroup
}

int vnx_gemv_w4(const void* x, int64_t ldx, const uint8_t* wq, int64_t ldw, const void* scales,
                int scale_dtype, int64_t lds, int64_t B, int64_t N, int64_t K, int group, float* y,
                int64_t ldy, void* workspace, size_t workspace_bytes, void* stream) {
  if (scale_dtype != VNX_F16 && scale_dtype != VNX_F32) return VNX_ERR_UNSUPPORTED;
  QGemvParams p{};
  p.x = static_cast<const uint16_t*>(x); p.ldx = ldx; p.w = wq; p.ldw = ldw; p.sc = scales; p.lds = lds;
  p.sc_f16 = scale_dtype == VNX_F16; p.B = B; p.N = N; p.K = K; p.G = group; p.y = y; p.ldy = ldy;
  p.gpg = group / kGK;
  const int st = qgemv_check(p, 4);
  if (st) return st;
  (void)workspace; (void)workspace_bytes;
  return qgemv_launch(p, 4, static_cast<hipStream_t>(stream));
}

int vnx_gemv_w4_swiglu(const void* x, int64_t ldx, const float* norm_w, float eps, const uint8_t* wq, int64_t ldw,
                       const void* scales, int scale_dtype, int64_t lds, int64_t B, int64_t N, int64_t K, int group,
                       void* y, int64_t ldy, void* stream) {
  if (scale_dtype != VNX_F16 && scale_dtype != VNX_F32) return VNX_ERR_UNSUPPORTED;
  if (!y) return VNX_ERR_INVALID_ARG;
  QGemvParams p{};
  if (norm_w) { p.xf = static_cast<const float*>(x); p.nw = norm_w; p.eps = eps; }
  p.x = static_cast<const uint16_t*>(x); p.ldx = ldx; p.w = wq; p.ldw = ldw; p.sc = scales; p.lds = lds;
  p.sc_f16 = scale_dtype == VNX_F16; p.B = B; p.N = N; p.K = K; p.G = group; p.yh = static_cast<uint16_t*>(y);
  p.ldy = ldy; p.gpg = group / kGK;
  const int st = qgemv_check(p, 4);
  if (st) return st;
  return qgemv_launch(p, 4, static_cast<hipStream_t>(stream));
}

int vnx_gemv_w4_rope_kv(const void* x, int64_t ldx, const float* norm_w, float eps, const uint8_t* wq, int64_t ldw,
                        const void* scales, int scale_dtype, int64_t lds, int64_t B, int64_t N, int64_t K, int group,
                        const vnx_rope_kv_args* rk, void* stream) {
  if (scale_dtype != VNX_F16 && scale_dtype != VNX_F32) return VNX_ERR_UNSUPPORTED;
  QGemvParams p{};
  if (norm_w) { p.xf = static_cast<const float*>(x); p.nw = norm_w; p.eps = eps; }
  const int rs = rope_out_from(rk, N, &p.ro);
  if (rs) return rs;
  if (B % rk->n) return VNX_ERR_INVALID_ARG;  // rows are whole sequences of n tokens
  p.x = static_cast<const uint16_t*>(x); p.ldx = ldx; p.w = wq; p.ldw = ldw; p.sc = scales; p.lds = lds;
  p.sc_f16 = scale_dtype == VNX_F16; p.B = B; p.N = N; p.K = K; p.G = group; p.rope_on = 1;
  p.gpg = group / kGK;
  const int st = qgemv_check(p, 4);
  if (st) return st;
  return qgemv_launch(p, 4, static_cast<hipStream_t>(stream));
}

int vnx_gemv_w4_rope_kv_embed(const int64_t* tokens, const void* emb, int emb_dtype, int64_t lde, int64_t vocab,
                              float scale, float* x_out, int64_t ldx, const float* norm_w, float eps,
                              const uint8_t* wq, int64_t ldw, const void* scales, int scale_dtype, int64_t lds,
                              int64_t B, int64_t N, int64_t K, int group, const vnx_rope_kv_args* rk, void* stream) {
  if (scale_dtype != VNX_F16 && scale_dtype != VNX_F32) return VNX_ERR_UNSUPPORTED;
  if (!tokens || !emb || !x_out || !norm_w || vocab < 1 || lde < K) return VNX_ERR_INVALID_ARG;
  if (emb_dtype != VNX_BF16) return VNX_ERR_UNSUPPORTED;
  if (lde % 8 || !aligned16(emb)) return VNX_ERR_UNSUPPORTED;  // 16-byte row loads
  QGemvParams p{};
  p.xf = x_out; p.nw = norm_w; p.eps = eps;
  p.ids = tokens; p.emb = static_cast<const uint16_t*>(emb); p.lde = lde; p.vocab = vocab; p.emb_scale = scale;
  p.xout = x_out;
  const int rs = rope_out_from(rk, N, &p.ro);
  if (rs) return rs;
  if (B % rk->n) return VNX_ERR_INVALID_ARG;  // rows are whole sequences of n tokens
  p.x = reinterpret_cast<const uint16_t*>(x_out); p.ldx = ldx; p.w = wq; p.ldw = ldw; p.sc = scales; p.lds = lds;
  p.sc_f16 = scale_dtype == VNX_F16; p.B = B; p.N = N; p.K = K; p.G = group; p.rope_on = 1;
  p.gpg = group / kGK;
  const int st = qgemv_check(p, 4);
  if (st) return st;
  return qgemv_launch(p, 4, static_cast<hipStream_t>(stream));
}

int vnx_gemv_w4_residual(const void* x, int64_t ldx, const uint8_t* wq, int64_t ldw, const void* scales,
                         int scale_dtype, int64_t lds, int64_t B, int64_t N, int64_t K, int group, float* res,
                         int64_t ldr, void* stream) {
  if (scale_dtype != VNX_F16 && scale_dtype != VNX_F32) return VNX_ERR_UNSUPPORTED;
  QGemvParams p{};
  p.x = static_cast<const uint16_t*>(x); p.ldx = ldx; p.w = wq; p.ldw = ldw; p.sc = scales; p.lds = lds;
  p.sc_f16 = scale_dtype == VNX_F16; p.B = B; p.N = N; p.K = K; p.G = group; p.y = res; p.ldy = ldr;
  p.gpg = group / kGK; p.resid = 1;
  const int st = qgemv_check(p, 4);
  if (st) return st;
  return qgemv_launch(p, 4, static_cast<hipStream_t>(stream));
}

size_t vnx_w4_tiles_bytes(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0 || K % kGK) return 0;
  return (size_t)((N + 15) / 16) * 16 * (size_t)(K / 2);
}

int vnx_pack_w4_tiles(const uint8_t* wq, int64_t ldw, int64_t N, int64_t K, uint8_t* out, void* stream) {
  if (!wq || !out || N <= 0 || K <= 0 || ldw < K / 2) return VNX_ERR_INVALID_ARG;
  if (K % kGK) return VNX_ERR_UNSUPPORTED;
  if (!aligned16(wq) || ldw % 16 || !aligned16(out)) return VNX_ERR_UNSUPPORTED;
  const int kg = (int)(K / kGK);
  const int64_t pieces = (N + 15) / 16 * kg * 64;
  hipLaunchKernelGGL(k_pack_w4_tiles, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), wq, ldw, N, kg, pieces, out);
  VNX_LAUNCH_CHECK();
  return VNX_OK;
}

int vnx_gemv_w4_tiles(const void* x, int64_t ldx, const uint8_t* wt, const void* scales, int64_t lds, int64_t B,
                      int64_t N, int64_t K, float* y, int64_t ldy, void* stream) {
  return vnx_gemv_w4_tiles_out(x, ldx, wt, scales, lds, B, N, K, y, VNX_F32, ldy, stream);
}

int vnx_gemv_w4_tiles_out(const void* x, int64_t ldx, const uint8_t* wt, const void* scales, int64_t lds, int64_t B,
                          int64_t N, int64_t K, void* y, int y_dtype, int64_t ldy, void* stream) {
  if (!x || !wt || !scales || !y || B < 0 || N <= 0 || K <= 0) return VNX_ERR_INVALID_ARG;
  if (y_dtype != VNX_F32 && y_dtype != VNX_BF16) return VNX_ERR_UNSUPPORTED;
  const bool ob = y_dtype == VNX_BF16;
  if (K != 512 && K != 1024) return VNX_ERR_UNSUPPORTED;
  if (ldx < K || ldy < N || lds < K / kGK) return VNX_ERR_INVALID_ARG;
  // 16-byte loads of x and of the tiles; 8- or 16-byte loads of a row's scales
  if (!aligned16(x) || ldx % 8 || !aligned16(wt) || !aligned16(scales) || lds % (K == 1024 ? 8 : 4))
    return VNX_ERR_UNSUPPORTED;
  if (B == 0) return VNX_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t tiles = (N + 15) / 16;
  for (int64_t b0 = 0; b0 < B; b0 += 32) {
    QGemvParams c{};
    c.x = static_cast<const uint16_t*>(x) + b0 * ldx; c.ldx = ldx; c.w = wt; c.sc = scales; c.lds = lds;
    c.sc_f16 = 1; c.B = min((int64_t)32, B - b0); c.N = N; c.K = K; c.G = kGK; c.gpg = 1;
    if (ob) c.yb = static_cast<uint16_t*>(y) + b0 * ldy;
    else c.y = static_cast<float*>(y) + b0 * ldy;
    c.ldy = ldy; c.row_off = b0;
    const bool two = c.B > 16;
    // one tile per step; up to 16 batch rows: 4-wave workgroups, about 4
    // per CU over the launch; beyond: 8-wave workgroups (one staged copy of
    // the 2 x 16 rows of x for twice the waves), about 2 per CU
    constexpr int TP = 1;
    const int64_t steps = (tiles + TP - 1) / TP;
    const int64_t wgs_target = (two ? 2 : 4) * device_cus();
    // a workgroup's range stays well inside the 32-bit buffer offsets
    const int64_t spw_max = ((int64_t)1 << 30) / (TP * (K / kGK) * 1024);
    const int64_t spw = min(spw_max, max((int64_t)4, (steps + wgs_target - 1) / wgs_target));
    const dim3 grid((unsigned)((steps + spw - 1) / spw));
    const size_t lds_bytes = (size_t)(two ? 2 : 1) * 16 * (K + kXPad) * 2;
#define VNX_QTILES(NC, KG, RS, NW, OCC) \
  do { \
    if (ob) hipLaunchKernelGGL((k_qgemv_tiles<NC, KG, TP, RS, NW, OCC, true>), grid, dim3(NW * 64), lds_bytes, s, c, \
                               (int)spw); \
    else hipLaunchKernelGGL((k_qgemv_tiles<NC, KG, TP, RS, NW, OCC>), grid, dim3(NW * 64), lds_bytes, s, c, (int)spw); \
  } while (0)
    // (measured on the 248,320 x 1024 head, three weight copies: one column
    // block with a 2-step ring at 4 waves per SIMD, B = 1 26.9 us; two blocks
    // with 8-wave workgroups and no ring (128 VGPRs, 4 waves per SIMD) 37.1
    // us, against 39.5 us for 4-wave workgroups with the ring at 2 waves per
    // SIMD and 67 us where the ring at 4 waves per SIMD spilled)
    if (K == 512) { if (two) VNX_QTILES(2, 4, 1, 8, 4); else VNX_QTILES(1, 4, 2, 4, 4); }
    else { if (two) VNX_QTILES(2, 8, 1, 8, 4); else VNX_QTILES(1, 8, 2, 4, 4); }
#undef VNX_QTILES
    VNX_LAUNCH_CHECK();
  }
  return VNX_OK;
}

int vnx_gemv_w8(const void* x, int64_t ldx, const int8_t* wq, int64_t ldw, const float* scale,
                int64_t B, int64_t N, int64_t K, float* y, int64_t ldy, void* workspace,
                size_t workspace_bytes, void* stream) {
  QGemvParams p{};
  p.x = static_cast<const uint16_t*>(x); p.ldx = ldx; p.w = reinterpret_cast<const uint8_t*>(wq); p.ldw = ldw;
  p.sc = scale; p.lds = 1; p.sc_f16 = 0; p.B = B; p.N = N; p.K = K; p.G = (int)K; p.y = y; p.ldy = ldy;
  p.gpg = (int)(K / kGK);
  const int st = qgemv_check(p, 8);
  if (st) return st;
  (void)workspace; (void)workspace_bytes;
  return qgemv_launch(p, 8, static_cast<hipStream_t>(stream));
}

int vnx_dequant_w4(const uint8_t* wq, int64_t ldw, const void* scales, int scale_dtype, int64_t lds,
                   int64_t N, int64_t K, int group, float* out, int64_t ldo, void* stream) {
  if (scale_dtype != VNX_F16 && scale_dtype != VNX_F32) return VNX_ERR_UNSUPPORTED;
  if (!wq || !scales || !out || N < 0 || K <= 0 || group <= 0 || K % group) return VNX_ERR_INVALID_ARG;
  if (ldw < (K + 1) / 2 || lds < K / group || ldo < K) return VNX_ERR_INVALID_ARG;
  if (N == 0) return VNX_OK;
  QGemvParams p{};
  p.w = wq; p.ldw = ldw; p.sc = scales; p.lds = lds; p.sc_f16 = scale_dtype == VNX_F16;
  p.N = N; p.K = K; p.G = group;
  const int64_t n = N * K;
  hipLaunchKernelGGL(k_dequant, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), p, 4, out, ldo);
  VNX_LAUNCH_CHECK();
  return VNX_OK;
}

int vnx_quantize_w4_g(const void* w, int dtype, int64_t N, int64_t K, int64_t ldw, int group, uint8_t* packed,
                      int64_t ldp, void* scales, int64_t lds, int32_t* bad_groups, void* stream) {
  if (dtype != VNX_F32 && dtype != VNX_BF16 && dtype != VNX_F16) return VNX_ERR_UNSUPPORTED;
  if (group != kGK) return VNX_ERR_UNSUPPORTED;
  if (!w || !packed || !scales || N < 0 || K <= 0 || K % kGK || ldw < K || ldp < K / 2 || lds < K / kGK)
    return VNX_ERR_INVALID_ARG;
  if (N == 0) return VNX_OK;
  const int64_t waves = N * (K / kGK);
  if ((waves + 3) / 4 >= INT32_MAX) return VNX_ERR_UNSUPPORTED;
  const dim3 grid((unsigned)((waves + 3) / 4));
  hipStream_t s = static_cast<hipStream_t>(stream);
  __half* sc = static_cast<__half*>(scales);
  if (dtype == VNX_F32)
    hipLaunchKernelGGL(k_quantize_w4_g<float>, grid, dim3(256), 0, s, static_cast<const float*>(w), N, K, ldw,
                       packed, ldp, sc, lds, bad_groups);
  else if (dtype == VNX_F16)
    hipLaunchKernelGGL(k_quantize_w4_g<__half>, grid, dim3(256), 0, s, static_cast<const __half*>(w), N, K, ldw,
                       packed, ldp, sc, lds, bad_groups);
  else
    hipLaunchKernelGGL(k_quantize_w4_g<__hip_bfloat16>, grid, dim3(256), 0, s,
                       static_cast<const __hip_bfloat16*>(w), N, K, ldw, packed, ldp, sc, lds, bad_groups);
  VNX_LAUNCH_CHECK();
  return VNX_OK;
}

int vnx_dequant_w8(const int8_t* wq, int64_t ldw, const float* scale, int64_t N, int64_t K, float* out,
                   int64_t ldo, void* stream) {
  if (!wq || !scale || !out || N < 0 || K <= 0 || ldw < K || ldo < K) return VNX_ERR_INVALID_ARG;
  if (N == 0) return VNX_OK;
  QGemvParams p{};
  p.w = reinterpret_cast<const uint8_t*>(wq); p.ldw = ldw; p.sc = scale; p.lds = 1; p.sc_f16 = 0;
  p.N = N; p.K = K; p.G = (int)K;
  const int64_t n = N * K;
  hipLaunchKernelGGL(k_dequant, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), p, 8, out, ldo);
  VNX_LAUNCH_CHECK();
  return VNX_OK;
}

}  // extern "C"
