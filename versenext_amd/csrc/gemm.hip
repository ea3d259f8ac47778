// Skinny bf16 GEMM for the verify forward (vnx_gemm_bf16): Y = X . W^T for
// the M <= a few hundred token rows of one speculative round (batch x (k+1)),
// X (M, K) bf16 activations, W (N, K) bf16 (the nn.Linear layout, packed once
// by vnx_pack_bf16), fp32 accumulation.  This is the Linear of the target's
// verify forward (packages/verse_torch/verse_torch/vnnn.py Linear.forward:
// x @ W^T), with the SwiGLU activation of SwiGLUMLP (vnnn.py:779-807) and the
// routing weight of a MoD expert (packages/verse_nex/verse_nex/mod.py:
// 466-600) optionally fused into the epilogue.
//
// At M ~ 224 the product sits near the machine balance (224 flops per weight
// byte): the weights stream from HBM once, the activations are re-read from
// L2 by every workgroup, and the per-CU L1 bandwidth decides the time.  So
// every load is a full-line wave access:
//  - W is packed into the v_mfma_f32_32x32x16_bf16 B-operand order: for row
//    tile t (32 rows), K chunk c (64) and k-step s, lane (r = lane % 32,
//    h = lane / 32) finds its 8 values W[t*32 + r][c*64 + h*32 + s*8 ..] at
//    packed[((t*nch + c)*4 + s)*512 + lane*8]: one contiguous KB per wave
//    load, four per chunk;
//  - X goes through LDS: the workgroup loads 32 rows x 64 k per chunk with
//    row-contiguous 16-byte lane loads, stores them with the 16-byte column
//    index XOR-swizzled by (row / 2) % 8 (conflict-free both ways), and each
//    wave reads its A operands (the same k permutation h*32 + s*8 as W, so
//    the dot product is unchanged).
// A workgroup owns a 32-row M tile and WN adjacent 32-column N tiles; its 4
// waves are WN (N tiles) x WK (K splits, chunks kw, kw + WK, ...), the K
// splits summed through LDS in split order (deterministic).  Workgroups are
// ordered so that the M tiles of one N group land on one XCD (ids t, t + 8,
// ...), whose L2 then serves that group's W rows to all of them.
#include <stdlib.h>

#include "vnx_internal.h"

namespace vnx {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kVgChunk = 64;  // K per chunk
constexpr int kVgXcds = 8;    // XCDs the dispatcher deals workgroups over
constexpr int kVgRowB = 128;  // bytes of one staged X row (64 bf16)
constexpr int kVgNormMaxK = 2048;  // NX: K of the normalized rows (norm weight staged in LDS)

struct VgParams {
  const uint16_t* x;
  const uint16_t* w;       // packed
  void* y;
  const float* comb;       // SwiGLU weights comb[m * ldc + z], or NULL
  int64_t ldx, sxb, swb, ldy, syb, ldc;
  int M, N, K;             // N = rows of W
  int mt, nt, ng;          // 32-row tiles of M and N; N groups of WN tiles
  int vec_out;             // N % 32 == 0, rows of y 16-byte aligned: tiles leave through LDS
  const float* xf;         // NX: the fp32 rows to normalize (x unused), pitch ldx
  const float* nw;         // NX: RMSNorm weight (K)
  float eps;
  // NX 2: the rows to normalize are the token embedding (xf unused): row m
  // is emb[ids[m]] * emb_scale (bf16 table, ids clamped to [0, vocab)); the
  // workgroups of N group c % ng write chunk c of their rows to xout (pitch ldx)
  const int64_t* ids;
  const uint16_t* emb;
  int64_t lde, vocab;
  float emb_scale;
  float* xout;
};



template <int OT>
__device__ __forceinline__ void vg_store(char* y, int64_t off, float v) {
  if constexpr (OT == 0) {
    reinterpret_cast<float*>(y)[off] = v;
  } else if constexpr (OT == 1) {
    reinterpret_cast<__bf16*>(y)[off] = static_cast<__bf16>(v);
  } else {
    reinterpret_cast<_Float16*>(y)[off] = static_cast<_Float16>(v);
  }
}

// Eight consecutive outputs of type OT from fp32 (16 bytes for bf16 / fp16,
// 32 for fp32).
template <int OT>
__device__ __forceinline__ void vg_store8(char* y, int64_t off, const float (&v)[8]) {
  if constexpr (OT == 0) {
    float* d = reinterpret_cast<float*>(y) + off;
    *reinterpret_cast<f32x4*>(d) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(d + 4) = f32x4{v[4], v[5], v[6], v[7]};
  } else if constexpr (OT == 1) {
    __bf16 t[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) t[e] = static_cast<__bf16>(v[e]);
    *reinterpret_cast<u32x4*>(reinterpret_cast<__bf16*>(y) + off) = __builtin_bit_cast(u32x4, t);
  } else {
    _Float16 t[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) t[e] = static_cast<_Float16>(v[e]);
    *reinterpret_cast<u32x4*>(reinterpret_cast<_Float16*>(y) + off) = __builtin_bit_cast(u32x4, t);
  }
}

__device__ __forceinline__ bf16x8 as_b8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// LDS byte offset of 16-byte column c16 (0..7) of staged row r (0..31).
__device__ __forceinline__ int xs_off(int r, int c16) { return r * kVgRowB + ((c16 ^ ((r >> 1) & 7)) << 4); }

// EPI 0: y[m, n] = acc.  EPI 1 (SwiGLU): W rows come in blocks of 32, the
// first 16 the gate rows and the last 16 the up rows of hidden units
// blk*16 .. +16; y[m, blk*16 + c] = comb * silu(gate) * up.  EPI 3
// (residual): y fp32, y[m, n] += acc.
// NX: X is RMSNorm(xf) (vnnn.py:593-615): rows of xf times the norm weight
// are staged as bf16, each thread also summing the squares of its row's
// values, and the epilogue scales row m by rstd_m = 1/sqrt(mean x^2 + eps)
// (the norm's per-row factor, applied to the fp32 accumulators).
template <int OT, int EPI, int WN, int NX = 0>
__global__ __launch_bounds__(256) void k_vgemm(VgParams p) {
  constexpr int WK = 4 / WN;
  constexpr int SLAB = WK * 32 * kVgRowB;  // staged X bytes per pass (WK chunks)
  constexpr int RED = 3 * 64 * 64;         // K-split partial tiles
  constexpr int TP = 36;                   // row pitch (floats) of the output transpose tiles
  constexpr int TR = WK > 1 ? RED : 0;     // their offset: past the partial tiles, else over the dead X buffers
  constexpr int TRB = TR + WN * 32 * TP * 4;
  constexpr int SMB = 2 * SLAB > TRB ? 2 * SLAB : TRB;
  static_assert(SMB >= RED, "the partial tiles fit");
  __shared__ __attribute__((aligned(16))) char smem[SMB];
  __shared__ float rsd[NX ? 32 : 1];
  __shared__ __attribute__((aligned(16))) float nws[NX ? kVgNormMaxK : 4];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave % WN, wk = wave / WN;
  const int z = blockIdx.y;
  const int t = blockIdx.x;
  // the M tiles of one N group on one XCD (ids t, t + 8, ...)
  const int grp = t / (kVgXcds * p.mt), rem = t - grp * (kVgXcds * p.mt);
  const int gi = grp * kVgXcds + rem % kVgXcds;
  const int mi = rem / kVgXcds;
  if (gi >= p.ng) return;  // uniform over the workgroup
  const int m0 = mi * 32;
  const int ni = gi * WN + wn;             // this wave's N tile (past nt: computes, never stores)
  const int nie = ni < p.nt ? ni : p.nt - 1;
  const int r = lane & 31, h = lane >> 5;
  const int nch = p.K / kVgChunk;
  const int npass = (nch + WK - 1) / WK;

  // X staging: thread tid loads, for j < WK, chunk (pass*WK + j), row
  // tid / 8, 16-byte column tid % 8.
  const int xr = tid >> 3, xc = tid & 7;
  const int xrc = min(m0 + xr, p.M - 1);
  const uint16_t* xrow = p.x + z * p.sxb + (int64_t)xrc * p.ldx + xc * 8;
  const float* xfrow = NX == 1 ? p.xf + (int64_t)xrc * p.ldx + xc * 8 : nullptr;
  const uint16_t* erow = nullptr;  // NX 2: this thread's embedding row, column xc*8
  if constexpr (NX == 2) {
    int64_t tok = p.ids[xrc];
    tok = tok < 0 ? 0 : (tok >= p.vocab ? p.vocab - 1 : tok);  // never outside the table
    erow = p.emb + tok * p.lde + xc * 8;
  }
  const uint32_t xkeep = m0 + xr < p.M ? 0xFFFFFFFFu : 0u;
  const uint16_t* wt = p.w + z * p.swb + (int64_t)nie * nch * 2048 + lane * 8;

  f32x16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
  // EPI 3: the residual values this lane adds to load now, under the K loop
  // (only split 0 stores).  vec_out: row m0 + lane/2, columns
  // ni*32 + 16 (lane % 2) .. +16, the layout of the transposed tile; else
  // rows 8i + 4h + e of column ni*32 + r, the accumulator layout.
  // The loads land in their final registers (a copy beside them would wait
  // for them at once), under a wave-uniform branch.
  f32x4 old[EPI == 3 ? 4 : 1];
  if constexpr (EPI == 3) {
    if (wk == 0) {
      if (p.vec_out) {
        const float* yf = reinterpret_cast<const float*>(p.y) + (int64_t)z * p.syb +
                          (int64_t)min(m0 + (lane >> 1), p.M - 1) * p.ldy + nie * 32 + 16 * (lane & 1);
#pragma unroll
        for (int q = 0; q < 4; ++q) old[q] = *reinterpret_cast<const f32x4*>(yf + 4 * q);
      } else {
        const float* yf = reinterpret_cast<const float*>(p.y) + (int64_t)z * p.syb + min(ni * 32 + r, p.N - 1);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) old[i][e] = yf[(int64_t)min(m0 + 8 * i + 4 * h + e, p.M - 1) * p.ldy];
      }
    }
  }
  float ss = 0.0f;  // NX: sum of squares of this thread's values of row xr
  // NX: the norm weight goes to LDS once per workgroup; its loads issue
  // before the ring's first loads, so their latencies overlap
  f32x4 nwr[NX ? kVgNormMaxK / 1024 : 1];
  if constexpr (NX) {
#pragma unroll
    for (int i = 0; i < kVgNormMaxK / 1024; ++i) {
      const int k = (tid + 256 * i) * 4;
      nwr[i] = k < p.K ? *reinterpret_cast<const f32x4*>(p.nw + k) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  // Loads run PD passes ahead of the math: pass ps lives in ring slot
  // ps % PD (the loop is unrolled by PD so the slots are registers).  NX
  // loads 8 fp32 per chunk instead of 8 bf16.
  constexpr int PD = NX ? 2 : (WK > 2 ? 2 : 4);
  constexpr int XW = NX ? 2 : 1;  // 16-byte loads per chunk
  u32x4 xv[PD][WK][XW], wv[PD][4];
  auto load_pass = [&](int ps, u32x4 (&xs)[WK][XW], u32x4 (&ws)[4]) {
#pragma unroll
    for (int j = 0; j < WK; ++j) {
      const int c = min(ps * WK + j, nch - 1);
      if constexpr (NX) {
        if constexpr (NX == 2) {
          xs[j][0] = *reinterpret_cast<const u32x4*>(erow + c * kVgChunk);
        } else {
          xs[j][0] = *reinterpret_cast<const u32x4*>(xfrow + c * kVgChunk);
          xs[j][1] = *reinterpret_cast<const u32x4*>(xfrow + c * kVgChunk + 4);
        }
      } else {
        xs[j][0] = *reinterpret_cast<const u32x4*>(xrow + c * kVgChunk);
      }
    }
    const int c = min(ps * WK + wk, nch - 1);
#pragma unroll
    for (int s = 0; s < 4; ++s)
      ws[s] = *reinterpret_cast<const u32x4*>(wt + (c * 4 + s) * 512);  // re-read by the M tiles: keep in L2
  };
#pragma unroll
  for (int j = 0; j < PD; ++j) load_pass(j, xv[j], wv[j]);
  if constexpr (NX) {
#pragma unroll
    for (int i = 0; i < kVgNormMaxK / 1024; ++i) {
      const int k = (tid + 256 * i) * 4;
      if (k < p.K) *reinterpret_cast<f32x4*>(&nws[k]) = nwr[i];
    }
    __syncthreads();
  }
  for (int ps0 = 0; ps0 < npass; ps0 += PD) {
#pragma unroll
    for (int j = 0; j < PD; ++j) {
      const int ps = ps0 + j;
      char* buf = smem + (ps & 1) * SLAB;
#pragma unroll
      for (int q = 0; q < WK; ++q) {
        u32x4 v;
        if constexpr (NX) {
          // bf16(x * w) of 8 consecutive columns; their squares into ss
          const bool live = ps * WK + q < nch;  // clamped re-reads are not summed
          const int c = min(ps * WK + q, nch - 1);
          f32x4 xa, xb;
          if constexpr (NX == 2) {
            // bf16 -> fp32 is exact; one rounding for the scale (the
            // residual stream's first value)
            const u32x4 e = xv[j][q][0];
            const float se = p.emb_scale;
            xa = f32x4{__builtin_bit_cast(float, e.x << 16) * se, __builtin_bit_cast(float, e.x & 0xFFFF0000u) * se,
                       __builtin_bit_cast(float, e.y << 16) * se, __builtin_bit_cast(float, e.y & 0xFFFF0000u) * se};
            xb = f32x4{__builtin_bit_cast(float, e.z << 16) * se, __builtin_bit_cast(float, e.z & 0xFFFF0000u) * se,
                       __builtin_bit_cast(float, e.w << 16) * se, __builtin_bit_cast(float, e.w & 0xFFFF0000u) * se};
            if (live && c % p.ng == gi && m0 + xr < p.M) {
              float* dst = p.xout + (int64_t)(m0 + xr) * p.ldx + c * kVgChunk + xc * 8;
              *reinterpret_cast<f32x4*>(dst) = xa;
              *reinterpret_cast<f32x4*>(dst + 4) = xb;
            }
          } else {
            xa = __builtin_bit_cast(f32x4, xv[j][q][0]);
            xb = __builtin_bit_cast(f32x4, xv[j][q][1]);
          }
          const f32x4 wa = *reinterpret_cast<const f32x4*>(&nws[c * kVgChunk + xc * 8]);
          const f32x4 wb = *reinterpret_cast<const f32x4*>(&nws[c * kVgChunk + xc * 8 + 4]);
          float t = 0.0f;
#pragma unroll
          for (int e = 0; e < 4; ++e) t = __builtin_fmaf(xa[e], xa[e], t);
#pragma unroll
          for (int e = 0; e < 4; ++e) t = __builtin_fmaf(xb[e], xb[e], t);
          ss += live ? t : 0.0f;
          bf16x8 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            o[e] = static_cast<__bf16>(xa[e] * wa[e]);
            o[4 + e] = static_cast<__bf16>(xb[e] * wb[e]);
          }
          v = __builtin_bit_cast(u32x4, o);
        } else {
          v = xv[j][q][0];
        }
        *reinterpret_cast<u32x4*>(buf + q * 32 * kVgRowB + xs_off(xr, xc)) = v & xkeep;
      }
      __syncthreads();  // pass ps's X is staged; the other buffer was read before it
      if (ps * WK + wk < nch) {  // uniform per wave
        const char* xb = buf + wk * 32 * kVgRowB;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(xb + xs_off(r, h * 4 + s));
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_b8(a), as_b8(wv[j][s]), acc, 0, 0, 0);
        }
      }
      // the slot's next pass, issued after its W operands are consumed: the
      // ring's registers then carry over the loop's back edge in place (a copy
      // of them would make the compiler wait for every load in flight there)
      load_pass(ps + PD, xv[j], wv[j]);  // past the end: clamped re-reads, never used
    }
  }

  if constexpr (WK == 1 && !NX) {
    if (p.vec_out) __syncthreads();  // the X buffers are dead before the transpose tiles reuse them
  }
  if constexpr (NX) {
    // row xr's sum of squares over its 8 threads (consecutive lanes)
    ss += __shfl_xor(ss, 1);
    ss += __shfl_xor(ss, 2);
    ss += __shfl_xor(ss, 4);
    if (xc == 0) rsd[xr] = 1.0f / __builtin_sqrtf(ss / (float)p.K + p.eps);
    if constexpr (WK == 1) __syncthreads();  // else the K-split reduction's barriers order it
  }
  if constexpr (WK > 1) {
    // K splits 1.. of each N tile -> LDS; split 0 adds them in split order
    __syncthreads();  // the X buffers are dead
    f32x16* red = reinterpret_cast<f32x16*>(smem);
    if (wk > 0) red[((wk - 1) * WN + wn) * 64 + lane] = acc;
    __syncthreads();
    if (wk > 0) return;
#pragma unroll
    for (int k = 1; k < WK; ++k) acc += red[((k - 1) * WN + wn) * 64 + lane];
  }
  if (ni >= p.nt) return;

  // lane holds D[row 8i + 4h + e][col r] in acc[4i + e]
  if constexpr (NX) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[4 * i + e] *= rsd[8 * i + 4 * h + e];
  }
  char* ybase = static_cast<char*>(p.y) + (int64_t)z * p.syb * (OT == 0 ? 4 : 2);
  if (p.vec_out) {
    // The tile leaves through this wave's LDS tile: lane (r, h) writes
    // D[8i + 4h + e][r], then lane l holds row l/2's columns 16 (l % 2) .. +16
    // and stores them as 16- or 32-byte pieces: one or two store
    // instructions per tile instead of 16 of 2-4 bytes.
    float* tr = reinterpret_cast<float*>(smem + TR) + wn * 32 * TP;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) tr[(8 * i + 4 * h + e) * TP + r] = acc[4 * i + e];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int hf = lane & 1, m = m0 + (lane >> 1);
    const float* row = tr + (lane >> 1) * TP;
    if (m >= p.M) return;
    if constexpr (EPI == 3) {
      float* yf = reinterpret_cast<float*>(ybase) + (int64_t)m * p.ldy + ni * 32 + 16 * hf;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(row + 16 * hf + 4 * q);
        *reinterpret_cast<f32x4*>(yf + 4 * q) =
            f32x4{old[q][0] + v[0], old[q][1] + v[1], old[q][2] + v[2], old[q][3] + v[3]};
      }
    } else if constexpr (EPI == 0) {
      float v0[8], v1[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) { v0[e] = row[16 * hf + e]; v1[e] = row[16 * hf + 8 + e]; }
      const int64_t o = (int64_t)m * p.ldy + ni * 32 + 16 * hf;
      vg_store8<OT>(ybase, o, v0);
      vg_store8<OT>(ybase, o + 8, v1);
    } else {
      // hidden units ni*16 + 8 (lane % 2) .. +8: gates in columns 0-15, ups in 16-31
      const float cw = p.comb ? p.comb[(int64_t)m * p.ldc + z] : 1.0f;
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float g = row[8 * hf + e], u = row[16 + 8 * hf + e];
        v[e] = g / (1.0f + __expf(-g)) * u;
        if (p.comb) v[e] *= cw;
      }
      vg_store8<OT>(ybase, (int64_t)m * p.ldy + ni * 16 + 8 * hf, v);
    }
    return;
  }
  if constexpr (EPI == 3) {
    // the residual values were loaded before the K loop (rows past M re-read
    // row M-1 and are not stored)
    const int n = ni * 32 + r;
    if (n >= p.N) return;
    float* yf = reinterpret_cast<float*>(ybase);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + 8 * i + 4 * h + e;
        if (m < p.M) yf[(int64_t)m * p.ldy + n] = old[i][e] + acc[4 * i + e];
      }
    return;
  }
  if constexpr (EPI == 0) {
    const int n = ni * 32 + r;
    if (n >= p.N) return;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + 8 * i + 4 * h + e;
        if (m < p.M) vg_store<OT>(ybase, (int64_t)m * p.ldy + n, acc[4 * i + e]);
      }
  } else {
    // lanes r < 16 hold the gate of hidden unit ni*16 + r; lane r + 16 its up
    float up[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) up[i] = __shfl_xor(acc[i], 16);
    if (r >= 16) return;
    const int j = ni * 16 + r;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + 8 * i + 4 * h + e;
        if (m >= p.M) continue;
        const float g = acc[4 * i + e];
        float v = g / (1.0f + __expf(-g)) * up[4 * i + e];
        if (p.comb) v *= p.comb[(int64_t)m * p.ldc + z];
        vg_store<OT>(ybase, (int64_t)m * p.ldy + j, v);
      }
  }
}

// ---------------------------------------------------------------------------
// Routed MoD expert products (vnx_expert_gemm_bf16).  Expert z multiplies only
// the rows routed to it (about top_k / E of them), and every expert's weight
// should stream from HBM once, so a workgroup owns WN adjacent 32-row tiles
// of W_z and a pass of up to 128 (gate-up) or 160 (down) of the expert's
// rows (four or five MFMA row tiles per wave, the W operand reused across
// them from registers): when one pass covers an expert's rows, the
// workgroups of further passes (grid.y) exit at once.  Its 4 waves are WN
// (N tiles) x WK (K splits), as in k_vgemm.  X (a pass's rows x WK chunks
// per step) is staged through LDS like k_vgemm's, the rows gathered through
// the row list.
//
// ROUTE: the row list of expert z is { m : comb[m*ldc + z] != 0 }, ascending;
// each workgroup builds it in LDS from comb (M <= 256: one ballot per wave),
// and the workgroup of N group 0, pass 0 publishes it (rows, counts, slots) for the
// products and the sum that follow.  Otherwise the expert's rows are the
// first counts[z] (all M when counts is NULL) rows of x + z*sxb.
// Output row j of expert z: y + z*syb + j*ldy (the compact order).
struct XgParams {
  const uint16_t* x;
  const uint16_t* w;       // packed; expert z at w + z*swb
  void* y;
  const float* comb;
  int32_t* rows;           // (E, M): expert z's row list at rows[z*M ..]
  int32_t* counts;         // (E)
  int32_t* slots;          // (M, E): slot of row m in expert z's list, or -1
  int64_t ldx, sxb, swb, ldy, syb, ldc;
  int M, N, K, E;
  int nt, ng;
  int xcd_group;           // the workgroups of one expert on one XCD
  int vec_out;             // rows of y 16-byte aligned (and N % 32 == 0 without SwiGLU): tiles leave through LDS
};

// MFMA row tiles of 32 per pass: 4 for the gate-up shape (WN 4), 5 for the
// down shape (a pass of 160 rows)
constexpr int xg_row_tiles(int wn) { return wn == 4 ? 4 : 5; }

template <int OT, int EPI, int WN, bool ROUTE>
__global__ __launch_bounds__(256, WN == 4 ? 3 : 2) void k_xgemm(XgParams p) {
  constexpr int WK = 4 / WN;
  constexpr int RT = xg_row_tiles(WN);
  constexpr int ROWS = 32 * RT;                       // rows per pass
  constexpr int SLAB = WK * ROWS * kVgRowB;           // staged X bytes per step
  constexpr int RED = (WK - 1) * WN * RT * 64 * 64;   // K-split partial tiles
  constexpr int SM = 2 * SLAB > RED ? 2 * SLAB : RED;
  __shared__ __attribute__((aligned(16))) char smem[SM];
  __shared__ int rl[256];
  __shared__ float cwl[ROWS];  // SwiGLU weights of the pass's rows
  __shared__ unsigned long long wmask[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wn = wave % WN, wk = wave / WN;
  // Workgroup t runs on XCD t % 8 (the dispatcher deals them round-robin;
  // gridDim.x is a multiple of 8 whenever xcd_group is set).  xcd_group:
  // the N groups of experts x, x + 8, ... run on XCD x, so each expert's X
  // rows are fetched into one L2 only (balanced routing, MoD's training
  // target).  Otherwise expert-major order: consecutive workgroups are N
  // groups of one expert, spread over every XCD, which keeps an even share
  // per XCD however unevenly the rows are routed.
  int z, gi;
  if (p.xcd_group) {
    const int t = blockIdx.x, slot = t >> 3;
    z = (t & 7) + 8 * (slot / p.ng);
    gi = slot % p.ng;
  } else {
    z = blockIdx.x / p.ng;
    gi = blockIdx.x % p.ng;
  }

  int cnt;
  if constexpr (ROUTE) {
    const bool sel = tid < p.M && p.comb[(int64_t)tid * p.ldc + z] != 0.0f;
    const unsigned long long b = __ballot(sel);
    if (lane == 0) wmask[wave] = b;
    __syncthreads();
    int before = 0;
    cnt = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int c = __popcll(wmask[w]);
      before += w < wave ? c : 0;
      cnt += c;
    }
    const int pos = before + __popcll(b & ((1ull << lane) - 1ull));
    if (sel) rl[pos] = tid;
    if (gi == 0 && blockIdx.y == 0) {
      if (tid < p.M) p.slots[(int64_t)tid * p.E + z] = sel ? pos : -1;
      if (sel) p.rows[(int64_t)z * p.M + pos] = tid;
      if (tid == 0) p.counts[z] = cnt;
    }
    __syncthreads();
  } else {
    cnt = p.counts ? min(p.counts[z], p.M) : p.M;
  }

  const int ni = gi * WN + wn;             // this wave's N tile (past nt: computes, never stores)
  const int nie = ni < p.nt ? ni : p.nt - 1;
  const int r = lane & 31, h = lane >> 5;
  const int nch = p.K / kVgChunk;
  const int nstep = (nch + WK - 1) / WK;
  const int xr = tid >> 3, xc = tid & 7;   // staging: rows xr + 32q, 16-byte column xc
  const uint16_t* wt = p.w + z * p.swb + (int64_t)nie * nch * 2048 + lane * 8;
  char* ybase = static_cast<char*>(p.y) + (int64_t)z * p.syb * (OT == 0 ? 4 : 2);

  // passes of ROWS rows are dealt over grid.y, so an expert with more rows
  // than one pass adds workgroups, not time to its workgroups' critical path
  for (int m0 = blockIdx.y * ROWS; m0 < cnt; m0 += gridDim.y * ROWS) {
    const int live = min(RT, (cnt - m0 + 31) / 32);  // row tiles of this pass
    // rows past the count re-read row cnt - 1: their outputs are computed
    // from finite values and never stored (MFMA rows are independent)
    // X through a buffer resource over the expert's M rows: 32-bit byte
    // offsets per row (the host bounds M * ldx), the chunk offset a scalar
    const uint16_t* xbase = ROUTE ? p.x : p.x + z * p.sxb;
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(xbase), (short)0, (int)((int64_t)p.M * p.ldx * 2), 0x00020000);
    uint32_t xoff[RT];
#pragma unroll
    for (int q = 0; q < RT; ++q) {
      const int j = m0 + xr + 32 * q;
      const int jc = min(j, cnt - 1);
      xoff[q] = (uint32_t)(((ROUTE ? rl[jc] : jc) * (int)p.ldx + xc * 8) * 2);
    }
    if (EPI == 1 && tid < ROWS) {
      // read before the epilogue: the K loop's barriers order it
      const int j = m0 + tid;
      cwl[tid] = p.comb && j < cnt ? p.comb[(int64_t)(ROUTE ? rl[j] : j) * p.ldc + z] : 1.0f;
    }
    f32x16 acc[RT];
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;

    // The W loads run PDW steps ahead of the math (step st in W slot
    // st % PDW), the X loads PDX steps (X slot st % PDX): W streams from HBM
    // and needs the deeper ring, X is re-read from L2.  The X registers are
    // free once staged, so the X loads of step st + PDX issue right after
    // the barrier; a W slot is reloaded only after this step's MFMAs have
    // read it (no register rotation, so nothing in flight has to be waited
    // for at the loop edge).
    // The gate-up shape (WN 4) keeps three workgroups per CU (<= 168
    // registers a lane, hence the shallow rings): at the MoD shapes its 16 x
    // 42 workgroups then all run at once, where two per CU left a second
    // wave of 160 (43.9 against 49.5 us).  The down shape (K split over two
    // waves) keeps two per CU with passes of 160 rows: the routed counts of
    // the config-5 target reach 140-154 rows for 2-4 of the 16 experts, and a
    // second pass re-reads such an expert's weights (30.9 against 38.9 us at
    // those counts, 30.7 against 27.3 when every expert has <= 128 rows);
    // one workgroup per CU with deeper rings measured slower.
    constexpr int PDW = WN == 4 ? 2 : 3, PDX = 1;
    constexpr int UN = PDW > PDX ? PDW : PDX;  // loop unroll: a multiple of both
    static_assert(UN % PDW == 0 && UN % PDX == 0, "ring depths must divide the unroll");
    u32x4 xv[PDX][WK][RT], wv[PDW][4];
    auto load_x = [&](int st, u32x4 (&xs)[WK][RT]) {
#pragma unroll
      for (int j = 0; j < WK; ++j) {
        const int c = min(st * WK + j, nch - 1);
#pragma unroll
        for (int q = 0; q < RT; ++q)
          xs[j][q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xres, xoff[q], c * kVgChunk * 2, 0));
      }
    };
    auto load_w = [&](int st, u32x4 (&ws)[4]) {
      const int c = min(st * WK + wk, nch - 1);
#pragma unroll
      for (int s = 0; s < 4; ++s) ws[s] = *reinterpret_cast<const u32x4*>(wt + (c * 4 + s) * 512);
    };
#pragma unroll
    for (int j = 0; j < PDW; ++j) load_w(j, wv[j]);
#pragma unroll
    for (int j = 0; j < PDX; ++j) load_x(j, xv[j]);
    for (int st0 = 0; st0 < nstep; st0 += UN) {
#pragma unroll
      for (int j = 0; j < UN; ++j) {
        const int st = st0 + j;
        char* buf = smem + (st & 1) * SLAB;
#pragma unroll
        for (int c = 0; c < WK; ++c)
#pragma unroll
          for (int q = 0; q < RT; ++q)
            *reinterpret_cast<u32x4*>(buf + c * ROWS * kVgRowB + xs_off(xr + 32 * q, xc)) = xv[j % PDX][c][q];
        __syncthreads();  // step st's X is staged; the other buffer was read before it
        load_x(st + PDX, xv[j % PDX]);  // past the end: clamped re-reads, never used
        if (st * WK + wk < nch) {  // uniform per wave
          const char* xb = buf + wk * ROWS * kVgRowB;
#pragma unroll
          for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < RT; ++i) {
              // every row tile (rows past the count are not stored)
              const u32x4 a = *reinterpret_cast<const u32x4*>(xb + xs_off(i * 32 + r, h * 4 + s));
              acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_b8(a), as_b8(wv[j % PDW][s]), acc[i], 0, 0, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        load_w(st + PDW, wv[j % PDW]);
      }
    }
    __syncthreads();  // the X buffers are dead
    if constexpr (WK > 1) {
      // K splits 1.. -> LDS; split 0 adds them in split order
      f32x16* red = reinterpret_cast<f32x16*>(smem);
      if (wk > 0)
#pragma unroll
        for (int i = 0; i < RT; ++i)
          if (i < live) red[(((wk - 1) * WN + wn) * RT + i) * 64 + lane] = acc[i];
      __syncthreads();
      if (wk == 0)
#pragma unroll
        for (int k = 1; k < WK; ++k)
#pragma unroll
          for (int i = 0; i < RT; ++i)
            if (i < live) acc[i] += red[(((k - 1) * WN + wn) * RT + i) * 64 + lane];
    }
    if (wk == 0 && ni < p.nt && p.vec_out) {
      // Each 32 x 32 tile leaves through this wave's LDS tile (the X
      // buffers and the reduction tiles are dead): lane (r, h) writes
      // D[8ii + 4h + e][r], then lane l reads row l/2's columns
      // 16 (l % 2) .. +16 and stores them as 16- or 32-byte pieces, so a row
      // tile is one or two store instructions instead of 16 of 2-4 bytes.
      constexpr int TP = 36;  // row pitch (floats): conflict-free writes, 16-byte aligned rows
      static_assert(RED + WN * 32 * TP * 4 <= SM, "the transpose tiles fit the dead staging LDS");
      float* tr = reinterpret_cast<float*>(smem + RED) + wn * 32 * TP;
      const int tr_row = lane >> 1, tr_half = lane & 1;
#pragma unroll
      for (int i = 0; i < RT; ++i) {
        if (i >= live) continue;
#pragma unroll
        for (int ii = 0; ii < 4; ++ii)
#pragma unroll
          for (int e = 0; e < 4; ++e) tr[(8 * ii + 4 * h + e) * TP + r] = acc[i][4 * ii + e];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int j = m0 + i * 32 + tr_row;
        const float* row = tr + tr_row * TP;
        if constexpr (EPI == 0) {
          // columns 16*half .. +16 of the tile
          float v0[8], v1[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) { v0[e] = row[16 * tr_half + e]; v1[e] = row[16 * tr_half + 8 + e]; }
          if (j < cnt) {
            const int64_t o = (int64_t)j * p.ldy + ni * 32 + 16 * tr_half;
            vg_store8<OT>(ybase, o, v0);
            vg_store8<OT>(ybase, o + 8, v1);
          }
        } else {
          // hidden units ni*16 + 8*half .. +8: gates in columns 0-15, ups in 16-31
          float v[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float g = row[8 * tr_half + e], u = row[16 + 8 * tr_half + e];
            v[e] = g / (1.0f + __expf(-g)) * u;
          }
          if (j < cnt) {
            if (p.comb) {
              const float cw = cwl[j - m0];
#pragma unroll
              for (int e = 0; e < 8; ++e) v[e] *= cw;
            }
            vg_store8<OT>(ybase, (int64_t)j * p.ldy + ni * 16 + 8 * tr_half, v);
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    } else if (wk == 0 && ni < p.nt) {
      // lane holds D[row 8ii + 4h + e][col r] of row tile i in acc[i][4ii + e]
#pragma unroll
      for (int i = 0; i < RT; ++i) {
        if (i >= live) continue;
        if constexpr (EPI == 0) {
          const int n = ni * 32 + r;
          if (n < p.N)
#pragma unroll
            for (int ii = 0; ii < 4; ++ii)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int j = m0 + i * 32 + 8 * ii + 4 * h + e;
                if (j < cnt) vg_store<OT>(ybase, (int64_t)j * p.ldy + n, acc[i][4 * ii + e]);
              }
        } else {
          float up[16];
#pragma unroll
          for (int e = 0; e < 16; ++e) up[e] = __shfl_xor(acc[i][e], 16);
          if (r < 16) {
            const int col = ni * 16 + r;
#pragma unroll
            for (int ii = 0; ii < 4; ++ii)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int j = m0 + i * 32 + 8 * ii + 4 * h + e;
                if (j >= cnt) continue;
                const float g = acc[i][4 * ii + e];
                float v = g / (1.0f + __expf(-g)) * up[4 * ii + e];
                if (p.comb) v *= cwl[j - m0];
                vg_store<OT>(ybase, (int64_t)j * p.ldy + col, v);
              }
          }
        }
      }
    }
    __syncthreads();  // the reduction tiles are read before the next pass stages X
  }
}

// Packing: one thread per 16 bytes of the packed layout (rows past N zero).
__global__ __launch_bounds__(256) void k_vpack(const uint16_t* w, int64_t ldw, int N, int K, uint16_t* out,
                                               int64_t total16) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total16) return;
  const int nch = K / kVgChunk;
  const int lane = (int)(i & 63);
  const int64_t q = i >> 6;               // (tile*nch + c)*4 + s
  const int s = (int)(q & 3);
  const int64_t tc = q >> 2;
  const int c = (int)(tc % nch);
  const int64_t tile = tc / nch;
  const int64_t row = tile * 32 + (lane & 31);
  const int k = c * kVgChunk + (lane >> 5) * 32 + s * 8;
  u32x4 v = {0u, 0u, 0u, 0u};
  if (row < N) v = *reinterpret_cast<const u32x4*>(w + row * ldw + k);
  *reinterpret_cast<u32x4*>(out + i * 8) = v;
}

// Launch shape and template dispatch of k_vgemm (p's pointers, strides and
// M / N / K set).  epi 3 is the residual epilogue (fp32 y); nx: RMSNorm input
// (bf16 output only).
int vg_run(VgParams p, int batch, int epi, int y_dtype, bool nx, hipStream_t s) {
  p.mt = (int)((p.M + 31) / 32);
  p.nt = (int)((p.N + 31) / 32);
  p.vec_out = aligned16(p.y) && p.ldy % 8 == 0 && p.syb % 8 == 0 && p.N % 32 == 0;
  // N tiles per workgroup: the most that still keep about three quarters of
  // the CUs busy (fewer tiles per workgroup split K over its waves instead)
  const int64_t cus = device_cus();
  int wn = 4;
  while (wn > 1 && (int64_t)p.mt * ((p.nt + wn - 1) / wn) * batch < cus * 3 / 4) wn /= 2;
  p.ng = (p.nt + wn - 1) / wn;
  const int64_t groups = (p.ng + kVgXcds - 1) / kVgXcds;
  const int64_t wgs = groups * kVgXcds * p.mt;
  if (wgs >= INT32_MAX) return VNX_ERR_UNSUPPORTED;
  const dim3 grid((unsigned)wgs, (unsigned)batch);
  auto launch = [&](auto ot, auto ep, auto nxc) {
    constexpr int OT = decltype(ot)::value, EP = decltype(ep)::value;
    constexpr int NXC = decltype(nxc)::value;
    if (wn == 4) hipLaunchKernelGGL((k_vgemm<OT, EP, 4, NXC>), grid, dim3(256), 0, s, p);
    else if (wn == 2) hipLaunchKernelGGL((k_vgemm<OT, EP, 2, NXC>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((k_vgemm<OT, EP, 1, NXC>), grid, dim3(256), 0, s, p);
  };
  if (epi == 3) {
    launch(IntC<0>{}, IntC<3>{}, IntC<0>{});
  } else if (nx) {
    if (p.emb) launch(IntC<1>{}, IntC<0>{}, IntC<2>{});  // embedding rows: no epilogue
    else if (epi == VNX_EPI_SWIGLU) launch(IntC<1>{}, IntC<1>{}, IntC<1>{});
    else launch(IntC<1>{}, IntC<0>{}, IntC<1>{});
  } else {
    auto by_epi = [&](auto ot) {
      if (epi == VNX_EPI_SWIGLU) launch(ot, IntC<1>{}, IntC<0>{});
      else launch(ot, IntC<0>{}, IntC<0>{});
    };
    if (y_dtype == VNX_F32) by_epi(IntC<0>{});
    else if (y_dtype == VNX_BF16) by_epi(IntC<1>{});
    else by_epi(IntC<2>{});
  }
  VNX_LAUNCH_CHECK();
  return VNX_OK;
}

}  // namespace
}  // namespace vnx

using namespace vnx;

extern "C" {

size_t vnx_pack_bf16_size(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0) return 0;
  return (size_t)((N + 31) / 32) * 32 * (size_t)K * 2;
}

int vnx_pack_bf16(const void* w, int64_t ldw, int64_t N, int64_t K, void* out, void* stream) {
  if (!w || !out || N <= 0 || K <= 0 || ldw < K) return VNX_ERR_INVALID_ARG;
  if (K % kVgChunk || ldw % 8 || !aligned16(w) || !aligned16(out)) return VNX_ERR_UNSUPPORTED;
  if (N >= INT32_MAX || K >= INT32_MAX) return VNX_ERR_UNSUPPORTED;
  const int64_t total16 = (N + 31) / 32 * 32 * K / 8;
  hipLaunchKernelGGL(k_vpack, dim3((unsigned)((total16 + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(w), ldw, (int)N, (int)K,
                     static_cast<uint16_t*>(out), total16);
  VNX_LAUNCH_CHECK();
  return VNX_OK;
}

int vnx_gemm_bf16(const void* x, int64_t ldx, int64_t sxb, const void* w_packed, int64_t swb, int64_t M,
                  int64_t N, int64_t K, int batch, int epilogue, const float* comb, int64_t ldc, void* y,
                  int y_dtype, int64_t ldy, int64_t syb, void* stream) {
  if (!x || !w_packed || !y || M < 0 || N < 0 || K <= 0 || batch < 0) return VNX_ERR_INVALID_ARG;
  if (epilogue != VNX_EPI_NONE && epilogue != VNX_EPI_SWIGLU) return VNX_ERR_INVALID_ARG;
  if (y_dtype != VNX_F32 && y_dtype != VNX_BF16 && y_dtype != VNX_F16) return VNX_ERR_UNSUPPORTED;
  const int64_t ncols = epilogue == VNX_EPI_SWIGLU ? N / 2 : N;
  if (ldx < K || ldy < ncols || sxb < 0 || swb < 0 || syb < 0) return VNX_ERR_INVALID_ARG;
  if (batch > 1 && swb < (N + 31) / 32 * 32 * K) return VNX_ERR_INVALID_ARG;
  if (epilogue == VNX_EPI_SWIGLU && N % 32) return VNX_ERR_INVALID_ARG;
  if (comb && (epilogue != VNX_EPI_SWIGLU || ldc < batch)) return VNX_ERR_INVALID_ARG;
  if (M == 0 || N == 0 || batch == 0) return VNX_OK;
  // 16-byte operand loads along K in 64-wide chunks
  if (K % kVgChunk || ldx % 8 || sxb % 8 || swb % 8 || !aligned16(x) || !aligned16(w_packed))
    return VNX_ERR_UNSUPPORTED;
  if (M >= INT32_MAX || N >= INT32_MAX || K >= INT32_MAX || batch > 65535) return VNX_ERR_UNSUPPORTED;
  VgParams p{};
  p.x = static_cast<const uint16_t*>(x); p.w = static_cast<const uint16_t*>(w_packed); p.y = y; p.comb = comb;
  p.ldx = ldx; p.sxb = sxb; p.swb = swb; p.ldy = ldy; p.syb = syb; p.ldc = ldc;
  p.M = (int)M; p.N = (int)N; p.K = (int)K;
  return vg_run(p, batch, epilogue, y_dtype, false, static_cast<hipStream_t>(stream));
}

int vnx_gemm_bf16_norm(const float* x, int64_t ldx, const float* norm_w, float eps, const void* w_packed,
                       int64_t M, int64_t N, int64_t K, int epilogue, void* y, int64_t ldy, void* stream) {
  if (!x || !norm_w || !w_packed || !y || M < 0 || N < 0 || K <= 0 || !(eps >= 0.0f)) return VNX_ERR_INVALID_ARG;
  if (epilogue != VNX_EPI_NONE && epilogue != VNX_EPI_SWIGLU) return VNX_ERR_INVALID_ARG;
  const int64_t ncols = epilogue == VNX_EPI_SWIGLU ? N / 2 : N;
  if (ldx < K || ldy < ncols || (epilogue == VNX_EPI_SWIGLU && N % 32)) return VNX_ERR_INVALID_ARG;
  if (M == 0 || N == 0) return VNX_OK;
  if (K % kVgChunk || K > kVgNormMaxK || ldx % 4 || !aligned16(x) || !aligned16(norm_w) || !aligned16(w_packed))
    return VNX_ERR_UNSUPPORTED;
  if (M >= INT32_MAX || N >= INT32_MAX) return VNX_ERR_UNSUPPORTED;
  VgParams p{};
  p.xf = x; p.nw = norm_w; p.eps = eps;
  p.x = reinterpret_cast<const uint16_t*>(x);  // not read (NX)
  p.w = static_cast<const uint16_t*>(w_packed); p.y = y;
  p.ldx = ldx; p.ldy = ldy;
  p.M = (int)M; p.N = (int)N; p.K = (int)K;
  return vg_run(p, 1, epilogue, VNX_BF16, true, static_cast<hipStream_t>(stream));
}

int vnx_gemm_bf16_norm_embed(const int64_t* tokens, const void* emb, int emb_dtype, int64_t lde, int64_t vocab,
                             float scale, float* x_out, int64_t ldx, const float* norm_w, float eps,
                             const void* w_packed, int64_t M, int64_t N, int64_t K, void* y, int64_t ldy,
                             void* stream) {
  if (!tokens || !emb || !x_out || !norm_w || !w_packed || !y || M < 0 || N < 0 || K <= 0 || !(eps >= 0.0f))
    return VNX_ERR_INVALID_ARG;
  if (vocab < 1 || lde < K || ldx < K || ldy < N) return VNX_ERR_INVALID_ARG;
  if (emb_dtype != VNX_BF16) return VNX_ERR_UNSUPPORTED;
  if (M == 0 || N == 0) return VNX_OK;
  if (K % kVgChunk || K > kVgNormMaxK || ldx % 4 || lde % 8 || !aligned16(x_out) || !aligned16(emb) ||
      !aligned16(norm_w) || !aligned16(w_packed))
    return VNX_ERR_UNSUPPORTED;
  if (M >= INT32_MAX || N >= INT32_MAX) return VNX_ERR_UNSUPPORTED;
  VgParams p{};
  p.xf = x_out; p.nw = norm_w; p.eps = eps;
  p.x = reinterpret_cast<const uint16_t*>(x_out);  // not read (NX)
  p.ids = tokens; p.emb = static_cast<const uint16_t*>(emb); p.lde = lde; p.vocab = vocab; p.emb_scale = scale;
  p.xout = x_out;
  p.w = static_cast<const uint16_t*>(w_packed); p.y = y;
  p.ldx = ldx; p.ldy = ldy;
  p.M = (int)M; p.N = (int)N; p.K = (int)K;
  return vg_run(p, 1, VNX_EPI_NONE, VNX_BF16, true, static_cast<hipStream_t>(stream));
}

int vnx_gemm_bf16_residual(const void* x, int64_t ldx, const void* w_packed, int64_t M, int64_t N, int64_t K,
                           float* res, int64_t ldr, void* stream) {
  if (!x || !w_packed || !res || M < 0 || N < 0 || K <= 0 || ldx < K || ldr < N) return VNX_ERR_INVALID_ARG;
  if (M == 0 || N == 0) return VNX_OK;
  if (K % kVgChunk || ldx % 8 || !aligned16(x) || !aligned16(w_packed)) return VNX_ERR_UNSUPPORTED;
  if (M >= INT32_MAX || N >= INT32_MAX || K >= INT32_MAX) return VNX_ERR_UNSUPPORTED;
  VgParams p{};
  p.x = static_cast<const uint16_t*>(x); p.w = static_cast<const uint16_t*>(w_packed); p.y = res;
  p.ldx = ldx; p.ldy = ldr;
  p.M = (int)M; p.N = (int)N; p.K = (int)K;
  return vg_run(p, 1, 3, VNX_F32, false, static_cast<hipStream_t>(stream));
}

int vnx_expert_gemm_bf16(const void* x, int64_t ldx, int64_t sxb, const void* w_packed, int64_t swb, int64_t M,
                         int64_t N, int64_t K, int experts, int epilogue, const float* comb, int64_t ldc, int route,
                         int32_t* rows, int32_t* counts, int32_t* slots, void* y, int y_dtype, int64_t ldy,
                         int64_t syb, void* stream) {
  if (!x || !w_packed || !y || M < 0 || N < 0 || K <= 0 || experts < 0) return VNX_ERR_INVALID_ARG;
  if (epilogue != VNX_EPI_NONE && epilogue != VNX_EPI_SWIGLU) return VNX_ERR_INVALID_ARG;
  if (y_dtype != VNX_F32 && y_dtype != VNX_BF16 && y_dtype != VNX_F16) return VNX_ERR_UNSUPPORTED;
  const int64_t ncols = epilogue == VNX_EPI_SWIGLU ? N / 2 : N;
  if (ldx < K || ldy < ncols || sxb < 0 || swb < 0 || syb < 0) return VNX_ERR_INVALID_ARG;
  if (experts > 1 && swb < (N + 31) / 32 * 32 * K) return VNX_ERR_INVALID_ARG;
  if (epilogue == VNX_EPI_SWIGLU && N % 32) return VNX_ERR_INVALID_ARG;
  if (comb && ((epilogue != VNX_EPI_SWIGLU && !route) || ldc < experts)) return VNX_ERR_INVALID_ARG;
  if (route) {
    // rows from the routing weights: comb, the three lists and a shared x
    if (!comb || !rows || !counts || !slots || sxb != 0) return VNX_ERR_INVALID_ARG;
    if (M > 256) return VNX_ERR_UNSUPPORTED;
  }
  if (M == 0 || N == 0 || experts == 0) return VNX_OK;
  if (K % kVgChunk || ldx % 8 || sxb % 8 || swb % 8 || !aligned16(x) || !aligned16(w_packed))
    return VNX_ERR_UNSUPPORTED;
  if (M >= INT32_MAX || N >= INT32_MAX || K >= INT32_MAX) return VNX_ERR_UNSUPPORTED;
  if (ldx >= INT32_MAX || M * ldx * 2 >= INT32_MAX) return VNX_ERR_UNSUPPORTED;  // 32-bit buffer offsets of x
  XgParams p{};
  p.x = static_cast<const uint16_t*>(x); p.w = static_cast<const uint16_t*>(w_packed); p.y = y; p.comb = comb;
  p.rows = rows; p.counts = counts; p.slots = slots;
  p.ldx = ldx; p.sxb = sxb; p.swb = swb; p.ldy = ldy; p.syb = syb; p.ldc = ldc;
  p.M = (int)M; p.N = (int)N; p.K = (int)K; p.E = experts;
  p.nt = (int)((N + 31) / 32);
  p.vec_out = aligned16(y) && ldy % 8 == 0 && syb % 8 == 0 && (epilogue == VNX_EPI_SWIGLU || N % 32 == 0);
  // 4 N tiles per workgroup unless that leaves the CUs short of workgroups;
  // then 2 N tiles and K split over 2 waves each
  const int64_t cus = device_cus();
  const int wn = (int64_t)((p.nt + 3) / 4) * experts >= cus ? 4 : 2;
  p.ng = (p.nt + wn - 1) / wn;
  // the down product (its X rows are K = expert hidden wide) groups an
  // expert's workgroups on one XCD; the routed gate-up keeps them spread
  p.xcd_group = (experts % 8 == 0 && route == 0) ? 1 : 0;
  const int64_t wgs = (int64_t)experts * p.ng;
  const int64_t passes = (M + 32 * xg_row_tiles(wn) - 1) / (32 * xg_row_tiles(wn));
  if (wgs >= INT32_MAX || passes > 65535) return VNX_ERR_UNSUPPORTED;
  const dim3 grid((unsigned)wgs, (unsigned)passes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool sw = epilogue == VNX_EPI_SWIGLU;
  auto go = [&](auto ot, auto rt) {
    constexpr int OT = decltype(ot)::value;
    constexpr bool RT = decltype(rt)::value != 0;
    if (sw) {
      if (wn == 4) hipLaunchKernelGGL((k_xgemm<OT, 1, 4, RT>), grid, dim3(256), 0, s, p);
      else hipLaunchKernelGGL((k_xgemm<OT, 1, 2, RT>), grid, dim3(256), 0, s, p);
    } else {
      if (wn == 4) hipLaunchKernelGGL((k_xgemm<OT, 0, 4, RT>), grid, dim3(256), 0, s, p);
      else hipLaunchKernelGGL((k_xgemm<OT, 0, 2, RT>), grid, dim3(256), 0, s, p);
    }
  };
  auto go_r = [&](auto ot) {
    if (route) go(ot, IntC<1>{});
    else go(ot, IntC<0>{});
  };
  if (y_dtype == VNX_F32) go_r(IntC<0>{});
  else if (y_dtype == VNX_BF16) go_r(IntC<1>{});
  else go_r(IntC<2>{});
  VNX_LAUNCH_CHECK();
  return VNX_OK;
}

}  // extern "C"
