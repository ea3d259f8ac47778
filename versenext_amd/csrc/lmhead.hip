// Verify-pass LM head on the matrix cores (vnx_lm_head):
//   logits (M, V) = X (M, K) . W (V, K)^T
// with X the final-norm hidden states of the B*(k+1) verified positions and W
// the tied embedding table, one row per vocab id (bf16 in, fp32 accumulate,
// fp32 or bf16 out).  This is CometSparkNexLM.head (cometspark.py:396-398,
// applied at :697 / :766; Linear.forward, vnnn.py:423-430) restricted to the
// rows the verifier reads (speculative.py:218-220).
//
// At the verify shape (M = 224, K = 1024, V = 248,320) the product has about
// 224 flop per byte of W, under the MI355X ridge (~312 flop/B for bf16): the
// kernel is built to stream W from HBM once, with enough bytes in flight:
//   * a workgroup (4 waves, one per SIMD) owns 256 consecutive vocab rows and
//     all M columns; wave w owns rows w*64 .. +64 (two 32-row MFMA A tiles)
//     and keeps their (64 x M) fp32 accumulators in registers;
//   * W fragments go straight from HBM to registers (the MFMA k index runs
//     along K, contiguous in W) through a ring of 4 64-k slabs, so 3 slabs
//     (96 KB per CU) are in flight ahead of the math;
//   * X is staged through LDS in 64-k slabs (double-buffered) and read as the
//     MFMA B operand by the 4 waves; each X fragment feeds both A tiles;
//   * v_mfma_f32_32x32x16_bf16: A = 32 vocab rows x 16 k, B = 16 k x 32
//     positions.  Inside a 64-k slab lane (r, h) (r = lane % 32, h = lane /
//     32) loads k = h*32 .. h*32+32 of its row (64 contiguous bytes) and
//     feeds k-step j with k = h*32 + j*8 .. +8; B uses the same k order, so
//     the dot product is unchanged;
//   * the 32x32 result gives each lane 4 runs of 4 consecutive vocab rows of
//     one position; the epilogue transposes the tile through LDS so every
//     store instruction writes one contiguous 1 KB (fp32) piece of a row.
#include "vnx_internal.h"

namespace vnx {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kLhRows = 256;                       // vocab rows per workgroup
constexpr int kLhSlab = 64;                        // k per slab (four MFMA k steps)
constexpr int kLhPitch = kLhSlab + 8;              // LDS row pitch of X (bf16)
constexpr int kLhOutPitch = kLhRows + 4;           // LDS row pitch of the output tile (fp32)
constexpr int kLhMaxM = 256;

typedef float f32x16 __attribute__((ext_vector_type(16)));

struct LhParams {
  const uint16_t* x;  // bf16 bits (M, K), row pitch ldx
  int64_t ldx;
  const uint16_t* w;  // bf16 bits (V, K), row pitch ldw
  int64_t ldw;
  void* out;          // (M, V), row pitch ldo (elements)
  int64_t ldo;
  int M, K;
  int64_t V;
};

__device__ __forceinline__ u32x4 ldg16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// MT: 32-column position tiles (M <= 32*MT); RING: W slabs held in registers
// (RING - 1 in flight ahead of the math), a divisor of K / 64; WAVES x TILES
// = 8: waves per workgroup and 32-row A tiles per wave (4 x 2: one wave per
// SIMD, each X fragment feeding two MFMAs; 8 x 1: two waves per SIMD).
template <int MT, int RING, bool OUT_BF16, int WAVES, int TILES>
__global__ __launch_bounds__(64 * WAVES, WAVES / 4) void k_lm_head(LhParams p) {
  static_assert(WAVES * TILES * 32 == kLhRows, "a workgroup covers kLhRows vocab rows");
  constexpr int kLhThreads = 64 * WAVES;
  constexpr int kLhTiles = TILES;
  constexpr size_t kXBytes = size_t(2) * MT * 32 * kLhPitch * 2;
  constexpr size_t kOBytes = size_t(32) * kLhOutPitch * 4;
  __shared__ __align__(16) char smem[kXBytes > kOBytes ? kXBytes : kOBytes];
  typedef uint16_t XBuf[MT * 32 * kLhPitch];
  XBuf* sx = reinterpret_cast<XBuf*>(smem);
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, r32 = lane & 31, h = lane >> 5;
  const int64_t n0 = (int64_t)blockIdx.x * kLhRows + w * (32 * kLhTiles);
  const int nslab = p.K / kLhSlab;

  // This lane's W rows (clamped inside V; rows past V are computed, not stored).
  const uint16_t* wrow[kLhTiles];
#pragma unroll
  for (int t = 0; t < kLhTiles; ++t) {
    int64_t n = n0 + t * 32 + r32;
    n = n < p.V ? n : p.V - 1;
    wrow[t] = p.w + n * p.ldw + h * 32;
  }
  typedef u32x4 WSlab[kLhTiles][4];
  auto load_w = [&](int s, WSlab& f) {
#pragma unroll
    for (int t = 0; t < kLhTiles; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) f[t][j] = ldg16(wrow[t] + s * kLhSlab + j * 8);
  };
  // X slab s: rows < M, 8 chunks of 16 bytes per row; rows past M are zero.
  constexpr int XCH = MT * 32 * (kLhSlab / 8);
  constexpr int XPT = (XCH + kLhThreads - 1) / kLhThreads;
  auto load_x = [&](int s, u32x4 (&xr)[XPT]) {
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
      const int idx = tid + j * kLhThreads;
      const int r = idx >> 3, c8 = idx & 7;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (idx < XCH && r < p.M) v = ldg16(p.x + (int64_t)r * p.ldx + s * kLhSlab + c8 * 8);
      xr[j] = v;
    }
  };
  auto store_x = [&](int buf, const u32x4 (&xr)[XPT]) {
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
      const int idx = tid + j * kLhThreads;
      if (idx < XCH) {
        const int r = idx >> 3, c8 = idx & 7;
        *reinterpret_cast<u32x4*>(&sx[buf][r * kLhPitch + c8 * 8]) = xr[j];
      }
    }
  };

  f32x16 acc[kLhTiles][MT];
#pragma unroll
  for (int t = 0; t < kLhTiles; ++t)
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[t][m][e] = 0.0f;

  // Loads are issued in a fixed order per step: X two slabs ahead, then W
  // RING - 1 slabs ahead.  s_waitcnt counts loads in issue order, so waiting
  // at the end of step s for X(s+1) (issued first in step s-1) leaves every
  // later prefetch in flight.  X(t) lives in register set t & 1 until it is
  // stored to LDS buffer t & 1 at the end of step t - 1.  nslab is a multiple
  // of RING (host), so the unrolled body has no branch; loads past the last
  // slab re-read it (in bounds, unused).
  WSlab ring[RING];
  u32x4 xr[2][XPT];
  const int last = nslab - 1;
#pragma unroll
  for (int j = 0; j < RING - 1; ++j) load_w(j < nslab ? j : last, ring[j]);
  load_x(0, xr[0]);
  store_x(0, xr[0]);
  load_x(1 < nslab ? 1 : last, xr[1]);
  __syncthreads();
  for (int sb = 0; sb < nslab; sb += RING) {
#pragma unroll
    for (int jr = 0; jr < RING; ++jr) {
      const int s = sb + jr;
      const int par = (RING % 2 == 0) ? (jr & 1) : (s & 1);
      if (RING % 2 == 0 || par == 0) load_x(s + 2 < nslab ? s + 2 : last, xr[0 ^ (RING % 2 == 0 ? (jr & 1) : 0)]);
      else load_x(s + 2 < nslab ? s + 2 : last, xr[1]);
      load_w(s + RING - 1 < nslab ? s + RING - 1 : last, ring[(jr + RING - 1) % RING]);
      const uint16_t* xs = sx[par] + r32 * kLhPitch + h * 32;
      // B fragments of k step j + 1 are read from LDS while the MFMAs of
      // step j run.
      bf16x8 bq[2][MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) bq[0][m] = as_bf16x8(*reinterpret_cast<const u32x4*>(xs + m * 32 * kLhPitch));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (j < 3) {
#pragma unroll
          for (int m = 0; m < MT; ++m)
            bq[(j + 1) & 1][m] = as_bf16x8(*reinterpret_cast<const u32x4*>(xs + m * 32 * kLhPitch + (j + 1) * 8));
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
#pragma unroll
          for (int t = 0; t < kLhTiles; ++t)
            acc[t][m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(ring[jr][t][j]), bq[j & 1][m], acc[t][m], 0, 0, 0);
        }
      }
      if (RING % 2 == 0) store_x(par ^ 1, xr[(jr & 1) ^ 1]);
      else if (par == 0) store_x(1, xr[1]);
      else store_x(0, xr[0]);
      __syncthreads();
    }
  }

  // Epilogue, one 32-position tile at a time: the waves' accumulators go to
  // LDS as [position][256 vocab rows], then every wave store writes 1 KB
  // (fp32) or 512 B (bf16) of one position row, so HBM sees whole lines.
  // acc[t][m][4*i + e] = logits[position m*32 + r32][vocab n0 + t*32 + 8*i + 4*h + e].
  float* so = reinterpret_cast<float*>(smem);
  const int64_t nw = (int64_t)blockIdx.x * kLhRows;
#pragma unroll
  for (int m = 0; m < MT; ++m) {
#pragma unroll
    for (int t = 0; t < kLhTiles; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 v = {acc[t][m][4 * i], acc[t][m][4 * i + 1], acc[t][m][4 * i + 2], acc[t][m][4 * i + 3]};
        *reinterpret_cast<f32x4*>(so + r32 * kLhOutPitch + w * (32 * kLhTiles) + t * 32 + 8 * i + 4 * h) = v;
      }
    __syncthreads();
    if constexpr (OUT_BF16) {
      // 32 positions x 256 values in passes of kLhThreads / 32 rows; a thread converts 8 values.
      constexpr int RPP = kLhThreads / 32;
#pragma unroll
      for (int q = 0; q < 32 / RPP; ++q) {
        const int rr = q * RPP + (tid >> 5), c = (tid & 31) * 8;
        const int r = m * 32 + rr;
        const int64_t n = nw + c;
        if (r < p.M && n < p.V) {
          const float* src = so + rr * kLhOutPitch + c;
          uint16_t* o = static_cast<uint16_t*>(p.out) + (int64_t)r * p.ldo + n;
          if (n + 8 <= p.V) {
            u32x4 pk;
            pk.x = (uint32_t)f32_to_bf16_rne(src[0]) | ((uint32_t)f32_to_bf16_rne(src[1]) << 16);
            pk.y = (uint32_t)f32_to_bf16_rne(src[2]) | ((uint32_t)f32_to_bf16_rne(src[3]) << 16);
            pk.z = (uint32_t)f32_to_bf16_rne(src[4]) | ((uint32_t)f32_to_bf16_rne(src[5]) << 16);
            pk.w = (uint32_t)f32_to_bf16_rne(src[6]) | ((uint32_t)f32_to_bf16_rne(src[7]) << 16);
            __builtin_nontemporal_store(pk, reinterpret_cast<u32x4*>(o));
          } else {
            for (int e = 0; e < 8 && n + e < p.V; ++e) o[e] = f32_to_bf16_rne(src[e]);
          }
        }
      }
    } else {
      // 32 positions x 256 values in passes of kLhThreads / 64 rows; a thread writes 4 values.
      constexpr int RPP = kLhThreads / 64;
#pragma unroll
      for (int q = 0; q < 32 / RPP; ++q) {
        const int rr = q * RPP + (tid >> 6), c = (tid & 63) * 4;
        const int r = m * 32 + rr;
        const int64_t n = nw + c;
        if (r < p.M && n < p.V) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(so + rr * kLhOutPitch + c);
          float* o = static_cast<float*>(p.out) + (int64_t)r * p.ldo + n;
          if (n + 4 <= p.V) {
            __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(o));
          } else {
            for (int e = 0; e < 4 && n + e < p.V; ++e) o[e] = v[e];
          }
        }
      }
    }
    __syncthreads();
  }
}

constexpr int kLhWaves = 8;  // 8 x 1 (two waves per SIMD) or 4 x 2

template <int MT, int RING>
void launch_ring(const LhParams& p, bool bf16_out, hipStream_t s) {
  constexpr int TILES = 8 / kLhWaves;
  const dim3 grid((unsigned)((p.V + kLhRows - 1) / kLhRows));
  if (bf16_out)
    hipLaunchKernelGGL((k_lm_head<MT, RING, true, kLhWaves, TILES>), grid, dim3(64 * kLhWaves), 0, s, p);
  else
    hipLaunchKernelGGL((k_lm_head<MT, RING, false, kLhWaves, TILES>), grid, dim3(64 * kLhWaves), 0, s, p);
}

// The ring depth divides the slab count: 4 when it can (3 slabs in flight;
// else 2, else 1.
template <int MT>
void launch_mt(const LhParams& p, bool bf16_out, hipStream_t s) {
  const int nslab = p.K / kLhSlab;
  if (nslab % 4 == 0) launch_ring<MT, 4>(p, bf16_out, s);
  else if (nslab % 2 == 0) launch_ring<MT, 2>(p, bf16_out, s);
  else launch_ring<MT, 1>(p, bf16_out, s);
}

}  // namespace
}  // namespace vnx

using namespace vnx;

extern "C" {

int vnx_lm_head(const void* x, int64_t ldx, const void* w, int64_t ldw, int64_t M, int64_t K, int64_t V,
                void* out, int out_dtype, int64_t ldo, void* stream) {
  if (M < 0 || K <= 0 || V <= 0) return VNX_ERR_INVALID_ARG;
  if (out_dtype != VNX_F32 && out_dtype != VNX_BF16) return VNX_ERR_UNSUPPORTED;
  if (ldx < K || ldw < K || ldo < V) return VNX_ERR_INVALID_ARG;
  if (M == 0) return VNX_OK;  // nothing is read or written: any pointers
  if (!x || !w || !out) return VNX_ERR_INVALID_ARG;
  if (M > kLhMaxM || K % kLhSlab != 0 || V >= ((int64_t)1 << 31)) return VNX_ERR_UNSUPPORTED;
  // 16-byte loads of X and W rows; 16-byte (fp32) or 8-byte (bf16) stores of
  // 4 consecutive vocab ids.
  if (!aligned16(x) || !aligned16(w) || ldx % 8 || ldw % 8) return VNX_ERR_UNSUPPORTED;
  if (out_dtype == VNX_F32 ? (!aligned16(out) || ldo % 4) : ((reinterpret_cast<uintptr_t>(out) & 7u) || ldo % 4))
    return VNX_ERR_UNSUPPORTED;
  LhParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.ldx = ldx;
  p.w = static_cast<const uint16_t*>(w);
  p.ldw = ldw;
  p.out = out;
  p.ldo = ldo;
  p.M = (int)M;
  p.K = (int)K;
  p.V = V;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bf = out_dtype == VNX_BF16;
  switch ((int)((M + 31) / 32)) {
    case 1: launch_mt<1>(p, bf, s); break;
    case 2: launch_mt<2>(p, bf, s); break;
    case 3: launch_mt<3>(p, bf, s); break;
    case 4: launch_mt<4>(p, bf, s); break;
    case 5: launch_mt<5>(p, bf, s); break;
    case 6: launch_mt<6>(p, bf, s); break;
    case 7: launch_mt<7>(p, bf, s); break;
    default: launch_mt<8>(p, bf, s); break;
  }
  VNX_LAUNCH_CHECK();
  return VNX_OK;
}

}  // extern "C"
