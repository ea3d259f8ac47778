// Tree-verify attention on gfx950 (vnx_tree_attn).
//
// For each batch row b, query head h and tree node i:
//   out[b,h,i,:] = sum_j softmax_j(q_i . k_j * scale + mask_ij) v_j
// over the keys j of the KV prefix (Tp rows, all visible) followed by the N
// tree rows, where node i sees tree row j iff bit j of anc[b,i] is set (its
// ancestors and itself).  This is DeviceBackend.attention
// (packages/verse_torch/verse_torch/device.py:260-270: scores = q k^T / sqrt(d)
// + additive mask, softmax, @ v) with the 0 / -inf mask of a token tree laid
// over a KV cache, the way TriSparse concatenates the cache before its new
// rows (packages/verse_nex/verse_nex/tri_sparse_attn.py:558-575).  GQA: query
// head h reads kv head h / (H / Hkv).
//
// Work split: one workgroup (4 waves) per (b, kv head, query group, key
// split).  The kv head's query rows (H/Hkv heads x N nodes, at most 64 per
// group) are the MFMA columns, so every K/V row is read from HBM once per
// query group.  Each wave walks 32-key steps of its split:
//   S^T[key][q] = K Q^T   v_mfma_f32_16x16x32_bf16, A = 16 K rows straight
//                         from HBM (the MFMA k index runs along the head
//                         dimension, which is contiguous in K), B = Q from LDS;
//   online softmax        keys are the MFMA rows, so a lane holds 8 keys of one
//                         query column: max/sum need two cross-row shuffles
//                         and the running (m, l) stays lane-local;
//   O^T[dim][q] += V^T P^T with P split into bf16 hi + lo parts (two MFMAs), so
//                         the fp32 result keeps ~2^-17 relative accuracy in P;
//                         V^T comes from a per-wave LDS tile (V is contiguous
//                         along dim, the MFMA needs it along keys).
// Waves merge their (m, l, O) through LDS; with several key splits the
// partial (m, l, O) go to the workspace and k_tree_merge combines them (a
// kernel boundary instead of cross-XCD fences).
#include "vnx_internal.h"

namespace vnx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kTaThreads = 256;  // 4 waves
constexpr int kTaMaxN = 64;      // tree nodes per sequence (one 64-bit mask word)

struct TreeAttnParams {
  const uint16_t* q;
  const uint16_t* kc;
  const uint16_t* vc;
  const uint16_t* kt;
  const uint16_t* vt;
  const uint64_t* anc;
  void* out;
  float* part_o;   // [B*H*N][S][D] unnormalised partial outputs (S > 1)
  float2* part_ml; // [B*H*N][S] (m, l) in the exp2 domain (S > 1)
  int64_t q_sb, q_sh, q_sr;
  int64_t c_sb, c_sh, c_sr;
  int64_t t_sb, t_sh, t_sr;
  int64_t o_sb, o_sh, o_sr;
  int64_t anc_sb;
  int B, H, Hkv, n_rep, Tp, N;
  int S, G, rows_per_group, chunk;  // key splits, query groups, keys per split
  const int32_t* tp_batch;          // per-batch prefix rows (<= Tp), or NULL
  int tree_follows_prefix;          // tree row j of batch b is tree row tp_b + j
  float c;                          // scale * log2(e)
};

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ u32x4 ldg16(const uint16_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// exp2 on the transcendental unit (v_exp_f32); exp2(-inf) = 0.
__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

// Orders this wave's LDS writes before its later LDS reads (and the reads of
// one step before the writes of the next): the LDS executes one wave's
// instructions in order, so only the compiler's ordering needs pinning.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int D, int QT>
struct TaSmem {
  static constexpr int R = D + 8;  // row pitch (bf16) of the Q and V tiles, 16-byte multiple
  static constexpr int DT = D / 16;
  static constexpr size_t q_bytes = size_t(QT) * 16 * R * 2;
  static constexpr size_t v_bytes = size_t(4) * 32 * R * 2;
  static constexpr size_t merge_bytes = size_t(2) * QT * DT * 64 * 16 + size_t(2) * QT * 16 * 8;
  static constexpr size_t bytes = (q_bytes + v_bytes > merge_bytes) ? q_bytes + v_bytes : merge_bytes;
};

// PF: issue the loads of a wave's next key step before the current step's
// math (more registers: chosen when the grid is at most one workgroup per CU,
// where latency, not occupancy, bounds the kernel).
template <int D, int QT, bool OUT_BF16, bool PF>
__global__ __launch_bounds__(kTaThreads) void k_tree_attn(TreeAttnParams p) {
  constexpr int KS = D / 32;          // MFMA k-steps over the head dimension
  constexpr int DT = D / 16;          // 16-wide dimension tiles of O
  constexpr int R = TaSmem<D, QT>::R;
  constexpr int LPR = D / 8;          // lanes per 16-byte-chunked row
  constexpr int VLD = D / 16;         // 16-byte V loads per lane per 32-key step
  __shared__ __align__(16) char smem[TaSmem<D, QT>::bytes];
  uint16_t* s_q = reinterpret_cast<uint16_t*>(smem);
  uint16_t* s_v = reinterpret_cast<uint16_t*>(smem + TaSmem<D, QT>::q_bytes);

  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, col = lane & 15, grp = lane >> 4;
  int bid = blockIdx.x;
  const int s = bid % p.S;
  bid /= p.S;
  const int g = bid % p.G;
  bid /= p.G;
  const int kvh = bid % p.Hkv;
  const int b = bid / p.Hkv;
  const int row0 = g * p.rows_per_group;
  const int nrows = min(p.rows_per_group, p.n_rep * p.N - row0);

  // Q rows of this group -> LDS (rows past nrows are zero).
  for (int idx = tid; idx < QT * 16 * LPR; idx += kTaThreads) {
    const int r = idx / LPR, c8 = idx - r * LPR;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (r < nrows) {
      const int rr = row0 + r, rep = rr / p.N, node = rr - rep * p.N;
      const int h = kvh * p.n_rep + rep;
      v = ldg16(p.q + b * p.q_sb + h * p.q_sh + node * p.q_sr + c8 * 8);
    }
    *reinterpret_cast<u32x4*>(s_q + r * R + c8 * 8) = v;
  }
  // Ancestor words of this lane's query columns.
  uint64_t anc[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int r = qt * 16 + col;
    anc[qt] = ~0ull;
    if (r < nrows) {
      const int rr = row0 + r, node = rr % p.N;
      anc[qt] = p.anc[b * p.anc_sb + node];
    }
  }
  __syncthreads();

  // This batch row's prefix: Tp rows, or tp_batch[b] (clamped to [0, Tp])
  // when the rows of a batch have different committed lengths.
  int Tp = p.Tp;
  if (p.tp_batch) Tp = min(max(p.tp_batch[b], 0), p.Tp);
  const int64_t cbase = b * p.c_sb + kvh * p.c_sh;
  const int64_t tbase = b * p.t_sb + kvh * p.t_sh + (p.tree_follows_prefix ? (int64_t)Tp * p.t_sr : 0);
  const int KT = Tp + p.N;
  // Row of key index `key` in K (or V): the prefix cache, then the tree rows;
  // keys past the end read tree row 0 (their scores are masked to -inf).
  auto krow = [&](int key, const uint16_t* cache, const uint16_t* tree) -> const uint16_t* {
    if (key < Tp) return cache + cbase + key * p.c_sr;
    const int j = key - Tp < p.N ? key - Tp : 0;
    return tree + tbase + j * p.t_sr;
  };

  float m[QT], l[QT];
  f32x4 o[QT][DT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m[qt] = kNegInf;
    l[qt] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[qt][dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  uint16_t* vt_w = s_v + w * 32 * R;  // this wave's 32-key V tile
  const int k_lo = s * p.chunk;
  const int k_hi = min(KT, k_lo + p.chunk);
  const int nsteps = (k_hi - k_lo + 31) >> 5;

  // One step's loads: K fragments (A rows = keys base + kt*16 + col, k = dims
  // ks*32 + grp*8 .. +8) and V rows, coalesced (load v covers keys
  // v*(64/LPR) + lane/LPR, chunk lane%LPR).  The loads of a wave's next step
  // are issued before the current step's math, so HBM latency overlaps it.
  auto load_step = [&](int base, u32x4 (&kf)[2][KS], u32x4 (&vv)[VLD]) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const uint16_t* r = krow(base + kt * 16 + col, p.kc, p.kt);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kf[kt][ks] = ldg16(r + ks * 32 + grp * 8);
    }
#pragma unroll
    for (int v = 0; v < VLD; ++v) {
      const int key = base + v * (64 / LPR) + lane / LPR;
      vv[v] = ldg16(krow(key, p.vc, p.vt) + (lane % LPR) * 8);
      if (key >= k_hi) vv[v] = u32x4{0u, 0u, 0u, 0u};
    }
  };
  u32x4 kf[2][KS], vv[VLD], kfn[2][KS], vvn[VLD];
  if (PF && w < nsteps) load_step(k_lo + w * 32, kf, vv);
  for (int st = w; st < nsteps; st += 4) {
    const int base = k_lo + st * 32;
    const bool more = PF && st + 4 < nsteps;
    if constexpr (PF) {
      if (more) load_step(base + 4 * 32, kfn, vvn);
    } else {
      load_step(base, kf, vv);
    }
    wave_lds_sync();  // previous step's V^T reads are done
#pragma unroll
    for (int v = 0; v < VLD; ++v)
      *reinterpret_cast<u32x4*>(vt_w + (v * (64 / LPR) + lane / LPR) * R + (lane % LPR) * 8) = vv[v];
    wave_lds_sync();
    // V^T A-operands: lane holds V[key kappa(grp, e)][dim dt*16 + col],
    // kappa = (e < 4 ? 0 : 16) + grp*4 + (e & 3): the keys whose scores this
    // lane holds for its query column (S^T rows grp*4 + j of both key tiles).
    bf16x8 va[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      uint16_t e8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) e8[e] = vt_w[((e < 4 ? 0 : 16) + grp * 4 + (e & 3)) * R + dt * 16 + col];
      va[dt] = __builtin_bit_cast(bf16x8, e8);
    }
    const bool edge = base + 32 > Tp;  // the step reaches tree keys or the end
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      f32x4 sa[2] = {f32x4{0.0f, 0.0f, 0.0f, 0.0f}, f32x4{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8 qf = as_bf16x8(*reinterpret_cast<const u32x4*>(s_q + (qt * 16 + col) * R + ks * 32 + grp * 8));
        sa[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kf[0][ks]), qf, sa[0], 0, 0, 0);
        sa[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kf[1][ks]), qf, sa[1], 0, 0, 0);
      }
      float x[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = sa[e >> 2][e & 3] * p.c;
      if (edge) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int key = base + (e < 4 ? 0 : 16) + grp * 4 + (e & 3);
          bool vis = key < k_hi;
          if (key >= Tp) vis = vis && ((anc[qt] >> (key - Tp)) & 1ull);
          x[e] = vis ? x[e] : kNegInf;
        }
      }
      float mx = x[0];
#pragma unroll
      for (int e = 1; e < 8; ++e) mx = __builtin_fmaxf(mx, x[e]);
      mx = __builtin_fmaxf(mx, __shfl_xor(mx, 16));
      mx = __builtin_fmaxf(mx, __shfl_xor(mx, 32));
      const float mn = __builtin_fmaxf(m[qt], mx);
      const float ms = mn == kNegInf ? 0.0f : mn;
      const float alpha = ex2(m[qt] - ms);
      m[qt] = mn;
      l[qt] *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[qt][dt] *= alpha;
      __bf16 ph[8], pl[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float pe = ex2(x[e] - ms);
        l[qt] += pe;
        ph[e] = static_cast<__bf16>(pe);
        pl[e] = static_cast<__bf16>(pe - static_cast<float>(ph[e]));
      }
      const bf16x8 bh = __builtin_bit_cast(bf16x8, ph), bl = __builtin_bit_cast(bf16x8, pl);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt], bh, o[qt][dt], 0, 0, 0);
        o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt], bl, o[qt][dt], 0, 0, 0);
      }
    }
    if (more) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) kf[kt][ks] = kfn[kt][ks];
#pragma unroll
      for (int v = 0; v < VLD; ++v) vv[v] = vvn[v];
    }
  }

  // Each lane summed l over its own 8 keys per step: add the 4 row groups.
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    l[qt] += __shfl_xor(l[qt], 16);
    l[qt] += __shfl_xor(l[qt], 32);
  }

  // Merge the 4 waves (same lane layout in every wave): 2,3 -> 0,1, then 1 -> 0.
  __syncthreads();  // Q / V tiles are dead; the merge slots alias them
  f32x4* s_o = reinterpret_cast<f32x4*>(smem);
  float2* s_ml = reinterpret_cast<float2*>(smem + size_t(2) * QT * DT * 64 * 16);
  auto put = [&](int slot) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) s_o[((slot * QT + qt) * DT + dt) * 64 + lane] = o[qt][dt];
      if (grp == 0) s_ml[(slot * QT + qt) * 16 + col] = make_float2(m[qt], l[qt]);
    }
  };
  auto take = [&](int slot) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const float2 ml = s_ml[(slot * QT + qt) * 16 + col];
      const float mn = __builtin_fmaxf(m[qt], ml.x);
      const float ms = mn == kNegInf ? 0.0f : mn;
      const float fa = ex2(m[qt] - ms), fb = ex2(ml.x - ms);
      m[qt] = mn;
      l[qt] = l[qt] * fa + ml.y * fb;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[qt][dt] = o[qt][dt] * fa + s_o[((slot * QT + qt) * DT + dt) * 64 + lane] * fb;
    }
  };
  if (w >= 2) put(w - 2);
  __syncthreads();
  if (w < 2) take(w);
  __syncthreads();
  if (w == 1) put(0);
  __syncthreads();
  if (w != 0) return;
  take(0);

#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int r = qt * 16 + col;
    if (r >= nrows) continue;
    const int rr = row0 + r, rep = rr / p.N, node = rr - rep * p.N;
    const int h = kvh * p.n_rep + rep;
    if (p.S == 1) {
      const float inv = l[qt] > 0.0f ? 1.0f / l[qt] : 0.0f;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int64_t off = b * p.o_sb + h * p.o_sh + node * p.o_sr + dt * 16 + grp * 4;
        const f32x4 v = o[qt][dt] * inv;
        if constexpr (OUT_BF16) {
          __bf16 t4[4] = {static_cast<__bf16>(v[0]), static_cast<__bf16>(v[1]), static_cast<__bf16>(v[2]),
                          static_cast<__bf16>(v[3])};
          *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.out) + off) = __builtin_bit_cast(uint2, t4);
        } else {
          *reinterpret_cast<f32x4*>(static_cast<float*>(p.out) + off) = v;
        }
      }
    } else {
      const int64_t prow = ((int64_t)(b * p.H + h) * p.N + node) * p.S + s;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        *reinterpret_cast<f32x4*>(p.part_o + prow * D + dt * 16 + grp * 4) = o[qt][dt];
      if (grp == 0) p.part_ml[prow] = make_float2(m[qt], l[qt]);
    }
  }
}

// Combines the S key-split partials of every output row: one thread per
// 4 consecutive dimensions.
template <int D, bool OUT_BF16>
__global__ __launch_bounds__(256) void k_tree_merge(TreeAttnParams p) {
  constexpr int TPR = D / 4;  // threads per row
  const int64_t rows = (int64_t)p.B * p.H * p.N;
  const int64_t row = (int64_t)blockIdx.x * (256 / TPR) + threadIdx.x / TPR;
  if (row >= rows) return;
  const int c4 = threadIdx.x % TPR;
  const float2* ml = p.part_ml + row * p.S;
  float M = kNegInf;
  for (int s = 0; s < p.S; ++s) M = __builtin_fmaxf(M, ml[s].x);
  const float Ms = M == kNegInf ? 0.0f : M;
  float L = 0.0f;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int s = 0; s < p.S; ++s) {
    const float f = ex2(ml[s].x - Ms);
    L += ml[s].y * f;
    acc += *reinterpret_cast<const f32x4*>(p.part_o + (row * p.S + s) * D + c4 * 4) * f;
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  const int node = (int)(row % p.N);
  const int64_t bh = row / p.N;
  const int h = (int)(bh % p.H), b = (int)(bh / p.H);
  const int64_t off = b * p.o_sb + h * p.o_sh + node * p.o_sr + c4 * 4;
  const f32x4 v = acc * inv;
  if constexpr (OUT_BF16) {
    __bf16 t4[4] = {static_cast<__bf16>(v[0]), static_cast<__bf16>(v[1]), static_cast<__bf16>(v[2]),
                    static_cast<__bf16>(v[3])};
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.out) + off) = __builtin_bit_cast(uint2, t4);
  } else {
    *reinterpret_cast<f32x4*>(static_cast<float*>(p.out) + off) = v;
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
struct TaPlan {
  int G, rows_per_group, QT, S, chunk;
};

// VNX_TA_SPLITS (>= 1) fixes the key splits for tuning sweeps.
static int ta_splits_override() {
  static const int v = [] {
    const char* e = getenv("VNX_TA_SPLITS");
    const int x = e ? atoi(e) : 0;
    return x > 0 ? x : 0;
  }();
  return v;
}

static TaPlan ta_plan(int B, int H, int Hkv, int N, int Tp, int d) {
  TaPlan pl{};
  const int qmax = d == 64 ? 64 : 32;  // query rows per group (register budget of O)
  const int rows = (H / Hkv) * N;
  pl.G = (rows + qmax - 1) / qmax;
  pl.rows_per_group = (rows + pl.G - 1) / pl.G;
  pl.QT = (pl.rows_per_group + 15) / 16;
  const int KT = Tp + N;
  const int steps = (KT + 31) / 32;
  const int64_t base = (int64_t)B * Hkv * pl.G;
  const int64_t target = (int64_t)device_cus() * 4 * wg_scale_pct() / 100;
  int S = (int)((target + base - 1) / base);
  // A split must carry enough keys to pay for the merge launch: at least 24
  // 32-key steps each (the config-3 sweep: 2 splits of 33 steps beat 4 of
  // 17; a verify step over ~800 keys runs best unsplit).
  const int sby_work = steps / 24 > 1 ? steps / 24 : 1;
  S = S < sby_work ? S : sby_work;
  const int smax = (steps + 3) / 4;  // at least one 32-key step per wave
  if (ta_splits_override()) S = ta_splits_override();
  S = S < 1 ? 1 : (S > smax ? smax : S);
  const int steps_per = (steps + S - 1) / S;
  pl.chunk = steps_per * 32;
  pl.S = (KT + pl.chunk - 1) / pl.chunk;
  return pl;
}

static size_t ta_ws_bytes(const TaPlan& pl, int B, int H, int N, int d) {
  if (pl.S <= 1) return 0;
  Carve c(nullptr);
  const int64_t prow = (int64_t)B * H * N * pl.S;
  c.take<float>(prow * d);
  c.take<float2>(prow);
  return c.bytes();
}

template <int D, bool OB, bool PF>
static void ta_launch_qt(const TreeAttnParams& p, int QT, dim3 grid, hipStream_t st) {
  switch (QT) {
    case 1: hipLaunchKernelGGL((k_tree_attn<D, 1, OB, PF>), grid, dim3(kTaThreads), 0, st, p); break;
    case 2: hipLaunchKernelGGL((k_tree_attn<D, 2, OB, PF>), grid, dim3(kTaThreads), 0, st, p); break;
    case 3:
      if constexpr (D == 64) hipLaunchKernelGGL((k_tree_attn<D, 3, OB, PF>), grid, dim3(kTaThreads), 0, st, p);
      break;
    default:
      if constexpr (D == 64) hipLaunchKernelGGL((k_tree_attn<D, 4, OB, PF>), grid, dim3(kTaThreads), 0, st, p);
      break;
  }
}

template <int D, bool OB>
static int ta_launch_d(const TreeAttnParams& p, int QT, hipStream_t st, hipEvent_t* ev) {
  const int64_t nwg = (int64_t)p.B * p.Hkv * p.G * p.S;
  const dim3 grid((unsigned)nwg);
  if (ev) VNX_HIP_CHECK(hipEventRecord(ev[0], st));
  if (nwg <= device_cus())
    ta_launch_qt<D, OB, true>(p, QT, grid, st);
  else
    ta_launch_qt<D, OB, false>(p, QT, grid, st);
  VNX_LAUNCH_CHECK();
  if (ev) VNX_HIP_CHECK(hipEventRecord(ev[1], st));
  if (p.S > 1) {
    const int64_t rows = (int64_t)p.B * p.H * p.N;
    const int rpb = 256 / (D / 4);
    hipLaunchKernelGGL((k_tree_merge<D, OB>), dim3((unsigned)((rows + rpb - 1) / rpb)), dim3(256), 0, st, p);
    VNX_LAUNCH_CHECK();
  }
  if (ev) VNX_HIP_CHECK(hipEventRecord(ev[2], st));
  return VNX_OK;
}

static bool strides_ok(int64_t sb, int64_t sh, int64_t sr, int unit) {
  return sb >= 0 && sh >= 0 && sr >= 0 && sb % unit == 0 && sh % unit == 0 && sr % unit == 0;
}

}  // namespace vnx

using namespace vnx;

extern "C" {

size_t vnx_tree_attn_workspace(int B, int H, int Hkv, int N, int Tp, int d) {
  if (B <= 0 || H <= 0 || Hkv <= 0 || H % Hkv || N <= 0 || N > kTaMaxN || Tp < 0 || (d != 64 && d != 128))
    return 256;
  const size_t n = ta_ws_bytes(ta_plan(B, H, Hkv, N, Tp, d), B, H, N, d);
  return n < 256 ? 256 : n;
}

int vnx_tree_attn(const vnx_tree_attn_args* a, void* workspace, size_t workspace_bytes, void* stream) {
  if (!a) return VNX_ERR_INVALID_ARG;
  const int B = a->B, H = a->H, Hkv = a->Hkv, N = a->N, Tp = a->Tp, d = a->d;
  if (B < 0 || H <= 0 || Hkv <= 0 || H % Hkv || N < 1 || Tp < 0) return VNX_ERR_INVALID_ARG;
  if (N > kTaMaxN || (d != 64 && d != 128)) return VNX_ERR_UNSUPPORTED;
  if (a->out_dtype != VNX_F32 && a->out_dtype != VNX_BF16) return VNX_ERR_UNSUPPORTED;
  if (B == 0) return VNX_OK;
  if (!a->q || !a->k_tree || !a->v_tree || !a->anc || !a->out) return VNX_ERR_INVALID_ARG;
  if (Tp > 0 && (!a->k_cache || !a->v_cache)) return VNX_ERR_INVALID_ARG;
  if (a->tp_batch && (reinterpret_cast<uintptr_t>(a->tp_batch) & 3u)) return VNX_ERR_INVALID_ARG;
  if (!(a->scale > 0.0f) || !__builtin_isfinite(a->scale)) return VNX_ERR_INVALID_ARG;
  if (a->anc_batch_stride < 0) return VNX_ERR_INVALID_ARG;
  // 16-byte loads of bf16 rows; 16-byte (fp32) / 8-byte (bf16) output stores.
  if (!strides_ok(a->q_strides[0], a->q_strides[1], a->q_strides[2], 8) ||
      !strides_ok(a->cache_strides[0], a->cache_strides[1], a->cache_strides[2], 8) ||
      !strides_ok(a->tree_strides[0], a->tree_strides[1], a->tree_strides[2], 8) ||
      !strides_ok(a->out_strides[0], a->out_strides[1], a->out_strides[2], 4))
    return VNX_ERR_UNSUPPORTED;
  if (!aligned16(a->q) || !aligned16(a->k_tree) || !aligned16(a->v_tree) || !aligned16(a->out) ||
      (Tp > 0 && (!aligned16(a->k_cache) || !aligned16(a->v_cache))) ||
      (reinterpret_cast<uintptr_t>(a->anc) & 7u))
    return VNX_ERR_UNSUPPORTED;
  const TaPlan pl = ta_plan(B, H, Hkv, N, Tp, d);
  if ((int64_t)B * Hkv * pl.G * pl.S >= INT32_MAX) return VNX_ERR_UNSUPPORTED;
  const size_t need = ta_ws_bytes(pl, B, H, N, d);
  if (need && (!workspace || workspace_bytes < need)) return VNX_ERR_WORKSPACE;

  TreeAttnParams p{};
  p.q = static_cast<const uint16_t*>(a->q);
  p.kc = static_cast<const uint16_t*>(Tp > 0 ? a->k_cache : a->k_tree);
  p.vc = static_cast<const uint16_t*>(Tp > 0 ? a->v_cache : a->v_tree);
  p.kt = static_cast<const uint16_t*>(a->k_tree);
  p.vt = static_cast<const uint16_t*>(a->v_tree);
  p.anc = a->anc;
  p.out = a->out;
  p.q_sb = a->q_strides[0]; p.q_sh = a->q_strides[1]; p.q_sr = a->q_strides[2];
  p.c_sb = a->cache_strides[0]; p.c_sh = a->cache_strides[1]; p.c_sr = a->cache_strides[2];
  p.t_sb = a->tree_strides[0]; p.t_sh = a->tree_strides[1]; p.t_sr = a->tree_strides[2];
  p.o_sb = a->out_strides[0]; p.o_sh = a->out_strides[1]; p.o_sr = a->out_strides[2];
  p.anc_sb = a->anc_batch_stride;
  p.B = B; p.H = H; p.Hkv = Hkv; p.n_rep = H / Hkv; p.Tp = Tp; p.N = N;
  p.S = pl.S; p.G = pl.G; p.rows_per_group = pl.rows_per_group; p.chunk = pl.chunk;
  p.tp_batch = a->tp_batch;
  p.tree_follows_prefix = a->tree_follows_prefix ? 1 : 0;
  p.c = (float)((double)a->scale * 1.4426950408889634);
  if (pl.S > 1) {
    Carve c(workspace);
    const int64_t prow = (int64_t)B * H * N * pl.S;
    p.part_o = c.take<float>(prow * d);
    p.part_ml = c.take<float2>(prow);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipEvent_t* ev = profile_slot(2);
  const bool ob = a->out_dtype == VNX_BF16;
  if (d == 64) return ob ? ta_launch_d<64, true>(p, pl.QT, st, ev) : ta_launch_d<64, false>(p, pl.QT, st, ev);
  return ob ? ta_launch_d<128, true>(p, pl.QT, st, ev) : ta_launch_d<128, false>(p, pl.QT, st, ev);
}

int vnx_tree_attn_plan(int B, int H, int Hkv, int N, int Tp, int d, int* splits, int* groups, int* chunk) {
  if (B <= 0 || H <= 0 || Hkv <= 0 || H % Hkv || N <= 0 || N > kTaMaxN || Tp < 0 || (d != 64 && d != 128))
    return VNX_ERR_INVALID_ARG;
  const TaPlan pl = ta_plan(B, H, Hkv, N, Tp, d);
  if (splits) *splits = pl.S;
  if (groups) *groups = pl.G;
  if (chunk) *chunk = pl.chunk;
  return VNX_OK;
}

}  // extern "C"
