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
//
// TriSparseAttention's paths (tri_sparse_attn.py:585-608) ride on the same
// walk: the global rows are a second key segment with waves of their own
// (softmax normalised apart, gated); with EXT the sliding window masks the
// keys of segment 1 whose position is window or more behind the query's
// (node i of batch row b sits at tp_b + depth(i), prefix row j at j; the
// first max(0, tp_b - window + 1) rows are skipped outright), and ALiBi is a
// third group of waves that walks segment 1's keys again without the window,
// adding -m_h * (query position - key position) to each score (the bias is
// per column, a multiply-add in the exp2 domain), its softmax gated by
// gates[2].
#include <climits>

#include "vnx_internal.h"

namespace vnx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kTaMaxN = 64;  // tree nodes per sequence (one 64-bit mask word)

struct TreeAttnParams {
  const uint16_t* q;
  const uint16_t* kc;
  const uint16_t* vc;
  const uint16_t* kt;
  const uint16_t* vt;
  const uint64_t* anc;
  void* out;
  float* part_o;   // [B*H*N][S+1][D] unnormalised partial outputs (S > 1)
  float2* part_ml; // [B*H*N][S+1] (m, l) in the exp2 domain (S > 1)
  int64_t q_sb, q_sh, q_sr;
  int64_t c_sb, c_sh, c_sr;
  int64_t t_sb, t_sh, t_sr;
  int64_t o_sb, o_sh, o_sr;
  int64_t anc_sb;
  int B, H, Hkv, n_rep, Tp, N;
  int S, G, rows_per_group, chunk;  // key splits, query groups, keys per split
  const int32_t* tp_batch;          // per-batch prefix rows (<= Tp), or NULL
  int tree_follows_prefix;          // tree row j of batch b is tree row tp_b + j
  // Second key segment: T2 rows visible to every node, normalised on its own
  // and mixed as gates[0] * segment 1 + gates[1] * segment 2 (T2 == 0: none).
  const uint16_t* k2;
  const uint16_t* v2;
  int64_t s2_sb, s2_sh, s2_sr;
  int T2, W2;                       // rows; waves of split 0 that walk them
  const float* gates;
  float c;                          // scale * log2(e)
  // EXT: sliding window (0: none) and ALiBi (slopes != NULL; the launch then
  // has one key split and W3 waves walking the third segment, for batch rows
  // with tp_b + N <= alibi_max)
  int window;
  const float* slopes;
  int alibi_max, W3;
  // qkv mode: queries from the projection rows (RoPE here), the tree rows'
  // keys / values written into the cache by every workgroup first
  const uint16_t* qkv;
  int64_t qkv_ld;
  const float* cos;
  const float* sin;
  int rope;
  int64_t cap;                      // rows at or past it are not written (and not rotated past the table)
};

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// 16 bytes from device memory, always as a global (not flat) load: flat
// loads also count against the LDS counter, which serialises the waits of a
// key loop that mixes them with LDS traffic.
__device__ __forceinline__ u32x4 ldg16(const uint16_t* p) {
  typedef const __attribute__((address_space(1))) u32x4* gptr;
  return *(gptr)(p);
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

// Four consecutive output elements: OT 0 fp32, 1 bf16, 2 fp16 (round to
// nearest even).
template <int OT>
__device__ __forceinline__ void ta_store4(void* out, int64_t off, f32x4 v) {
  if constexpr (OT == 0) {
    *reinterpret_cast<f32x4*>(static_cast<float*>(out) + off) = v;
  } else if constexpr (OT == 1) {
    __bf16 t4[4] = {static_cast<__bf16>(v[0]), static_cast<__bf16>(v[1]), static_cast<__bf16>(v[2]),
                    static_cast<__bf16>(v[3])};
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + off) = __builtin_bit_cast(uint2, t4);
  } else {
    _Float16 t4[4] = {static_cast<_Float16>(v[0]), static_cast<_Float16>(v[1]), static_cast<_Float16>(v[2]),
                      static_cast<_Float16>(v[3])};
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + off) = __builtin_bit_cast(uint2, t4);
  }
}

template <int D, int QT, int NW>
struct TaSmem {
  static constexpr int R = D + 8;  // row pitch (bf16) of the Q and V tiles, 16-byte multiple
  static constexpr int DT = D / 16;
  static constexpr size_t q_bytes = size_t(QT) * 16 * R * 2;
  static constexpr size_t v_bytes = size_t(NW) * 32 * R * 2;
  static constexpr size_t o_bytes = size_t(NW) * QT * DT * 64 * 16;
  static constexpr size_t merge_bytes = o_bytes + size_t(NW) * QT * 16 * 8;
  static constexpr size_t bytes = (q_bytes + v_bytes > merge_bytes) ? q_bytes + v_bytes : merge_bytes;
};

// The (D, QT, NW, PF) variants that fit: at most 64 KB of LDS, the VGPRs of
// NW waves per CU (16 waves: 128 each), and prefetch rings only at 4 waves
// (PF 2 for d = 64 and 128, and at 8 waves for d = 64; the deeper rings, one
// workgroup per CU, d = 64).
constexpr bool ta_variant_ok(int D, int QT, int NW, int PF) {
  if (PF && NW != 4 && NW != 8) return false;
  if (PF > 2 && (D != 64 || NW != 4)) return false;
  if (PF && NW == 8) return D == 64 && QT <= 4;  // merge area up to 135 KB of the 160 KB LDS
  if (D == 64) return NW == 4 ? QT <= 4 : NW == 8 ? QT <= 2 : NW == 16 ? QT == 1 : false;
  if (D == 128) return NW == 4 ? QT <= 2 : NW == 8 ? QT == 1 : false;
  return false;
}

// One workgroup of NW waves per (b, kv head, query group, key split).  PF > 0:
// a ring of PF register sets, the loads of a wave's next PF - 1 key steps in
// flight during a step's math.  PF 2 with d = 64 fits two 4-wave workgroups
// per CU (<= 256 registers a lane), so grids of up to two workgroups per CU
// keep every wave resident; deeper rings take one workgroup per CU (up to
// 512 registers a lane, VGPRs and AGPRs) and keep more bytes in flight.
template <int D, int QT, int OT, int NW, int PF, bool EXT>
__global__ __launch_bounds__(NW * 64, (PF == 2 && D == 64 && NW == 4) ? 2 : 1) void k_tree_attn(TreeAttnParams p) {
  constexpr int KS = D / 32;          // MFMA k-steps over the head dimension
  constexpr int DT = D / 16;          // 16-wide dimension tiles of O
  constexpr int R = TaSmem<D, QT, NW>::R;
  constexpr int LPR = D / 8;          // lanes per 16-byte-chunked row
  constexpr int VLD = D / 16;         // 16-byte V loads per lane per 32-key step
  static_assert(PF == 0 || (PF >= 2 && PF <= 6), "prefetch ring of 2-6 register sets");
  __shared__ __align__(16) char smem[TaSmem<D, QT, NW>::bytes];
  uint16_t* s_q = reinterpret_cast<uint16_t*>(smem);
  uint16_t* s_v = reinterpret_cast<uint16_t*>(smem + TaSmem<D, QT, NW>::q_bytes);

  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, col = lane & 15,
            grp = lane >> 4;
  int bid = blockIdx.x;
  const int s = bid % p.S;
  bid /= p.S;
  const int g = bid % p.G;
  bid /= p.G;
  const int kvh = bid % p.Hkv;
  const int b = bid / p.Hkv;
  const int row0 = g * p.rows_per_group;
  const int nrows = min(p.rows_per_group, p.n_rep * p.N - row0);

  if (p.qkv) {
    // qkv mode.  Element pairs (j, j + D/2) of a head rotate together: item
    // (r, c) takes 8-dim chunk c < LPR/2 and its partner chunk c + LPR/2.
    const int tpb = __builtin_amdgcn_readfirstlane(min(max(p.tp_batch[b], 0), p.Tp));
    auto rot8 = [&](const uint16_t* src, int64_t pos, int c, u32x4& lo, u32x4& hi) {
      const u32x4 a = ldg16(src + c * 8), z = ldg16(src + D / 2 + c * 8);
      if (!p.rope) { lo = a; hi = z; return; }
      const __bf16* av = reinterpret_cast<const __bf16*>(&a);
      const __bf16* zv = reinterpret_cast<const __bf16*>(&z);
      // the table entries of dims c*8 .. +8 and their partners: 16-byte loads
      // (tables 16-byte aligned, D a multiple of 16)
      f32x4 tc[4], ts[4];
      const f32x4* cr = reinterpret_cast<const f32x4*>(p.cos + pos * D + c * 8);
      const f32x4* sr = reinterpret_cast<const f32x4*>(p.sin + pos * D + c * 8);
      tc[0] = cr[0]; tc[1] = cr[1]; tc[2] = cr[D / 8]; tc[3] = cr[D / 8 + 1];
      ts[0] = sr[0]; ts[1] = sr[1]; ts[2] = sr[D / 8]; ts[3] = sr[D / 8 + 1];
      __bf16 lo8[8], hi8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x0 = static_cast<float>(av[e]), x1 = static_cast<float>(zv[e]);
        const float c0 = tc[e >> 2][e & 3], c1 = tc[2 + (e >> 2)][e & 3];
        const float s0 = ts[e >> 2][e & 3], s1 = ts[2 + (e >> 2)][e & 3];
        lo8[e] = static_cast<__bf16>(x0 * c0 - x1 * s0);   // rotate_half(x)[j] = -x[j + D/2]
        hi8[e] = static_cast<__bf16>(x1 * c1 + x0 * s1);   // rotate_half(x)[j + D/2] = x[j]
      }
      lo = __builtin_bit_cast(u32x4, lo8);
      hi = __builtin_bit_cast(u32x4, hi8);
    };
    // Three kinds of items, each starting on a wave boundary so their load ->
    // math -> store chains run in different waves side by side: the tree
    // rows' rotated keys (item (i, c): chunk c < LPR/2 of row i and its
    // partner), the group's rotated queries into LDS (rows past nrows are
    // zero), and the tree rows' values (two chunks per item), copied.
    const int nk = p.N * (LPR / 2), nq = QT * 16 * (LPR / 2);
    const int oq = (nk + 63) / 64 * 64, ov = oq + (nq + 63) / 64 * 64;
    for (int slot = tid; slot < ov + nk; slot += NW * 64) {
      if (slot < nk) {
        const int i = slot / (LPR / 2), c = slot - i * (LPR / 2);
        const int64_t pos = (int64_t)tpb + i;
        if (pos < p.cap) {
          const uint16_t* row = p.qkv + (int64_t)(b * p.N + i) * p.qkv_ld;
          uint16_t* kd = const_cast<uint16_t*>(p.kt) + b * p.t_sb + kvh * p.t_sh + pos * p.t_sr;
          u32x4 lo, hi;
          rot8(row + (int64_t)(p.H + kvh) * D, pos, c, lo, hi);
          *reinterpret_cast<u32x4*>(kd + c * 8) = lo;
          *reinterpret_cast<u32x4*>(kd + D / 2 + c * 8) = hi;
        }
      } else if (slot >= oq && slot < oq + nq) {
        const int idx = slot - oq;
        const int r = idx / (LPR / 2), c = idx - r * (LPR / 2);
        u32x4 lo = {0u, 0u, 0u, 0u}, hi = {0u, 0u, 0u, 0u};
        if (r < nrows) {
          const int rr = row0 + r, rep = rr / p.N, node = rr - rep * p.N;
          const int h = kvh * p.n_rep + rep;
          const int64_t pos = min((int64_t)tpb + node, p.cap - 1);
          rot8(p.qkv + (int64_t)(b * p.N + node) * p.qkv_ld + (int64_t)h * D, pos, c, lo, hi);
        }
        *reinterpret_cast<u32x4*>(s_q + r * R + c * 8) = lo;
        *reinterpret_cast<u32x4*>(s_q + r * R + D / 2 + c * 8) = hi;
      } else if (slot >= ov) {
        const int j = slot - ov;
        const int i = j / (LPR / 2), cv = j - i * (LPR / 2);
        const int64_t pos = (int64_t)tpb + i;
        if (pos < p.cap) {
          const uint16_t* vs = p.qkv + (int64_t)(b * p.N + i) * p.qkv_ld + (int64_t)(p.H + p.Hkv + kvh) * D;
          uint16_t* vd = const_cast<uint16_t*>(p.vt) + b * p.t_sb + kvh * p.t_sh + pos * p.t_sr;
          const u32x4 v0 = ldg16(vs + cv * 8), v1 = ldg16(vs + D / 2 + cv * 8);
          *reinterpret_cast<u32x4*>(vd + cv * 8) = v0;
          *reinterpret_cast<u32x4*>(vd + D / 2 + cv * 8) = v1;
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0);  // the cache rows are written before any wave reads them
  } else {
    // Q rows of this group -> LDS (rows past nrows are zero).
    for (int idx = tid; idx < QT * 16 * LPR; idx += NW * 64) {
      const int r = idx / LPR, c8 = idx - r * LPR;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (r < nrows) {
        const int rr = row0 + r, rep = rr / p.N, node = rr - rep * p.N;
        const int h = kvh * p.n_rep + rep;
        v = ldg16(p.q + b * p.q_sb + h * p.q_sh + node * p.q_sr + c8 * 8);
      }
      *reinterpret_cast<u32x4*>(s_q + r * R + c8 * 8) = v;
    }
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

  // Segment 1: this batch row's prefix of Tp rows, or tp_batch[b] (clamped
  // to [0, Tp]) when the rows of a batch have different committed lengths,
  // then the N tree rows.  Segment 2: T2 rows, no tree.  Segment 3 (EXT with
  // ALiBi): segment 1's keys again.
  int Tp = p.Tp;
  if (p.tp_batch) Tp = min(max(p.tp_batch[b], 0), p.Tp);
  // One value per workgroup, read by a vector load: made wave-uniform, so the
  // key bounds and step tests below are scalar.
  Tp = __builtin_amdgcn_readfirstlane(Tp);
  // The segment this wave walks: split 0 gives its last W2 waves the second
  // segment and, with ALiBi, the W3 before them the third (wave-uniform, so
  // the selects below are scalar).
  const bool has2 = p.T2 > 0 && s == 0;
  const bool alibi = EXT && p.slopes != nullptr;
  const bool has3 = alibi && Tp + p.N <= p.alibi_max;
  const int w2 = has2 ? p.W2 : 0, w3 = alibi ? p.W3 : 0;
  const int nw1 = NW - w2 - w3;
  const bool seg3 = alibi && w >= nw1 && w < nw1 + w3;
  const bool seg2 = has2 && w >= nw1 + w3;
  const int wi = seg2 ? w - nw1 - w3 : seg3 ? w - nw1 : w;  // index among the segment's waves
  const int nws = seg2 ? w2 : seg3 ? w3 : nw1;               // waves walking the segment
  const bool win = EXT && p.window > 0 && !seg2 && !seg3;
  const uint16_t* kc = seg2 ? p.k2 : p.kc;
  const uint16_t* vc = seg2 ? p.v2 : p.vc;
  const int64_t cbase = seg2 ? b * p.s2_sb + kvh * p.s2_sh : b * p.c_sb + kvh * p.c_sh;
  const int64_t csr = seg2 ? p.s2_sr : p.c_sr;
  const int Tpe = seg2 ? p.T2 : Tp;
  const int KT = seg2 ? p.T2 : Tp + p.N;
  const int64_t tbase = b * p.t_sb + kvh * p.t_sh + (p.tree_follows_prefix ? (int64_t)Tp * p.t_sr : 0);
  // Row of key index `key` in K (or V): the prefix rows, then the tree rows;
  // keys past the end read a valid row (their scores are masked to -inf).
  auto krow = [&](int key, const uint16_t* cache, const uint16_t* tree) -> const uint16_t* {
    if (key < Tpe) return cache + cbase + key * csr;
    if (seg2) return cache + cbase;
    const int j = key - Tpe < p.N ? key - Tpe : 0;
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
  // segment 1 under a window starts at the first row any node can see
  const int kbase = win ? max(0, Tp - p.window + 1) : 0;
  const int k_lo = (seg2 || seg3) ? 0 : kbase + s * p.chunk;
  const int k_hi = seg2 ? p.T2 : seg3 ? (has3 ? KT : 0) : min(KT, k_lo + p.chunk);
  const int nsteps = k_hi > k_lo ? (k_hi - k_lo + 31) >> 5 : 0;
  // Per query column: its position (prefix rows + depth), the window's first
  // visible key, the ALiBi slope times -log2(e).
  int qpos[EXT ? QT : 1], kmin[EXT ? QT : 1];
  float cb[EXT ? QT : 1];
  if constexpr (EXT) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int r = qt * 16 + col;
      const int dep = r < nrows ? __builtin_popcountll(anc[qt]) - 1 : 0;
      qpos[qt] = Tp + dep;
      kmin[qt] = win ? qpos[qt] - p.window + 1 : INT_MIN;
      cb[qt] = 0.0f;
      if (seg3 && r < nrows) {
        const int h = kvh * p.n_rep + (row0 + r) / p.N;
        cb[qt] = -p.slopes[h] * 1.4426950408889634f;
      }
    }
  }
  // the last key index below some column's window start
  const int wlim = win ? Tp + p.N - p.window : INT_MIN;

  // One step's loads: K fragments (A rows = keys base + kt*16 + col, k = dims
  // ks*32 + grp*8 .. +8) and V rows, coalesced (load v covers keys
  // v*(64/LPR) + lane/LPR, chunk lane%LPR).
  // Lane offsets of a step whose keys are all cache rows (the usual step):
  // then every load is a uniform row pointer plus one of these.
  const bool small_stride = csr <= (1 << 24);
  int koff[2], voff[VLD];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) koff[kt] = (kt * 16 + col) * (int)csr + grp * 8;
#pragma unroll
  for (int v = 0; v < VLD; ++v) voff[v] = (v * (64 / LPR) + lane / LPR) * (int)csr + (lane % LPR) * 8;
  // The two paths choose row addresses only; the loads after them are the
  // same instructions whichever path ran, so the wait counts stay exact.
  auto load_step = [&](int base, u32x4 (&kf)[2][KS], u32x4 (&vv)[VLD]) {
    const uint16_t* kr[2];
    const uint16_t* vr[VLD];
    if (base + 32 <= Tpe && small_stride) {
      const uint16_t* kb = kc + cbase + base * csr;
      const uint16_t* vb = vc + cbase + base * csr;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) kr[kt] = kb + koff[kt];
#pragma unroll
      for (int v = 0; v < VLD; ++v) vr[v] = vb + voff[v];
    } else {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) kr[kt] = krow(base + kt * 16 + col, kc, p.kt) + grp * 8;
#pragma unroll
      for (int v = 0; v < VLD; ++v) vr[v] = krow(base + v * (64 / LPR) + lane / LPR, vc, p.vt) + (lane % LPR) * 8;
    }
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kf[kt][ks] = ldg16(kr[kt] + ks * 32);
#pragma unroll
    for (int v = 0; v < VLD; ++v) vv[v] = ldg16(vr[v]);
  };

  // One step's math on its loaded K fragments and V rows.
  auto step = [&](const int base, const u32x4 (&kf)[2][KS], const u32x4 (&vv)[VLD]) {
    // masks: the step reaches tree keys or the end, or keys below a window
    const bool edge = base + 32 > Tpe || (EXT && base < wlim);
    wave_lds_sync();  // previous step's V^T reads are done
    // V rows of keys past the split enter the tile as zeros (only a step that
    // reaches the end has any).  The select sits here, where the store waits
    // for the loads anyway: right after a prefetch it would wait for the next
    // step's loads at once.
    if (base + 32 > k_hi) {
#pragma unroll
      for (int v = 0; v < VLD; ++v) {
        const int key = base + v * (64 / LPR) + lane / LPR;
        *reinterpret_cast<u32x4*>(vt_w + (v * (64 / LPR) + lane / LPR) * R + (lane % LPR) * 8) =
            key < k_hi ? vv[v] : u32x4{0u, 0u, 0u, 0u};
      }
    } else {
#pragma unroll
      for (int v = 0; v < VLD; ++v)
        *reinterpret_cast<u32x4*>(vt_w + (v * (64 / LPR) + lane / LPR) * R + (lane % LPR) * 8) = vv[v];
    }
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
    int kpos[EXT ? 8 : 1];
    if constexpr (EXT) {
      if (seg3) {
        // key positions: prefix row j at j, tree row j at Tp + depth(j)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int key = base + (e < 4 ? 0 : 16) + grp * 4 + (e & 3);
          const int j = key - Tpe;
          kpos[e] = key < Tpe ? key
                              : (j < p.N ? Tp + __builtin_popcountll(p.anc[b * p.anc_sb + j]) - 1 : Tp);
        }
      }
    }
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      f32x4 sa[2] = {f32x4{0.0f, 0.0f, 0.0f, 0.0f}, f32x4{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8 qf = as_bf16x8(*reinterpret_cast<const u32x4*>(s_q + (qt * 16 + col) * R + ks * 32 + grp * 8));
        sa[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kf[0][ks]), qf, sa[0], 0, 0, 0);
        sa[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kf[1][ks]), qf, sa[1], 0, 0, 0);
      }
      // Raw scores q.k: the scale c (> 0) enters with the max (the max of the
      // scaled scores is c times the raw max, rounding being monotone) and in
      // each exponent's fma.  ALiBi rows are scaled and biased here.
      float x[8];
      float cs = p.c;
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = sa[e >> 2][e & 3];
      if constexpr (EXT) {
        if (seg3) {
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = __builtin_fmaf(cb[qt], (float)(qpos[qt] - kpos[e]), x[e] * p.c);
          cs = 1.0f;
        }
      }
      if (edge) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int key = base + (e < 4 ? 0 : 16) + grp * 4 + (e & 3);
          // selects, not branches: tree keys by their ancestor bit, prefix
          // keys by the window
          const bool tree_vis = (anc[qt] >> ((unsigned)(key - Tpe) & 63u)) & 1ull;
          const bool pre_vis = EXT ? key >= kmin[qt] : true;
          const bool vis = key < k_hi && (key >= Tpe ? tree_vis : pre_vis);
          x[e] = vis ? x[e] : kNegInf;
        }
      }
      float mx = x[0];
#pragma unroll
      for (int e = 1; e < 8; ++e) mx = __builtin_fmaxf(mx, x[e]);
      mx = __builtin_fmaxf(mx, __shfl_xor(mx, 16));
      mx = __builtin_fmaxf(mx, __shfl_xor(mx, 32));
      mx *= cs;
      const float mn = __builtin_fmaxf(m[qt], mx);
      const float ms = mn == kNegInf ? 0.0f : mn;
      // (l, O) are rescaled only when some lane's finite running max moved:
      // otherwise alpha is exactly 1 (or they are still zero).
      if (__builtin_amdgcn_ballot_w64(mn != m[qt] && m[qt] != kNegInf)) {
        const float alpha = ex2(m[qt] - ms);
        l[qt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[qt][dt] *= alpha;
      }
      m[qt] = mn;
      __bf16 ph[8], pl[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float pe = ex2(__builtin_fmaf(x[e], cs, -ms));
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
  };

  // The ancestor words (and the prologue's other loads) land before the walk,
  // so no mask test inside it waits on the vector-memory counter, which would
  // also wait for a prefetched step.
  __builtin_amdgcn_s_waitcnt(0);
  if constexpr (PF >= 2) {
    // PF register sets in turn: a step's math runs while the next PF - 1
    // steps' loads are in flight.  The loads are unconditional (past the last
    // step they fetch the last step's rows again, an L2 hit) and nothing is
    // copied between the sets, so each step waits only for its own loads.
    u32x4 kS[PF][2][KS], vS[PF][VLD];
    int st = wi;
    if (st < nsteps) {
      const int last = nsteps - 1;
#pragma unroll
      for (int r = 0; r < PF - 1; ++r) load_step(k_lo + min(st + r * nws, last) * 32, kS[r], vS[r]);
      // step st from set `cur`, then the loads of step st + (PF - 1) * nws into
      // set `nxt` (the one the previous step consumed); true once done
      auto stage = [&](const u32x4 (&kc)[2][KS], const u32x4 (&vc)[VLD], u32x4 (&kn)[2][KS],
                       u32x4 (&vn)[VLD]) -> bool {
        load_step(k_lo + min(st + (PF - 1) * nws, last) * 32, kn, vn);
        step(k_lo + st * 32, kc, vc);
        st += nws;
        return st >= nsteps;
      };
      for (;;) {
        if (stage(kS[0], vS[0], kS[PF - 1], vS[PF - 1])) break;
        if (stage(kS[1], vS[1], kS[0], vS[0])) break;
        if constexpr (PF > 2) {
          if (stage(kS[2 % PF], vS[2 % PF], kS[1], vS[1])) break;
        }
        if constexpr (PF > 3) {
          if (stage(kS[3 % PF], vS[3 % PF], kS[2 % PF], vS[2 % PF])) break;
        }
        if constexpr (PF > 4) {
          if (stage(kS[4 % PF], vS[4 % PF], kS[3 % PF], vS[3 % PF])) break;
        }
        if constexpr (PF > 5) {
          if (stage(kS[5 % PF], vS[5 % PF], kS[4 % PF], vS[4 % PF])) break;
        }
      }
    }
  } else {
    for (int st = wi; st < nsteps; st += nws) {
      u32x4 kf[2][KS], vv[VLD];
      load_step(k_lo + st * 32, kf, vv);
      step(k_lo + st * 32, kf, vv);
    }
  }

  // Each lane summed l over its own 8 keys per step: add the 4 row groups.
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    l[qt] += __shfl_xor(l[qt], 16);
    l[qt] += __shfl_xor(l[qt], 32);
  }

  // Merge: every wave parks (m, l, O) in LDS (the Q / V tiles are dead), then
  // wave t combines dimension tile t of the segment-1 waves (and, apart, of
  // the segment-2 waves) for all query columns.
  __syncthreads();
  f32x4* s_o = reinterpret_cast<f32x4*>(smem);
  float2* s_ml = reinterpret_cast<float2*>(smem + TaSmem<D, QT, NW>::o_bytes);
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) s_o[((w * QT + qt) * DT + dt) * 64 + lane] = o[qt][dt];
    if (grp == 0) s_ml[(w * QT + qt) * 16 + col] = make_float2(m[qt], l[qt]);
  }
  __syncthreads();
  const float g1 = (has2 || alibi) && p.S == 1 ? p.gates[0] : 1.0f;
  const float g2 = has2 && p.S == 1 ? p.gates[1] : 0.0f;
  const float g3 = has3 ? p.gates[2] : 0.0f;  // ALiBi launches have one split
  for (int t = w; t < QT * DT; t += NW) {
    const int qt = t / DT, dt = t - qt * DT;
    // (M, L, O) of waves [a, e) for this lane's column and 4 dimensions.
    auto combine = [&](int a, int e, float& M, float& L, f32x4& O) {
      M = kNegInf;
      for (int i = a; i < e; ++i) M = __builtin_fmaxf(M, s_ml[(i * QT + qt) * 16 + col].x);
      const float Ms = M == kNegInf ? 0.0f : M;
      L = 0.0f;
      O = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      for (int i = a; i < e; ++i) {
        const float2 ml = s_ml[(i * QT + qt) * 16 + col];
        const float f = ex2(ml.x - Ms);
        L += ml.y * f;
        O += s_o[((i * QT + qt) * DT + dt) * 64 + lane] * f;
      }
    };
    float M1, L1, M2 = kNegInf, L2 = 0.0f, M3 = kNegInf, L3 = 0.0f;
    f32x4 O1, O2 = {0.0f, 0.0f, 0.0f, 0.0f}, O3 = {0.0f, 0.0f, 0.0f, 0.0f};
    combine(0, nw1, M1, L1, O1);
    if (has3) combine(nw1, nw1 + w3, M3, L3, O3);
    if (has2) combine(nw1 + w3, NW, M2, L2, O2);
    const int r = qt * 16 + col;
    if (r >= nrows) continue;
    const int rr = row0 + r, rep = rr / p.N, node = rr - rep * p.N;
    const int h = kvh * p.n_rep + rep;
    if (p.S == 1) {
      f32x4 v = O1 * (L1 > 0.0f ? g1 / L1 : 0.0f);
      if (has2) v += O2 * (L2 > 0.0f ? g2 / L2 : 0.0f);
      if (has3) v += O3 * (L3 > 0.0f ? g3 / L3 : 0.0f);
      ta_store4<OT>(p.out, b * p.o_sb + h * p.o_sh + node * p.o_sr + dt * 16 + grp * 4, v);
    } else {
      const int64_t prow = ((int64_t)(b * p.H + h) * p.N + node) * (p.S + 1);
      *reinterpret_cast<f32x4*>(p.part_o + (prow + s) * D + dt * 16 + grp * 4) = O1;
      if (dt == 0 && grp == 0) p.part_ml[prow + s] = make_float2(M1, L1);
      if (has2) {
        *reinterpret_cast<f32x4*>(p.part_o + (prow + p.S) * D + dt * 16 + grp * 4) = O2;
        if (dt == 0 && grp == 0) p.part_ml[prow + p.S] = make_float2(M2, L2);
      }
    }
  }
}

// Combines the S key-split partials of every output row (and the gated
// second segment, kept in slot S): one thread per 4 consecutive dimensions.
template <int D, int OT>
__global__ __launch_bounds__(256) void k_tree_merge(TreeAttnParams p) {
  constexpr int TPR = D / 4;  // threads per row
  const int64_t rows = (int64_t)p.B * p.H * p.N;
  const int64_t row = (int64_t)blockIdx.x * (256 / TPR) + threadIdx.x / TPR;
  if (row >= rows) return;
  const int c4 = threadIdx.x % TPR;
  const int SS = p.S + 1;
  const float2* ml = p.part_ml + row * SS;
  float M = kNegInf;
  for (int s = 0; s < p.S; ++s) M = __builtin_fmaxf(M, ml[s].x);
  const float Ms = M == kNegInf ? 0.0f : M;
  float L = 0.0f;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int s = 0; s < p.S; ++s) {
    const float f = ex2(ml[s].x - Ms);
    L += ml[s].y * f;
    acc += *reinterpret_cast<const f32x4*>(p.part_o + (row * SS + s) * D + c4 * 4) * f;
  }
  f32x4 v;
  if (p.T2 > 0) {
    const float L2 = ml[p.S].y;
    const f32x4 o2 = *reinterpret_cast<const f32x4*>(p.part_o + (row * SS + p.S) * D + c4 * 4);
    v = acc * (L > 0.0f ? p.gates[0] / L : 0.0f) + o2 * (L2 > 0.0f ? p.gates[1] / L2 : 0.0f);
  } else {
    v = acc * (L > 0.0f ? 1.0f / L : 0.0f);
  }
  const int node = (int)(row % p.N);
  const int64_t bh = row / p.N;
  const int h = (int)(bh % p.H), b = (int)(bh / p.H);
  ta_store4<OT>(p.out, b * p.o_sb + h * p.o_sh + node * p.o_sr + c4 * 4, v);
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
struct TaPlan {
  int G, rows_per_group, QT, S, chunk;
};

// force_splits (>= 1) fixes the key splits (the args' field; 0: the plan's).
// window > 0: only the last window - 1 prefix rows (plus the tree) are walked.
// alibi: one split (the third segment walks all keys in split 0).
static TaPlan ta_plan(int B, int H, int Hkv, int N, int Tp, int d, int force_splits = 0, int window = 0,
                      bool alibi = false) {
  TaPlan pl{};
  const int qmax = d == 64 ? 64 : 32;  // query rows per group (register budget of O)
  const int rows = (H / Hkv) * N;
  pl.G = (rows + qmax - 1) / qmax;
  pl.rows_per_group = (rows + pl.G - 1) / pl.G;
  pl.QT = (pl.rows_per_group + 15) / 16;
  const int KT = (window > 0 && Tp > window - 1 ? window - 1 : Tp) + N;
  const int steps = (KT + 31) / 32;
  const int64_t base = (int64_t)B * Hkv * pl.G;
  // Key splits only to give every CU a workgroup: a grid that already has
  // one per CU runs unsplit (config 3, 256 workgroups of 66 key steps: 32.7
  // us unsplit against 35-36 us in two splits plus the merge launch), and a
  // split carries at least 8 key steps.
  const int64_t cus = device_cus();
  int S = base >= cus ? 1 : (int)((cus + base - 1) / base);
  const int sby_work = steps / 8 > 1 ? steps / 8 : 1;
  S = S < sby_work ? S : sby_work;
  const int smax = (steps + 3) / 4;  // at least one 32-key step per wave
  if (force_splits > 0) S = force_splits;
  if (alibi) S = 1;
  S = S < 1 ? 1 : (S > smax ? smax : S);
  const int steps_per = (steps + S - 1) / S;
  pl.chunk = steps_per * 32;
  pl.S = (KT + pl.chunk - 1) / pl.chunk;
  return pl;
}

static size_t ta_ws_bytes(const TaPlan& pl, int B, int H, int N, int d) {
  if (pl.S <= 1) return 0;
  Carve c(nullptr);
  const int64_t prow = (int64_t)B * H * N * (pl.S + 1);  // + the second segment's slot
  c.take<float>(prow * d);
  c.take<float2>(prow);
  return c.bytes();
}

// Workgroup shapes (the args' force_waves codes): 4, 8, 16 waves; 5 = 4
// waves and 9 = 8 waves with the next key step's loads in flight (a ring of
// two register sets).
struct TaShape {
  int nw, pf;
};
static TaShape ta_shape(int code) {
  if (code == 5) return {4, 2};
  if (code == 9) return {8, 2};
  return {code, 0};
}

// The shape of a launch.  A grid of at most one workgroup per CU gets 8 waves
// (8 with prefetch when the query tile is 3 or 4, 16 when neither fits), so
// each wave walks few key steps and more loads are in flight per CU; up to
// two per CU, 8 waves where the query tile fits them, else (d = 64) 4 waves
// with prefetch; larger grids keep 4 waves.  force (the args' force_waves)
// overrides the choice where the shape fits.  EXT launches (window / ALiBi)
// have 4 or 8 waves.
static int ta_waves(int D, int QT, int64_t nwg, int force, bool ext) {
  auto ok = [&](int code) {
    const TaShape sh = ta_shape(code);
    if (ext && (sh.pf || (sh.nw != 4 && sh.nw != 8))) return false;
    return ta_variant_ok(D, QT, sh.nw, sh.pf);
  };
  if (force && ok(force)) return force;
  if (ext) return ok(8) && nwg <= 2 * device_cus() ? 8 : 4;
  const int64_t cus = device_cus();
  if (nwg <= cus) {
    if (ok(8)) return 8;  // (measured at least as fast as 16 at decode shapes, with twice the registers)
    if (ok(9)) return 9;
    if (ok(16)) return 16;
    return 5;
  }
  if (nwg <= 2 * cus) {
    if (ok(8)) return 8;
    if (D == 64 && ok(5)) return 5;
  }
  return 4;
}

template <int D, int OT, int NW, int PF, bool EXT>
static void ta_launch_qt(const TreeAttnParams& p, int QT, dim3 grid, hipStream_t st) {
  const dim3 block(NW * 64);
  switch (QT) {
    case 1:
      if constexpr (ta_variant_ok(D, 1, NW, PF))
        hipLaunchKernelGGL((k_tree_attn<D, 1, OT, NW, PF, EXT>), grid, block, 0, st, p);
      break;
    case 2:
      if constexpr (ta_variant_ok(D, 2, NW, PF))
        hipLaunchKernelGGL((k_tree_attn<D, 2, OT, NW, PF, EXT>), grid, block, 0, st, p);
      break;
    case 3:
      if constexpr (ta_variant_ok(D, 3, NW, PF))
        hipLaunchKernelGGL((k_tree_attn<D, 3, OT, NW, PF, EXT>), grid, block, 0, st, p);
      break;
    default:
      if constexpr (ta_variant_ok(D, 4, NW, PF))
        hipLaunchKernelGGL((k_tree_attn<D, 4, OT, NW, PF, EXT>), grid, block, 0, st, p);
      break;
  }
}

template <int D, int OT>
static int ta_launch_d(TreeAttnParams p, int QT, bool ext, int force_waves, hipStream_t st, hipEvent_t* ev) {
  const int64_t nwg = (int64_t)p.B * p.Hkv * p.G * p.S;
  const dim3 grid((unsigned)nwg);
  const int nw = ta_waves(D, QT, nwg, force_waves, ext);
  const int waves = ta_shape(nw).nw;
  if (p.T2 > 0) {
    // split 0's share of waves for the second segment: a quarter, at most
    // one per 32-row step of it
    const int steps2 = (p.T2 + 31) / 32;
    p.W2 = waves / 4 < steps2 ? waves / 4 : steps2;
    if (p.W2 < 1) p.W2 = 1;
  }
  if (p.slopes) {
    // the ALiBi segment walks as many keys as segment 1: half the rest
    p.W3 = (waves - (p.T2 > 0 ? p.W2 : 0)) / 2;
    if (p.W3 < 1) p.W3 = 1;
  }
  if (ev) VNX_HIP_CHECK(hipEventRecord(ev[0], st));
  if (ext) {
    if (nw == 8) ta_launch_qt<D, OT, 8, 0, true>(p, QT, grid, st);
    else ta_launch_qt<D, OT, 4, 0, true>(p, QT, grid, st);
  } else {
    switch (nw) {
      case 16: ta_launch_qt<D, OT, 16, 0, false>(p, QT, grid, st); break;
      case 8: ta_launch_qt<D, OT, 8, 0, false>(p, QT, grid, st); break;
      case 5: ta_launch_qt<D, OT, 4, 2, false>(p, QT, grid, st); break;
      case 9: ta_launch_qt<D, OT, 8, 2, false>(p, QT, grid, st); break;
      default: ta_launch_qt<D, OT, 4, 0, false>(p, QT, grid, st); break;
    }
  }
  VNX_LAUNCH_CHECK();
  if (ev) VNX_HIP_CHECK(hipEventRecord(ev[1], st));
  if (p.S > 1) {
    const int64_t rows = (int64_t)p.B * p.H * p.N;
    const int rpb = 256 / (D / 4);
    hipLaunchKernelGGL((k_tree_merge<D, OT>), dim3((unsigned)((rows + rpb - 1) / rpb)), dim3(256), 0, st, p);
    VNX_LAUNCH_CHECK();
  }
  if (ev) VNX_HIP_CHECK(hipEventRecord(ev[2], st));
  return VNX_OK;
}

static bool strides_ok(int64_t sb, int64_t sh, int64_t sr, int unit) {
  return sb >= 0 && sh >= 0 && sr >= 0 && sb % unit == 0 && sh % unit == 0 && sr % unit == 0;
}

// ---------------------------------------------------------------------------
// fp32 rows with small heads (d = 8 / 16 / 32: the fp32 TriSparse models).
// One wave per query row (b, h, node i).  The lanes walk the row's keys 64
// apart, each lane keeping its own online softmax (running max m, sum l,
// output o[D]) for path A (prefix + tree keys inside the window) and path C
// (the same keys, no window, score + -(m_h * distance): ALiBi), sharing
// every key's q . k; the wave then merges the 64 lane states.  The second
// segment (path B, the global rows) follows in a loop of its own.  A chain
// (anc == NULL) lets node i see tree rows j <= i, so N is not held to one
// mask word and prefill chunks of any length run here.  Scores follow the
// reference's fp32 computation (tri_sparse_attn.py:258-378 window,
// :469-495 global rows, :489-530 ALiBi, mixed as :585-608).

struct F32RowsParams {
  const float* q;
  const float* kc;
  const float* vc;
  const float* kt;
  const float* vt;
  const uint64_t* anc;   // NULL: chain
  void* out;
  int64_t q_sb, q_sh, q_sr;
  int64_t c_sb, c_sh, c_sr;
  int64_t t_sb, t_sh, t_sr;
  int64_t o_sb, o_sh, o_sr;
  int64_t anc_sb;
  const float* k2;
  const float* v2;
  int64_t s2_sb, s2_sh, s2_sr;
  int T2;
  const float* gates;
  const float* slopes;
  int alibi_max, window;
  const int32_t* tp_batch;
  int follows;
  int B, H, N, Tp, n_rep;
  float scale;
};

template <int D>
struct RowSoftmax {
  float m, l;
  float o[D];
};

template <int D>
__device__ __forceinline__ void rs_init(RowSoftmax<D>& a) {
  a.m = -INFINITY;
  a.l = 0.0f;
#pragma unroll
  for (int d = 0; d < D; ++d) a.o[d] = 0.0f;
}

// e^x for x <= 0 on the transcendental unit
__device__ __forceinline__ float rs_exp(float x) { return ex2(x * 1.4426950408889634f); }

template <int D>
__device__ __forceinline__ void rs_add(RowSoftmax<D>& a, float s, const float (&v)[D]) {
  if (s > a.m) {
    const float c = rs_exp(a.m - s);  // 0 while a.m is -inf
    a.l *= c;
#pragma unroll
    for (int d = 0; d < D; ++d) a.o[d] *= c;
    a.m = s;
  }
  const float e = rs_exp(s - a.m);
  a.l += e;
#pragma unroll
  for (int d = 0; d < D; ++d) a.o[d] = fmaf(e, v[d], a.o[d]);
}

__device__ __forceinline__ float rs_wave_sum(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// Merges the 64 lane states; every lane returns the row's softmax output
// (sum_j e_j v_j / sum_j e_j), zeros when no lane saw a key.
template <int D>
__device__ __forceinline__ void rs_merge(RowSoftmax<D>& a) {
  float M = a.m;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
  const float c = a.m == -INFINITY ? 0.0f : rs_exp(a.m - M);
  const float L = rs_wave_sum(a.l * c);
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
#pragma unroll
  for (int d = 0; d < D; ++d) a.o[d] = rs_wave_sum(a.o[d] * c) * inv;
}

template <int D>
__device__ __forceinline__ void load_row_f32(const float* src, float (&r)[D]) {
#pragma unroll
  for (int d = 0; d < D; d += 4) {
    const f32x4 t = *reinterpret_cast<const f32x4*>(src + d);
    r[d] = t[0]; r[d + 1] = t[1]; r[d + 2] = t[2]; r[d + 3] = t[3];
  }
}

template <int D>
__device__ __forceinline__ float dot_f32(const float (&q)[D], const float (&k)[D]) {
  float s = 0.0f;
#pragma unroll
  for (int d = 0; d < D; ++d) s = fmaf(q[d], k[d], s);
  return s;
}

template <int D, int OT>
__global__ __launch_bounds__(256) void k_attn_rows_f32(F32RowsParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= (int64_t)p.B * p.H * p.N) return;  // whole waves leave; no barriers below
  const int i = (int)(r % p.N);
  const int h = (int)((r / p.N) % p.H);
  const int b = (int)(r / ((int64_t)p.N * p.H));
  const int kvh = h / p.n_rep;
  int tp = p.Tp;
  if (p.tp_batch) {
    const int t = p.tp_batch[b];
    tp = t < 0 ? 0 : t > p.Tp ? p.Tp : t;
  }
  float q[D];
  load_row_f32<D>(p.q + b * p.q_sb + h * p.q_sh + i * p.q_sr, q);
  const uint64_t* anc = p.anc ? p.anc + b * p.anc_sb : nullptr;
  const uint64_t w = anc ? anc[i] : 0;
  const int pos_i = tp + (anc ? __popcll(w) - 1 : i);
  const int nk = tp + (anc ? p.N : i + 1);
  const bool alibi = p.slopes && tp + p.N <= p.alibi_max;
  const float slope = alibi ? p.slopes[h] : 0.0f;
  // prefix rows (position = index) a window leaves out are skipped outright
  int lo = 0;
  if (p.window > 0 && !alibi) {
    lo = pos_i - p.window + 1;
    lo = lo < 0 ? 0 : lo > tp ? tp : lo;
  }
  RowSoftmax<D> A, C;
  rs_init(A);
  rs_init(C);
  for (int t = lo + lane; t < nk; t += 64) {
    int64_t off;
    const float* kb;
    const float* vb;
    int kpos;
    if (t < tp) {
      off = b * p.c_sb + kvh * p.c_sh + t * p.c_sr;
      kb = p.kc;
      vb = p.vc;
      kpos = t;
    } else {
      const int j = t - tp;
      if (anc && !((w >> j) & 1ull)) continue;
      off = b * p.t_sb + kvh * p.t_sh + (int64_t)(p.follows ? tp + j : j) * p.t_sr;
      kb = p.kt;
      vb = p.vt;
      kpos = tp + (anc ? __popcll(anc[j]) - 1 : j);
    }
    float k[D], v[D];
    load_row_f32<D>(kb + off, k);
    load_row_f32<D>(vb + off, v);
    const float s = dot_f32<D>(q, k) * p.scale;
    const int dist = pos_i - kpos;
    if (p.window <= 0 || dist < p.window) rs_add<D>(A, s, v);
    if (alibi) rs_add<D>(C, s + -(slope * (float)dist), v);
  }
  rs_merge<D>(A);
  if (alibi) rs_merge<D>(C);
  const bool has2 = p.T2 > 0;
  const float g1 = (has2 || p.slopes) ? p.gates[0] : 1.0f;
  RowSoftmax<D> S2;
  rs_init(S2);
  if (has2) {
    const int64_t base = b * p.s2_sb + kvh * p.s2_sh;
    for (int t = lane; t < p.T2; t += 64) {
      float k[D], v[D];
      load_row_f32<D>(p.k2 + base + t * p.s2_sr, k);
      load_row_f32<D>(p.v2 + base + t * p.s2_sr, v);
      rs_add<D>(S2, dot_f32<D>(q, k) * p.scale, v);
    }
    rs_merge<D>(S2);
  }
  if (lane != 0) return;
  const float g2 = has2 ? p.gates[1] : 0.0f;
  const float g3 = alibi ? p.gates[2] : 0.0f;
  const int64_t ob = b * p.o_sb + h * p.o_sh + i * p.o_sr;
#pragma unroll
  for (int d = 0; d < D; d += 4) {
    f32x4 y;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float t = g1 * A.o[d + e];
      if (has2) t = t + g2 * S2.o[d + e];
      if (alibi) t = t + g3 * C.o[d + e];
      y[e] = t;
    }
    ta_store4<OT>(p.out, ob + d, y);
  }
}

template <int D>
static void attn_rows_launch(const F32RowsParams& p, int ot, hipStream_t st) {
  const int64_t rows = (int64_t)p.B * p.H * p.N;
  const dim3 grid((unsigned)((rows + 3) / 4));
  if (ot == 0) hipLaunchKernelGGL((k_attn_rows_f32<D, 0>), grid, dim3(256), 0, st, p);
  else if (ot == 1) hipLaunchKernelGGL((k_attn_rows_f32<D, 1>), grid, dim3(256), 0, st, p);
  else hipLaunchKernelGGL((k_attn_rows_f32<D, 2>), grid, dim3(256), 0, st, p);
}

// vnx_tree_attn with f32_rows set: the argument checks of that path, then one
// launch (no workspace).
static int tree_attn_f32(const vnx_tree_attn_args* a, void* stream) {
  const int B = a->B, H = a->H, Hkv = a->Hkv, N = a->N, Tp = a->Tp, d = a->d;
  if (d != 8 && d != 16 && d != 32) return VNX_ERR_UNSUPPORTED;
  if (a->qkv) return VNX_ERR_UNSUPPORTED;  // queries and rows come in ready
  if (a->anc && N > kTaMaxN) return VNX_ERR_UNSUPPORTED;
  if (a->window < 0 || a->alibi_max_keys < 0 || a->T2 < 0) return VNX_ERR_INVALID_ARG;
  if (B == 0) return VNX_OK;
  if (!a->q || !a->k_tree || !a->v_tree || !a->out) return VNX_ERR_INVALID_ARG;
  if (Tp > 0 && (!a->k_cache || !a->v_cache)) return VNX_ERR_INVALID_ARG;
  if ((a->T2 > 0 || a->alibi_slopes) && (!a->gates || (reinterpret_cast<uintptr_t>(a->gates) & 3u)))
    return VNX_ERR_INVALID_ARG;
  if (a->alibi_slopes && (reinterpret_cast<uintptr_t>(a->alibi_slopes) & 3u)) return VNX_ERR_INVALID_ARG;
  if (a->T2 > 0 && (!a->k_seg2 || !a->v_seg2)) return VNX_ERR_INVALID_ARG;
  if (a->tp_batch && (reinterpret_cast<uintptr_t>(a->tp_batch) & 3u)) return VNX_ERR_INVALID_ARG;
  if (!(a->scale > 0.0f) || !__builtin_isfinite(a->scale)) return VNX_ERR_INVALID_ARG;
  if (a->anc_batch_stride < 0) return VNX_ERR_INVALID_ARG;
  if (((int64_t)B * H * N + 3) / 4 >= INT32_MAX) return VNX_ERR_UNSUPPORTED;  // one wave per row, 4 per workgroup
  // 16-byte loads of fp32 rows; 4-element output stores
  if (!strides_ok(a->q_strides[0], a->q_strides[1], a->q_strides[2], 4) ||
      !strides_ok(a->cache_strides[0], a->cache_strides[1], a->cache_strides[2], 4) ||
      !strides_ok(a->tree_strides[0], a->tree_strides[1], a->tree_strides[2], 4) ||
      !strides_ok(a->out_strides[0], a->out_strides[1], a->out_strides[2], 4) ||
      (a->T2 > 0 && !strides_ok(a->seg2_strides[0], a->seg2_strides[1], a->seg2_strides[2], 4)))
    return VNX_ERR_UNSUPPORTED;
  if (!aligned16(a->q) || !aligned16(a->k_tree) || !aligned16(a->v_tree) || !aligned16(a->out) ||
      (Tp > 0 && (!aligned16(a->k_cache) || !aligned16(a->v_cache))) ||
      (a->T2 > 0 && (!aligned16(a->k_seg2) || !aligned16(a->v_seg2))) ||
      (a->anc && (reinterpret_cast<uintptr_t>(a->anc) & 7u)))
    return VNX_ERR_UNSUPPORTED;
  F32RowsParams p{};
  p.q = static_cast<const float*>(a->q);
  p.kc = static_cast<const float*>(Tp > 0 ? a->k_cache : a->k_tree);
  p.vc = static_cast<const float*>(Tp > 0 ? a->v_cache : a->v_tree);
  p.kt = static_cast<const float*>(a->k_tree);
  p.vt = static_cast<const float*>(a->v_tree);
  p.anc = a->anc;
  p.out = a->out;
  p.q_sb = a->q_strides[0]; p.q_sh = a->q_strides[1]; p.q_sr = a->q_strides[2];
  p.c_sb = a->cache_strides[0]; p.c_sh = a->cache_strides[1]; p.c_sr = a->cache_strides[2];
  p.t_sb = a->tree_strides[0]; p.t_sh = a->tree_strides[1]; p.t_sr = a->tree_strides[2];
  p.o_sb = a->out_strides[0]; p.o_sh = a->out_strides[1]; p.o_sr = a->out_strides[2];
  p.anc_sb = a->anc_batch_stride;
  if (a->T2 > 0) {
    p.k2 = static_cast<const float*>(a->k_seg2);
    p.v2 = static_cast<const float*>(a->v_seg2);
    p.s2_sb = a->seg2_strides[0]; p.s2_sh = a->seg2_strides[1]; p.s2_sr = a->seg2_strides[2];
    p.T2 = a->T2;
  }
  p.gates = a->gates;
  p.slopes = a->alibi_slopes;
  p.alibi_max = a->alibi_max_keys;
  p.window = a->window;
  p.tp_batch = a->tp_batch;
  p.follows = a->tree_follows_prefix ? 1 : 0;
  p.B = B; p.H = H; p.N = N; p.Tp = Tp; p.n_rep = H / Hkv;
  p.scale = a->scale;
  const int ot = a->out_dtype == VNX_F32 ? 0 : a->out_dtype == VNX_BF16 ? 1 : 2;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (d == 8) attn_rows_launch<8>(p, ot, st);
  else if (d == 16) attn_rows_launch<16>(p, ot, st);
  else attn_rows_launch<32>(p, ot, st);
  VNX_LAUNCH_CHECK();
  return VNX_OK;
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

size_t vnx_tree_attn_workspace_args(const vnx_tree_attn_args* a) {
  if (!a) return 256;
  const int B = a->B, H = a->H, Hkv = a->Hkv, N = a->N, Tp = a->Tp, d = a->d;
  if (B <= 0 || H <= 0 || Hkv <= 0 || H % Hkv || N <= 0 || N > kTaMaxN || Tp < 0 || (d != 64 && d != 128) ||
      a->window < 0 || a->force_splits < 0)
    return 256;
  const bool ext = a->alibi_slopes || (a->window > 0 && Tp + N > a->window);
  const TaPlan pl = ta_plan(B, H, Hkv, N, Tp, d, a->force_splits, ext ? a->window : 0, a->alibi_slopes != nullptr);
  const size_t n = ta_ws_bytes(pl, B, H, N, d);
  return n < 256 ? 256 : n;
}

int vnx_tree_attn(const vnx_tree_attn_args* a, void* workspace, size_t workspace_bytes, void* stream) {
  if (!a) return VNX_ERR_INVALID_ARG;
  const int B = a->B, H = a->H, Hkv = a->Hkv, N = a->N, Tp = a->Tp, d = a->d;
  if (B < 0 || H <= 0 || Hkv <= 0 || H % Hkv || N < 1 || Tp < 0) return VNX_ERR_INVALID_ARG;
  if (a->out_dtype != VNX_F32 && a->out_dtype != VNX_BF16 && a->out_dtype != VNX_F16) return VNX_ERR_UNSUPPORTED;
  if (a->f32_rows) return tree_attn_f32(a, stream);
  if (N > kTaMaxN || (d != 64 && d != 128)) return VNX_ERR_UNSUPPORTED;
  if (a->T2 < 0) return VNX_ERR_INVALID_ARG;
  if (B == 0) return VNX_OK;
  if ((!a->q && !a->qkv) || !a->k_tree || !a->v_tree || !a->anc || !a->out) return VNX_ERR_INVALID_ARG;
  if (a->qkv) {
    // the projection rows: RoPE and the tree rows' cache write here
    if (!a->tree_follows_prefix || !a->tp_batch || a->cap < 1) return VNX_ERR_INVALID_ARG;
    if (a->qkv_ld < (int64_t)(H + 2 * Hkv) * d) return VNX_ERR_INVALID_ARG;
    if (a->rope && (!a->cos_table || !a->sin_table || a->table_rows < 1)) return VNX_ERR_INVALID_ARG;
    if (a->rope && (!aligned16(a->cos_table) || !aligned16(a->sin_table))) return VNX_ERR_UNSUPPORTED;
    if (!aligned16(a->qkv) || a->qkv_ld % 8) return VNX_ERR_UNSUPPORTED;
  }
  if (a->window < 0 || a->alibi_max_keys < 0 || a->force_splits < 0 || a->force_waves < 0)
    return VNX_ERR_INVALID_ARG;
  if (a->window > 0 && a->window < N) return VNX_ERR_UNSUPPORTED;  // tree keys always inside the window
  if (a->alibi_slopes && (!a->gates || (reinterpret_cast<uintptr_t>(a->gates) & 3u) ||
                          (reinterpret_cast<uintptr_t>(a->alibi_slopes) & 3u)))
    return VNX_ERR_INVALID_ARG;
  if (a->T2 > 0) {
    if (!a->k_seg2 || !a->v_seg2 || !a->gates || (reinterpret_cast<uintptr_t>(a->gates) & 3u))
      return VNX_ERR_INVALID_ARG;
    if (!strides_ok(a->seg2_strides[0], a->seg2_strides[1], a->seg2_strides[2], 8) ||
        !aligned16(a->k_seg2) || !aligned16(a->v_seg2))
      return VNX_ERR_UNSUPPORTED;
  }
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
  if ((a->q && !aligned16(a->q)) || !aligned16(a->k_tree) || !aligned16(a->v_tree) || !aligned16(a->out) ||
      (Tp > 0 && (!aligned16(a->k_cache) || !aligned16(a->v_cache))) ||
      (reinterpret_cast<uintptr_t>(a->anc) & 7u))
    return VNX_ERR_UNSUPPORTED;
  // EXT variant: ALiBi, or a window some row's keys reach past
  const bool ext = a->alibi_slopes || (a->window > 0 && Tp + N > a->window);
  const int window = ext ? a->window : 0;
  const TaPlan pl = ta_plan(B, H, Hkv, N, Tp, d, a->force_splits, window, a->alibi_slopes != nullptr);
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
  if (a->T2 > 0) {
    p.k2 = static_cast<const uint16_t*>(a->k_seg2);
    p.v2 = static_cast<const uint16_t*>(a->v_seg2);
    p.s2_sb = a->seg2_strides[0]; p.s2_sh = a->seg2_strides[1]; p.s2_sr = a->seg2_strides[2];
    p.T2 = a->T2;
    p.gates = a->gates;
  }
  p.c = (float)((double)a->scale * 1.4426950408889634);
  p.window = window;
  p.slopes = a->alibi_slopes;
  p.alibi_max = a->alibi_max_keys;
  if (p.slopes) p.gates = a->gates;
  if (a->qkv) {
    p.qkv = static_cast<const uint16_t*>(a->qkv);
    p.qkv_ld = a->qkv_ld;
    p.cos = a->cos_table;
    p.sin = a->sin_table;
    p.rope = a->rope ? 1 : 0;
    p.cap = a->rope ? (a->cap < a->table_rows ? a->cap : a->table_rows) : a->cap;
  }
  if (pl.S > 1) {
    Carve c(workspace);
    const int64_t prow = (int64_t)B * H * N * (pl.S + 1);
    p.part_o = c.take<float>(prow * d);
    p.part_ml = c.take<float2>(prow);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipEvent_t* ev = profile_slot(2);
  const int ot = a->out_dtype == VNX_F32 ? 0 : a->out_dtype == VNX_BF16 ? 1 : 2;
  const int fw = a->force_waves;
  if (d == 64)
    return ot == 0   ? ta_launch_d<64, 0>(p, pl.QT, ext, fw, st, ev)
           : ot == 1 ? ta_launch_d<64, 1>(p, pl.QT, ext, fw, st, ev)
                     : ta_launch_d<64, 2>(p, pl.QT, ext, fw, st, ev);
  return ot == 0   ? ta_launch_d<128, 0>(p, pl.QT, ext, fw, st, ev)
         : ot == 1 ? ta_launch_d<128, 1>(p, pl.QT, ext, fw, st, ev)
                   : ta_launch_d<128, 2>(p, pl.QT, ext, fw, st, ev);
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
