// Row top-b: the b best ids of each vocab row (tree expansion: a node's
// children take the best ids of its parent's draft row).
//
// Order: value descending, ties to the lower id, NaN above every number (the
// numpy.argmax order, so b = 1 is argmax); -inf ranks below every number.
// Two launches, no cross-workgroup
// signalling: k_topk_filter (rows of up to 64 chunks of 8,192) or
// k_topk_chunk (longer rows) reduces one chunk of one row per workgroup and
// writes its best KB (b rounded up to a power of two) to the workspace;
// k_topk_merge merges a row's chunk lists in one wave.
#include "rowred.h"
#include "vnx_internal.h"

namespace vnx {
namespace {

constexpr int kTNT = 256;
constexpr int kTNB = 4;
constexpr int kTopMaxChunks = 64;
constexpr int kTopMaxB = 16;

// Order key of (value, id): the value's bits made unsigned-monotone (NaN
// above +inf, -inf above an empty slot, -0 equal to +0), the id inverted
// below them, so
// a larger key is a better element in the numpy.argmax order.
__device__ __forceinline__ uint32_t vkey(float x) {
  const uint32_t u = x == 0.0f ? 0u : __float_as_uint(x);  // -0 ties with +0
  const uint32_t k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return __builtin_isnan(x) ? 0xFFFFFFFFu : k;
}

__device__ __forceinline__ float vkey_value(uint32_t k) {
  if (k == 0xFFFFFFFFu) return __builtin_nanf("");
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

__device__ __forceinline__ uint64_t full_key(uint32_t vk, int64_t id) {
  return ((uint64_t)vk << 32) | (uint32_t)~(uint32_t)id;
}

// Per-thread best KB of the elements this thread sees, in arrival order
// (increasing ids): a strictly larger value key displaces, so an equal value
// that arrives later never passes an earlier one (lower id first).  The
// insertion is a branchless compare-exchange network (one compare and four
// selects per level).  Ids are offsets inside the chunk.
template <int KB>
struct TopList {
  uint32_t k[KB];
  uint32_t i[KB];
  __device__ __forceinline__ void init() {
#pragma unroll
    for (int q = 0; q < KB; ++q) { k[q] = 0u; i[q] = 0xFFFFFFFFu; }
  }
  __device__ __forceinline__ void push(uint32_t x, uint32_t ix) {
#pragma unroll
    for (int q = 0; q < KB; ++q) {
      const bool c = x > k[q];
      const uint32_t nk = c ? x : k[q], ni = c ? ix : i[q];
      x = c ? k[q] : x;
      ix = c ? i[q] : ix;
      k[q] = nk;
      i[q] = ni;
    }
  }
};

// A merged list of full 64-bit keys (best first).
template <int KB>
struct KeyList {
  uint64_t k[KB];
  // Drops the head (after it won a merge round).
  __device__ __forceinline__ void pop() {
#pragma unroll
    for (int q = 0; q < KB - 1; ++q) k[q] = k[q + 1];
    k[KB - 1] = 0ull;
  }
};

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t w = __shfl_xor(v, o, VNX_WAVE);
    v = w > v ? w : v;
  }
  return v;
}

struct TopkParams {
  const void* x;
  int64_t rows, V, ld;
  int chunks;
  int64_t chunk_len;  // multiple of the vector width
  uint64_t* part;     // (rows, chunks, KB) full keys, best first
  int b;
  int64_t* ids;       // (rows, ldo)
  float* vals;        // (rows, ldo) or NULL
  int64_t ldo;
};

template <typename Tin, int KB>
__global__ __launch_bounds__(kTNT) void k_topk_chunk(TopkParams p) {
  constexpr int VE = Vec<Tin>::N;
  __shared__ uint64_t sk[kTNT / VNX_WAVE];
  const int64_t r = blockIdx.x / p.chunks;
  const int c = blockIdx.x % p.chunks;
  const Tin* row = static_cast<const Tin*>(p.x) + r * p.ld;
  const int64_t c0 = (int64_t)c * p.chunk_len;
  const int64_t c1 = c0 + p.chunk_len < p.V ? c0 + p.chunk_len : p.V;
  const int tid = threadIdx.x;
  TopList<KB> L;
  L.init();
  const int64_t n = c1 - c0;
  const int64_t nvec = n / VE;
  const int64_t nfull = nvec / ((int64_t)kTNT * kTNB) * ((int64_t)kTNT * kTNB);
  for (int64_t v0 = 0; v0 < nfull; v0 += (int64_t)kTNT * kTNB) {
    float x[kTNB * VE];
#pragma unroll
    for (int j = 0; j < kTNB; ++j) Vec<Tin>::load(row + c0 + (v0 + tid + (int64_t)kTNT * j) * VE, &x[j * VE]);
#pragma unroll
    for (int j = 0; j < kTNB; ++j) {
      const uint32_t off = (uint32_t)((v0 + tid + (int64_t)kTNT * j) * VE);
#pragma unroll
      for (int e = 0; e < VE; ++e) L.push(vkey(x[j * VE + e]), off + e);
    }
  }
  for (int64_t vi = nfull + tid; vi < nvec; vi += kTNT) {
    float x[VE];
    Vec<Tin>::load(row + c0 + vi * VE, x);
#pragma unroll
    for (int e = 0; e < VE; ++e) L.push(vkey(x[e]), (uint32_t)(vi * VE + e));
  }
  // Scalar tail (fewer than VE elements after the last full vector).
  const int64_t tail0 = nvec * VE;
  if (tid < n - tail0) L.push(vkey(Vec<Tin>::load1(row + c0 + tail0 + tid)), (uint32_t)(tail0 + tid));

  // Block merge: KB rounds of a block max over the list heads (full keys,
  // unique across threads since ids are).
  KeyList<KB> K;
#pragma unroll
  for (int q = 0; q < KB; ++q) K.k[q] = L.i[q] == 0xFFFFFFFFu ? 0ull : full_key(L.k[q], c0 + L.i[q]);
  uint64_t* out = p.part + ((size_t)r * p.chunks + c) * KB;
  const int w = tid / VNX_WAVE, l = tid % VNX_WAVE;
#pragma unroll
  for (int q = 0; q < KB; ++q) {
    const uint64_t wm = wave_max_u64(K.k[0]);
    __syncthreads();
    if (l == 0) sk[w] = wm;
    __syncthreads();
    uint64_t best = sk[0];
#pragma unroll
    for (int j = 1; j < kTNT / VNX_WAVE; ++j) best = sk[j] > best ? sk[j] : best;
    if (K.k[0] == best && best != 0ull) K.pop();
    if (tid == 0) out[q] = best;
  }
}

// Chunks of kFiltLen elements (32 per thread, all loaded at once): each
// thread's largest key, then per wave the KB-th largest of its 64 lanes'
// maxima, t_w -- KB threads of that wave hold an element >= t_w, so t_w is a
// lower bound of the chunk's KB-th best, and so is t = max_w t_w.  Only
// elements with key >= t enter the per-thread lists (a few per chunk), so
// the per-element cost is the key and two compares instead of the insertion
// network; the lists are then merged as in k_topk_chunk.
constexpr int kFiltPer = 32;                    // elements per thread
constexpr int64_t kFiltLen = (int64_t)kTNT * kFiltPer;

template <typename Tin, int KB>
__global__ __launch_bounds__(kTNT) void k_topk_filter(TopkParams p) {
  constexpr int VE = Vec<Tin>::N;
  constexpr int NV = kFiltPer / VE;             // vectors per thread
  __shared__ uint64_t sk[kTNT / VNX_WAVE];
  __shared__ uint32_t st[kTNT / VNX_WAVE];
  const int64_t r = blockIdx.x / p.chunks;
  const int c = blockIdx.x % p.chunks;
  const Tin* row = static_cast<const Tin*>(p.x) + r * p.ld;
  const int64_t c0 = (int64_t)c * p.chunk_len;
  const int64_t c1 = c0 + p.chunk_len < p.V ? c0 + p.chunk_len : p.V;
  const int64_t n = c1 - c0;
  const int tid = threadIdx.x;
  const int w = tid / VNX_WAVE, l = tid % VNX_WAVE;
  // vector j of this thread covers offsets (tid + kTNT*j)*VE .. +VE
  // Every full vector's load first (raw bits), the keys after: a conversion
  // beside its load would wait there for every load in flight.
  // The loads carry no condition (vectors past the chunk re-read its last full
  // vector; their keys come from the element loads below), so no select or
  // copy sits beside them.
  uint32_t key[kFiltPer];
  u32x4 raw[NV];
  if (n >= VE) {  // uniform
    const int64_t last = (n / VE - 1) * VE;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t off = (int64_t)(tid + kTNT * j) * VE;
      raw[j] = Vec<Tin>::load_raw(row + c0 + (off + VE <= n ? off : last));
    }
  }
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t off = (int64_t)(tid + kTNT * j) * VE;
    if (off + VE <= n) {
      float x[VE];
      Vec<Tin>::cvt_raw(raw[j], x);
#pragma unroll
      for (int e = 0; e < VE; ++e) key[j * VE + e] = vkey(x[e]);
    } else {
#pragma unroll
      for (int e = 0; e < VE; ++e)
        key[j * VE + e] = off + e < n ? vkey(Vec<Tin>::load1(row + c0 + off + e)) : 0u;  // 0: no element
    }
  }
  uint32_t tmax = 0u;
#pragma unroll
  for (int q = 0; q < kFiltPer; ++q) tmax = key[q] > tmax ? key[q] : tmax;
  // the wave's KB-th largest lane maximum (lane index breaks ties)
  uint64_t cur = ((uint64_t)tmax << 32) | (uint32_t)l;
  uint32_t tw = 0u;
#pragma unroll
  for (int q = 0; q < KB; ++q) {
    const uint64_t m = wave_max_u64(cur);
    if (cur == m) cur = 0ull;
    tw = (uint32_t)(m >> 32);
  }
  if (l == 0) st[w] = tw;
  __syncthreads();
  uint32_t t = st[0];
#pragma unroll
  for (int j = 1; j < kTNT / VNX_WAVE; ++j) t = st[j] > t ? st[j] : t;
  TopList<KB> L;
  L.init();
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int e = 0; e < VE; ++e) {
      const uint32_t k = key[j * VE + e];
      if (k != 0u && k >= t) L.push(k, (uint32_t)((tid + kTNT * j) * VE + e));
    }
  KeyList<KB> K;
#pragma unroll
  for (int q = 0; q < KB; ++q) K.k[q] = L.i[q] == 0xFFFFFFFFu ? 0ull : full_key(L.k[q], c0 + L.i[q]);
  uint64_t* out = p.part + ((size_t)r * p.chunks + c) * KB;
#pragma unroll
  for (int q = 0; q < KB; ++q) {
    const uint64_t wm = wave_max_u64(K.k[0]);
    __syncthreads();
    if (l == 0) sk[w] = wm;
    __syncthreads();
    uint64_t best = sk[0];
#pragma unroll
    for (int j = 1; j < kTNT / VNX_WAVE; ++j) best = sk[j] > best ? sk[j] : best;
    if (K.k[0] == best && best != 0ull) K.pop();
    if (tid == 0) out[q] = best;
  }
}

// One wave per row: lane c holds chunk c's sorted list.
template <int KB>
__global__ __launch_bounds__(kTNT) void k_topk_merge(TopkParams p) {
  const int lane = threadIdx.x % VNX_WAVE;
  const int64_t r = (int64_t)blockIdx.x * (kTNT / VNX_WAVE) + threadIdx.x / VNX_WAVE;
  if (r >= p.rows) return;
  KeyList<KB> K;
#pragma unroll
  for (int q = 0; q < KB; ++q) K.k[q] = lane < p.chunks ? p.part[((size_t)r * p.chunks + lane) * KB + q] : 0ull;
#pragma unroll
  for (int q = 0; q < KB; ++q) {
    const uint64_t best = wave_max_u64(K.k[0]);
    if (K.k[0] == best && best != 0ull) K.pop();
    if (lane == 0 && q < p.b) {
      p.ids[r * p.ldo + q] = (int64_t)(uint32_t)~(uint32_t)best;
      if (p.vals) p.vals[r * p.ldo + q] = vkey_value((uint32_t)(best >> 32));
    }
  }
}

template <typename Tin, int KB>
void launch_topk(const TopkParams& p, hipStream_t s) {
  if (p.chunk_len == kFiltLen)
    hipLaunchKernelGGL((k_topk_filter<Tin, KB>), dim3((unsigned)(p.rows * p.chunks)), dim3(kTNT), 0, s, p);
  else
    hipLaunchKernelGGL((k_topk_chunk<Tin, KB>), dim3((unsigned)(p.rows * p.chunks)), dim3(kTNT), 0, s, p);
  hipLaunchKernelGGL(k_topk_merge<KB>, dim3((unsigned)((p.rows + 3) / 4)), dim3(kTNT), 0, s, p);
}

int kb_of(int b) {
  int kb = 1;
  while (kb < b) kb <<= 1;
  return kb;
}

// Rows of at most kTopMaxChunks filter chunks take the filter kernel (one
// chunk of kFiltLen per workgroup); longer rows the streaming kernel.
void topk_plan(int64_t rows, int64_t V, int dtype, int* chunks, int64_t* len) {
  const int ve = dtype == VNX_F32 ? 4 : 8;
  if (V <= kFiltLen * kTopMaxChunks) {
    *len = kFiltLen;
    *chunks = (int)((V + kFiltLen - 1) / kFiltLen);
    return;
  }
  const int c = pick_chunks(rows, V, ve, kTopMaxChunks, 2048);
  const int64_t l = ((V + c - 1) / c + ve - 1) / ve * ve;
  *len = l;
  *chunks = (int)((V + l - 1) / l);
}

}  // namespace
}  // namespace vnx

using namespace vnx;

extern "C" {

size_t vnx_row_topk_workspace(int64_t rows, int64_t V, int b) {
  if (rows <= 0 || V <= 0 || b < 1 || b > kTopMaxB) return 256;
  int c;
  int64_t len;
  topk_plan(rows, V, VNX_F32, &c, &len);  // fp32 plans the most chunks
  const int kb = kb_of(b);
  Carve cv(nullptr);
  cv.take<uint64_t>((size_t)rows * c * kb);
  return cv.bytes();
}

int vnx_row_topk(const void* logits, int dtype, int64_t rows, int64_t V, int64_t ld, int b,
                 int64_t* ids, float* vals, int64_t ldo, void* workspace, size_t workspace_bytes,
                 void* stream) {
  if (dtype != VNX_F32 && dtype != VNX_BF16) return VNX_ERR_UNSUPPORTED;
  if (rows < 0 || V <= 0 || b < 1 || b > kTopMaxB || b > V || ldo < b) return VNX_ERR_INVALID_ARG;
  if (rows == 0) return VNX_OK;  // nothing is read or written: any pointers
  if (!ids) return VNX_ERR_INVALID_ARG;
  // Ids travel as 32-bit offsets inside 64-bit keys.
  if (rows > (1 << 24) || V >= ((int64_t)1 << 31)) return VNX_ERR_UNSUPPORTED;
  const int ve = dtype == VNX_F32 ? 4 : 8;
  if (!logits || ld < V) return VNX_ERR_INVALID_ARG;
  if (!aligned16(logits) || ld % ve != 0) return VNX_ERR_UNSUPPORTED;
  int c;
  int64_t len;
  topk_plan(rows, V, dtype, &c, &len);
  if (rows * (int64_t)c >= INT32_MAX) return VNX_ERR_UNSUPPORTED;
  const int kb = kb_of(b);
  Carve cv(workspace);
  TopkParams p{};
  p.part = cv.take<uint64_t>((size_t)rows * c * kb);
  if (!workspace || workspace_bytes < cv.bytes()) return VNX_ERR_WORKSPACE;
  p.x = logits; p.rows = rows; p.V = V; p.ld = ld; p.chunks = c; p.chunk_len = len;
  p.b = b; p.ids = ids; p.vals = vals; p.ldo = ldo;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto go = [&](auto tin) {
    using Tin = decltype(tin);
    switch (kb) {
      case 1: launch_topk<Tin, 1>(p, s); break;
      case 2: launch_topk<Tin, 2>(p, s); break;
      case 4: launch_topk<Tin, 4>(p, s); break;
      case 8: launch_topk<Tin, 8>(p, s); break;
      default: launch_topk<Tin, 16>(p, s); break;
    }
  };
  if (dtype == VNX_F32) go(float{});
  else go(__hip_bfloat16{});
  VNX_LAUNCH_CHECK();
  return VNX_OK;
}

}  // extern "C"
