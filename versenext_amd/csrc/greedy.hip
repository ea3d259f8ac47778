// Greedy verify (the reference semantics, batched): one launch, grid
// B*rows_t*C of argmax chunks; the last workgroup of batch row b merges the
// row argmaxes and applies the longest-prefix rule.
#include "rowred.h"
#include "vnx_internal.h"

namespace vnx {

constexpr int kNT = 256;
constexpr int kNB = 8;
constexpr int kMaxK = 64;
constexpr int kMaxChunks = 64;

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

// Last workgroup of batch row b: pred[i] (and main_pred[b, i] when given) =
// the argmax of row i < rows_t from its chunk partials.  The partials of b
// are contiguous (row-major by i): read in tiles of kNT with one coherent
// load per thread, merged per row from LDS in chunk order.  Ends with a
// barrier, so every thread sees pred[].
__device__ void merge_row_argmax(const float* part_v, const int64_t* part_i, int64_t b, int rows_t,
                                 int chunks, int64_t* pred, int64_t* main_pred) {
  __shared__ float tile_v[kNT];
  __shared__ int64_t tile_i[kNT];
  const int tid = threadIdx.x;
  float bv = kNegInf;
  int64_t bi = INT64_MAX;
  const int64_t base = b * rows_t * chunks;
  const int total = rows_t * chunks;
  for (int t0 = 0; t0 < total; t0 += kNT) {
    if (t0 + tid < total) {
      tile_v[tid] = ld_agent(&part_v[base + t0 + tid]);
      tile_i[tid] = ld_agent(&part_i[base + t0 + tid]);
    }
    __syncthreads();
    if (tid < rows_t) {
      const int lo = max(tid * chunks, t0), hi = min((tid + 1) * chunks, min(t0 + kNT, total));
      for (int i = lo; i < hi; ++i)
        if (argmax_better(tile_v[i - t0], tile_i[i - t0], bv, bi)) { bv = tile_v[i - t0]; bi = tile_i[i - t0]; }
    }
    __syncthreads();
  }
  if (tid < rows_t) {
    pred[tid] = bi;
    if (main_pred) main_pred[b * rows_t + tid] = bi;
  }
  __syncthreads();
}

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
  const TScale one{1.0f, 1.0f};
  ChunkResult cr = reduce_chunk<Tin, SM_ID, false, false, true, kNT, kNB>(row, c0, c1, one, kNegInf, lds);
  const int64_t slot = (b * p.rows_t + i) * p.chunks + c;
  if (threadIdx.x == 0) {
    st_agent(&p.part_v[slot], cr.av);
    st_agent(&p.part_i[slot], cr.ai);
  }
  if (!arrive_last(&p.cnt[b], (unsigned)(p.rows_t * p.chunks), &last_flag)) return;
  merge_row_argmax(p.part_v, p.part_i, b, p.rows_t, p.chunks, pred, p.main_pred);
  const int tid = threadIdx.x;
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

// ---------------------------------------------------------------------------
// Greedy tree verification.  Node i (BFS order, parent[i] < i) is accepted
// iff its token equals the argmax of its parent's target row (row 0 for the
// root's children, 1 + parent otherwise) and every ancestor is accepted.  The
// chosen node is the deepest accepted one (lowest index among equally deep
// ones); its root path is emitted, then the argmax of its own row (row 0 when
// no node is accepted) as the bonus token.
// ---------------------------------------------------------------------------
constexpr int kMaxNodes = 64;

struct TreeShape {
  uint64_t anc[kMaxNodes];  // ancestor-or-self words
  int8_t prow[kMaxNodes];   // target row holding the prediction for node i
};

struct TreeGreedyParams {
  const void* tgt;
  int64_t B;
  int N;
  int64_t V, ld, sb;
  int chunks;
  int64_t chunk_len;
  const int64_t* tokens;
  int64_t ld_tok;
  int32_t* accept_len;
  int32_t* best;
  int64_t* out_ids;
  int64_t* pred_out;
  float* part_v;
  int64_t* part_i;
  unsigned* cnt;
  TreeShape ts;
};

template <typename Tin>
__global__ __launch_bounds__(kNT) void k_tree_greedy(TreeGreedyParams p) {
  __shared__ ReduceLds lds;
  __shared__ int last_flag;
  __shared__ int64_t pred[kMaxNodes + 1];
  const int rows_t = p.N + 1;
  const int c = blockIdx.x % p.chunks;
  const int64_t t = blockIdx.x / p.chunks;
  const int64_t b = t % p.B;
  const int i = (int)(t / p.B);
  const Tin* row = static_cast<const Tin*>(p.tgt) + b * p.sb + i * p.ld;
  const int64_t c0 = (int64_t)c * p.chunk_len;
  const int64_t c1 = c0 + p.chunk_len < p.V ? c0 + p.chunk_len : p.V;
  const TScale one{1.0f, 1.0f};
  ChunkResult cr = reduce_chunk<Tin, SM_ID, false, false, true, kNT, kNB>(row, c0, c1, one, kNegInf, lds);
  const int64_t slot = (b * rows_t + i) * p.chunks + c;
  if (threadIdx.x == 0) {
    st_agent(&p.part_v[slot], cr.av);
    st_agent(&p.part_i[slot], cr.ai);
  }
  if (!arrive_last(&p.cnt[b], (unsigned)(rows_t * p.chunks), &last_flag)) return;
  merge_row_argmax(p.part_v, p.part_i, b, rows_t, p.chunks, pred, p.pred_out);
  const int lane = threadIdx.x;
  if (lane >= VNX_WAVE) return;
  // One wave: lane n < N tests node n.
  const bool live = lane < p.N;
  const uint64_t w = live ? p.ts.anc[lane] : 0ull;
  const bool match = live && p.tokens[b * p.ld_tok + lane] == pred[live ? p.ts.prow[lane] : 0];
  const uint64_t M = __ballot(match);
  const bool acc = live && (w & ~M) == 0ull;
  // Deepest accepted node, lowest index among equals: key = depth * 128 + (127 - n).
  int key = acc ? (__popcll(w) << 7) | (127 - lane) : 0;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) key = max(key, __shfl_xor(key, o, VNX_WAVE));
  const int depth = key >> 7;
  const int bestn = key ? 127 - (key & 127) : -1;
  const uint64_t path = bestn >= 0 ? p.ts.anc[bestn] : 0ull;
  int64_t* out = p.out_ids + b * rows_t;
  // Lane j < depth emits the j-th node of the path (the j-th set bit of its
  // ancestor word: ancestors precede descendants in BFS order).
  for (int j = lane; j < rows_t; j += VNX_WAVE) {
    int64_t v = -1;
    if (j < depth) {
      uint64_t m = path;
      for (int q = 0; q < j; ++q) m &= m - 1;
      v = p.tokens[b * p.ld_tok + __builtin_ctzll(m)];
    } else if (j == depth) {
      v = pred[bestn + 1];
    }
    out[j] = v;
  }
  if (lane == 0) {
    p.accept_len[b] = depth;
    if (p.best) p.best[b] = bestn;
  }
}

}  // namespace vnx

using namespace vnx;

extern "C" {

// Chunks per target row of the greedy verify: about two workgroups per CU
// in all (the rows' chunks count into one arrival counter per batch row;
// B 4 x 7 rows of 248,320: 30 us against 46 us at 64 chunks per row; B 32:
// 44 us against 46).
static int64_t gv_wgs() { return 2 * (int64_t)device_cus(); }

size_t vnx_greedy_verify_workspace(int64_t B, int rows_t, int64_t V) {
  if (B <= 0 || rows_t <= 0 || V <= 0) return 256;
  const int c = pick_chunks(B * rows_t, V, 4, kMaxChunks, gv_wgs());
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
  int c = pick_chunks(B * rows_t, V, ve, kMaxChunks, gv_wgs());
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

extern "C" {

// Chunks per target row: about two workgroups per CU in all, and no more --
// the rows' workgroups all count into one arrival counter per batch row, and
// at config 3 (656 rows) whole rows per workgroup ran 104 us against 111 us
// for 4 chunks per row and 145 us for 13.
static int tree_plan(int64_t B, int N, int64_t V, int dtype, int* chunks, int64_t* len) {
  const int ve = dtype == VNX_F32 ? 4 : 8;
  int c = pick_chunks(B * (N + 1), V, ve, kMaxChunks, 2 * (int64_t)device_cus());
  const int64_t l = ((V + c - 1) / c + ve - 1) / ve * ve;
  *len = l;
  *chunks = (int)((V + l - 1) / l);
  return 0;
}

size_t vnx_tree_greedy_workspace(int64_t B, int N, int64_t V) {
  if (B <= 0 || N <= 0 || V <= 0) return 256;
  int c;
  int64_t len;
  tree_plan(B, N, V, VNX_F32, &c, &len);  // fp32 plans the most chunks
  Carve cv(nullptr);
  cv.take<unsigned>(B);
  cv.take<float>((size_t)B * (N + 1) * c);
  cv.take<int64_t>((size_t)B * (N + 1) * c);
  return cv.bytes();
}

int vnx_tree_greedy(const void* target, int dtype, int64_t B, int N, int64_t V, int64_t ld, int64_t sb,
                    const int64_t* tokens, int64_t ld_tok, const int32_t* parent, int32_t* accept_len,
                    int32_t* best, int64_t* out_ids, int64_t* pred, void* workspace, size_t workspace_bytes,
                    void* stream) {
  if (dtype != VNX_F32 && dtype != VNX_BF16) return VNX_ERR_UNSUPPORTED;
  if (B < 0 || N < 1 || N > kMaxNodes || V <= 0) return VNX_ERR_INVALID_ARG;
  if (B == 0) return VNX_OK;
  if (!parent) return VNX_ERR_INVALID_ARG;
  if (B > (1 << 20) || V > ((int64_t)1 << 31)) return VNX_ERR_UNSUPPORTED;
  int st = check_rows(target, dtype, ld, sb, N + 1, V);
  if (st) return st;
  if (!tokens || ld_tok < N || !accept_len || !out_ids) return VNX_ERR_INVALID_ARG;
  TreeGreedyParams p{};
  for (int i = 0; i < N; ++i) {
    const int par = parent[i];
    if (par < -1 || par >= i) return VNX_ERR_INVALID_ARG;
    p.ts.anc[i] = (1ull << i) | (par >= 0 ? p.ts.anc[par] : 0ull);
    p.ts.prow[i] = (int8_t)(par + 1);
  }
  int c;
  int64_t len;
  tree_plan(B, N, V, dtype, &c, &len);
  if (B * (N + 1) * (int64_t)c >= INT32_MAX) return VNX_ERR_UNSUPPORTED;
  Carve cv(workspace);
  p.cnt = cv.take<unsigned>(B);
  p.part_v = cv.take<float>((size_t)B * (N + 1) * c);
  p.part_i = cv.take<int64_t>((size_t)B * (N + 1) * c);
  if (!workspace || workspace_bytes < cv.bytes()) return VNX_ERR_WORKSPACE;
  p.tgt = target; p.B = B; p.N = N; p.V = V; p.ld = ld; p.sb = sb;
  p.chunks = c; p.chunk_len = len; p.tokens = tokens; p.ld_tok = ld_tok;
  p.accept_len = accept_len; p.best = best; p.out_ids = out_ids; p.pred_out = pred;
  hipStream_t s = static_cast<hipStream_t>(stream);
  st = zero_counters(p.cnt, B, s);
  if (st) return st;
  dim3 g((unsigned)(B * (N + 1) * c));
  if (dtype == VNX_F32)
    hipLaunchKernelGGL(k_tree_greedy<float>, g, dim3(kNT), 0, s, p);
  else
    hipLaunchKernelGGL(k_tree_greedy<__hip_bfloat16>, g, dim3(kNT), 0, s, p);
  VNX_LAUNCH_CHECK();
  return VNX_OK;
}

}  // extern "C"
