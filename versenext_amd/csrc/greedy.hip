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
  // Partials of b are contiguous (row-major by i): read in tiles of kNT with
  // one coherent load per thread, merged per row from LDS.
  __shared__ float tile_v[kNT];
  __shared__ int64_t tile_i[kNT];
  const int tid = threadIdx.x;
  float bv = kNegInf;
  int64_t bi = INT64_MAX;
  {
    const int64_t base = b * p.rows_t * p.chunks;
    const int total = p.rows_t * p.chunks;
    for (int t0 = 0; t0 < total; t0 += kNT) {
      if (t0 + tid < total) {
        tile_v[tid] = ld_agent(&p.part_v[base + t0 + tid]);
        tile_i[tid] = ld_agent(&p.part_i[base + t0 + tid]);
      }
      __syncthreads();
      if (tid < p.rows_t) {
        const int lo = max(tid * p.chunks, t0), hi = min((tid + 1) * p.chunks, min(t0 + kNT, total));
        for (int i = lo; i < hi; ++i)
          if (argmax_better(tile_v[i - t0], tile_i[i - t0], bv, bi)) { bv = tile_v[i - t0]; bi = tile_i[i - t0]; }
      }
      __syncthreads();
    }
  }
  if (tid < p.rows_t) {
    pred[tid] = bi;
    if (p.main_pred) p.main_pred[b * p.rows_t + tid] = bi;
  }
  __syncthreads();
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

}  // namespace vnx

using namespace vnx;

extern "C" {

size_t vnx_greedy_verify_workspace(int64_t B, int rows_t, int64_t V) {
  if (B <= 0 || rows_t <= 0 || V <= 0) return 256;
  const int c = pick_chunks(B * rows_t, V, 4, kMaxChunks, 2048);
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
  int c = pick_chunks(B * rows_t, V, ve, kMaxChunks, 2048);
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
