// Vocab-row reductions: row LSE (+ max / argmax), row argmax, softmax.
// Grid: one workgroup per (row, chunk); the last workgroup of a row merges
// the chunk partials (fp64) and writes the row's outputs.
#include "rowred.h"
#include "vnx_internal.h"

namespace vnx {

constexpr int kNT = 256;
constexpr int kNB = 8;

struct RowParams {
  const void* x;
  int64_t rows, V, ld;
  int chunks;
  int64_t chunk_len;  // multiple of the vector width
  TScale sc;
  const float* thr;
  double* lse;
  float* rowmax;
  int64_t* argmax;
  float* part_m;
  double* part_s;
  float* part_v;
  int64_t* part_i;
  unsigned* counters;
};

template <typename Tin, int SM, bool THR, bool LSE, bool ARGMAX>
__global__ __launch_bounds__(kNT) void k_row_reduce(RowParams p) {
  __shared__ ReduceLds lds;
  __shared__ int last_flag;
  const int64_t r = blockIdx.x / p.chunks;
  const int c = blockIdx.x % p.chunks;
  const Tin* row = static_cast<const Tin*>(p.x) + r * p.ld;
  const int64_t c0 = (int64_t)c * p.chunk_len;
  const int64_t c1 = c0 + p.chunk_len < p.V ? c0 + p.chunk_len : p.V;
  const float thr = (THR && p.thr) ? p.thr[r] : kNegInf;
  ChunkResult cr = reduce_chunk<Tin, SM, THR, LSE, ARGMAX, kNT, kNB>(row, c0, c1, p.sc, thr, lds);
  const int64_t slot = r * p.chunks + c;
  if (threadIdx.x == 0) {
    if constexpr (LSE) { st_agent(&p.part_m[slot], cr.m); st_agent(&p.part_s[slot], cr.s); }
    if constexpr (ARGMAX) { st_agent(&p.part_v[slot], cr.av); st_agent(&p.part_i[slot], cr.ai); }
  }
  if (!arrive_last(&p.counters[r], (unsigned)p.chunks, &last_flag)) return;
  // Last workgroup of row r: the chunk partials go to LDS with one coherent
  // load per thread (chunks <= kNT), then thread 0 merges them in order.
  __shared__ float t_m[kNT], t_v[kNT];
  __shared__ double t_s[kNT];
  __shared__ int64_t t_i[kNT];
  const int j = threadIdx.x;
  if (j < p.chunks) {
    if constexpr (LSE) { t_m[j] = ld_agent(&p.part_m[slot - c + j]); t_s[j] = ld_agent(&p.part_s[slot - c + j]); }
    if constexpr (ARGMAX) { t_v[j] = ld_agent(&p.part_v[slot - c + j]); t_i[j] = ld_agent(&p.part_i[slot - c + j]); }
  }
  __syncthreads();
  if (threadIdx.x != 0) return;
  if constexpr (LSE) {
    float M = kNegInf;
    double S = 0.0;
    for (int q = 0; q < p.chunks; ++q) merge_partial(M, S, t_m[q], t_s[q]);
    p.lse[r] = lse_of(M, S);
    if (p.rowmax) p.rowmax[r] = M;
  }
  if constexpr (ARGMAX) {
    float bv = kNegInf;
    int64_t bi = INT64_MAX;
    for (int q = 0; q < p.chunks; ++q)
      if (argmax_better(t_v[q], t_i[q], bv, bi)) { bv = t_v[q]; bi = t_i[q]; }
    p.argmax[r] = bi;
  }
}

// out = exp(a - L) in fp32, L the row LSE: the exponent a*log2(e) - L*log2(e)
// is formed with both products split into hi + lo parts.
template <typename Tin, int SM, bool THR>
__global__ __launch_bounds__(kNT) void k_softmax_write(const Tin* __restrict__ x, int64_t V, int64_t ld,
                                                       TScale sc, const float* thr_p, const double* lse,
                                                       float* __restrict__ out, int64_t ldo, int chunks,
                                                       int64_t chunk_len) {
  const int64_t r = blockIdx.x / chunks;
  const int c = blockIdx.x % chunks;
  const int64_t c0 = (int64_t)c * chunk_len;
  const int64_t c1 = c0 + chunk_len < V ? c0 + chunk_len : V;
  const float thr = (THR && thr_p) ? thr_p[r] : kNegInf;
  const double L = lse[r];
  const double Lt = L * 1.4426950408889634074;
  const float hi = (float)Lt;
  const float lo = (float)(Lt - (double)hi);
  const bool finite = __builtin_isfinite(L);
  const Tin* row = x + r * ld;
  float* orow = out + r * ldo;
  for (int64_t j = c0 + threadIdx.x; j < c1; j += kNT) {
    const float a = scaled<SM, THR>(Vec<Tin>::load1(row + j), sc, thr);
    float t = __builtin_fmaf(a, kL2eHi, -hi);
    t = __builtin_fmaf(a, kL2eLo, t) - lo;
    orow[j] = finite ? __builtin_amdgcn_exp2f(t) : (L == -__builtin_inf() ? 0.0f : __builtin_nanf(""));
  }
}

static int row_common_check(const void* x, int dtype, int64_t rows, int64_t V, int64_t ld) {
  if (rows < 0 || V <= 0 || ld < V) return VNX_ERR_INVALID_ARG;
  if (dtype != VNX_F32 && dtype != VNX_BF16) return VNX_ERR_UNSUPPORTED;
  if (rows == 0) return VNX_OK;  // nothing is read or written: any pointers
  if (!x) return VNX_ERR_INVALID_ARG;
  const int ve = dtype == VNX_F32 ? 4 : 8;
  if (!aligned16(x) || ld % ve != 0) return VNX_ERR_UNSUPPORTED;
  return VNX_OK;
}

struct RowPlan {
  int chunks;
  int64_t chunk_len;
};

static RowPlan row_plan(int64_t rows, int64_t V, int dtype) {
  const int ve = dtype == VNX_F32 ? 4 : 8;
  RowPlan pl;
  // at least 8 vectors per thread per chunk (few rows: fewer, longer
  // chunks); about two workgroups per CU, and two chunks per row for long
  // row sets (V 248,320, fp32 row LSE: 32 rows 17 us against 25 us at 30
  // chunks per row, 224 rows 42 against 47, 1,088 rows 172 us at 2 chunks
  // per row against 180 at 1)
  pl.chunks = pick_chunks(rows, V, ve * 8, 64, std::max<int64_t>(2 * (int64_t)device_cus(), 2 * rows));
  int64_t len = (V + pl.chunks - 1) / pl.chunks;
  len = (len + ve - 1) / ve * ve;
  pl.chunk_len = len;
  pl.chunks = (int)((V + len - 1) / len);
  return pl;
}

static size_t row_ws(int64_t rows, int64_t V, int dtype, RowParams*) {
  RowPlan pl = row_plan(rows, V, dtype);
  Carve cv(nullptr);
  size_t n = (size_t)rows * pl.chunks;
  cv.take<unsigned>(rows);
  cv.take<float>(n);
  cv.take<double>(n);
  cv.take<float>(n);
  cv.take<int64_t>(n);
  return cv.bytes();
}

static void row_carve(void* ws, int64_t rows, const RowPlan& pl, RowParams& p) {
  Carve cv(ws);
  size_t n = (size_t)rows * pl.chunks;
  p.counters = cv.take<unsigned>(rows);
  p.part_m = cv.take<float>(n);
  p.part_s = cv.take<double>(n);
  p.part_v = cv.take<float>(n);
  p.part_i = cv.take<int64_t>(n);
}

template <bool LSE, bool ARGMAX>
static int launch_row_reduce(RowParams& p, int dtype, int sm, hipStream_t st) {
  int zs = zero_counters(p.counters, p.rows, st);
  if (zs) return zs;
  dim3 grid((unsigned)(p.rows * p.chunks));
  return dispatch_tsm(dtype, sm, p.thr != nullptr, [&](auto tin, auto smc, auto thrc) {
    using Tin = decltype(tin);
    hipLaunchKernelGGL((k_row_reduce<Tin, decltype(smc)::value, decltype(thrc)::value, LSE, ARGMAX>), grid,
                       dim3(kNT), 0, st, p);
    VNX_LAUNCH_CHECK();
    return (int)VNX_OK;
  });
}

}  // namespace vnx

using namespace vnx;

extern "C" {

size_t vnx_row_lse_workspace(int64_t rows, int64_t V) {
  if (rows <= 0 || V <= 0) return 256;
  // Sized for the worse (fp32) plan; bf16 plans use fewer chunks.
  return row_ws(rows, V, VNX_F32, nullptr);
}

int vnx_row_lse(const void* logits, int dtype, int64_t rows, int64_t V, int64_t ld,
                float temperature, const float* thresholds, double* lse, float* rowmax,
                int64_t* argmax, void* workspace, size_t workspace_bytes, void* stream) {
  int st = row_common_check(logits, dtype, rows, V, ld);
  if (st) return st;
  if (!(temperature > 0.0f) || !__builtin_isfinite(temperature)) return VNX_ERR_INVALID_ARG;
  if (rows == 0) return VNX_OK;
  if (!lse) return VNX_ERR_INVALID_ARG;
  if (rows > (int64_t)1 << 24) return VNX_ERR_UNSUPPORTED;
  RowPlan pl = row_plan(rows, V, dtype);
  if (!workspace || workspace_bytes < row_ws(rows, V, dtype, nullptr)) return VNX_ERR_WORKSPACE;
  RowParams p{};
  p.x = logits; p.rows = rows; p.V = V; p.ld = ld;
  p.chunks = pl.chunks; p.chunk_len = pl.chunk_len;
  const int sm = make_scale(temperature, &p.sc);
  p.thr = thresholds; p.lse = lse; p.rowmax = rowmax; p.argmax = argmax;
  row_carve(workspace, rows, pl, p);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (argmax) return launch_row_reduce<true, true>(p, dtype, sm, s);
  return launch_row_reduce<true, false>(p, dtype, sm, s);
}

int vnx_row_argmax(const void* logits, int dtype, int64_t rows, int64_t V, int64_t ld,
                   int64_t* argmax, void* workspace, size_t workspace_bytes, void* stream) {
  int st = row_common_check(logits, dtype, rows, V, ld);
  if (st) return st;
  if (rows == 0) return VNX_OK;
  if (!argmax) return VNX_ERR_INVALID_ARG;
  if (rows > (int64_t)1 << 24) return VNX_ERR_UNSUPPORTED;
  RowPlan pl = row_plan(rows, V, dtype);
  if (!workspace || workspace_bytes < row_ws(rows, V, dtype, nullptr)) return VNX_ERR_WORKSPACE;
  RowParams p{};
  p.x = logits; p.rows = rows; p.V = V; p.ld = ld;
  p.chunks = pl.chunks; p.chunk_len = pl.chunk_len;
  const int sm = make_scale(1.0f, &p.sc);
  p.argmax = argmax;
  row_carve(workspace, rows, pl, p);
  return launch_row_reduce<false, true>(p, dtype, sm, static_cast<hipStream_t>(stream));
}

int vnx_softmax(const void* logits, int dtype, int64_t rows, int64_t V, int64_t ld,
                float temperature, const float* thresholds, float* out, int64_t ldo,
                void* workspace, size_t workspace_bytes, void* stream) {
  int st = row_common_check(logits, dtype, rows, V, ld);
  if (st) return st;
  if (ldo < V || !(temperature > 0.0f) || !__builtin_isfinite(temperature)) return VNX_ERR_INVALID_ARG;
  if (rows == 0) return VNX_OK;
  if (!out) return VNX_ERR_INVALID_ARG;
  if (rows > (int64_t)1 << 24) return VNX_ERR_UNSUPPORTED;
  RowPlan pl = row_plan(rows, V, dtype);
  Carve cv(workspace);
  double* lse = cv.take<double>(rows);
  size_t need = cv.bytes() + row_ws(rows, V, dtype, nullptr);
  if (!workspace || workspace_bytes < need) return VNX_ERR_WORKSPACE;
  RowParams p{};
  p.x = logits; p.rows = rows; p.V = V; p.ld = ld;
  p.chunks = pl.chunks; p.chunk_len = pl.chunk_len;
  const int sm = make_scale(temperature, &p.sc);
  p.thr = thresholds; p.lse = lse;
  row_carve(static_cast<char*>(workspace) + cv.bytes(), rows, pl, p);
  hipStream_t s = static_cast<hipStream_t>(stream);
  st = launch_row_reduce<true, false>(p, dtype, sm, s);
  if (st) return st;
  dim3 grid((unsigned)(rows * pl.chunks));
  return dispatch_tsm(dtype, sm, thresholds != nullptr, [&](auto tin, auto smc, auto thrc) {
    using Tin = decltype(tin);
    hipLaunchKernelGGL((k_softmax_write<Tin, decltype(smc)::value, decltype(thrc)::value>), grid, dim3(kNT), 0,
                       s, static_cast<const Tin*>(logits), V, ld, p.sc, thresholds, lse, out, ldo, pl.chunks,
                       pl.chunk_len);
    VNX_LAUNCH_CHECK();
    return (int)VNX_OK;
  });
}

size_t vnx_softmax_workspace(int64_t rows, int64_t V) {
  Carve cv(nullptr);
  cv.take<double>(rows > 0 ? rows : 1);
  return cv.bytes() + vnx_row_lse_workspace(rows, V);
}

}  // extern "C"
