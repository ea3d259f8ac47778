/*
 * vnx — MI355X (gfx950) speculative-decoding verification kernels, C ABI.
 *
 * Drop-in boundary for VerseNext's speculative-decode path: the Python
 * `SpeculativeDecoder` and the `DeviceBackend` "rocm" device call these entry
 * points through ctypes.  Every reference citation below is relative to the
 * CUI-hyg/VerseNext source tree.
 *
 * Conventions (all entry points):
 *   - every pointer argument is a caller-owned DEVICE pointer unless noted;
 *   - nothing here allocates device memory: entry points that need scratch
 *     take `workspace` + `workspace_bytes` (query the size with the matching
 *     *_workspace() function).  Its contents need no initialisation (each
 *     call clears the counters it uses with a small kernel); calls that may
 *     run concurrently (different streams) must not share a workspace;
 *   - `stream` is a hipStream_t (NULL = the null stream); calls are
 *     asynchronous on that stream;
 *   - return value: VNX_OK (0) or a negative vnx_status; no exception or
 *     longjmp crosses the ABI.  Argument checks happen on the host before
 *     anything is launched.  The verification entry points (vnx_row_lse,
 *     vnx_row_argmax, vnx_softmax, vnx_spec_accept, vnx_sample,
 *     vnx_sampler_sample, vnx_greedy_verify, vnx_tree_attn, vnx_tree_greedy,
 *     vnx_row_topk, vnx_lm_head) return VNX_OK for an empty batch (no rows)
 *     after the size and dtype checks, without reading any pointer;
 *   - dtype codes: VNX_F32 (fp32), VNX_BF16 (bfloat16) for logits;
 *   - token ids are int64, like the reference's int64 token arrays
 *     (packages/verse_nex/verse_nex/speculative.py:161, :202-203);
 *   - thread-compatible: the library keeps no mutable state after vnx_init()
 *     except a host-side cache of checked temperatures (mutex-protected).
 */
#ifndef VNX_H_
#define VNX_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum vnx_status {
  VNX_OK = 0,
  VNX_ERR_INVALID_ARG = -1,   /* shape / pointer / range error  -> ValueError   */
  VNX_ERR_WORKSPACE = -2,     /* workspace missing or too small -> ValueError   */
  VNX_ERR_UNSUPPORTED = -3,   /* dtype / size outside the kernels' range        */
  VNX_ERR_HIP = -4,           /* a HIP runtime call failed      -> RuntimeError */
  VNX_ERR_NO_DEVICE = -5,     /* no gfx950 device / bad ordinal -> RuntimeError */
  VNX_ERR_TOO_LARGE = -6      /* input needs more than an allocation-free entry
                                 point's fixed scratch          -> ValueError   */
};

enum vnx_dtype { VNX_F32 = 0, VNX_BF16 = 1, VNX_F16 = 2 };

/* Flags written by vnx_spec_accept, one byte per (row, position). */
enum vnx_accept_flag {
  VNX_FLAG_NEAR_TIE = 1,      /* |u - p/q| < 1e-6 at this position                     */
  VNX_FLAG_LSE_EDGE = 2,      /* a row LSE lies within 1e-7 of an fp32 rounding edge   */
  VNX_FLAG_CDF_EDGE = 4,      /* the sampled CDF step lies within 1e-12*mass of u*mass */
  VNX_FLAG_ZERO_RESIDUAL = 8, /* max(0,p-q) had zero mass; sampled from p instead      */
  VNX_FLAG_BAD_ID = 16        /* draft id outside [0, V): treated as rejected          */
};

/* Library ABI version (major*10000 + minor*100 + patch). */
int vnx_version(void);

/* Static text for a vnx_status code. */
const char* vnx_status_string(int status);

/* Text of the last HIP error seen by this thread ("" if none). */
const char* vnx_last_hip_error(void);

/* Phase profiling (a measurement aid with no counterpart in the reference).
 * vnx_profile_begin(max_calls) creates events for up to max_calls entry-point
 * calls; while active, each vnx_spec_accept call records an event before each
 * of its two launches (the LSE pass; acceptance, masses and draw) and one
 * after the last, on its own stream (vnx_tree_attn's bf16 path records its
 * attention and merge launches the same way).  vnx_profile_end waits for the recorded events, writes the
 * summed milliseconds of each phase into phase_ms[0..nphase) and the number of
 * profiled calls into *ncalls, and releases the events.  Not for use while
 * calls run concurrently on several streams. */
int vnx_profile_begin(int max_calls);
int vnx_profile_end(double* phase_ms, int nphase, int* ncalls);

/* Selects `device` and checks it is a gfx950 GPU.  Safe to call repeatedly.
 * Replaces: get_backend("rocm"/"rocm:N") device selection,
 * packages/verse_torch/verse_torch/device.py:346-386 and
 * packages/verse_torch/verse_torch/backend_torch.py:65-98. */
int vnx_init(int device);

/* ---------------------------------------------------------------------------
 * Vocab-row reductions.
 * logits: `rows` rows of `V` elements, row pitch `ld` elements (ld >= V).
 * temperature: > 0; rows are scaled as RN(l / temperature) before the LSE
 *   (sampler.py:95).  thresholds: NULL, or one float per row: scaled values
 *   below it are masked to -inf (top-k keep rule `scaled >= kth`, sampler.py:98-102).
 * ------------------------------------------------------------------------- */
size_t vnx_row_lse_workspace(int64_t rows, int64_t V);

/* lse[r] = log(sum_j exp(a_rj)) in fp64, rowmax[r] = max_j a_rj (fp32),
 * argmax[r] = first index of the maximum of the RAW logits (numpy.argmax).
 * rowmax / argmax may be NULL.
 * Replaces the row reductions inside NumpyBackend.softmax (device.py:305-308),
 * Tensor.softmax (packages/verse_torch/verse_torch/tensor.py:965-975) and
 * Sampler.sample steps 1-3 (sampler.py:94-111). */
int vnx_row_lse(const void* logits, int dtype, int64_t rows, int64_t V, int64_t ld,
                float temperature, const float* thresholds,
                double* lse, float* rowmax, int64_t* argmax,
                void* workspace, size_t workspace_bytes, void* stream);

/* argmax[r] = numpy.argmax(logits[r, :V]) (first maximal index, NaN wins).
 * Replaces np.argmax at speculative.py:158 and :220. */
int vnx_row_argmax(const void* logits, int dtype, int64_t rows, int64_t V, int64_t ld,
                   int64_t* argmax, void* workspace, size_t workspace_bytes, void* stream);

/* out[r, j] = softmax(RN(l/temperature))[j] in fp32 (row pitch ldo).
 * Replaces DeviceBackend.softmax (device.py:246-248, :305-308). */
size_t vnx_softmax_workspace(int64_t rows, int64_t V);

int vnx_softmax(const void* logits, int dtype, int64_t rows, int64_t V, int64_t ld,
                float temperature, const float* thresholds, float* out, int64_t ldo,
                void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Stochastic speculative acceptance (Leviathan et al. 2023, Alg. 1).
 * target: B x (k+1) rows, row (b,i) at target + b*sb_t + i*ld_t,
 * draft:  B x k rows,     row (b,i) at draft  + b*sb_d + i*ld_d
 * (strides in elements; contiguous (B,k+1,V) is ld_t = V, sb_t = (k+1)*V),
 * p_i = softmax(target_i / T), q_i = softmax(draft_i / T) (optional per-row
 * thresholds thr_t (B*(k+1)) / thr_d (B*k), NULL = no top-k).
 * draft_ids (B,k) int64, uniforms (B,k+1) fp32 in [0,1).
 * Position i is accepted iff u_i < 1 and u_i*q_i(x_i) < p_i(x_i) (i.e.
 * u_i < min(1, p/q)); n = first rejected position (k if none).  The emitted
 * token at n is the inverse-CDF draw with u_k from norm(max(0, p_n - q_n))
 * (n < k) or from p_k (n == k).
 * Outputs: accept_len (B) int32 = n; out_ids (B, k+1) int64 = x_0..x_{n-1},
 * the drawn token, then -1; flags (B, k+1) uint8 (vnx_accept_flag, may be
 * NULL); lse_t (B*(k+1)) / lse_d (B*k) fp32 row LSEs as used (may be NULL).
 * The reference verifier is the greedy special case of this rule:
 * SpeculativeDecoder.verify / verify_then_commit, speculative.py:168-310.
 * ------------------------------------------------------------------------- */
size_t vnx_spec_accept_workspace(int64_t B, int k, int64_t V);

int vnx_spec_accept(const void* target, const void* draft, int dtype,
                    int64_t B, int k, int64_t V,
                    int64_t ld_t, int64_t sb_t, int64_t ld_d, int64_t sb_d,
                    const int64_t* draft_ids, const float* uniforms, float temperature,
                    const float* thr_t, const float* thr_d,
                    int32_t* accept_len, int64_t* out_ids, uint8_t* flags,
                    float* lse_t, float* lse_d,
                    void* workspace, size_t workspace_bytes, void* stream);

/* vnx_spec_accept for a caller whose draws already computed the draft rows'
 * log-sum-exps (the k draws of a speculative round, vnx_sample with its lse
 * and flags outputs, at the same temperature and without top-k): lse_d_in
 * [i * ld_in + b] is RN32 of the LSE of draft row i of batch row b, and
 * flags_d_in (same layout, may be NULL) their flags, whose VNX_FLAG_LSE_EDGE
 * bit carries over to the positions those rows decide.  The first launch
 * then streams only the k + 1 target rows per batch row (and reads the draft
 * rows at the draft ids), so the draft logits are not read twice in a round;
 * the decisions equal vnx_spec_accept's given the same draft LSEs.  No
 * per-row thresholds.  Workspace: vnx_spec_accept_workspace(B, k, V). */
int vnx_spec_accept_draft_lse(const void* target, const void* draft, int dtype, int64_t B, int k, int64_t V,
                              int64_t ld_t, int64_t sb_t, int64_t ld_d, int64_t sb_d,
                              const int64_t* draft_ids, const float* uniforms, float temperature,
                              const float* lse_d_in, const uint8_t* flags_d_in, int64_t ld_in,
                              int32_t* accept_len, int64_t* out_ids, uint8_t* flags, float* lse_t, void* workspace,
                              size_t workspace_bytes, void* stream);

/* Sampler.sample, one call per batch of rows: out_ids[b] = the token the
 * reference's Sampler draws from logits row b with temperature, top_k, top_p
 * and the uniform uniforms[b] in place of its RNG
 * (packages/verse_infra/verse_infra/verse_inference/sampler.py:70-138):
 * temperature 0 -> numpy.argmax of the raw row; a = RN(l/T); top_k in (0, V):
 * kth = the kth largest a (numpy.partition order, NaN largest), a = a >= kth ?
 * a : -inf; max(a) not finite -> numpy.argmax of the raw row; p =
 * vnx_exp_canon(a - RN32(row LSE)); top_p < 1: the first cutoff + 1 tokens
 * in (p descending, id ascending) order, cutoff = the first position whose
 * cumulative floor(p * 2^60) reaches floor(top_p * 2^60), at most V - 1;
 * the draw is the inverse CDF over the kept p (numpy's Generator.choice
 * rule).  Each row is split over several workgroups (a short chain of
 * launches: with 0 < top_k <= 256 a candidate search, one read of the row;
 * the workspace of vnx_sampler_workspace(B, V, dtype) bytes, no
 * initialisation, holds the candidates, histograms and partials).
 * mode (bit flags) selects the sampling step of CometSparkNexLM's
 * _generate_with_logits (packages/verse_nex/verse_nex/cometspark.py:868-910):
 *   VNX_SAMPLE_CALIBRATE  l -> l / sqrt(var(l) + calib_eps) * calib_factor
 *                         first (cometspark.py:922-948, fused: two more passes
 *                         over the row, the same arithmetic as
 *                         vnx_logit_calibrate), greedy included;
 *   VNX_SAMPLE_EXACT_K    argpartition(-a, k-1)[:k]: exactly k tokens, NaN
 *                         ranked below every value, ties at the kth value
 *                         taken by lower id (numpy leaves them open); the
 *                         draw runs over the kept ids in id order;
 *   VNX_SAMPLE_UNIFORM_F64 uniforms holds B doubles (else B floats): the
 *                         float64 value numpy's Generator.random() gives the
 *                         reference's choice, used without rounding.
 * Optional outputs (NULL to skip): flags (VNX_FLAG_CDF_EDGE / LSE_EDGE), lse
 * = RN32(row LSE), kth (the top-k threshold, -inf if off), p_star / j_star
 * (the last kept token's probability and id, -1 if top_p is off), k_star (the
 * id of the last kept tie at kth under VNX_SAMPLE_EXACT_K, else -1).  Errors:
 * temperature < 0 or not finite, top_k < 0, top_p outside (0, 1], unknown
 * mode bits, a calibration factor that is not finite or eps < 0 ->
 * VNX_ERR_INVALID_ARG (the reference's ValueError, sampler.py:54-59). */
#define VNX_SAMPLE_EXACT_K 1
#define VNX_SAMPLE_CALIBRATE 2
#define VNX_SAMPLE_UNIFORM_F64 4

size_t vnx_sampler_workspace(int64_t B, int64_t V, int dtype);

int vnx_sampler_sample(const void* logits, int dtype, int64_t B, int64_t V, int64_t ld, float temperature,
                       int64_t top_k, float top_p, int mode, float calib_factor, float calib_eps,
                       const void* uniforms, int64_t* out_ids, uint8_t* flags, float* lse, float* kth,
                       float* p_star, int64_t* j_star, int64_t* k_star, void* workspace, size_t workspace_bytes,
                       void* stream);

/* Logit calibration of VMPC-compressed models
 * (CometSparkNexLM._apply_logit_calibration, packages/verse_nex/verse_nex/
 * cometspark.py:922-948): out row b = logits row b / sqrt(var + eps) *
 * calib_factor, var the row's population variance (taken in fp64, then
 * rounded to fp32; the rest in fp32 in the reference's order).  out is fp32
 * (it may alias fp32 logits with ld_out == ld); var (B) fp64 may be NULL. */
int vnx_logit_calibrate(const void* logits, int dtype, int64_t B, int64_t V, int64_t ld, float calib_factor,
                        float eps, float* out, int64_t ld_out, double* var, void* stream);

/* Allocation-free vnx_spec_accept.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory or pass a workspace (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, kernels and results as vnx_spec_accept
 * without workspace / workspace_bytes: its scratch is a fixed static device
 * array of vnx_spec_accept_noalloc_max_bytes() bytes (8 MiB) per GPU, held
 * until the process ends.  Inputs for which vnx_spec_accept_workspace(B, k,
 * V) exceeds that size (at V = 248,320 and k = 8: B above about 1,000)
 * return VNX_ERR_TOO_LARGE before anything is launched.  Every call on one GPU
 * shares that GPU's array (each call leaves it in a state the next call does
 * not read): calls that overlap on one GPU (concurrent streams) race.  The
 * first call with a new temperature adds one entry to the host-side
 * temperature cache (host memory only).  vnx_init(device) resolves the
 * array's address for that device; otherwise the first call does. */
size_t vnx_spec_accept_noalloc_max_bytes(void);

int vnx_spec_accept_noalloc(const void* target, const void* draft, int dtype,
                            int64_t B, int k, int64_t V,
                            int64_t ld_t, int64_t sb_t, int64_t ld_d, int64_t sb_d,
                            const int64_t* draft_ids, const float* uniforms, float temperature,
                            const float* thr_t, const float* thr_d,
                            int32_t* accept_len, int64_t* out_ids, uint8_t* flags,
                            float* lse_t, float* lse_d, void* stream);

/* Sampling (the draft's proposals, and any caller of Sampler.sample):
 * out_ids[b] = the inverse-CDF draw with uniforms[b] from softmax(logits row
 * b / T) (optional per-row top-k thresholds, NULL = none), the same draw the
 * acceptance kernels make for the bonus token (the numpy Generator.choice
 * rule, sampler.py:135-137, with the uniform given).  logits: B rows of V,
 * row pitch ld.  flags (B) uint8 and lse (B) fp32 may be NULL.
 * Replaces Sampler.sample steps 1-4 (sampler.py:94-138) and the draw of
 * _generate_with_logits (cometspark.py:880, :903-911), with host uniforms
 * in place of the RNG stream. */
size_t vnx_sample_workspace(int64_t B, int64_t V);

int vnx_sample(const void* logits, int dtype, int64_t B, int64_t V, int64_t ld, const float* uniforms,
               float temperature, const float* thresholds, int64_t* out_ids, uint8_t* flags, float* lse,
               void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Greedy verify, the reference semantics batched:
 * main_pred[b,i] = argmax(target row (b,i)) for i < rows_t (rows_t = k or k+1,
 * row (b,i) at target + b*sb + i*ld), accepted[b,i] = draft_ids[b,i] ==
 * main_pred[b,i] (i < k), accept_len[b] = length of the accepted prefix,
 * out_ids[b,:] = accepted prefix, then main_pred at the first mismatch
 * ("blessed" token), or main_pred[b,k] when all k match and rows_t == k+1
 * (bonus), then -1.
 * Replaces SpeculativeDecoder.verify (speculative.py:218-223) and the
 * prefix loop of verify_then_commit (speculative.py:277-287), for all rows
 * instead of batch row 0 only.  accepted / main_pred may be NULL.
 * ------------------------------------------------------------------------- */
size_t vnx_greedy_verify_workspace(int64_t B, int rows_t, int64_t V);

int vnx_greedy_verify(const void* target, int dtype, int64_t B, int k, int rows_t,
                      int64_t V, int64_t ld, int64_t sb, const int64_t* draft_ids,
                      uint8_t* accepted, int64_t* main_pred,
                      int32_t* accept_len, int64_t* out_ids,
                      void* workspace, size_t workspace_bytes, void* stream);

/* RoPE + KV-cache write of a q|k|v projection (vnx_rope_kv's work, done in
 * the projection's epilogue).  Projection row m is token (m / n, m % n) at
 * position lens[m / n] + m % n; heads are H query heads, then Hkv key heads,
 * then Hkv value heads of d dims (d % 16 == 0).  Queries (rotated when rope)
 * go to q_out (B, H, n, d) bf16; keys (rotated) and values to the bf16 caches
 * at b*c_sb + head*c_sh + pos*c_sr; rows at or past cap (and table_rows when
 * rope) are skipped.  NeoX rotate-half with the (table_rows, d) fp32 cos / sin
 * tables.  The projection weight's rows must be permuted per head (see
 * vnx_gemv_w4_rope_kv) so that each output tile holds rotate-half pairs. */
typedef struct vnx_rope_kv_args {
  const int32_t* lens;
  int n, H, Hkv, d;
  const float* cos_table;
  const float* sin_table;
  int64_t table_rows;
  int rope;
  void* q_out;
  void* k_cache;
  void* v_cache;
  int64_t c_sb, c_sh, c_sr, cap;
} vnx_rope_kv_args;

/* ---------------------------------------------------------------------------
 * Weight-only quantized GEMV / skinny GEMM (draft decode, tied LM head):
 * y (B, N) fp32, row pitch ldy = x (B, K) fp16 (row pitch ldx) . W^T with W
 * the dequantized (N, K) weight.  Matrix-core kernels (MFMA f16 -> f32); any
 * B (processed 32 columns at a time).  K must be a multiple of 128; x and
 * each weight row must start 16-byte aligned (ldx % 8 == 0, ldw % 16 == 0).
 * Small N splits K over workgroups: the fp32 partials go to the workspace
 * (vnx_gemv_workspace bytes; no initialisation needed) and are added in a
 * fixed order, so results do not depend on scheduling.
 * ------------------------------------------------------------------------- */

size_t vnx_gemv_workspace(int64_t B, int64_t N, int64_t K);

/* W4: wq (N, ceil(K/2)) bytes, row pitch ldw, two int4 per byte with the low
 * nibble at the even column (the packing of quantize.py:36-68, _pack_int4);
 * scales (N, K/group), row pitch lds, fp16 (VNX_F16) or fp32 (VNX_F32); the
 * weight is q * s[n][k / group].  group = K with fp32 scales is the
 * reference's per-channel INT4 (quantize_int4, quantize.py:231-258;
 * matmul_int4, :277-309); group = 128 with fp16 scales is the group-128
 * format.  Replaces matmul_int4 / QuantizedLinear.forward_fused
 * (quantize.py:506-533). */
int vnx_gemv_w4(const void* x, int64_t ldx, const uint8_t* wq, int64_t ldw, const void* scales,
                int scale_dtype, int64_t lds, int64_t B, int64_t N, int64_t K, int group,
                float* y, int64_t ldy, void* workspace, size_t workspace_bytes, void* stream);

/* vnx_gemv_w4 (group-128 fp16 scales, K = 512 or 1024) on a tiled copy of
 * the packed weight, for large N (a draft's tied LM head): vnx_pack_w4_tiles
 * writes it (vnx_w4_tiles_bytes(N, K) bytes, rows padded to a multiple of 16
 * with zeros): 16-row tile t holds K/128 pieces of 1 KB, piece g holding for
 * l = 0..63 the 16 bytes W[16t + l % 16][64g + 16(l / 16) .. +16] of the
 * row-major packing with every nibble in offset form (q + 8 = q ^ 8; a
 * reordering and an exact recoding, so the product is vnx_gemv_w4's bit for
 * bit).  scales (N, K/128) fp16 with row pitch lds (a multiple of 8 for
 * K = 1024, of 4 for K = 512), x and wt 16-byte aligned, ldx % 8 == 0.
 * Replaces matmul_int4 / QuantizedLinear.forward_fused (quantize.py:277-309,
 * :506-533) for the tied head of an INT4 draft (cometspark.py:396-398). */
size_t vnx_w4_tiles_bytes(int64_t N, int64_t K);
int vnx_pack_w4_tiles(const uint8_t* wq, int64_t ldw, int64_t N, int64_t K, uint8_t* out, void* stream);
int vnx_gemv_w4_tiles(const void* x, int64_t ldx, const uint8_t* wt, const void* scales, int64_t lds, int64_t B,
                      int64_t N, int64_t K, float* y, int64_t ldy, void* stream);

/* vnx_gemv_w4_tiles with the output dtype chosen: y_dtype VNX_F32 (the
 * vnx_gemv_w4_tiles call) or VNX_BF16 (each fp32 sum rounded to nearest even
 * once), for a draft head whose logits are kept in the model's bf16, as the
 * reference's head Linear returns them in the module dtype
 * (spark/src/base_model.py:207, :271). */
int vnx_gemv_w4_tiles_out(const void* x, int64_t ldx, const uint8_t* wt, const void* scales, int64_t lds, int64_t B,
                          int64_t N, int64_t K, void* y, int y_dtype, int64_t ldy, void* stream);

/* vnx_gemv_w4 of a fused [gate; up] weight with SwiGLU fused (SwiGLUMLP,
 * packages/verse_torch/verse_torch/vnnn.py:779-807, on QuantizedLinear
 * projections): W (N, K) has its rows interleaved in blocks of 16, the 8 gate
 * rows of hidden units 8t .. 8t+7 then their 8 up rows (N % 16 == 0,
 * N < 32768); y (B, N/2) fp16, row pitch ldy, y[b, j] = silu(acc[b, gate_j])
 * * acc[b, up_j] in fp32, rounded once.
 * norm_w (here and in vnx_gemv_w4_rope_kv): NULL, x is fp16 (B, K); else x is
 * the fp32 residual rows (B, K), row pitch ldx, and the product's input is
 * RMSNorm(x) * norm_w (vnnn.py:593-615, the block's norm fused): fp16(x *
 * norm_w) times W, each row's sum scaled by rstd = 1/sqrt(mean(x^2) + eps). */
int vnx_gemv_w4_swiglu(const void* x, int64_t ldx, const float* norm_w, float eps, const uint8_t* wq, int64_t ldw,
                       const void* scales, int scale_dtype, int64_t lds, int64_t B, int64_t N, int64_t K, int group,
                       void* y, int64_t ldy, void* stream);

/* vnx_gemv_w4 (group-128 fp16 scales) of a q|k|v projection with RoPE and
 * the KV-cache write in the epilogue (rk; B rows = tokens): rows of W (and of
 * its scales) permuted per head in 16-row tiles: tile t of head h holds dims
 * t*8 .. t*8+7 then d/2 + t*8 .. d/2 + t*8+7.  N = (H + 2*Hkv)*d < 32768. */
int vnx_gemv_w4_rope_kv(const void* x, int64_t ldx, const float* norm_w, float eps, const uint8_t* wq, int64_t ldw,
                        const void* scales, int scale_dtype, int64_t lds, int64_t B, int64_t N, int64_t K, int group,
                        const vnx_rope_kv_args* rk, void* stream);

/* vnx_gemv_w4_rope_kv with the first block's input gathered from the token
 * embedding (CometSparkV05LM.forward, spark/src/base_model.py:170-208:
 * tok_emb(idx) x scale, then norm1, then the q|k|v projection), replacing
 * vnx_embed_rmsnorm + vnx_gemv_w4_rope_kv on a quantized draft's first layer:
 * x_out[b] = emb[tokens[b]] * scale (fp32, row pitch ldx; emb bf16 with row
 * pitch lde, a multiple of 8; ids clamped to [0, vocab)), written by the
 * call, and the product's input is RMSNorm(x_out) * norm_w as with norm_w in
 * vnx_gemv_w4_rope_kv. */
int vnx_gemv_w4_rope_kv_embed(const int64_t* tokens, const void* emb, int emb_dtype, int64_t lde, int64_t vocab,
                              float scale, float* x_out, int64_t ldx, const float* norm_w, float eps,
                              const uint8_t* wq, int64_t ldw, const void* scales, int scale_dtype, int64_t lds,
                              int64_t B, int64_t N, int64_t K, int group, const vnx_rope_kv_args* rk, void* stream);

/* vnx_gemv_w4 with the residual add fused: res[b*ldr + n] += (x . W^T)[b, n]
 * (fp32; N < 32768), the `x = x + proj(...)` of VerseNexBlock.forward
 * (cometspark.py:236-247) on a quantized projection. */
int vnx_gemv_w4_residual(const void* x, int64_t ldx, const uint8_t* wq, int64_t ldw, const void* scales,
                         int scale_dtype, int64_t lds, int64_t B, int64_t N, int64_t K, int group, float* res,
                         int64_t ldr, void* stream);

/* W8: wq (N, K) int8, row pitch ldw; scale (N) fp32 per output row (the
 * per-channel INT8 of quantize_int8, quantize.py:187-214).  Replaces
 * QuantizedLinear.forward for qtype="int8" (quantize.py:467-505). */
int vnx_gemv_w8(const void* x, int64_t ldx, const int8_t* wq, int64_t ldw, const float* scale,
                int64_t B, int64_t N, int64_t K, float* y, int64_t ldy, void* workspace,
                size_t workspace_bytes, void* stream);

/* INT4 group-128 quantization on the device (the writer of the format above;
 * quantize_int4_g of the product's quant.py, restating the group variant of
 * QuantizedLinear's INT4 path, quantize.py:231-258, with fp16 group scales):
 * rows w (N, K) in dtype VNX_F32 / VNX_BF16 / VNX_F16, row pitch ldw
 * elements -> packed (N, K/2) bytes (pitch ldp) and fp16 scales (N, K/128)
 * (pitch lds); per group s = RN16(RN32(max|w| / 7)) (1/7 for an all-zero
 * group), q = clamp(rint(w / s), -8, 7).  group must be 128, K a multiple of
 * it.  bad_groups (device int32, zeroed by the caller; NULL to skip) counts
 * groups with a non-finite weight or a scale that underflows fp16 (the
 * host-side quantizer's ValueError).  Used to stream .vn weights into the
 * GEMV buffers chunk by chunk without a full-precision copy. */
int vnx_quantize_w4_g(const void* w, int dtype, int64_t N, int64_t K, int64_t ldw, int group, uint8_t* packed,
                      int64_t ldp, void* scales, int64_t lds, int32_t* bad_groups, void* stream);

/* out[n][k] = q[n][k] * s (fp32, one rounded multiply): the weights the GEMV
 * kernels use.  Replaces dequantize_int4 (quantize.py:261-274) and
 * dequantize_int8 (quantize.py:216-224). */
int vnx_dequant_w4(const uint8_t* wq, int64_t ldw, const void* scales, int scale_dtype, int64_t lds,
                   int64_t N, int64_t K, int group, float* out, int64_t ldo, void* stream);
int vnx_dequant_w8(const int8_t* wq, int64_t ldw, const float* scale, int64_t N, int64_t K,
                   float* out, int64_t ldo, void* stream);

/* ---------------------------------------------------------------------------
 * Tree-verify attention over a KV cache.
 * For batch row b, query head h and tree node i (i < N):
 *   out[b,h,i,:] = sum_j softmax_j(scale * q[b,h,i,:] . k_j + mask_ij) v_j
 * over the Tp prefix rows of the cache (all visible) followed by the N tree
 * rows, tree row j visible to node i iff bit j of anc[b*anc_batch_stride + i]
 * is set (ancestors-or-self; a chain tree gives causal attention).  Query head
 * h reads kv head h / (H / Hkv).  This is DeviceBackend.attention
 * (packages/verse_torch/verse_torch/device.py:260-270, scale 1/sqrt(d), an
 * additive 0 / -inf mask) over the cache concatenated with the new rows as
 * TriSparse does (packages/verse_nex/verse_nex/tri_sparse_attn.py:558-575),
 * and the SDPA call of TorchBackend.attention (backend_torch.py:356-379).
 * q (B,H,N,d), caches (B,Hkv,Tp,d), tree rows (B,Hkv,N,d): bf16 with the head
 * dimension contiguous and strides {batch, head, row} in elements (multiples
 * of 8, pointers 16-byte aligned).  The tree rows may live inside the cache
 * (k_tree = k_cache + Tp*row stride).  out (B,H,N,d): fp32, bf16 or fp16
 * (round to nearest even), strides multiples of 4.  d in {64, 128}; 1 <= N <= 64
 * (f32_rows below: fp32 rows, d in {8, 16, 32}, chains of any N).
 * A node that sees no key (Tp == 0 and an empty mask word) gets zeros.
 * The workspace (vnx_tree_attn_workspace bytes, no initialisation) holds the
 * per-split partials when the keys are split over several workgroups.
 * ------------------------------------------------------------------------- */
typedef struct vnx_tree_attn_args {
  const void* q;              /* bf16 (B, H, N, d)                              */
  int64_t q_strides[3];       /* batch, head, row                               */
  const void* k_cache;        /* bf16 (B, Hkv, Tp, d); may be NULL when Tp == 0 */
  const void* v_cache;
  int64_t cache_strides[3];   /* shared by k_cache and v_cache                  */
  const void* k_tree;         /* bf16 (B, Hkv, N, d)                            */
  const void* v_tree;
  int64_t tree_strides[3];    /* shared by k_tree and v_tree                    */
  const uint64_t* anc;        /* (B, N) ancestor-or-self words                  */
  int64_t anc_batch_stride;   /* 0: one tree shared by all batch rows           */
  void* out;
  int out_dtype;              /* VNX_F32, VNX_BF16 or VNX_F16                   */
  int64_t out_strides[3];
  int B, H, Hkv, Tp, N, d;
  float scale;                /* > 0; 1/sqrt(d) in the reference               */
  /* Ragged batches (per-sequence KV lengths, the commit / rollback of
   * ParallelKVCache.batch_update / per_seq_lens, kv_cache_parallel.py:42-286):
   * tp_batch, when not NULL, is a device array of B int32; batch row b then
   * has min(max(tp_batch[b], 0), Tp) prefix rows (Tp is the maximum).  With
   * tree_follows_prefix != 0 the tree rows of batch row b start right after
   * its prefix: tree row j is read at k_tree + b*s0 + kvh*s1 + (tp_b + j)*s2
   * (pass k_tree = k_cache and the cache strides to verify rows written into
   * the cache in place). */
  const int32_t* tp_batch;
  int tree_follows_prefix;
  /* Gated second key segment (TriSparse's global-token path,
   * tri_sparse_attn.py:469-495, mixed with the sigmoid gates, :585-608):
   * when T2 > 0, every node also attends to the T2 rows of k_seg2 / v_seg2
   * (all visible, softmax normalised on their own) and
   *   out = gates[0] * (attention over prefix + tree) + gates[1] * (attention
   *         over the T2 rows)
   * with gates a device array of 2 fp32.  seg2_strides {batch, head, row} in
   * elements (batch 0: one segment shared by all rows), multiples of 8.
   * T2 == 0 (or zero-initialised trailing fields): no second segment. */
  const void* k_seg2;
  const void* v_seg2;
  int64_t seg2_strides[3];
  int T2;
  const float* gates;
  /* RoPE and the cache write of the new rows done here (the work of
   * vnx_rope_kv, TriSparseAttention._apply_rope, tri_sparse_attn.py:182-221):
   * when qkv is not NULL (bf16, row pitch qkv_ld; row b*N + i holds the H
   * query, Hkv key and Hkv value heads of tree row i), q is not read: the
   * queries are those rows' query heads rotated at position tp_batch[b] + i,
   * and each workgroup first writes the rows' rotated keys and their values
   * into k_tree / v_tree at tree row tp_b + i (rows at or past cap skipped).
   * Needs tree_follows_prefix and tp_batch; rope == 0: no rotation; cos /
   * sin tables (table_rows, d) fp32, 16-byte aligned (else
   * VNX_ERR_UNSUPPORTED).  NULL (or zero-initialised trailing
   * fields): q holds the queries and the tree rows are already written. */
  const void* qkv;
  int64_t qkv_ld;
  const float* cos_table;
  const float* sin_table;
  int64_t table_rows;
  int rope;
  int64_t cap;
  /* TriSparse's sliding window and ALiBi paths (tri_sparse_attn.py:258-378,
   * :489-530).  Positions: node i of batch row b sits at tp_b + depth(i)
   * (depth = its ancestor count, 0 for a root; a chain's row i at tp_b + i),
   * prefix row j at j, tree row j at tp_b + depth(j).
   * window > 0: the prefix + tree attention keeps only keys with
   *   pos(i) - pos(key) < window (needs window >= N, else
   *   VNX_ERR_UNSUPPORTED: the tree keys then always fall inside it).
   * alibi_slopes (device array of H fp32, e.g. m_h = 2^(-h/H), h = 1..H) not
   *   NULL: a third softmax over the same prefix + tree keys, no window, with
   *   scores + -m_h * (pos(i) - pos(key)), added as gates[2] * it for batch
   *   rows with tp_b + N <= alibi_max_keys (the reference's T_k <= 1024 rule,
   *   :600-607); gates then holds 3 fp32 (gates[1] unused without a second
   *   segment) and out = gates[0] * path A + gates[1] * path B + gates[2] *
   *   path C.
   * Zero (the zero-initialised default): no window, no ALiBi. */
  int window;
  const float* alibi_slopes;
  int alibi_max_keys;
  /* Tuning: force_splits >= 1 fixes the key splits, force_waves (4, 5 = 4
   * with prefetch, 8, 9 = 8 with prefetch, 16) the workgroup shape where the
   * query tile fits;
   * 0: the launch plan's choice.  (Size the workspace with
   * vnx_tree_attn_workspace_args when forcing splits.) */
  int force_splits;
  int force_waves;
  /* fp32 rows (nonzero): q, the cache and tree rows and the second segment
   * are fp32 (TriSparse on fp32 weights, tri_sparse_attn.py:258-378,
   * :469-530), d in {8, 16, 32}, strides multiples of 4 elements, pointers
   * 16-byte aligned; qkv must be NULL and no workspace is used.  anc may be
   * NULL: a chain (node i sees tree rows j <= i and sits at tp_b + i), and
   * then any N >= 1 (prefill chunks); the window may be shorter than N.
   * Zero: the bf16 rows above. */
  int f32_rows;
} vnx_tree_attn_args;

/* Workspace bytes of the automatic plan without a window (an upper bound for
 * any window and for ALiBi). */
size_t vnx_tree_attn_workspace(int B, int H, int Hkv, int N, int Tp, int d);

/* Workspace bytes of exactly this call (forced splits, window, ALiBi
 * included); 256 for invalid arguments. */
size_t vnx_tree_attn_workspace_args(const vnx_tree_attn_args* args);

int vnx_tree_attn(const vnx_tree_attn_args* args, void* workspace, size_t workspace_bytes,
                  void* stream);

/* The launch shape vnx_tree_attn uses: key splits, query groups (of at most
 * 64 rows for d = 64, 32 for d = 128) and keys per split. */
int vnx_tree_attn_plan(int B, int H, int Hkv, int N, int Tp, int d, int* splits, int* groups,
                       int* chunk);

/* ---------------------------------------------------------------------------
 * Greedy tree verification: the reference's greedy rule on a token tree.
 * target: B x (N+1) rows at target + b*sb + i*ld (row 0: the prediction after
 * the last committed token, row 1+n: after tree node n); tokens (B, N) int64,
 * row pitch ld_tok; parent: a HOST array of N int32 (BFS order, parent[n] <
 * n, -1 for the root's children) shared by all batch rows, 1 <= N <= 64.
 * Node n is accepted iff tokens[b,n] == argmax(target row of its parent)
 * (numpy.argmax order) and its parent is accepted.  accept_len[b] = depth of
 * the deepest accepted node (lowest index among equally deep; 0 if none),
 * best[b] = that node or -1 (may be NULL), out_ids (B, N+1) = its root path,
 * the argmax of its own row (row 0 when none) as the bonus token, then -1;
 * pred (B, N+1) = the row argmaxes (may be NULL).
 * A chain tree (parent[n] = n-1) is the reference's verify + prefix rule
 * (speculative.py:218-223, :277-287) with the bonus token of the full match.
 * ------------------------------------------------------------------------- */
size_t vnx_tree_greedy_workspace(int64_t B, int N, int64_t V);

int vnx_tree_greedy(const void* target, int dtype, int64_t B, int N, int64_t V, int64_t ld, int64_t sb,
                    const int64_t* tokens, int64_t ld_tok, const int32_t* parent, int32_t* accept_len,
                    int32_t* best, int64_t* out_ids, int64_t* pred, void* workspace,
                    size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Row top-b (tree expansion): ids (rows, ldo) int64 = the b best ids of each
 * row of raw logits (row pitch ld), value descending, ties to the lower id,
 * NaN above every number (the numpy.argmax order, so b = 1 is argmax);
 * vals (rows, ldo) fp32 their values (may be NULL).  1 <= b <= 16, b <= V.
 * Replaces the top-k selection of Sampler.sample (np.partition,
 * packages/verse_infra/verse_infra/verse_inference/sampler.py:98-102) and of
 * _generate_with_logits (np.argpartition, cometspark.py:896-904) where a tree
 * draft needs the ids themselves, in a fixed order.
 * ------------------------------------------------------------------------- */
size_t vnx_row_topk_workspace(int64_t rows, int64_t V, int b);

int vnx_row_topk(const void* logits, int dtype, int64_t rows, int64_t V, int64_t ld, int b,
                 int64_t* ids, float* vals, int64_t ldo, void* workspace, size_t workspace_bytes,
                 void* stream);

/* ---------------------------------------------------------------------------
 * Verify-pass LM head on the matrix cores: out (M, V) = x (M, K) . w (V, K)^T,
 * x the final-norm hidden states of the verified positions (M = B*(k+1) <=
 * 256), w the tied embedding table (one row per vocab id), both bf16 with K
 * contiguous; fp32 accumulation; out fp32 (VNX_F32) or bf16 (VNX_BF16, round
 * to nearest even), row pitch ldo.  K a multiple of 64; x, w 16-byte aligned
 * with ldx, ldw multiples of 8; ldo a multiple of 4.  With out (B, k+1, V)
 * contiguous the result feeds vnx_spec_accept / vnx_greedy_verify directly.
 * Replaces the tied head CometSparkNexLM.head (cometspark.py:396-398, applied
 * at :697 / :766; Linear.forward, packages/verse_torch/verse_torch/vnnn.py:
 * 423-430) over the k+1 positions the verifier reads (speculative.py:218-220).
 * ------------------------------------------------------------------------- */
int vnx_lm_head(const void* x, int64_t ldx, const void* w, int64_t ldw, int64_t M, int64_t K, int64_t V,
                void* out, int out_dtype, int64_t ldo, void* stream);

/* ---------------------------------------------------------------------------
 * Fused per-layer work of the CometSpark forward (verify and draft steps).
 * Activation dtypes: VNX_F32, VNX_BF16 or VNX_F16; matrices row-major with
 * the given row pitches (elements).
 *
 * vnx_rmsnorm: per row m < M of D <= 4096 values, s = x[m] + res[m] (res may
 * be NULL), x_out[m] = s (x_out may be x, or NULL), y[m] = s / sqrt(mean(s^2)
 * + eps) * w.  RMSNorm (packages/verse_torch/verse_torch/vnnn.py:593-615,
 * :468-508) with the residual adds of VerseNexBlock.forward
 * (packages/verse_nex/verse_nex/cometspark.py:236-247).
 *
 * vnx_rope_kv: qkv (B*n rows of (H + 2*Hkv) * d values, heads q | k | v);
 * row (b, i) sits at position lens[b] + i.  q_out (B, H, n, d) contiguous =
 * q with RoPE (rotate-half, x*cos + rotate_half(x)*sin with the cos / sin
 * tables of table_rows x d fp32 values; rope = 0 copies), k with RoPE and v
 * are written into the caches at (b, kv head, position) via the strides
 * {c_sb, c_sh, c_sr}.  q_out and the caches are out_dtype (VNX_F32 or
 * VNX_BF16).  Rows whose position is not below cap (nor, with RoPE, below
 * table_rows) are skipped.  TriSparseAttention._apply_rope and its KV-cache
 * concat (packages/verse_nex/verse_nex/tri_sparse_attn.py:182-221, :558-575).
 *
 * vnx_swiglu: out[m, c] = silu(gu[m, c]) * gu[m, Hf + c], c < Hf: the
 * activation of SwiGLUMLP (vnnn.py:779-807) on a fused gate | up product.
 *
 * vnx_axpby: out[t] = coef[0] * a[t] + coef[1] * b[t], t < n, coef a device
 * array: the sigmoid-gated sum of the TriSparse paths (tri_sparse_attn.py:
 * 585-608).
 * ------------------------------------------------------------------------- */
int vnx_rmsnorm(const float* x, int64_t ldx, const void* res, int res_dtype, int64_t ldr, const float* w,
                float eps, int64_t M, int64_t D, float* x_out, int64_t ldxo, void* y, int y_dtype, int64_t ldy,
                void* stream);

/* vnx_embed_rmsnorm: the first block's norm with the token embedding folded
 * in (CometSparkV05LM.forward, spark/src/base_model.py:170-208: tok_emb(idx)
 * x sqrt(D), then norm1): x_out[m] = emb[tokens[m]] * scale (fp32, emb row
 * pitch lde, emb_dtype VNX_F32 / VNX_BF16 / VNX_F16; token ids clamped to
 * [0, vocab)), y[m] = RMSNorm(x_out[m]) * w as vnx_rmsnorm. */
int vnx_embed_rmsnorm(const int64_t* tokens, const void* emb, int emb_dtype, int64_t lde, int64_t vocab,
                      float scale, const float* w, float eps, int64_t M, int64_t D, float* x_out, int64_t ldxo,
                      void* y, int y_dtype, int64_t ldy, void* stream);

int vnx_rope_kv(const void* qkv, int dtype, int64_t ldq, int64_t B, int n, int H, int Hkv, int d,
                const int32_t* lens, const float* cos_table, const float* sin_table, int64_t table_rows, int rope,
                void* q_out, void* k_cache, void* v_cache, int out_dtype, int64_t c_sb, int64_t c_sh,
                int64_t c_sr, int64_t cap, void* stream);

int vnx_swiglu(const void* gu, int dtype, int64_t ldg, int64_t M, int64_t Hf, void* out, int out_dtype,
               int64_t ldo, void* stream);

int vnx_axpby(const float* a, const float* b, const float* coef, int64_t n, void* out, int out_dtype,
              void* stream);

/* MoD routing (Router.forward, packages/verse_nex/verse_nex/mod.py:337-440;
 * MoDLayer.forward, :779-803): logits (M, P + P*E) fp32 = [part-router
 * logits | the P expert routers' logits, part-major]; comb (M, P*E) fp32 =
 * softmax(part logits)[p] x softmax over part p's top-k expert logits
 * (larger first, ties to the lower index) for the selected experts, 0
 * elsewhere.  P <= 8, E <= 16, P + P*E <= 64, 1 <= topk <= E. */
int vnx_mod_route(const float* logits, int64_t ld, int64_t M, int P, int E, int topk, float* comb, int64_t ldc,
                  void* stream);

/* vnx_mod_route with the router products folded in: logits[m, r] =
 * sum_c h[m*ldh + c] * wr[r*ldw + c] (fp32, r < P + P*E <= 32: the part
 * router's rows, then each part's expert-router rows), then the same
 * routing weights into comb.  The router Linear (mod.py:337-440,
 * `self.gate(router_input)`) and the top-k rule in one launch.  With x_out
 * (bf16, not NULL) it also writes `copies` bf16 copies of h, copy q at
 * x_out + q*sxo (row pitch ldxo): the experts' input rows.  With norm_w
 * (not NULL) h is the raw residual row and the routing input is its RMSNorm,
 * RMSNorm(h) = h * rstd * norm_w, rstd = 1/sqrt(mean(h^2) + eps) (the block's
 * norm2 fused: the products use h * norm_w and the logits are scaled by
 * rstd; the bf16 copies are bf16(h * rstd * norm_w)). */
int vnx_mod_route_x(const float* h, int64_t ldh, const float* norm_w, float eps, const float* wr, int64_t ldw,
                    int64_t M, int64_t D, int P, int E, int topk, float* comb, int64_t ldc, void* x_out, int64_t ldxo,
                    int64_t sxo, int copies, void* stream);

/* The routed, weighted expert activations (DensePart / Expert,
 * mod.py:466-600): for row m and expert x < PE, with g = gu + m*ldg + x*sxg
 * and o = out + m*ldo + x*sxo, o[j] = comb[m, x] * silu(g[j]) * g[He + j],
 * j < He (0 for unselected experts).  Row-major (M, PE*2He) input is
 * sxg = 2He, ldg = PE*2He; expert-major (PE, M, 2He) is ldg = 2He,
 * sxg = M*2He (the same choices for out with He). */
int vnx_mod_swiglu(const void* gu, int dtype, int64_t ldg, int64_t sxg, const float* comb, int64_t ldc, int64_t M,
                   int PE, int64_t He, void* out, int out_dtype, int64_t ldo, int64_t sxo, void* stream);

/* out (M, D) fp32 = sum over x < PE of y[x] (y (PE, M, D) contiguous): the sum
 * of the experts' (weighted) down projections (MoDLayer.forward, mod.py:779-803). */
int vnx_sum_experts(const void* y, int dtype, int64_t M, int PE, int64_t D, float* out, void* stream);

/* out[m*ldo + c] (fp32) = the sum, over experts z < E in ascending order
 * with slots[m*E + z] >= 0, of y[z*syb + slots[m*E + z]*ldy + c], c < D: the
 * expert sum of MoDLayer.forward (mod.py:779-803) over compact per-expert
 * outputs (vnx_expert_gemm_bf16's row lists).  Equal to vnx_sum_experts of
 * the dense outputs, whose unrouted rows are zero.  accumulate != 0: out[m*ldo
 * + c] += that sum (the block's residual add, x + sum). */
int vnx_sum_expert_rows(const void* y, int dtype, int64_t ldy, int64_t syb, const int32_t* slots, int64_t M,
                        int E, int64_t D, float* out, int64_t ldo, int accumulate, void* stream);

/* Commit of one speculative round for all B sequences (the accept-and-advance
 * step of SpeculativeDecoder.verify_then_commit, packages/verse_nex/
 * verse_nex/speculative.py:277-310, with per-sequence KV lengths as in
 * ParallelKVCache.batch_update, kv_cache_parallel.py:42-286): with n_b =
 * clamp(accept_len[b], 0, k), ids[b*ld_ids + 0 .. n_b] (accepted drafts and
 * the drawn / bonus token) are appended to out[b*ld_out + count[b] ...]
 * (positions >= n_cap dropped), count[b], lens_t[b] and lens_d[b] advance by
 * n_b + 1, c[b] = ids[b*ld_ids + n_b], and info = {min count, max lens_t,
 * max lens_d, sum n_b} (int64).  B <= 1024; one launch. */
int vnx_spec_commit(const int32_t* accept_len, const int64_t* out_ids, int64_t ld_ids, int B, int k, int64_t* out,
                    int64_t ld_out, int64_t n_cap, int64_t* count, int64_t* c, int32_t* lens_t, int32_t* lens_d,
                    int64_t* info, void* stream);

/* ---------------------------------------------------------------------------
 * Skinny bf16 GEMM of the verify forward: for batch z < batch,
 *   acc[m, n] = sum_k x[z*sxb + m*ldx + k] * W_z[n, k]   (fp32 accumulation)
 * x (M, K) bf16 activations; W_z (N, K) bf16 weights in the nn.Linear layout,
 * given packed by vnx_pack_bf16 (batch z at w_packed + z*swb elements); y in
 * y_dtype (VNX_F32, VNX_BF16 or VNX_F16, round to nearest even).  Replaces
 * the Linear of the verifier's target forward (packages/verse_torch/
 * verse_torch/vnnn.py Linear.forward, x @ W^T) for the M = batch x (k+1)
 * rows of one round.  epilogue VNX_EPI_NONE: y[z*syb + m*ldy + n] = acc[m, n].
 * VNX_EPI_SWIGLU: W rows come in blocks of 32 (16 gate rows, then the 16 up
 * rows of the same hidden units) and
 *   y[z*syb + m*ldy + blk*16 + c] = comb[m*ldc + z] * silu(acc[m, blk*32 + c])
 *                                   * acc[m, blk*32 + 16 + c]
 * (comb NULL: weight 1): SwiGLUMLP's activation (vnnn.py:779-807) and a MoD
 * expert's routing weight (packages/verse_nex/verse_nex/mod.py:466-600).
 * K multiple of 64; x 16-byte aligned, ldx and sxb multiples of 8 (sxb = 0
 * shares x over the batch).  Deterministic (fixed summation order).
 *
 * vnx_pack_bf16: packs W (N, K) bf16, row pitch ldw, into the
 * vnx_pack_bf16_size(N, K) bytes at out (16-byte aligned) that vnx_gemm_bf16
 * reads: the matrix-core operand order, rows padded with zeros to a multiple
 * of 32.  Done once per weight.
 * ------------------------------------------------------------------------- */
enum vnx_epilogue { VNX_EPI_NONE = 0, VNX_EPI_SWIGLU = 1 };


size_t vnx_pack_bf16_size(int64_t N, int64_t K);
int vnx_pack_bf16(const void* w, int64_t ldw, int64_t N, int64_t K, void* out, void* stream);

int vnx_gemm_bf16(const void* x, int64_t ldx, int64_t sxb, const void* w_packed, int64_t swb, int64_t M,
                  int64_t N, int64_t K, int batch, int epilogue, const float* comb, int64_t ldc, void* y,
                  int y_dtype, int64_t ldy, int64_t syb, void* stream);

/* vnx_gemm_bf16 (batch 1) whose input is RMSNorm of the fp32 rows x (M, K),
 * row pitch ldx (vnnn.py:593-615, the block's norm1 / norm2 fused):
 *   acc[m, n] = rstd_m * sum_k bf16(x[m, k] * norm_w[k]) * W[n, k],
 *   rstd_m = 1/sqrt(mean_k x[m, k]^2 + eps),
 * then the epilogue (VNX_EPI_NONE or VNX_EPI_SWIGLU) into bf16 y.  K <= 2048;
 * x and norm_w 16-byte aligned, ldx % 4 == 0. */
int vnx_gemm_bf16_norm(const float* x, int64_t ldx, const float* norm_w, float eps, const void* w_packed,
                       int64_t M, int64_t N, int64_t K, int epilogue, void* y, int64_t ldy, void* stream);

/* vnx_gemm_bf16_norm of the first block, its input gathered from the token
 * embedding (CometSparkV05LM.forward, spark/src/base_model.py:170-208:
 * tok_emb(idx) x scale, then norm1, then the q|k|v projection), replacing
 * vnx_embed_rmsnorm + vnx_gemm_bf16 on the target's first layer: x_out[m] =
 * emb[tokens[m]] * scale (fp32, row pitch ldx; emb bf16 with row pitch lde, a
 * multiple of 8; ids clamped to [0, vocab)), written by the call, and y (M, N)
 * bf16 = RMSNorm(x_out) * norm_w times W as vnx_gemm_bf16_norm (no epilogue). */
int vnx_gemm_bf16_norm_embed(const int64_t* tokens, const void* emb, int emb_dtype, int64_t lde, int64_t vocab,
                             float scale, float* x_out, int64_t ldx, const float* norm_w, float eps,
                             const void* w_packed, int64_t M, int64_t N, int64_t K, void* y, int64_t ldy,
                             void* stream);

/* vnx_gemm_bf16 (batch 1) with the residual add fused: res[m*ldr + n] +=
 * acc[m, n] (fp32), the `x = x + proj(...)` of VerseNexBlock.forward
 * (cometspark.py:236-247). */
int vnx_gemm_bf16_residual(const void* x, int64_t ldx, const void* w_packed, int64_t M, int64_t N, int64_t K,
                           float* res, int64_t ldr, void* stream);

/* Routed MoD expert products (the expert FFNs of DensePart / Expert,
 * packages/verse_nex/verse_nex/mod.py:466-600, evaluated only on the rows
 * routed to each expert).  For expert z < experts, with its row list
 * L_z = (l_0 < l_1 < ...) of n_z rows:
 *   acc[j, n] = sum_k X_z[j, k] * W_z[n, k]  (fp32), j < n_z,
 * written to y + z*syb + j*ldy (compact order) with the epilogue of
 * vnx_gemm_bf16 (VNX_EPI_SWIGLU weights row j by comb[l_j*ldc + z]).
 * route != 0: L_z = { m < M : comb[m*ldc + z] != 0 } (M <= 256; with
 *   VNX_EPI_NONE comb only selects the rows), X_z[j] =
 *   x[l_j] (x shared, sxb = 0); the call also writes rows[z*M + j] = l_j,
 *   counts[z] = n_z and slots[m*experts + z] = j for m = l_j, else -1.
 * route == 0: X_z[j] = x[z*sxb + j*ldx], n_z = counts[z] (counts NULL: M),
 *   rows / slots unused.
 * W_z packed by vnx_pack_bf16 at w_packed + z*swb elements; K multiple of
 * 64; M * ldx * 2 < 2^31 (VNX_ERR_UNSUPPORTED otherwise).  Each element's
 * summation order depends on the shapes only, not on the row lists
 * (deterministic). */
int vnx_expert_gemm_bf16(const void* x, int64_t ldx, int64_t sxb, const void* w_packed, int64_t swb, int64_t M,
                         int64_t N, int64_t K, int experts, int epilogue, const float* comb, int64_t ldc, int route,
                         int32_t* rows, int32_t* counts, int32_t* slots, void* y, int y_dtype, int64_t ldy,
                         int64_t syb, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VNX_H_ */
