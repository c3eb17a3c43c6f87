/*
 * egpt.h - C ABI of libegpt_hip.so, the MI355X (gfx950) batch-1 decode kernels.
 *
 * Every entry point:
 *   - takes caller-owned DEVICE pointers (no allocation, no host<->device copies,
 *     no device->host reads: the decode position is read on the device), so each
 *     call can be captured into a hipGraph;
 *   - launches on the caller's stream and returns without synchronising;
 *   - returns EGPT_OK (0) or a negative status (bad argument, unsupported shape,
 *     or a failed launch), never aborts.
 *
 * Strides are in ELEMENTS. Activations are bf16 (passed as raw 16-bit storage),
 * weights int8 row-major [N, K] (the nn.Linear layout), per-output-channel scales
 * fp32 [N].
 */
#ifndef EGPT_H_
#define EGPT_H_

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  EGPT_OK = 0,
  EGPT_ERR_INVALID = -1,      /* bad pointer, size, stride or alignment */
  EGPT_ERR_UNSUPPORTED = -2,  /* shape or dtype outside what the kernels implement */
  EGPT_ERR_LAUNCH = -3,       /* the HIP launch failed (hipGetLastError) */
  EGPT_ERR_WORKSPACE = -4     /* workspace missing or smaller than required */
};

enum { EGPT_F32 = 0, EGPT_BF16 = 1, EGPT_F16 = 2 };

/* Largest M (rows of x) the GEMV kernels take; the reference's MAX_DECODE_ROWS
 * (research/realmodel/int8_linear.py:18). */
#define EGPT_MAX_DECODE_ROWS 16

int egpt_abi_version(void);
const char *egpt_status_string(int status);

/*
 * Weight-only int8 GEMV:  y[m, n] = bf16( scale[n] * sum_k x[m, k] * w[n, k] ),
 * fp32 accumulation, scale applied once after the K reduction, one rounding to
 * bf16 (round to nearest even). 1 <= M <= 16.
 * Replaces int8_matmul / the Triton _dot16 kernel
 * (research/realmodel/int8_linear.py:67-85 and :26-38).
 */
int egpt_int8_gemv(const void *x, int64_t ldx, const int8_t *w, int64_t ldw, const float *scale,
                   void *y, int64_t ldy, int M, int N, int K, hipStream_t stream);

/*
 * Split-K form of the same product: `splits` partial sums over K chunks are
 * written as fp32 [splits, M, N] into the workspace, then reduced in a fixed
 * order (no atomics, deterministic), scaled and rounded once.
 * Replaces the Triton _part / _reduce pair (research/realmodel/int8_linear.py:41-64,
 * launched at :79-84).
 */
int egpt_int8_gemv_splitk_workspace(int M, int N, int K, int splits, size_t *bytes);
int egpt_int8_gemv_splitk(const void *x, int64_t ldx, const int8_t *w, int64_t ldw, const float *scale,
                          void *y, int64_t ldy, int M, int N, int K, int splits,
                          void *workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * Per-output-channel symmetric int8 quantisation of a float matrix w [N, K] (row
 * stride ldw) into codes q int8 [N, K] (row stride ldq) and steps s fp32 [N]:
 *   s[n]    = max(max_k |w[n, k]| / 127, 1e-12)        (fp32, correctly rounded)
 *   q[n, k] = clamp(round_half_even(w[n, k] / s[n]), -127, 127)
 * dtype: EGPT_F32 / EGPT_BF16 / EGPT_F16, converted exactly to fp32 first. Each
 * step is one correctly rounded fp32 operation, so the bits equal the formula on
 * the CPU. Codes of rows holding NaN or infinity are unspecified.
 * Replaces quantize_weight for device tensors (research/realmodel/int8_linear.py:106-117).
 */
int egpt_quantize_rows(int dtype, const void *w, int64_t ldw, int N, int K, int8_t *q, int64_t ldq, float *s,
                       hipStream_t stream);

/*
 * Int8-weight GEMM for prefill (any M, typically > 16 rows):
 *   y[m, n] = bf16( fp32( bf16( sum_k x[m, k] * w[n, k] ) ) * scale[n] )
 * fp32 accumulation on bf16 MFMA with the weights' exact bf16 image, rounded once to
 * bf16, then the scale in fp32 and a second rounding: the reference's prefill formula
 * `((x2 @ w.to(bfloat16).t()).float() * s).to(bfloat16)` (research/realmodel/int8_linear.py:96-97),
 * without materialising the bf16 weights. x bf16 [M, K] (row stride ldx), w int8 [N, K]
 * (ldw), y bf16 [M, N] (ldy). The MFMA kernel takes K a multiple of 64, ldx % 8 == 0,
 * ldw % 16 == 0, 16-byte aligned x and w and operands under 2 GiB; any other shape runs
 * a generic kernel (fp32 sums over lane-strided K, the same two roundings), slower but
 * with the same contract.
 */
int egpt_int8_gemm(const void *x, int64_t ldx, const int8_t *w, int64_t ldw, const float *scale,
                   void *y, int64_t ldy, int M, int N, int K, hipStream_t stream);
/* The same product with a workspace, which lets short-M shapes (M <= 128 whose
 * 64 x 64 output tiles leave CUs idle) split K: each split's fp32 tile goes to the
 * workspace and a second launch adds the splits in order, then rounds as above.
 * egpt_int8_gemm_workspace gives the bytes the split needs for this shape (0: no
 * split; the workspace may then be NULL). Same result contract as egpt_int8_gemm
 * (the fp32 sum in another order). Replaces the same reference formula
 * (research/realmodel/int8_linear.py:96-97); the split mirrors the reference's
 * split-K GEMV (:41-64) for the GEMM. */
int egpt_int8_gemm_workspace(int M, int N, int K, size_t *bytes);
int egpt_int8_gemm_ws(const void *x, int64_t ldx, const int8_t *w, int64_t ldw, const float *scale,
                      void *y, int64_t ldy, int M, int N, int K, void *workspace, size_t workspace_bytes,
                      hipStream_t stream);
/* The product of a gate/up weight pair followed by SwiGLU: w holds `inter` gate rows then `inter` up rows
 * (int8 [2 inter, K], scales fp32 [2 inter]); for each row m and feature f, g and u are the product's values of
 * rows f and inter + f (the two roundings above) and act[m, f] = bf16(bf16(silu(g)) * u), transformers' bf16
 * Qwen3MLP rounding (models/qwen3/modeling_qwen3.py:49-62). The same bits as egpt_int8_gemm into a
 * [M, 2 inter] buffer followed by egpt_silu_mul, without that buffer. For K a multiple of 64, aligned rows and
 * operands under 2 GiB, and not for shapes whose plain product splits K (egpt_int8_gemm_workspace > 0);
 * EGPT_ERR_UNSUPPORTED otherwise, before any launch (the caller runs the two calls). Replaces, with the product, the reference's prefill formula
 * for gate_proj / up_proj (research/realmodel/int8_linear.py:96-97) and the SwiGLU its Inductor graph fuses
 * after them. */
int egpt_int8_gemm_swiglu(const void *x, int64_t ldx, const int8_t *w, int64_t ldw, const float *scale,
                          void *act, int64_t ld_act, int M, int inter, int K, hipStream_t stream);
/* The split-K product followed by the residual update and RMSNorm of each output row, the pair that follows
 * o_proj and down_proj in a prompt pass (transformers' Qwen3 decoder layer, models/qwen3/modeling_qwen3.py:285-322:
 * residual add, then the next RMSNorm): o = the product above, resid = bf16(resid + o) (written back), y =
 * RMSNorm(resid) * norm_w (as egpt_add_rmsnorm). The splits' sum, both roundings, the residual and the norm run in
 * one launch after the split slices, bit-identical to egpt_int8_gemm_ws followed by egpt_add_rmsnorm; o itself is
 * not stored. Only for shapes that split K (egpt_int8_gemm_workspace > 0, the same workspace) and N <= 16384;
 * EGPT_ERR_UNSUPPORTED otherwise, before any launch (the caller runs the two calls). Replaces, with
 * egpt_int8_gemm_ws, the reference's prefill formula (research/realmodel/int8_linear.py:96-97) and the residual +
 * RMSNorm its Inductor graph fuses after it. */
int egpt_int8_gemm_add_rmsnorm(const void *x, int64_t ldx, const int8_t *w, int64_t ldw, const float *scale,
                               void *resid, int64_t ld_resid, const void *norm_w, void *y, int64_t ldy,
                               int M, int N, int K, float eps, void *workspace, size_t workspace_bytes,
                               hipStream_t stream);
/* The split-K product of the fused QKV weights (w [(Hq + 2 Hkv) D, K]) followed by egpt_qk_norm_rope on its rows,
 * the pair at the start of a prompt pass's attention (transformers' Qwen3Attention.forward, the projections then
 * q_norm / k_norm, RoPE and the cache update, models/qwen3/modeling_qwen3.py:252-263): the splits' sum and both
 * roundings of each qkv element, then its head's norm, rotation and store, in one launch after the split slices;
 * bit-identical to egpt_int8_gemm_ws into a qkv buffer followed by egpt_qk_norm_rope, and the qkv rows themselves
 * are not stored. Only for shapes that split K (egpt_int8_gemm_workspace(M, (Hq + 2 Hkv) D, K) > 0, the same
 * workspace), D in {32, 64, 128} and 16-byte aligned rows and strides; EGPT_ERR_UNSUPPORTED otherwise, before any
 * launch (the caller runs the two calls). Replaces, with egpt_int8_gemm_ws, the reference's prefill formula for
 * q_proj / k_proj / v_proj (research/realmodel/int8_linear.py:96-97) and what its Inductor graph fuses after it. */
int egpt_int8_gemm_qk_norm_rope(const void *x, int64_t ldx, const int8_t *w, int64_t ldw, const float *scale,
                                const int64_t *positions, const void *q_norm_w, const void *k_norm_w,
                                const void *cos_t, const void *sin_t, void *q_out, int64_t ld_q, void *k_cache,
                                void *v_cache, int64_t cache_head_stride, int64_t cache_slot_stride, int M, int Hq,
                                int Hkv, int D, int K, int cap, float eps, void *workspace, size_t workspace_bytes,
                                hipStream_t stream);

/*
 * Split-K GQA decode attention (flash decoding) with its partial-softmax reduce.
 *   q   [B, Hq, 1, D]     strides (q_sb, q_sh), last dim contiguous
 *   k,v [B, Hkv, cap, D]  strides (sb, sh, sn), last dim contiguous
 *   position int64 [B] (pos_stride elements apart; pos_stride 0 = one shared value):
 *     query row b attends to slots 0..position[b] (clamped to cap-1); slots past it
 *     are never read.
 *   out [B, Hq, 1, D]     strides (o_sb, o_sh), in the input dtype.
 * Query head h reads kv head h / (Hq / Hkv). fp32 math, online softmax per split,
 * partials (max, sum, acc[D]) reduced in fp32. dtype: EGPT_F32 / EGPT_BF16 / EGPT_F16.
 * D in {32, 64, 128}; Hq / Hkv in {1, 2, 4, 8}. nsplit <= 0 picks the default.
 * With Hkv == Hq this is the reference's MHA contract.
 * Replaces _split_kernel + _combine_kernel and the NSPLIT choice
 * (research/phase5/decode_attention.py:22-71, :74-103); nsplit 1 is the
 * single-pass kernel (:106-151): one launch, which writes out directly.
 */
/* The default split count: 1 up to 256 slots (no combine launch), then about one
 * block per CU, at least 64 slots per split, at most 256 splits. */
int egpt_decode_attn_default_splits(int B, int Hkv, int cap);
int egpt_decode_attn_workspace(int B, int Hq, int Hkv, int cap, int D, int nsplit, size_t *bytes);
int egpt_decode_attn(int dtype,
                     const void *q, int64_t q_sb, int64_t q_sh,
                     const void *k, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                     const void *v, int64_t v_sb, int64_t v_sh, int64_t v_sn,
                     const int64_t *position, int64_t pos_stride,
                     void *out, int64_t o_sb, int64_t o_sh,
                     void *workspace, size_t workspace_bytes,
                     int B, int Hq, int Hkv, int cap, int D, int nsplit, float scale,
                     hipStream_t stream);

/*
 * egpt_decode_attn without a workspace and without any allocation: the split
 * partials go to a scratch array that the library holds in device memory, one copy
 * per device, for the life of the process. No counterpart in the reference; it is
 * for callers that cannot allocate device memory (code under graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Same arguments and result as
 * egpt_decode_attn minus the workspace. Limits: the partials of B * Hq * nsplit
 * (query row, split) pairs, egpt_decode_attn_workspace bytes, must fit in
 * EGPT_NOALLOC_SCRATCH_BYTES (else EGPT_ERR_WORKSPACE: at D 128, 8,065 pairs, e.g.
 * 16 query heads x 504 splits). The device that runs the call must be current
 * (EGPT_ERR_INVALID if `stream` belongs to another). Calls that overlap on one
 * device share the array and race; the first call on a device looks up the array's
 * address there, so make it before a graph capture: made while `stream` is being
 * captured it returns EGPT_ERR_INVALID and launches nothing. A failed lookup is not
 * remembered; the next call looks up again.
 */
#define EGPT_NOALLOC_SCRATCH_BYTES (4u << 20)
int egpt_decode_attn_noalloc(int dtype,
                             const void *q, int64_t q_sb, int64_t q_sh,
                             const void *k, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                             const void *v, int64_t v_sb, int64_t v_sh, int64_t v_sn,
                             const int64_t *position, int64_t pos_stride,
                             void *out, int64_t o_sb, int64_t o_sh,
                             int B, int Hq, int Hkv, int cap, int D, int nsplit, float scale,
                             hipStream_t stream);

/*
 * Decode-step kernels of the Qwen3 layer around the two hot kernels. They replace
 * the elementwise work the reference leaves to transformers' modules compiled by
 * Inductor inside its graph step (research/realmodel/fast_decode.py:42-49); the
 * arithmetic is transformers' bf16 Qwen3 (models/qwen3/modeling_qwen3.py).
 * Activations are bf16 [rows, n] with row strides ld*.
 */

/* y = bf16(w * bf16(x * rsqrt(mean(x^2) + eps))), fp32 statistics
 * (Qwen3RMSNorm, modeling_qwen3.py:30-46). n <= 16384. */
int egpt_rmsnorm(const void *x, int64_t ldx, const void *w, void *y, int64_t ldy, int rows, int n, float eps,
                 hipStream_t stream);

/* Residual add then RMSNorm: x = bf16(x + a) in place, y = RMSNorm(x)
 * (the `residual + hidden_states` / next-norm pair of Qwen3DecoderLayer, modeling_qwen3.py:285-322). */
int egpt_add_rmsnorm(void *x, int64_t ldx, const void *a, int64_t lda, const void *w, void *y, int64_t ldy,
                     int rows, int n, float eps, hipStream_t stream);

/* q_norm / k_norm (RMSNorm over head_dim), RoPE with bf16 cos/sin tables [cap, D],
 * and the static-cache write of the new key and value at slot positions[r]
 * (Qwen3Attention.forward up to past_key_values.update, modeling_qwen3.py:252-263;
 * the reference's `keys.index_copy_(2, position, k)`, research/phase5/compiled_baseline.py:44-45).
 * qkv rows are [q (Hq*D) | k (Hkv*D) | v (Hkv*D)]; rotated queries go to q_out [rows, Hq*D];
 * caches are [Hkv, cap, D] with strides (cache_head_stride, cache_slot_stride). D in {32, 64, 128}. */
int egpt_qk_norm_rope(const void *qkv, int64_t ld_qkv, const int64_t *positions, const void *q_norm_w,
                      const void *k_norm_w, const void *cos_t, const void *sin_t, void *q_out, int64_t ld_q,
                      void *k_cache, void *v_cache, int64_t cache_head_stride, int64_t cache_slot_stride,
                      int rows, int Hq, int Hkv, int D, int cap, float eps, hipStream_t stream);

/* Causal attention of a prompt block: query row t (position pos0 + t, head hq of
 * kv head hq / (Hq / Hkv)) attends cache slots 0 .. pos0 + t,
 *   out[t, hq] = softmax((q[t, hq] . k[s]) * scale) v,
 * the prompt pass of the reference's Qwen3 path (Qwen3Attention.forward over the
 * prompt: SDPA with the causal mask over the static cache, modeling_qwen3.py:252-280,
 * integrations/sdpa_attention.py:79-102). bf16 q [rows, Hq*D] (row stride q_ld, the
 * rotated queries of egpt_qk_norm_rope), caches [Hkv, cap, D] (strides cache_head_stride,
 * cache_slot_stride) already holding slots 0 .. pos0 + rows - 1, bf16 out [rows, Hq*D]
 * (row stride o_ld). fp32 logits and softmax; the probabilities multiply v as bf16.
 * scale > 0 (else EGPT_ERR_INVALID). D 128, Hq / Hkv in {1, 2, 4, 8} (else
 * EGPT_ERR_UNSUPPORTED: the caller keeps its library attention). */
int egpt_prefill_attn(const void *q, int64_t q_ld, const void *k_cache, const void *v_cache,
                      int64_t cache_head_stride, int64_t cache_slot_stride, void *out, int64_t o_ld, int rows,
                      int Hq, int Hkv, int D, int cap, int pos0, float scale, hipStream_t stream);

/* act = bf16(bf16(silu(gate)) * up) over rows laid out [gate (inter) | up (inter)]
 * (Qwen3MLP, modeling_qwen3.py:49-62). */
int egpt_silu_mul(const void *gu, int64_t ld_gu, int inter, void *out, int64_t ld_out, int rows,
                  hipStream_t stream);

/* out[r] = table[tokens[r]] (embed_tokens gather; ids clamped to [0, vocab)). */
int egpt_embed(const int64_t *tokens, int rows, const void *table, int64_t ld_table, int vocab, void *out,
               int64_t ld_out, int n, hipStream_t stream);

/* Greedy pick: *token = first index of the largest bf16 logit (torch.argmax), and
 * *position += 1 when position is non-null: the token/position update of the
 * reference's graph step (research/realmodel/fast_decode.py:48-49). */
int egpt_argmax_workspace(int n, size_t *bytes);
int egpt_argmax(const void *logits, int n, void *workspace, size_t workspace_bytes, int64_t *token,
                int64_t *position, hipStream_t stream);

/*
 * One int8 weight-only GEMV of a single activation row (M = 1) with a fused
 * prologue and epilogue: the building block of the decode step below, and the
 * batch-1 form of the reference's int8 linear (research/realmodel/int8_linear.py:26-38,
 * y = bf16(s * fp32 sum)) with the elementwise work around it
 * (transformers' Qwen3 RMSNorm / residual / SwiGLU, models/qwen3/modeling_qwen3.py).
 *
 * Activation (bf16, K elements), one of:
 *   x                       the row x[0..K)
 *   x + *x_token * x_ld     a table row selected on the device (token clamped to [0, x_rows))
 *   merge_m/_l/_acc != NULL the split-K attention partials of K / head_dim heads
 *                           (merge_splits splits, the layout of egpt_decode_attn's
 *                           workspace for B = 1), merged as in the combine
 * optionally RMS-normalised first: h = bf16(norm_w * bf16(x * rsqrt(mean x^2 + eps))).
 * Epilogue on the fp32 sums acc[n] (weights int8 [rows, K] with row stride ldw,
 * fp32 scale per row):
 *   EGPT_EPI_STORE     y[n] = bf16(scale[n] acc[n])                         n < N
 *   EGPT_EPI_RESIDUAL  y[n] = bf16(resid[n] + bf16(scale[n] acc[n]))       (resid: row, or table row
 *                      by *resid_token like x; y may alias resid)
 *   EGPT_EPI_SWIGLU    y[n] = bf16(bf16(silu(g)) * u), g = bf16(scale[n] acc[n]) from row n,
 *                      u = bf16(scale[N + n] acc[N + n]) from row N + n    (rows 2N)
 *   EGPT_EPI_ARGMAX    y[n] = bf16(scale[n] acc[n]) if y != NULL, and per-block maxima
 *                      (value, first index) to part_v / part_i (egpt_int8_gemv_fused_parts
 *                      entries); egpt_argmax_parts() then picks the token.
 * Supported: STORE with or without norm; RESIDUAL from a row or a merge, no
 * norm; SWIGLU and ARGMAX with norm. K a multiple of 16, K <= 12288 (merge:
 * K <= 4096, merge_splits <= 16); 16-byte aligned x, norm_w, w rows, merge_acc.
 */
enum { EGPT_EPI_STORE = 0, EGPT_EPI_RESIDUAL = 1, EGPT_EPI_SWIGLU = 2, EGPT_EPI_ARGMAX = 3 };

typedef struct egpt_gemv_fused {
  int epilogue;
  int N, K;
  const void *x;
  const int64_t *x_token;
  int64_t x_ld;
  int x_rows;
  const void *norm_w;
  float eps;
  const float *merge_m, *merge_l, *merge_acc;
  int merge_splits, head_dim;
  const int8_t *w;
  int64_t ldw;
  const float *scale;
  void *y;
  const void *resid;
  const int64_t *resid_token;
  int64_t resid_ld;
  float *part_v;
  int *part_i;
} egpt_gemv_fused;

int egpt_int8_gemv_fused_parts(const egpt_gemv_fused *g, int *parts);
int egpt_int8_gemv_fused(const egpt_gemv_fused *g, hipStream_t stream);

/* Greedy pick over per-block maxima: *token = index of the largest value
 * (first index on ties, torch.argmax), *position += 1 when position != NULL. */
int egpt_argmax_parts(const float *part_v, const int *part_i, int parts, int64_t *token, int64_t *position,
                      hipStream_t stream);

/*
 * Whole batch-1 decode step of a Qwen3 decoder with int8 weight-only linears,
 * fused into 5 launches per layer plus one for the head (RMSNorm in the GEMV
 * prologues; residual adds and SwiGLU in the GEMV epilogues; q/k-norm, RoPE,
 * the K/V cache write and the split-K combine inside the attention kernel; the
 * embedding gather inside layer 0; lm_head + argmax + position advance in the
 * last launch). Consumes *token at *position, writes K/V slot *position of every
 * layer, leaves the greedy next token in *token and advances *position by one.
 * Replaces the reference's captured decode step, the Inductor-compiled HF
 * forward + argmax + token/position update (research/realmodel/fast_decode.py:45-49),
 * with every linear on its int8 GEMV contract (research/realmodel/int8_linear.py:26-38).
 *
 * Weights are device pointers, row-major [rows, cols]:
 *   qkv_w [(heads + 2 kv_heads) head_dim, hidden]  (q rows, then k, then v)
 *   o_w   [hidden, heads head_dim]
 *   gu_w  [2 inter, hidden]                        (gate rows, then up rows)
 *   down_w [hidden, inter],  head_w [vocab, hidden]
 * with fp32 per-row scales; norms bf16; caches bf16 [kv_heads, cap, head_dim];
 * rope_cos / rope_sin bf16 [cap, head_dim]; x / qkv / attn / act / logits are
 * bf16 rows of hidden / (heads + 2 kv_heads) head_dim / heads head_dim / inter /
 * vocab elements (logits may be NULL). `layer` is a HOST array of `layers` entries.
 * The workspace (egpt_qwen3_step_workspace bytes, 256-byte aligned) holds the
 * attention and argmax partials; every step writes them before reading them, so
 * its contents on entry do not matter.
 * Sizes: hidden, inter and heads*head_dim multiples of 16 and <= 12288;
 * head_dim in {32, 64, 128}; heads / kv_heads in {1, 2, 4, 8}.
 */
typedef struct egpt_qwen3_layer {
  const int8_t *qkv_w;
  const float *qkv_s;
  const int8_t *o_w;
  const float *o_s;
  const int8_t *gu_w;
  const float *gu_s;
  const int8_t *down_w;
  const float *down_s;
  const void *in_norm;
  const void *post_norm;
  const void *q_norm;
  const void *k_norm;
  void *k_cache;
  void *v_cache;
} egpt_qwen3_layer;

typedef struct egpt_qwen3_step {
  int layers, hidden, inter, heads, kv_heads, head_dim, vocab, cap, nsplit;
  float eps;
  const egpt_qwen3_layer *layer;
  const void *embed;
  const void *final_norm;
  const int8_t *head_w;
  const float *head_s;
  const void *rope_cos;
  const void *rope_sin;
  int64_t *token;
  int64_t *position;
  void *x;
  void *qkv;
  void *attn;
  void *act;
  void *logits;
  void *workspace;
  size_t workspace_bytes;
  /* Optional (NULL: unused): each step also stores its greedy token to
   * token_ring[new position % token_ring_slots], where the new position is the
   * one it leaves in *position. Pinned host memory (hipHostMalloc) lets a host
   * loop read every step's token once that step has completed, with no copy
   * launched per token; device memory works too. */
  int64_t *token_ring;
  int token_ring_slots;
} egpt_qwen3_step;

int egpt_qwen3_step_workspace(const egpt_qwen3_step *step, size_t *bytes);
/* The step's split count for `nsplit`. Up to 3072 slots, where the step's
 * attention blocks serve one query head each: one split per 64 slots, at most 4
 * up to 512 slots and 8 past that, merged in the o_proj GEMV's prologue. Past
 * 3072 slots (blocks of a kv head's whole group): about one block per CU and at
 * least 64 slots per split, merged in one small launch past 16. Unlike the
 * stand-alone attention, the step splits short caches too, since its merge needs
 * no launch of its own. Has no counterpart in the reference, whose step reads
 * SDPA. */
int egpt_qwen3_step_default_splits(int heads, int kv_heads, int head_dim, int cap);
int egpt_qwen3_decode_step(const egpt_qwen3_step *step, hipStream_t stream);

/* The step's fused GEMV launches as egpt_gemv_fused descriptions, in launch
 * order (4 per layer, then the head): *count = 4 layers + 1; `out` (capacity
 * entries) may be NULL to query the count. Replaying them through
 * egpt_int8_gemv_fused runs exactly the GEMVs of egpt_qwen3_decode_step. */
int egpt_qwen3_step_gemvs(const egpt_qwen3_step *step, egpt_gemv_fused *out, int capacity, int *count);

#ifdef __cplusplus
}
#endif

#endif /* EGPT_H_ */
