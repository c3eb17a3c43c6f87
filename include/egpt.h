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
 * Split-K GQA decode attention (flash decoding) with its partial-softmax reduce.
 *   q   [B, Hq, 1, D]     strides (q_sb, q_sh), last dim contiguous
 *   k,v [B, Hkv, cap, D]  strides (sb, sh, sn), last dim contiguous
 *   position int64 [B] (pos_stride elements apart; pos_stride 0 = one shared value):
 *     query row b attends to slots 0..position[b] (clamped to cap-1); slots past it
 *     are never read.
 *   out [B, Hq, 1, D]     strides (o_sb, o_sh), in the input dtype.
 * Query head h reads kv head h / (Hq / Hkv). fp32 math, online softmax per split,
 * partials (max, sum, acc[D]) reduced in fp32. dtype: EGPT_F32 / EGPT_BF16 / EGPT_F16.
 * D in {64, 128}; Hq / Hkv in {1, 2, 4, 8}. nsplit <= 0 picks the default.
 * With Hkv == Hq this is the reference's MHA contract.
 * Replaces _split_kernel + _combine_kernel and the NSPLIT choice
 * (research/phase5/decode_attention.py:22-71, :74-103); nsplit 1 is the
 * single-pass kernel (:106-151).
 */
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

#ifdef __cplusplus
}
#endif

#endif /* EGPT_H_ */
