// Device helpers of the fused decode-step kernels (qwen3_fused.hip): the int8 x
// bf16 dot product of the GEMV tiles, bf16 unpacking, the greedy (argmax)
// reduction and the per-head RMSNorm + RoPE of queries and keys.
#pragma once

#include "attn_core.h"

namespace egpt {

__device__ __forceinline__ float bf16r(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// 16 int8 weights times 16 fp32 activations, biased form: (w + 128) converts
// with one v_cvt_f32_ubyteN; 128 * sum(x) is removed once after the reduction.
__device__ __forceinline__ float dot16_biased(const u32x4 wq, const float* xf, float acc) {
  const uint32_t d[4] = {wq.x ^ 0x80808080u, wq.y ^ 0x80808080u, wq.z ^ 0x80808080u, wq.w ^ 0x80808080u};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    acc = fmaf((float)(d[j] & 0xffu), xf[4 * j + 0], acc);
    acc = fmaf((float)((d[j] >> 8) & 0xffu), xf[4 * j + 1], acc);
    acc = fmaf((float)((d[j] >> 16) & 0xffu), xf[4 * j + 2], acc);
    acc = fmaf((float)(d[j] >> 24), xf[4 * j + 3], acc);
  }
  return acc;
}

__device__ __forceinline__ void unpack_bf16x16(const u32x4 a, const u32x4 b, float* xf) {
  const uint32_t u[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    xf[2 * i] = bf16_lo(u[i]);
    xf[2 * i + 1] = bf16_hi(u[i]);
  }
}

struct ArgBest {
  float v;
  int i;
};

// torch.argmax's order: NaN ranks above every number, then the larger value;
// ties (NaN against NaN included) go to the smaller index.
__device__ __forceinline__ ArgBest arg_better(ArgBest a, ArgBest b) {
  const bool an = a.v != a.v, bn = b.v != b.v;
  const bool b_wins = an ? (bn && b.i < a.i) : (bn || b.v > a.v || (b.v == a.v && b.i < a.i));
  return b_wins ? b : a;
}

template <int W>
__device__ __forceinline__ ArgBest block_argbest(ArgBest x) {
  __shared__ float sv[W];
  __shared__ int si[W];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    ArgBest o;
    o.v = __shfl_xor(x.v, off, kWave);
    o.i = __shfl_xor(x.i, off, kWave);
    x = arg_better(x, o);
  }
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) {
    sv[wave] = x.v;
    si[wave] = x.i;
  }
  lds_barrier();
  ArgBest r{sv[0], si[0]};
#pragma unroll
  for (int j = 1; j < W; ++j) r = arg_better(r, ArgBest{sv[j], si[j]});
  lds_barrier();
  return r;
}

__device__ __forceinline__ const uint16_t* token_row(const uint16_t* base, const int64_t* token, int64_t ld,
                                                     int rows) {
  if (!token) return base;
  int64_t t = *token;
  t = t < 0 ? 0 : (t >= rows ? rows - 1 : t);
  return base + t * ld;
}

// Head-wise RMSNorm + RoPE of one head held by an LPS-lane group (EPL elements
// per lane, element d0 + e; x, norm weight, cos and sin rows already loaded).
// rotate_half pairs element i with i +- D/2, which sits in lane (sub ^ LPS/2)
// at the same e.
template <int D, int EPL, int LPS>
__device__ __forceinline__ void head_norm_rope(const u32x4 xr, const u32x4 wr, const u32x4 cr, const u32x4 sr, int d0,
                                               float eps, float (&out)[EPL]) {
  float xv[EPL], w[EPL], cs[EPL], sn[EPL];
  Elem<__bf16>::unpack(xr, xv);
  Elem<__bf16>::unpack(wr, w);
  Elem<__bf16>::unpack(cr, cs);
  Elem<__bf16>::unpack(sr, sn);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) ss = fmaf(xv[e], xv[e], ss);
  const float inv = rsqrtf(group_sum<LPS>(ss) / (float)D + eps);
  float nv[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) nv[e] = bf16r(w[e] * bf16r(xv[e] * inv));
  const bool lower = d0 < D / 2;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const float p = LPS == 16 ? xor8(nv[e]) : __shfl_xor(nv[e], LPS / 2, kWave);
    const float rh = lower ? -p : p;
    out[e] = bf16r(bf16r(nv[e] * cs[e]) + bf16r(rh * sn[e]));
  }
}

}  // namespace egpt
