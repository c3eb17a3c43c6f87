// Elementwise / normalisation kernels of the Qwen3 decode step on gfx950.
//
// Rounding follows transformers' bf16 Qwen3 (models/qwen3/modeling_qwen3.py), op by op:
//   RMSNorm      y = bf16( w * bf16( x * rsqrt(mean(x^2) + eps) ) ), statistics in fp32  (:30-46)
//   residual     x = bf16( x + a )                                                      (:285-322)
//   q/k norm     RMSNorm over head_dim on each head                                      (:237-238, :255-256)
//   RoPE         bf16( bf16(x * cos) + bf16(rotate_half(x) * sin) ), cos/sin tables bf16 (:139-166)
//   SwiGLU       bf16( bf16(silu(gate)) * up )                                           (:49-62)
//   argmax       first index of the largest logit (torch.argmax), next token + position
//                advance of the reference's graph step (research/realmodel/fast_decode.py:45-49)
// All activations are bf16 stored as uint16.
#include "step_core.h"

namespace egpt {
namespace {

constexpr int kNormThreads = 256;

__device__ __forceinline__ float bf16r(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Block-wide sum with a fixed order: wave sums, then the four wave totals in order.
__device__ __forceinline__ float block_sum_256(float v, float* red) {
  v = wave_sum(v);
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) red[wave] = v;
  __syncthreads();
  const float total = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return total;
}

// One block per row. If `a` is non-null the residual is updated first:
// x = bf16(x + a) (written back), then y = RMSNorm(x).
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(uint16_t* __restrict__ x, int64_t ldx,
                                                                   const uint16_t* __restrict__ a, int64_t lda,
                                                                   const uint16_t* __restrict__ w,
                                                                   uint16_t* __restrict__ y, int64_t ldy, int n,
                                                                   float eps) {
  __shared__ float red[kNormThreads / kWave];
  extern __shared__ float rowbuf[];  // n floats: the (updated) residual row
  const int64_t row = blockIdx.x;
  uint16_t* xr = x + row * ldx;
  float ss = 0.f;
  for (int i = threadIdx.x; i < n; i += kNormThreads) {
    float v = bf16_to_f32(xr[i]);
    if (a) {
      v = bf16r(v + bf16_to_f32(a[row * lda + i]));
      xr[i] = f32_to_bf16(v);
    }
    rowbuf[i] = v;
    ss = fmaf(v, v, ss);
  }
  const float total = block_sum_256(ss, red);
  const float inv = rsqrtf(total / (float)n + eps);
  uint16_t* yr = y + row * ldy;
  for (int i = threadIdx.x; i < n; i += kNormThreads) {
    yr[i] = f32_to_bf16(bf16_to_f32(w[i]) * bf16r(rowbuf[i] * inv));
  }
}

// Element e of a row in the vector form: thread t owns 8-element groups t, t + 256, ... (16-byte accesses).
// The same arithmetic per element as add_rmsnorm_kernel; the sum of squares runs in this element order.
__device__ __forceinline__ void unpack8(const u32x4 v, float (&f)[8]) {
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_lo(u[i]);
    f[2 * i + 1] = bf16_hi(u[i]);
  }
}
__device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
  uint32_t u[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) u[i] = (uint32_t)f32_to_bf16(f[2 * i]) | ((uint32_t)f32_to_bf16(f[2 * i + 1]) << 16);
  return u32x4{u[0], u[1], u[2], u[3]};
}

// add_rmsnorm_kernel for rows of a multiple of 8 elements, 16-byte aligned: every access 16 bytes wide (the
// scalar form issues one 2-byte access per element and per thread, 0.25-0.3 of HBM peak at 8192 rows).
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_v8_kernel(uint16_t* __restrict__ x, int64_t ldx,
                                                                      const uint16_t* __restrict__ a, int64_t lda,
                                                                      const uint16_t* __restrict__ w,
                                                                      uint16_t* __restrict__ y, int64_t ldy, int n,
                                                                      float eps) {
  __shared__ float red[kNormThreads / kWave];
  extern __shared__ float rowbuf[];  // n floats: the (updated) residual row
  const int64_t row = blockIdx.x;
  uint16_t* xr = x + row * ldx;
  float ss = 0.f;
  for (int g = threadIdx.x; g * 8 < n; g += kNormThreads) {
    float v[8];
    unpack8(ld16(xr + g * 8), v);
    if (a) {
      float av[8];
      unpack8(ld16(a + row * lda + g * 8), av);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = bf16r(v[e] + av[e]);
      *(u32x4*)(xr + g * 8) = pack8(v);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      rowbuf[g * 8 + e] = v[e];
      ss = fmaf(v[e], v[e], ss);
    }
  }
  const float total = block_sum_256(ss, red);
  const float inv = rsqrtf(total / (float)n + eps);
  uint16_t* yr = y + row * ldy;
  for (int g = threadIdx.x; g * 8 < n; g += kNormThreads) {
    float wv[8], o[8];
    unpack8(ld16(w + g * 8), wv);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = wv[e] * bf16r(rowbuf[g * 8 + e] * inv);
    *(u32x4*)(yr + g * 8) = pack8(o);
  }
}

// q/k RMSNorm + RoPE + cache write. One wavefront per (row, head); heads
// 0..Hq-1 are query heads (written to q_out), Hq..Hq+Hkv-1 key heads (normed,
// rotated, written to the key cache at the row's position), the last Hkv value
// heads (copied to the value cache). Row layout of qkv: [q(Hq*D) | k(Hkv*D) | v(Hkv*D)].
template <int D>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    const uint16_t* __restrict__ qkv, int64_t ld_qkv, const int64_t* __restrict__ positions,
    const uint16_t* __restrict__ qn_w, const uint16_t* __restrict__ kn_w, const uint16_t* __restrict__ cos_t,
    const uint16_t* __restrict__ sin_t, uint16_t* __restrict__ q_out, int64_t ld_q, uint16_t* __restrict__ k_cache,
    uint16_t* __restrict__ v_cache, int64_t c_sh, int64_t c_sn, int rows, int Hq, int Hkv, int cap, float eps) {
  constexpr int EPT = D >= kWave ? D / kWave : 1;  // elements per lane (2 for D = 128)
  static_assert(D % kWave == 0 || kWave % D == 0, "head_dim must divide or be a multiple of 64");
  const int lane = threadIdx.x & (kWave - 1);
  const bool live = lane < D;  // D < 64: the upper lanes hold no element
  const int64_t job = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  const int heads = Hq + 2 * Hkv;
  if (job >= (int64_t)rows * heads) return;
  const int64_t row = job / heads;
  const int head = (int)(job % heads);
  int64_t pos = positions[row];
  pos = pos < 0 ? 0 : (pos >= cap ? cap - 1 : pos);
  const uint16_t* src = qkv + row * ld_qkv + (int64_t)head * D;
  if (head >= Hq + Hkv) {  // value head: straight copy into the cache
    uint16_t* dst = v_cache + (int64_t)(head - Hq - Hkv) * c_sh + pos * c_sn;
    if (live) {
#pragma unroll
      for (int e = 0; e < EPT; ++e) dst[lane + e * kWave] = src[lane + e * kWave];
    }
    return;
  }
  const bool is_q = head < Hq;
  const uint16_t* nw = is_q ? qn_w : kn_w;
  float xv[EPT];
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    xv[e] = live ? bf16_to_f32(src[lane + e * kWave]) : 0.f;
    ss = fmaf(xv[e], xv[e], ss);
  }
  const float inv = rsqrtf(wave_sum(ss) / (float)D + eps);
  // Normed values. Lane l holds elements l + 64 e; rotate_half pairs element i
  // with i +- D/2, which for D = 128 sits in the same lane (e +- 1) and for
  // D = 64 in lane l ^ 32 (same e).
  float nv[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) nv[e] = live ? bf16r(bf16_to_f32(nw[lane + e * kWave]) * bf16r(xv[e] * inv)) : 0.f;
  const uint16_t* cr = cos_t + pos * D;
  const uint16_t* sr = sin_t + pos * D;
  uint16_t out[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const int i = lane + e * kWave;
    float partner;
    if constexpr (D / 2 >= kWave) {
      constexpr int kHalf = D / 2 / kWave;
      partner = e < kHalf ? nv[(e + kHalf) % EPT] : nv[(e + EPT - kHalf) % EPT];
    } else {
      partner = __shfl_xor(nv[e], D / 2, kWave);
    }
    const float rh = i % D < D / 2 ? -partner : partner;
    out[e] = live ? f32_to_bf16(bf16r(nv[e] * bf16_to_f32(cr[i])) + bf16r(rh * bf16_to_f32(sr[i]))) : 0;
  }
  uint16_t* dst = is_q ? q_out + row * ld_q + (int64_t)head * D
                       : k_cache + (int64_t)(head - Hq) * c_sh + pos * c_sn;
  if (live) {
#pragma unroll
    for (int e = 0; e < EPT; ++e) dst[lane + e * kWave] = out[e];
  }
}

// act = bf16( bf16(silu(gate)) * up ), gate/up interleaved per row as [gate(inter) | up(inter)].
// qk_norm_rope_kernel for 16-byte aligned rows: a (row, head) job per group of D / 8 lanes, 8 elements per lane
// and 16-byte accesses (the wavefront-per-head form issues 2-byte accesses). Query and key heads take the decode
// step's head_norm_rope (the same per-element roundings and the same lane layout and sum order as the step's
// attention kernel), value heads a 16-byte copy. Groups past the last job compute the last one and store nothing.
// The q/k/v operands of one launch of the 16-byte form.
struct QkRope {
  const int64_t* positions;
  const uint16_t* qn_w;
  const uint16_t* kn_w;
  const uint16_t* cos_t;
  const uint16_t* sin_t;
  uint16_t* q_out;
  int64_t ld_q;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t c_sh, c_sn;
  int rows, Hq, Hkv, cap;
  float eps;
};

// The (row, head) job of this lane group and the lane's first element.
struct QkJob {
  int64_t row;
  int head;
  int d0;
  bool store;
};

template <int D>
__device__ __forceinline__ QkJob qk_job(const QkRope& a) {
  constexpr int LPS = D / 8;  // lanes per head: 16 at D 128
  const int heads = a.Hq + 2 * a.Hkv;
  const int64_t jobs = (int64_t)a.rows * heads;
  const int64_t job_raw = (int64_t)blockIdx.x * (256 / LPS) + threadIdx.x / LPS;
  QkJob j;
  j.store = job_raw < jobs;
  const int64_t job = j.store ? job_raw : jobs - 1;
  j.row = job / heads;
  j.head = (int)(job % heads);
  j.d0 = (threadIdx.x % LPS) * 8;
  return j;
}

// The rest of a job once the lane's 8 elements of its head (xr) are in: value heads copy into the cache, query
// and key heads take head_norm_rope into q_out / the key cache.
template <int D>
__device__ __forceinline__ void qk_finish(const QkRope& a, const QkJob& j, const u32x4 xr) {
  constexpr int EPL = 8;
  constexpr int LPS = D / EPL;
  const int64_t row = j.row;
  const int head = j.head, d0 = j.d0, Hq = a.Hq, Hkv = a.Hkv;
  const bool store = j.store;
  const uint16_t* qn_w = a.qn_w;
  const uint16_t* kn_w = a.kn_w;
  const uint16_t* cos_t = a.cos_t;
  const uint16_t* sin_t = a.sin_t;
  uint16_t* q_out = a.q_out;
  uint16_t* k_cache = a.k_cache;
  uint16_t* v_cache = a.v_cache;
  const int64_t ld_q = a.ld_q, c_sh = a.c_sh, c_sn = a.c_sn;
  const float eps = a.eps;
  int64_t pos = a.positions[row];
  pos = pos < 0 ? 0 : (pos >= a.cap ? a.cap - 1 : pos);
  if (head >= Hq + Hkv) {  // value head: straight copy into the cache (group-uniform)
    if (store) *(u32x4*)(v_cache + (int64_t)(head - Hq - Hkv) * c_sh + pos * c_sn + d0) = xr;
    return;
  }
  const bool is_q = head < Hq;
  const u32x4 wr = ld16((is_q ? qn_w : kn_w) + d0);
  const u32x4 cr = ld16(cos_t + pos * D + d0);
  const u32x4 sr = ld16(sin_t + pos * D + d0);
  float o[EPL];
  head_norm_rope<D, EPL, LPS>(xr, wr, cr, sr, d0, eps, o);
  uint32_t pk[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) pk[e] = (uint32_t)f32_to_bf16(o[2 * e]) | ((uint32_t)f32_to_bf16(o[2 * e + 1]) << 16);
  uint16_t* dst = is_q ? q_out + row * ld_q + (int64_t)head * D : k_cache + (int64_t)(head - Hq) * c_sh + pos * c_sn;
  if (store) *(u32x4*)(dst + d0) = u32x4{pk[0], pk[1], pk[2], pk[3]};
}

template <int D>
__global__ __launch_bounds__(256) void qk_norm_rope_v8_kernel(const uint16_t* __restrict__ qkv, int64_t ld_qkv,
                                                              const QkRope a) {
  const QkJob j = qk_job<D>(a);
  qk_finish<D>(a, j, ld16(qkv + j.row * ld_qkv + (int64_t)j.head * D + j.d0));
}

// launch_reduce_qk_norm_rope's kernel: the lane's 8 elements of the qkv row from the S split partials
// [S][rows][(Hq + 2 Hkv) D] of the prefill GEMM, added and rounded as int8_gemm_reduce_kernel does (every
// slice's loads issued before the first addition; bf16(bf16(v0 + v1 + ...) * scale)), then qk_norm_rope_v8's job.
template <int D, int S>
__global__ __launch_bounds__(256) void reduce_qk_norm_rope_v8_kernel(const float* __restrict__ part,
                                                                     const float* __restrict__ scale, const QkRope a) {
  const QkJob j = qk_job<D>(a);
  const int64_t n = (int64_t)(a.Hq + 2 * a.Hkv) * D;
  const int64_t mn = (int64_t)a.rows * n;
  const int64_t col = (int64_t)j.head * D + j.d0;
  const float* p = part + j.row * n + col;
  u32x4 v[S][2];
#pragma unroll
  for (int sp = 0; sp < S; ++sp) {
    v[sp][0] = ld16(p + sp * mn);
    v[sp][1] = ld16(p + sp * mn + 4);
  }
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    auto part_e = [&](int sp) {
      const u32x4& q = v[sp][e / 4];
      const uint32_t w = (e % 4 == 0) ? q.x : (e % 4 == 1) ? q.y : (e % 4 == 2) ? q.z : q.w;
      return __uint_as_float(w);
    };
    float acc = part_e(0);
#pragma unroll
    for (int sp = 1; sp < S; ++sp) acc += part_e(sp);
    o[e] = bf16r(bf16r(acc) * scale[col + e]);
  }
  qk_finish<D>(a, j, pack8(o));
}

__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ gu, int64_t ld_gu, int inter,
                                                       uint16_t* __restrict__ out, int64_t ld_out, int rows) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)rows * inter) return;
  const int64_t row = i / inter;
  const int c = (int)(i % inter);
  const float g = bf16_to_f32(gu[row * ld_gu + c]);
  const float u = bf16_to_f32(gu[row * ld_gu + inter + c]);
  const float sg = bf16r(g / (1.0f + expf(-g)));
  out[row * ld_out + c] = f32_to_bf16(sg * u);
}

// silu_mul_kernel with 8 elements per thread and 16-byte accesses, block (column chunk, row): for inter, the
// row strides and the pointers multiples of 8 elements / 16 bytes. The same arithmetic per element.
__global__ __launch_bounds__(256) void silu_mul_v8_kernel(const uint16_t* __restrict__ gu, int64_t ld_gu, int inter,
                                                          uint16_t* __restrict__ out, int64_t ld_out) {
  const int64_t row = blockIdx.y;
  const int c = ((int)blockIdx.x * 256 + (int)threadIdx.x) * 8;
  if (c >= inter) return;
  float g[8], u[8], o[8];
  unpack8(ld16(gu + row * ld_gu + c), g);
  unpack8(ld16(gu + row * ld_gu + inter + c), u);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float sg = bf16r(g[e] / (1.0f + expf(-g[e])));
    o[e] = sg * u[e];
  }
  *(u32x4*)(out + row * ld_out + c) = pack8(o);
}

// Embedding gather: out[r, :] = table[token[r], :].
__global__ __launch_bounds__(256) void embed_kernel(const int64_t* __restrict__ tokens, const uint16_t* __restrict__ table,
                                                    int64_t ld_table, int vocab, uint16_t* __restrict__ out,
                                                    int64_t ld_out, int n) {
  const int64_t row = blockIdx.y;
  int64_t t = tokens[row];
  t = t < 0 ? 0 : (t >= vocab ? vocab - 1 : t);
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    out[row * ld_out + i] = table[t * ld_table + i];
}

// argmax, stage 1: each block reduces a contiguous range to (max, first index),
// in torch.argmax's order (step_core.h arg_better: NaN above every number).

__device__ __forceinline__ ArgBest wave_arg(ArgBest x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    ArgBest o;
    o.v = __shfl_xor(x.v, off, kWave);
    o.i = __shfl_xor(x.i, off, kWave);
    x = arg_better(x, o);
  }
  return x;
}

constexpr int kArgThreads = 256;

__device__ ArgBest block_arg(ArgBest x) {
  __shared__ float sv[kArgThreads / kWave];
  __shared__ int si[kArgThreads / kWave];
  x = wave_arg(x);
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) {
    sv[wave] = x.v;
    si[wave] = x.i;
  }
  __syncthreads();
  ArgBest r{sv[0], si[0]};
#pragma unroll
  for (int j = 1; j < kArgThreads / kWave; ++j) r = arg_better(r, ArgBest{sv[j], si[j]});
  return r;
}

__global__ __launch_bounds__(kArgThreads) void argmax_partial_kernel(const uint16_t* __restrict__ logits, int n,
                                                                     int per_block, float* __restrict__ pv,
                                                                     int* __restrict__ pi) {
  const int begin = blockIdx.x * per_block;
  const int end = min(n, begin + per_block);
  ArgBest best{-INFINITY, 0x7fffffff};
  for (int i = begin + threadIdx.x; i < end; i += kArgThreads) best = arg_better(best, ArgBest{bf16_to_f32(logits[i]), i});
  best = block_arg(best);
  if (threadIdx.x == 0) {
    pv[blockIdx.x] = best.v;
    pi[blockIdx.x] = best.i;
  }
}

__global__ __launch_bounds__(kArgThreads) void argmax_final_kernel(const float* __restrict__ pv,
                                                                   const int* __restrict__ pi, int parts,
                                                                   int64_t* __restrict__ token,
                                                                   int64_t* __restrict__ position) {
  ArgBest best{-INFINITY, 0x7fffffff};
  for (int j = threadIdx.x; j < parts; j += kArgThreads) best = arg_better(best, ArgBest{pv[j], pi[j]});
  best = block_arg(best);
  if (threadIdx.x == 0) {
    *token = best.i == 0x7fffffff ? 0 : best.i;  // no logits at all: token 0
    if (position) *position += 1;
  }
}

constexpr int kArgParts = 256;

// launch_reduce_add_rmsnorm's kernel: S split partials per element, every load of an element issued before its
// first addition (the reduce kernel's order: v0 + v1 + ... + v(S-1)).
template <int S, bool V8>
__global__ __launch_bounds__(kNormThreads) void reduce_add_rmsnorm_kernel(const float* __restrict__ part,
                                                                         const float* __restrict__ scale,
                                                                         uint16_t* __restrict__ x, int64_t ldx,
                                                                         const uint16_t* __restrict__ w,
                                                                         uint16_t* __restrict__ y, int64_t ldy, int M,
                                                                         int n, float eps) {
  __shared__ float red[kNormThreads / kWave];
  extern __shared__ float rowbuf[];  // n floats: the updated residual row
  const int64_t row = blockIdx.x;
  const int64_t mn = (int64_t)M * n;
  const float* pr = part + row * n;
  uint16_t* xr = x + row * ldx;
  float ss = 0.f;
  if (V8) {  // add_rmsnorm_v8_kernel's element order (8-element groups per thread)
    for (int g = threadIdx.x; g * 8 < n; g += kNormThreads) {
      float xv[8], r[8];
      unpack8(ld16(xr + g * 8), xv);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int i = g * 8 + e;
        float v[S];
#pragma unroll
        for (int sp = 0; sp < S; ++sp) v[sp] = pr[sp * mn + i];
        float acc = v[0];
#pragma unroll
        for (int sp = 1; sp < S; ++sp) acc += v[sp];
        const float o = bf16r(bf16r(acc) * scale[i]);
        r[e] = bf16r(xv[e] + o);
        rowbuf[i] = r[e];
        ss = fmaf(r[e], r[e], ss);
      }
      *(u32x4*)(xr + g * 8) = pack8(r);
    }
  } else {
    for (int i = threadIdx.x; i < n; i += kNormThreads) {
      float v[S];
#pragma unroll
      for (int sp = 0; sp < S; ++sp) v[sp] = pr[sp * mn + i];
      float acc = v[0];
#pragma unroll
      for (int sp = 1; sp < S; ++sp) acc += v[sp];
      const float o = bf16r(bf16r(acc) * scale[i]);  // the GEMM's output element, as the reduce kernel rounds it
      const float r = bf16r(bf16_to_f32(xr[i]) + o);
      xr[i] = f32_to_bf16(r);
      rowbuf[i] = r;
      ss = fmaf(r, r, ss);
    }
  }
  const float total = block_sum_256(ss, red);
  const float inv = rsqrtf(total / (float)n + eps);
  uint16_t* yr = y + row * ldy;
  if (V8) {
    for (int g = threadIdx.x; g * 8 < n; g += kNormThreads) {
      float wv[8], o[8];
      unpack8(ld16(w + g * 8), wv);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = wv[e] * bf16r(rowbuf[g * 8 + e] * inv);
      *(u32x4*)(yr + g * 8) = pack8(o);
    }
  } else {
    for (int i = threadIdx.x; i < n; i += kNormThreads)
      yr[i] = f32_to_bf16(bf16_to_f32(w[i]) * bf16r(rowbuf[i] * inv));
  }
}

constexpr int kReduceNormMaxSplits = 16;

bool aligned16p(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Whether a norm's rows take the vector form: whole 8-element groups, 16-byte aligned rows.
bool v8_row(const void* x, int64_t ldx, const void* w, const void* y, int64_t ldy, int n, const void* a = nullptr,
            int64_t lda = 0) {
  return n % 8 == 0 && ldx % 8 == 0 && ldy % 8 == 0 && lda % 8 == 0 && aligned16p(x) && aligned16p(w) &&
         aligned16p(y) && aligned16p(a);
}

template <int S>
int launch_reduce_norm(int splits, dim3 grid, size_t lds, hipStream_t st, const float* part, const float* scale,
                       uint16_t* x, int64_t ldx, const uint16_t* w, uint16_t* y, int64_t ldy, int M, int n,
                       float eps) {
  if constexpr (S < 2) {
    return EGPT_ERR_UNSUPPORTED;
  } else {
    if (splits != S)
      return launch_reduce_norm<S - 1>(splits, grid, lds, st, part, scale, x, ldx, w, y, ldy, M, n, eps);
    if (v8_row(x, ldx, w, y, ldy, n))
      hipLaunchKernelGGL((reduce_add_rmsnorm_kernel<S, true>), grid, dim3(kNormThreads), lds, st, part, scale, x, ldx,
                         w, y, ldy, M, n, eps);
    else
      hipLaunchKernelGGL((reduce_add_rmsnorm_kernel<S, false>), grid, dim3(kNormThreads), lds, st, part, scale, x,
                         ldx, w, y, ldy, M, n, eps);
    return EGPT_LAUNCH_STATUS();
  }
}

}  // namespace

int launch_reduce_add_rmsnorm(const float* part, int splits, const float* scale, void* resid, int64_t ld_resid,
                              const void* norm_w, void* y, int64_t ldy, int M, int N, float eps, hipStream_t st) {
  if (!part || !scale || !resid || !norm_w || !y || M < 1 || N < 1 || ld_resid < N || ldy < N)
    return EGPT_ERR_INVALID;
  if (splits < 2 || splits > kReduceNormMaxSplits || (size_t)N * sizeof(float) > 64 * 1024)
    return EGPT_ERR_UNSUPPORTED;
  return launch_reduce_norm<kReduceNormMaxSplits>(splits, dim3(M), (size_t)N * sizeof(float), st, part, scale,
                                                  (uint16_t*)resid, ld_resid, (const uint16_t*)norm_w, (uint16_t*)y,
                                                  ldy, M, N, eps);
}

namespace {

template <int D, int S>
int launch_rqk(int splits, dim3 grid, hipStream_t st, const float* part, const float* scale, const QkRope& a) {
  if constexpr (S < 2) {
    return EGPT_ERR_UNSUPPORTED;
  } else {
    if (splits != S) return launch_rqk<D, S - 1>(splits, grid, st, part, scale, a);
    hipLaunchKernelGGL((reduce_qk_norm_rope_v8_kernel<D, S>), grid, dim3(256), 0, st, part, scale, a);
    return EGPT_LAUNCH_STATUS();
  }
}

}  // namespace

int check_reduce_qk_norm_rope(int splits, const int64_t* positions, const void* q_norm_w, const void* k_norm_w,
                              const void* cos_t, const void* sin_t, const void* q_out, int64_t ld_q,
                              const void* k_cache, const void* v_cache, int64_t cache_head_stride,
                              int64_t cache_slot_stride, int rows, int Hq, int Hkv, int D, int cap) {
  if (!positions || !q_norm_w || !k_norm_w || !cos_t || !sin_t || !q_out || !k_cache || !v_cache)
    return EGPT_ERR_INVALID;
  if (rows < 1 || Hq < 1 || Hkv < 1 || cap < 1 || ld_q < (int64_t)Hq * D) return EGPT_ERR_INVALID;
  if (splits < 2 || splits > kReduceNormMaxSplits || (D != 128 && D != 64 && D != 32)) return EGPT_ERR_UNSUPPORTED;
  if (ld_q % 8 || cache_head_stride % 8 || cache_slot_stride % 8 || !aligned16p(q_out) || !aligned16p(k_cache) ||
      !aligned16p(v_cache) || !aligned16p(q_norm_w) || !aligned16p(k_norm_w) || !aligned16p(cos_t) ||
      !aligned16p(sin_t))
    return EGPT_ERR_UNSUPPORTED;
  return EGPT_OK;
}

int launch_reduce_qk_norm_rope(const float* part, int splits, const float* scale, const int64_t* positions,
                               const void* q_norm_w, const void* k_norm_w, const void* cos_t, const void* sin_t,
                               void* q_out, int64_t ld_q, void* k_cache, void* v_cache, int64_t cache_head_stride,
                               int64_t cache_slot_stride, int rows, int Hq, int Hkv, int D, int cap, float eps,
                               hipStream_t st) {
  const int c = check_reduce_qk_norm_rope(splits, positions, q_norm_w, k_norm_w, cos_t, sin_t, q_out, ld_q, k_cache,
                                          v_cache, cache_head_stride, cache_slot_stride, rows, Hq, Hkv, D, cap);
  if (c != EGPT_OK) return c;
  if (!part || !scale || (uintptr_t)part % 16) return EGPT_ERR_INVALID;
  const QkRope a{positions, (const uint16_t*)q_norm_w, (const uint16_t*)k_norm_w, (const uint16_t*)cos_t,
                 (const uint16_t*)sin_t, (uint16_t*)q_out, ld_q, (uint16_t*)k_cache, (uint16_t*)v_cache,
                 cache_head_stride, cache_slot_stride, rows, Hq, Hkv, cap, eps};
  const int64_t jobs = (int64_t)rows * (Hq + 2 * Hkv);
  const int per_block = 256 / (D / 8);
  const dim3 grid((unsigned)((jobs + per_block - 1) / per_block));
  if (D == 128) return launch_rqk<128, kReduceNormMaxSplits>(splits, grid, st, part, scale, a);
  if (D == 64) return launch_rqk<64, kReduceNormMaxSplits>(splits, grid, st, part, scale, a);
  return launch_rqk<32, kReduceNormMaxSplits>(splits, grid, st, part, scale, a);
}

}  // namespace egpt

using namespace egpt;

extern "C" int egpt_rmsnorm(const void* x, int64_t ldx, const void* w, void* y, int64_t ldy, int rows, int n, float eps,
                            hipStream_t stream) {
  if (!x || !w || !y || rows < 0 || n < 1 || ldx < n || ldy < n) return EGPT_ERR_INVALID;
  if ((size_t)n * sizeof(float) > 64 * 1024) return EGPT_ERR_UNSUPPORTED;
  if (rows == 0) return EGPT_OK;
  hipLaunchKernelGGL(v8_row(x, ldx, w, y, ldy, n) ? add_rmsnorm_v8_kernel : add_rmsnorm_kernel, dim3(rows),
                     dim3(kNormThreads), n * sizeof(float), stream, (uint16_t*)x, ldx, (const uint16_t*)nullptr, 0,
                     (const uint16_t*)w, (uint16_t*)y, ldy, n, eps);
  return EGPT_LAUNCH_STATUS();
}

extern "C" int egpt_add_rmsnorm(void* x, int64_t ldx, const void* a, int64_t lda, const void* w, void* y, int64_t ldy,
                                int rows, int n, float eps, hipStream_t stream) {
  if (!x || !a || !w || !y || rows < 0 || n < 1 || ldx < n || lda < n || ldy < n) return EGPT_ERR_INVALID;
  if ((size_t)n * sizeof(float) > 64 * 1024) return EGPT_ERR_UNSUPPORTED;
  if (rows == 0) return EGPT_OK;
  hipLaunchKernelGGL(v8_row(x, ldx, w, y, ldy, n, a, lda) ? add_rmsnorm_v8_kernel : add_rmsnorm_kernel, dim3(rows),
                     dim3(kNormThreads), n * sizeof(float), stream, (uint16_t*)x, ldx, (const uint16_t*)a, lda,
                     (const uint16_t*)w, (uint16_t*)y, ldy, n, eps);
  return EGPT_LAUNCH_STATUS();
}

extern "C" int egpt_qk_norm_rope(const void* qkv, int64_t ld_qkv, const int64_t* positions, const void* q_norm_w,
                                 const void* k_norm_w, const void* cos_t, const void* sin_t, void* q_out, int64_t ld_q,
                                 void* k_cache, void* v_cache, int64_t cache_head_stride, int64_t cache_slot_stride,
                                 int rows, int Hq, int Hkv, int D, int cap, float eps, hipStream_t stream) {
  if (!qkv || !positions || !q_norm_w || !k_norm_w || !cos_t || !sin_t || !q_out || !k_cache || !v_cache)
    return EGPT_ERR_INVALID;
  if (rows < 0 || Hq < 1 || Hkv < 1 || cap < 1 || ld_qkv < (int64_t)(Hq + 2 * Hkv) * D || ld_q < (int64_t)Hq * D)
    return EGPT_ERR_INVALID;
  if (rows == 0) return EGPT_OK;
  const int64_t jobs = (int64_t)rows * (Hq + 2 * Hkv);
  const bool v8 = ld_qkv % 8 == 0 && ld_q % 8 == 0 && cache_head_stride % 8 == 0 && cache_slot_stride % 8 == 0 &&
                  aligned16p(qkv) && aligned16p(q_out) && aligned16p(k_cache) && aligned16p(v_cache) &&
                  aligned16p(q_norm_w) && aligned16p(k_norm_w) && aligned16p(cos_t) && aligned16p(sin_t);
  if (v8 && (D == 128 || D == 64 || D == 32)) {
    const int per_block = 256 / (D / 8);  // (row, head) jobs per block
    const dim3 g8((unsigned)((jobs + per_block - 1) / per_block));
    const QkRope qa{positions, (const uint16_t*)q_norm_w, (const uint16_t*)k_norm_w, (const uint16_t*)cos_t,
                    (const uint16_t*)sin_t, (uint16_t*)q_out, ld_q, (uint16_t*)k_cache, (uint16_t*)v_cache,
                    cache_head_stride, cache_slot_stride, rows, Hq, Hkv, cap, eps};
#define EGPT_QKV8(DD) \
  hipLaunchKernelGGL((qk_norm_rope_v8_kernel<DD>), g8, dim3(256), 0, stream, (const uint16_t*)qkv, ld_qkv, qa)
    if (D == 128) EGPT_QKV8(128);
    else if (D == 64) EGPT_QKV8(64);
    else EGPT_QKV8(32);
#undef EGPT_QKV8
    return EGPT_LAUNCH_STATUS();
  }
  dim3 grid((unsigned)((jobs + 3) / 4));
  if (D == 128) {
    hipLaunchKernelGGL((qk_norm_rope_kernel<128>), grid, dim3(256), 0, stream, (const uint16_t*)qkv, ld_qkv, positions,
                       (const uint16_t*)q_norm_w, (const uint16_t*)k_norm_w, (const uint16_t*)cos_t,
                       (const uint16_t*)sin_t, (uint16_t*)q_out, ld_q, (uint16_t*)k_cache, (uint16_t*)v_cache,
                       cache_head_stride, cache_slot_stride, rows, Hq, Hkv, cap, eps);
  } else if (D == 64) {
    hipLaunchKernelGGL((qk_norm_rope_kernel<64>), grid, dim3(256), 0, stream, (const uint16_t*)qkv, ld_qkv, positions,
                       (const uint16_t*)q_norm_w, (const uint16_t*)k_norm_w, (const uint16_t*)cos_t,
                       (const uint16_t*)sin_t, (uint16_t*)q_out, ld_q, (uint16_t*)k_cache, (uint16_t*)v_cache,
                       cache_head_stride, cache_slot_stride, rows, Hq, Hkv, cap, eps);
  } else if (D == 32) {
    hipLaunchKernelGGL((qk_norm_rope_kernel<32>), grid, dim3(256), 0, stream, (const uint16_t*)qkv, ld_qkv, positions,
                       (const uint16_t*)q_norm_w, (const uint16_t*)k_norm_w, (const uint16_t*)cos_t,
                       (const uint16_t*)sin_t, (uint16_t*)q_out, ld_q, (uint16_t*)k_cache, (uint16_t*)v_cache,
                       cache_head_stride, cache_slot_stride, rows, Hq, Hkv, cap, eps);
  } else {
    return EGPT_ERR_UNSUPPORTED;
  }
  return EGPT_LAUNCH_STATUS();
}

extern "C" int egpt_silu_mul(const void* gu, int64_t ld_gu, int inter, void* out, int64_t ld_out, int rows,
                             hipStream_t stream) {
  if (!gu || !out || inter < 1 || rows < 0 || ld_gu < 2 * (int64_t)inter || ld_out < inter) return EGPT_ERR_INVALID;
  if (rows == 0) return EGPT_OK;
  if (inter % 8 == 0 && ld_gu % 8 == 0 && ld_out % 8 == 0 && aligned16p(gu) && aligned16p(out) && rows <= 65535) {
    hipLaunchKernelGGL(silu_mul_v8_kernel, dim3((unsigned)((inter / 8 + 255) / 256), (unsigned)rows), dim3(256), 0,
                       stream, (const uint16_t*)gu, ld_gu, inter, (uint16_t*)out, ld_out);
    return EGPT_LAUNCH_STATUS();
  }
  const int64_t total = (int64_t)rows * inter;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream,
                     (const uint16_t*)gu, ld_gu, inter, (uint16_t*)out, ld_out, rows);
  return EGPT_LAUNCH_STATUS();
}

extern "C" int egpt_embed(const int64_t* tokens, int rows, const void* table, int64_t ld_table, int vocab, void* out,
                          int64_t ld_out, int n, hipStream_t stream) {
  if (!tokens || !table || !out || rows < 0 || vocab < 1 || n < 1 || ld_table < n || ld_out < n)
    return EGPT_ERR_INVALID;
  if (rows == 0) return EGPT_OK;
  dim3 grid((unsigned)((n + 255) / 256 < 8 ? (n + 255) / 256 : 8), (unsigned)rows);
  hipLaunchKernelGGL(embed_kernel, grid, dim3(256), 0, stream, tokens, (const uint16_t*)table, ld_table, vocab,
                     (uint16_t*)out, ld_out, n);
  return EGPT_LAUNCH_STATUS();
}

extern "C" int egpt_argmax_workspace(int n, size_t* bytes) {
  if (!bytes || n < 1) return EGPT_ERR_INVALID;
  *bytes = (size_t)kArgParts * (sizeof(float) + sizeof(int));
  return EGPT_OK;
}

extern "C" int egpt_argmax(const void* logits, int n, void* workspace, size_t workspace_bytes, int64_t* token,
                           int64_t* position, hipStream_t stream) {
  if (!logits || !token || n < 1) return EGPT_ERR_INVALID;
  size_t need = 0;
  egpt_argmax_workspace(n, &need);
  if (!workspace || workspace_bytes < need || (uintptr_t)workspace % 16) return EGPT_ERR_WORKSPACE;
  const int per_block = (n + kArgParts - 1) / kArgParts;
  const int parts = (n + per_block - 1) / per_block;
  float* pv = (float*)workspace;
  int* pi = (int*)((char*)workspace + kArgParts * sizeof(float));
  hipLaunchKernelGGL(argmax_partial_kernel, dim3(parts), dim3(kArgThreads), 0, stream, (const uint16_t*)logits, n,
                     per_block, pv, pi);
  if (hipGetLastError() != hipSuccess) return EGPT_ERR_LAUNCH;
  hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kArgThreads), 0, stream, pv, pi, parts, token, position);
  return EGPT_LAUNCH_STATUS();
}
