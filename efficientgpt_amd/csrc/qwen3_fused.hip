// Fused batch-1 Qwen3 decode step on gfx950 (MI355X): six launches per layer
// instead of ten, and two for the head, so the step is bound by weight streaming
// rather than by kernel count.
//
// Per layer (x is the bf16 residual stream, one row):
//   1. qkv  = int8 GEMV( RMSNorm(x; input_layernorm) )               [norm in the GEMV prologue]
//   2. attn = split-K GQA attention over slots 0..p of q_norm/k_norm + RoPE
//             of qkv, which also writes K/V slot p; then a small kernel merges
//             the partial softmax states
//   3. x    = bf16( x + int8 GEMV(attn; o_proj) )                    [residual in the epilogue]
//   4. act  = SwiGLU( int8 GEMV( RMSNorm(x; post_attention_layernorm) ; gate|up ) )
//   5. x    = bf16( x + int8 GEMV(act; down_proj) )
// Head: logits = int8 GEMV( RMSNorm(x; norm) ; lm_head ) with per-block maxima,
//       then one block reduces them: argmax -> token, position += 1.
// Layer 0 reads its input row straight from the embedding table at the device
// token, so the embedding gather needs no launch of its own.
//
// The rounding of every op is transformers' bf16 Qwen3 (models/qwen3/modeling_qwen3.py):
// RMSNorm bf16(w * bf16(x * rsqrt(mean x^2 + eps))) (:30-46), the residual adds
// bf16(x + y) (:285-322), RoPE bf16(bf16(x cos) + bf16(rotate_half(x) sin))
// (:139-166), SwiGLU bf16(bf16(silu(g)) * u) (:49-62); every int8 linear is the
// reference's decode contract bf16(s * fp32 sum) (research/realmodel/int8_linear.py:26-38).
// The step replaces the reference's captured graph step
// (research/realmodel/fast_decode.py:45-49: compiled forward + argmax + position).
//
// No block ever waits for, or signals, another block of the same launch: every
// cross-block reduction (split-K combine, argmax) is a separate launch, ordered
// by the kernel boundary. (A last-block-done hand-off inside the lm_head launch
// needs a device-scope fence per block; 9.5k blocks of L2 write-back/invalidate
// made that launch 30x slower than the stream itself.)
#include "attn_core.h"

namespace egpt {
namespace {

constexpr int kFWaves = 4;
constexpr int kFThreads = kFWaves * kWave;
constexpr int kFChunk = kWave * 16;  // int8 weights covered by one 16-byte load per lane
constexpr int kMaxChunks = 12;       // K <= 12288

enum { kEpiStore = 0, kEpiResid = 1, kEpiSwiGLU = 2, kEpiArgmax = 3 };

__device__ __forceinline__ float bf16r(float f) { return bf16_to_f32(f32_to_bf16(f)); }

struct FusedGemv {
  const uint16_t* x;       // activation row, or a table when x_token is set
  const int64_t* x_token;  // device id selecting row x + token * x_ld (the embedding gather)
  int64_t x_ld;
  int x_rows;
  const uint16_t* norm_w;  // RMSNorm weight [K] (NORM kernels)
  float eps;
  const int8_t* w;         // int8 [rows, K] row-major; SwiGLU: gate rows [0, N) then up rows [N, 2N)
  int64_t ldw;
  const float* scale;      // fp32 per row
  int N;                   // output features
  int K;
  uint16_t* y;             // output row (Argmax: the logits, may be null)
  const uint16_t* resid;   // Resid: residual row, or a table when resid_token is set
  const int64_t* resid_token;
  int64_t resid_ld;
  float* part_v;           // Argmax: per-block maxima (value, first index)
  int* part_i;
};

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

// larger value wins; equal values: the smaller index (torch.argmax's first maximum)
__device__ __forceinline__ ArgBest arg_better(ArgBest a, ArgBest b) {
  return (b.v > a.v || (b.v == a.v && b.i < a.i)) ? b : a;
}

__device__ __forceinline__ ArgBest block_argbest(ArgBest x) {
  __shared__ float sv[kFWaves];
  __shared__ int si[kFWaves];
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
  __syncthreads();
  ArgBest r{sv[0], si[0]};
#pragma unroll
  for (int j = 1; j < kFWaves; ++j) r = arg_better(r, ArgBest{sv[j], si[j]});
  __syncthreads();
  return r;
}

__device__ __forceinline__ const uint16_t* token_row(const uint16_t* base, const int64_t* token, int64_t ld,
                                                     int rows) {
  if (!token) return base;
  int64_t t = *token;
  t = t < 0 ? 0 : (t >= rows ? rows - 1 : t);
  return base + t * ld;
}

// One int8 GEMV of a single activation row with a fused prologue / epilogue.
// A block is 4 wavefronts; a wavefront owns RH output features (R weight rows:
// SwiGLU pairs each gate row with its up row) and streams them with 16-byte
// loads, all NCH chunks of all R rows issued before any arithmetic. With NORM,
// each wavefront reduces mean(x^2) over its own copy of the row (every lane
// holds 16 * NCH elements, which together tile the row once).
template <int R, int NCH, int EPI, bool NORM>
__global__ __launch_bounds__(kFThreads) void fused_gemv_kernel(const FusedGemv a) {
  constexpr int RH = EPI == kEpiSwiGLU ? R / 2 : R;
  static_assert(EPI != kEpiSwiGLU || R % 2 == 0, "SwiGLU pairs rows");
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t f0 = ((int64_t)blockIdx.x * kFWaves + wave) * RH;
  const bool active = f0 < a.N;

  const int8_t* wrow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t f = min(f0 + (r % RH), (int64_t)a.N - 1);
    wrow[r] = a.w + ((EPI == kEpiSwiGLU && r >= RH) ? f + a.N : f) * a.ldw;
  }
  // Weights first: they do not depend on the activation.
  u32x4 wv[NCH][R];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int k = c * kFChunk + lane * 16;
    const bool kin = k < a.K;
#pragma unroll
    for (int r = 0; r < R; ++r) wv[c][r] = kin ? ld16_stream(wrow[r] + k) : u32x4{0u, 0u, 0u, 0u};
  }

  const uint16_t* xr = token_row(a.x, a.x_token, a.x_ld, a.x_rows);
  float xf[NCH][16];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int k = c * kFChunk + lane * 16;
    if (k < a.K) {
      unpack_bf16x16(ld16(xr + k), ld16(xr + k + 8), xf[c]);
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) xf[c][e] = 0.f;
    }
  }
  if constexpr (NORM) {
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int e = 0; e < 16; ++e) ss = fmaf(xf[c][e], xf[c][e], ss);
    const float inv = rsqrtf(wave_sum(ss) / (float)a.K + a.eps);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int k = c * kFChunk + lane * 16;
      if (k < a.K) {
        float nw[16];
        unpack_bf16x16(ld16(a.norm_w + k), ld16(a.norm_w + k + 8), nw);
#pragma unroll
        for (int e = 0; e < 16; ++e) xf[c][e] = bf16r(nw[e] * bf16r(xf[c][e] * inv));
      }
    }
  }

  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  float sx = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    float t = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) t += xf[c][e];
    sx += t;
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = dot16_biased(wv[c][r], xf[c], acc[r]);
  }

  // Row totals (wave-uniform); lane j < RH keeps feature f0 + j.
  float mine = 0.f, mine_up = 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float v = wave_sum(acc[r] - 128.f * sx);
    if (r < RH) {
      if (lane == r) mine = v;
    } else {
      if (lane == r - RH) mine_up = v;
    }
  }
  const int64_t f = f0 + lane;
  const bool own = active && lane < RH && f < a.N;

  if constexpr (EPI == kEpiStore) {
    if (own) a.y[f] = f32_to_bf16(mine * a.scale[f]);
  } else if constexpr (EPI == kEpiResid) {
    if (own) {
      const float o = bf16r(mine * a.scale[f]);
      const uint16_t* rr = token_row(a.resid, a.resid_token, a.resid_ld, a.x_rows);
      a.y[f] = f32_to_bf16(bf16_to_f32(rr[f]) + o);
    }
  } else if constexpr (EPI == kEpiSwiGLU) {
    if (own) {
      const float g = bf16r(mine * a.scale[f]);
      const float u = bf16r(mine_up * a.scale[a.N + f]);
      const float sg = bf16r(g / (1.0f + expf(-g)));
      a.y[f] = f32_to_bf16(sg * u);
    }
  } else {  // per-block maximum of the logits
    ArgBest b{-INFINITY, 0x7fffffff};
    if (own) {
      const uint16_t lg = f32_to_bf16(mine * a.scale[f]);
      if (a.y) a.y[f] = lg;
      b = ArgBest{bf16_to_f32(lg), (int)f};
    }
    b = block_argbest(b);
    if (threadIdx.x == 0) {
      a.part_v[blockIdx.x] = b.v;
      a.part_i[blockIdx.x] = b.i;
    }
  }
}

// Greedy pick over the per-block maxima: token = first index of the largest
// logit (torch.argmax), position += 1. One block.
__global__ __launch_bounds__(kFThreads) void argmax_final_kernel(const float* __restrict__ part_v,
                                                                 const int* __restrict__ part_i, int parts,
                                                                 int64_t* __restrict__ token,
                                                                 int64_t* __restrict__ position) {
  ArgBest best{-INFINITY, 0x7fffffff};
  for (int j = threadIdx.x; j < parts; j += kFThreads) best = arg_better(best, ArgBest{part_v[j], part_i[j]});
  best = block_argbest(best);
  if (threadIdx.x == 0) {
    *token = best.i == 0x7fffffff ? 0 : best.i;  // all-NaN logits: token 0
    *position += 1;
  }
}

struct AttnStep {
  const uint16_t* qkv;  // raw projections [(Hq + 2 Hkv) * D]
  const uint16_t* q_norm_w;
  const uint16_t* k_norm_w;
  const uint16_t* cos_t;  // [cap, D]
  const uint16_t* sin_t;
  const int64_t* position;
  uint16_t* k_cache;  // [Hkv, cap, D]
  uint16_t* v_cache;
  int64_t c_sh, c_sn;
  float* ws_m;
  float* ws_l;
  float* ws_acc;
  int Hkv, cap, nsplit;
  float eps, scale;
};

// Head-wise RMSNorm + RoPE of one head held by an LPS-lane group (EPL elements
// per lane, element d0 + e). rotate_half pairs element i with i +- D/2, which
// sits in lane (sub ^ LPS/2) at the same e.
template <int D, int EPL, int LPS>
__device__ __forceinline__ void head_norm_rope(const uint16_t* src, const uint16_t* nw, const uint16_t* cr,
                                               const uint16_t* sr, int d0, float eps, float (&out)[EPL]) {
  float xv[EPL], w[EPL], cs[EPL], sn[EPL];
  Elem<__bf16>::unpack(ld16(src + d0), xv);
  Elem<__bf16>::unpack(ld16(nw + d0), w);
  Elem<__bf16>::unpack(ld16(cr + d0), cs);
  Elem<__bf16>::unpack(ld16(sr + d0), sn);
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
    const float p = __shfl_xor(nv[e], LPS / 2, kWave);
    const float rh = lower ? -p : p;
    out[e] = bf16r(bf16r(nv[e] * cs[e]) + bf16r(rh * sn[e]));
  }
}

// Attention partials of one decode step: block (kv head, split). Query and new
// key are normalised and rotated in the prologue (each block redoes its G query
// heads: 2 x 128 elements); the block whose split holds slot p writes the new K
// and V rows there before reading its range, and no other block touches slot p.
template <int D, int G>
__global__ __launch_bounds__(kAttnThreads) void attn_step_kernel(const AttnStep a) {
  constexpr int EPL = AttnGeom<__bf16, D>::EPL;
  constexpr int LPS = AttnGeom<__bf16, D>::LPS;
  const int tid = threadIdx.x;
  const int d0 = (tid % LPS) * EPL;
  const int hk = blockIdx.x;
  const int split = blockIdx.y;
  const int Hq = a.Hkv * G;

  int64_t pos = *a.position;
  pos = pos < 0 ? 0 : (pos >= a.cap ? a.cap - 1 : pos);
  const int64_t len = pos + 1;
  int64_t start, end;
  attn_split_range(len, a.nsplit, split, start, end);
  const int64_t chunk = (len + a.nsplit - 1) / a.nsplit;
  const bool owner = split == (int)((len - 1) / chunk);

  const uint16_t* cr = a.cos_t + pos * D;
  const uint16_t* sr = a.sin_t + pos * D;
  float qf[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) head_norm_rope<D, EPL, LPS>(a.qkv + (int64_t)(hk * G + g) * D, a.q_norm_w, cr, sr, d0, a.eps, qf[g]);

  uint16_t* kc = a.k_cache + (int64_t)hk * a.c_sh;
  uint16_t* vc = a.v_cache + (int64_t)hk * a.c_sh;
  if (owner) {  // block-uniform
    float kn[EPL];
    head_norm_rope<D, EPL, LPS>(a.qkv + (int64_t)(Hq + hk) * D, a.k_norm_w, cr, sr, d0, a.eps, kn);
    if (tid < LPS) {
      uint32_t packed[EPL / 2];
#pragma unroll
      for (int e = 0; e < EPL / 2; ++e)
        packed[e] = (uint32_t)f32_to_bf16(kn[2 * e]) | ((uint32_t)f32_to_bf16(kn[2 * e + 1]) << 16);
      *(u32x4*)(kc + pos * a.c_sn + d0) = u32x4{packed[0], packed[1], packed[2], packed[3]};
      *(u32x4*)(vc + pos * a.c_sn + d0) = ld16(a.qkv + (int64_t)(Hq + a.Hkv + hk) * D + d0);
    }
    __syncthreads();
  }

  attn_partial<__bf16, D, G>(qf, (const __bf16*)kc, a.c_sn, (const __bf16*)vc, a.c_sn, start, end, a.scale, a.ws_m,
                             a.ws_l, a.ws_acc, (int64_t)(hk * G) * a.nsplit + split, a.nsplit);
}

// Merge of the split partials: one block per query head, one thread per element.
template <int D>
__global__ __launch_bounds__(D) void attn_merge_kernel(const float* __restrict__ ws_m, const float* __restrict__ ws_l,
                                                       const float* __restrict__ ws_acc, uint16_t* __restrict__ out,
                                                       int nsplit) {
  const int h = blockIdx.x;
  const int d = threadIdx.x;
  out[(int64_t)h * D + d] = f32_to_bf16(attn_combine_one(ws_m + (int64_t)h * nsplit, ws_l + (int64_t)h * nsplit,
                                                         ws_acc + (int64_t)h * nsplit * D, nsplit, D, d));
}

// ------------------------------------------------------------------ host side

int chunks_for(int K) {
  const int n = (K + kFChunk - 1) / kFChunk;
  if (n <= 4) return n < 1 ? 1 : n;
  if (n <= 6) return 6;
  if (n <= 8) return 8;
  return 12;
}

// Output features per wavefront: the largest of 4 / 2 / 1 that still gives the
// 256 CUs at least 256 blocks.
int features_per_wave(int64_t n, bool pairs) {
  const int hi = pairs ? 2 : 4;
  for (int rh = hi; rh > 1; rh /= 2)
    if ((n + (int64_t)kFWaves * rh - 1) / ((int64_t)kFWaves * rh) >= 256) return rh;
  return 1;
}

template <int EPI, bool NORM, int R>
int launch_r(const FusedGemv& a, int nch, unsigned blocks, hipStream_t st) {
  switch (nch) {
#define EGPT_CASE(C) \
  case C: hipLaunchKernelGGL((fused_gemv_kernel<R, C, EPI, NORM>), dim3(blocks), dim3(kFThreads), 0, st, a); break;
    EGPT_CASE(1) EGPT_CASE(2) EGPT_CASE(3) EGPT_CASE(4) EGPT_CASE(6) EGPT_CASE(8) EGPT_CASE(12)
#undef EGPT_CASE
    default: return EGPT_ERR_UNSUPPORTED;
  }
  return EGPT_LAUNCH_STATUS();
}

template <int EPI, bool NORM>
int launch_fused(const FusedGemv& a, hipStream_t st) {
  const bool pairs = EPI == kEpiSwiGLU;
  const int rh = features_per_wave(a.N, pairs);
  const unsigned blocks = (unsigned)((a.N + (int64_t)kFWaves * rh - 1) / ((int64_t)kFWaves * rh));
  const int nch = chunks_for(a.K);
  if constexpr (EPI == kEpiSwiGLU) {
    return rh >= 2 ? launch_r<EPI, NORM, 4>(a, nch, blocks, st) : launch_r<EPI, NORM, 2>(a, nch, blocks, st);
  } else {
    if (rh >= 4) return launch_r<EPI, NORM, 4>(a, nch, blocks, st);
    if (rh >= 2) return launch_r<EPI, NORM, 2>(a, nch, blocks, st);
    return launch_r<EPI, NORM, 1>(a, nch, blocks, st);
  }
}

unsigned head_blocks(int vocab) {
  const int rh = features_per_wave(vocab, false);
  return (unsigned)((vocab + (int64_t)kFWaves * rh - 1) / ((int64_t)kFWaves * rh));
}

struct StepLayout {
  size_t ml, acc, part_v, part_i, total;
};

StepLayout step_layout(const egpt_qwen3_step* s) {
  auto up = [](size_t b) { return (b + 255) / 256 * 256; };
  StepLayout L;
  const size_t rows = (size_t)s->heads * (size_t)s->nsplit;
  L.ml = up(rows * sizeof(float));
  L.acc = up(rows * (size_t)s->head_dim * sizeof(float));
  const size_t hb = head_blocks(s->vocab);
  L.part_v = up(hb * sizeof(float));
  L.part_i = up(hb * sizeof(int));
  L.total = 2 * L.ml + L.acc + L.part_v + L.part_i;
  return L;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_step(const egpt_qwen3_step* s) {
  if (!s || !s->layer || !s->embed || !s->final_norm || !s->head_w || !s->head_s || !s->rope_cos || !s->rope_sin ||
      !s->token || !s->position || !s->x || !s->qkv || !s->attn || !s->act)
    return EGPT_ERR_INVALID;
  if (s->layers < 1 || s->hidden < 16 || s->inter < 16 || s->heads < 1 || s->kv_heads < 1 || s->vocab < 1 ||
      s->cap < 1 || s->nsplit < 1 || s->heads % s->kv_heads != 0)
    return EGPT_ERR_INVALID;
  if (s->hidden % 16 || s->inter % 16 || s->hidden > kMaxChunks * kFChunk || s->inter > kMaxChunks * kFChunk ||
      s->heads * s->head_dim > kMaxChunks * kFChunk)
    return EGPT_ERR_UNSUPPORTED;
  if (s->head_dim != 128 && s->head_dim != 64 && s->head_dim != 32) return EGPT_ERR_UNSUPPORTED;
  const int g = s->heads / s->kv_heads;
  if (g != 1 && g != 2 && g != 4 && g != 8) return EGPT_ERR_UNSUPPORTED;
  const void* ptrs[] = {s->embed, s->final_norm, s->head_w, s->rope_cos, s->rope_sin, s->x, s->qkv, s->attn, s->act};
  for (const void* p : ptrs)
    if (!aligned16(p)) return EGPT_ERR_INVALID;
  for (int i = 0; i < s->layers; ++i) {
    const egpt_qwen3_layer& L = s->layer[i];
    const void* lp[] = {L.qkv_w, L.qkv_s, L.o_w, L.o_s, L.gu_w, L.gu_s, L.down_w, L.down_s,
                        L.in_norm, L.post_norm, L.q_norm, L.k_norm, L.k_cache, L.v_cache};
    for (const void* p : lp)
      if (!p || !aligned16(p)) return EGPT_ERR_INVALID;
  }
  const StepLayout lay = step_layout(s);
  if (!s->workspace || s->workspace_bytes < lay.total || ((uintptr_t)s->workspace & 255u)) return EGPT_ERR_WORKSPACE;
  return EGPT_OK;
}

template <int D>
int launch_attn_step(const AttnStep& a, int G, uint16_t* out, hipStream_t st) {
  dim3 grid((unsigned)a.Hkv, (unsigned)a.nsplit);
  switch (G) {
    case 1: hipLaunchKernelGGL((attn_step_kernel<D, 1>), grid, dim3(kAttnThreads), 0, st, a); break;
    case 2: hipLaunchKernelGGL((attn_step_kernel<D, 2>), grid, dim3(kAttnThreads), 0, st, a); break;
    case 4: hipLaunchKernelGGL((attn_step_kernel<D, 4>), grid, dim3(kAttnThreads), 0, st, a); break;
    case 8: hipLaunchKernelGGL((attn_step_kernel<D, 8>), grid, dim3(kAttnThreads), 0, st, a); break;
    default: return EGPT_ERR_UNSUPPORTED;
  }
  if (hipGetLastError() != hipSuccess) return EGPT_ERR_LAUNCH;
  hipLaunchKernelGGL((attn_merge_kernel<D>), dim3((unsigned)(a.Hkv * G)), dim3(D), 0, st, a.ws_m, a.ws_l, a.ws_acc,
                     out, a.nsplit);
  return EGPT_LAUNCH_STATUS();
}

}  // namespace
}  // namespace egpt

using namespace egpt;

extern "C" int egpt_qwen3_step_workspace(const egpt_qwen3_step* s, size_t* bytes) {
  if (!s || !bytes || s->heads < 1 || s->kv_heads < 1 || s->nsplit < 1 || s->head_dim < 1 || s->vocab < 1)
    return EGPT_ERR_INVALID;
  *bytes = step_layout(s).total;
  return EGPT_OK;
}

extern "C" int egpt_qwen3_decode_step(const egpt_qwen3_step* s, hipStream_t stream) {
  int st = check_step(s);
  if (st != EGPT_OK) return st;
  const StepLayout lay = step_layout(s);
  char* ws = (char*)s->workspace;
  float* ws_m = (float*)ws;
  float* ws_l = (float*)(ws + lay.ml);
  float* ws_acc = (float*)(ws + 2 * lay.ml);
  float* part_v = (float*)(ws + 2 * lay.ml + lay.acc);
  int* part_i = (int*)(ws + 2 * lay.ml + lay.acc + lay.part_v);

  const int D = s->head_dim;
  const int G = s->heads / s->kv_heads;
  const int n_qkv = (s->heads + 2 * s->kv_heads) * D;
  const uint16_t* x = (const uint16_t*)s->x;
  for (int i = 0; i < s->layers; ++i) {
    const egpt_qwen3_layer& L = s->layer[i];
    const bool first = i == 0;
    // 1. RMSNorm + QKV
    FusedGemv g{};
    g.x = first ? (const uint16_t*)s->embed : x;
    g.x_token = first ? s->token : nullptr;
    g.x_ld = s->hidden;
    g.x_rows = s->vocab;
    g.norm_w = (const uint16_t*)L.in_norm;
    g.eps = s->eps;
    g.w = L.qkv_w;
    g.ldw = s->hidden;
    g.scale = L.qkv_s;
    g.N = n_qkv;
    g.K = s->hidden;
    g.y = (uint16_t*)s->qkv;
    if ((st = launch_fused<kEpiStore, true>(g, stream)) != EGPT_OK) return st;
    // 2. attention
    AttnStep at{};
    at.qkv = (const uint16_t*)s->qkv;
    at.q_norm_w = (const uint16_t*)L.q_norm;
    at.k_norm_w = (const uint16_t*)L.k_norm;
    at.cos_t = (const uint16_t*)s->rope_cos;
    at.sin_t = (const uint16_t*)s->rope_sin;
    at.position = s->position;
    at.k_cache = (uint16_t*)L.k_cache;
    at.v_cache = (uint16_t*)L.v_cache;
    at.c_sh = (int64_t)s->cap * D;
    at.c_sn = D;
    at.ws_m = ws_m;
    at.ws_l = ws_l;
    at.ws_acc = ws_acc;
    at.Hkv = s->kv_heads;
    at.cap = s->cap;
    at.nsplit = s->nsplit;
    at.eps = s->eps;
    at.scale = 1.0f / sqrtf((float)D);
    uint16_t* attn_out = (uint16_t*)s->attn;
    if (D == 128) st = launch_attn_step<128>(at, G, attn_out, stream);
    else if (D == 64) st = launch_attn_step<64>(at, G, attn_out, stream);
    else st = launch_attn_step<32>(at, G, attn_out, stream);
    if (st != EGPT_OK) return st;
    // 3. o_proj + residual (layer 0: the residual is the embedding row)
    FusedGemv o{};
    o.x = (const uint16_t*)s->attn;
    o.x_rows = s->vocab;
    o.w = L.o_w;
    o.ldw = (int64_t)s->heads * D;
    o.scale = L.o_s;
    o.N = s->hidden;
    o.K = s->heads * D;
    o.y = (uint16_t*)s->x;
    o.resid = first ? (const uint16_t*)s->embed : x;
    o.resid_token = first ? s->token : nullptr;
    o.resid_ld = s->hidden;
    if ((st = launch_fused<kEpiResid, false>(o, stream)) != EGPT_OK) return st;
    // 4. RMSNorm + gate/up + SwiGLU
    FusedGemv gu{};
    gu.x = x;
    gu.x_rows = 1;
    gu.norm_w = (const uint16_t*)L.post_norm;
    gu.eps = s->eps;
    gu.w = L.gu_w;
    gu.ldw = s->hidden;
    gu.scale = L.gu_s;
    gu.N = s->inter;
    gu.K = s->hidden;
    gu.y = (uint16_t*)s->act;
    if ((st = launch_fused<kEpiSwiGLU, true>(gu, stream)) != EGPT_OK) return st;
    // 5. down + residual
    FusedGemv dn{};
    dn.x = (const uint16_t*)s->act;
    dn.x_rows = 1;
    dn.w = L.down_w;
    dn.ldw = s->inter;
    dn.scale = L.down_s;
    dn.N = s->hidden;
    dn.K = s->inter;
    dn.y = (uint16_t*)s->x;
    dn.resid = x;
    if ((st = launch_fused<kEpiResid, false>(dn, stream)) != EGPT_OK) return st;
  }
  // head: final norm + lm_head + per-block maxima, then the greedy pick
  FusedGemv h{};
  h.x = x;
  h.x_rows = 1;
  h.norm_w = (const uint16_t*)s->final_norm;
  h.eps = s->eps;
  h.w = s->head_w;
  h.ldw = s->hidden;
  h.scale = s->head_s;
  h.N = s->vocab;
  h.K = s->hidden;
  h.y = (uint16_t*)s->logits;
  h.part_v = part_v;
  h.part_i = part_i;
  if ((st = launch_fused<kEpiArgmax, true>(h, stream)) != EGPT_OK) return st;
  hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kFThreads), 0, stream, part_v, part_i,
                     (int)head_blocks(s->vocab), s->token, s->position);
  return EGPT_LAUNCH_STATUS();
}
