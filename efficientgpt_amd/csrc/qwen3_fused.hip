// Fused batch-1 Qwen3 decode step on gfx950 (MI355X): five launches per layer
// (six past 16 attention splits) instead of ten, and two for the head.
//
// Per layer (x is the bf16 residual stream, one row):
//   1. qkv  = int8 GEMV( RMSNorm(x; input_layernorm) )               [norm in the GEMV prologue]
//   2. split-K GQA attention partials over slots 0..p of q_norm/k_norm + RoPE
//      of qkv, which also writes K/V slot p
//   3. x    = bf16( x + int8 GEMV(merge(partials); o_proj) )         [merge in the prologue,
//                                                                     residual in the epilogue]
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
#include "step_core.h"

namespace egpt {
namespace {

constexpr int kFWaves = 4;
constexpr int kFThreads = kFWaves * kWave;
constexpr int kFChunk = kWave * 16;  // int8 weights covered by one 16-byte load per lane
constexpr int kMaxChunks = 12;       // K <= 12288

enum { kEpiStore = 0, kEpiResid = 1, kEpiSwiGLU = 2, kEpiArgmax = 3 };

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
  int64_t y_ld;            // two-row GEMV: row stride of y (x rows are x_ld apart)
  const uint16_t* resid;   // Resid: residual row, or a table when resid_token is set
  const int64_t* resid_token;
  int64_t resid_ld;
  float* part_v;           // Argmax: per-block maxima (value, first index)
  int* part_i;
  const float* ws_m;       // merge sources: split-K partials of K / head_dim heads
  const float* ws_l;
  const float* ws_acc;
  int nsplit;
  int head_dim;
};

// Activation source of a fused GEMV: XSRC = kXRow reads a row; XSRC = 4, 8 or
// 16 merges the attention partials of at most that many splits.
enum { kXRow = 0 };

// Largest split count the o_proj prologue merges itself: all of a thread's
// partial loads are issued together, unrolled to the launch's bound.
constexpr int kMergeInGemvMaxSplits = 16;

// Unroll bound of the merge for a split count: the smallest of 4, 8, 16 that
// holds it, so the unrolled prologue is not much longer than the launch needs.
constexpr int merge_bound(int nsplit) { return nsplit <= 4 ? 4 : nsplit <= 8 ? 8 : 16; }

// Stage the activation row of a fused GEMV in LDS as bf16 (the value every
// wavefront of the block multiplies), once per block:
//   kXRow, NORM: h = bf16(w * bf16(x * rsqrt(mean x^2 + eps)))   (x from a row or table[token])
//   kXRow:       h = x
//   merge:       h = bf16(sum_s w_s acc_s / sum_s w_s l_s), w_s = exp(m_s - max m),
//                the split-K merge over K / head_dim heads, splits in order
// Each thread owns 8 consecutive elements per pass; elements from K up to the
// end of the last 1 KiB chunk are stored as 0. The loads are issued by
// stage_load() BEFORE the kernel's weight loads: vector loads retire in order,
// so the activation can then be used without waiting for the weight stream.
template <int NTHREADS, int NCH, int XSRC>
struct Staged {
  static constexpr int kPasses = (NCH * kFChunk + NTHREADS * 8 - 1) / (NTHREADS * 8);
  static constexpr int kSplits = XSRC == kXRow ? 1 : XSRC;
  u32x4 xv[kPasses], nv[kPasses];
  float mv[kSplits], lv[kSplits];
  u32x4 lo[kSplits], hi[kSplits];
};

template <int NTHREADS, int NCH, bool NORM, int XSRC>
__device__ __forceinline__ void stage_load(const FusedGemv& a, Staged<NTHREADS, NCH, XSRC>& st) {
  const int tid = threadIdx.x;
  const u32x4 z{0u, 0u, 0u, 0u};
  if constexpr (XSRC != kXRow) {
    // One pass: K <= NTHREADS * 8 is checked on the host. Threads past K load
    // nothing (whole wavefronts when K is a multiple of 512). Slots past the
    // split count are not masked here, since a select on the loaded values
    // would put a wait for the partials ahead of the weight loads:
    // stage_finish() gives them weight 0.
    const int k8 = tid * 8;
    if (k8 < a.K) {
      const int D = a.head_dim;
      const int h = k8 / D;
      const int d = k8 - h * D;
      const int last = a.nsplit - 1;
      const float* mrow = a.ws_m + (int64_t)h * a.nsplit;
      const float* lrow = a.ws_l + (int64_t)h * a.nsplit;
      const float* arow = a.ws_acc + (int64_t)h * a.nsplit * D + d;
#pragma unroll
      for (int sp = 0; sp < XSRC; ++sp) {
        int sl = sp;
        if constexpr (XSRC > 8) {
          // Re-read the last split past the count: no early exit, so the loop
          // unrolls and the partials stay in registers (an exit here left the
          // 16-slot arrays in scratch memory: the 1.7B step at 16 splits ran at
          // 885 instead of 1376 tok/s).
          sl = sp < last ? sp : last;
        } else {
          if (sp > last) break;  // wave-uniform: 1.5% faster than re-reading at 7 splits
        }
        st.mv[sp] = gload(mrow + sl);
        st.lv[sp] = gload(lrow + sl);
        st.lo[sp] = ld16(arow + (int64_t)sl * D);
        st.hi[sp] = ld16(arow + (int64_t)sl * D + 4);
      }
    }
  } else {
    const uint16_t* xr = token_row(a.x, a.x_token, a.x_ld, a.x_rows);
#pragma unroll
    for (int p = 0; p < Staged<NTHREADS, NCH, XSRC>::kPasses; ++p) {
      const int k8 = (p * NTHREADS + tid) * 8;
      const bool in = k8 < a.K;
      st.xv[p] = in ? ld16(xr + k8) : z;
      if constexpr (NORM) st.nv[p] = in ? ld16(a.norm_w + k8) : z;
    }
  }
}

template <int NTHREADS, int NCH, bool NORM, int XSRC>
__device__ __forceinline__ void stage_finish(const FusedGemv& a, const Staged<NTHREADS, NCH, XSRC>& st, uint16_t* hs) {
  const int tid = threadIdx.x;
  if constexpr (XSRC != kXRow) {
    const int k8 = tid * 8;
    if (k8 >= a.K) {
      if (k8 < NCH * kFChunk) *(u32x4*)(hs + k8) = u32x4{0u, 0u, 0u, 0u};
    } else {
      float mx = -INFINITY;
#pragma unroll
      for (int sp = 0; sp < XSRC; ++sp) mx = fmaxf(mx, sp < a.nsplit ? st.mv[sp] : -INFINITY);
      float acc8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      float ls = 0.f;
#pragma unroll
      for (int sp = 0; sp < XSRC; ++sp) {
        if (sp >= a.nsplit || st.mv[sp] == -INFINITY) continue;  // past the split count, or empty: weight 0
        const float wgt = exp2f((st.mv[sp] - mx) * kLog2e);
        const float v8[8] = {__uint_as_float(st.lo[sp].x), __uint_as_float(st.lo[sp].y),
                             __uint_as_float(st.lo[sp].z), __uint_as_float(st.lo[sp].w),
                             __uint_as_float(st.hi[sp].x), __uint_as_float(st.hi[sp].y),
                             __uint_as_float(st.hi[sp].z), __uint_as_float(st.hi[sp].w)};
#pragma unroll
        for (int e = 0; e < 8; ++e) acc8[e] = fmaf(wgt, v8[e], acc8[e]);
        ls = fmaf(wgt, st.lv[sp], ls);
      }
      uint32_t pk[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        pk[e] = (uint32_t)f32_to_bf16(acc8[2 * e] / ls) | ((uint32_t)f32_to_bf16(acc8[2 * e + 1] / ls) << 16);
      *(u32x4*)(hs + k8) = u32x4{pk[0], pk[1], pk[2], pk[3]};
    }
  } else if constexpr (NORM) {
    __shared__ float red[NTHREADS / kWave];
    float ss = 0.f;
#pragma unroll
    for (int p = 0; p < Staged<NTHREADS, NCH, XSRC>::kPasses; ++p) {
      float v[8];
      Elem<__bf16>::unpack(st.xv[p], v);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(v[e], v[e], ss);
    }
    ss = wave_sum(ss);
    if ((tid & (kWave - 1)) == 0) red[tid / kWave] = ss;
    lds_barrier();
    float total = 0.f;
#pragma unroll
    for (int j = 0; j < NTHREADS / kWave; ++j) total += red[j];
    const float inv = rsqrtf(total / (float)a.K + a.eps);
#pragma unroll
    for (int p = 0; p < Staged<NTHREADS, NCH, XSRC>::kPasses; ++p) {
      const int k8 = (p * NTHREADS + tid) * 8;
      if (k8 < NCH * kFChunk) {  // past K, x and w load as 0 and h is 0
        float v[8], w[8];
        Elem<__bf16>::unpack(st.xv[p], v);
        Elem<__bf16>::unpack(st.nv[p], w);
        uint32_t pk[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          pk[e] = (uint32_t)f32_to_bf16(w[2 * e] * bf16r(v[2 * e] * inv)) |
                  ((uint32_t)f32_to_bf16(w[2 * e + 1] * bf16r(v[2 * e + 1] * inv)) << 16);
        *(u32x4*)(hs + k8) = u32x4{pk[0], pk[1], pk[2], pk[3]};
      }
    }
  } else {
#pragma unroll
    for (int p = 0; p < Staged<NTHREADS, NCH, XSRC>::kPasses; ++p) {
      const int k8 = (p * NTHREADS + tid) * 8;
      if (k8 < NCH * kFChunk) *(u32x4*)(hs + k8) = st.xv[p];  // 0 past K
    }
  }
  lds_barrier();
}

// Weight rows of wave tile t: RH output features; SwiGLU: RH gate rows then the
// RH matching up rows. Rows past N are clamped to N - 1 and never stored.
template <int R, int EPI>
__device__ __forceinline__ void tile_rows(const FusedGemv& a, int64_t t, const int8_t* (&rows)[R]) {
  constexpr int RH = EPI == kEpiSwiGLU ? R / 2 : R;
  const int64_t f0 = t * RH;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t fr = min(f0 + (r % RH), (int64_t)a.N - 1);
    rows[r] = a.w + ((EPI == kEpiSwiGLU && r >= RH) ? fr + a.N : fr) * a.ldw;
  }
}

// Epilogue operands of the feature lane j < RH stores in tile t.
struct GemvEpi {
  float sc, sc_up, res;
};

template <int R, int EPI>
__device__ __forceinline__ GemvEpi tile_epi(const FusedGemv& a, int64_t t, int lane) {
  constexpr int RH = EPI == kEpiSwiGLU ? R / 2 : R;
  const int64_t fc = min(t * RH + (lane < RH ? lane : 0), (int64_t)a.N - 1);
  GemvEpi e;
  e.sc = a.scale[fc];
  e.sc_up = EPI == kEpiSwiGLU ? a.scale[a.N + fc] : 0.f;
  e.res = EPI == kEpiResid ? bf16_to_f32(token_row(a.resid, a.resid_token, a.resid_ld, a.x_rows)[fc]) : 0.f;
  return e;
}

// CG chunks (1 KiB each) of R weight rows, in registers. Every lane loads:
// a lane past K (K is a multiple of 16) reads column 0 instead, and its
// activation values are zero, so those weights add exactly 0. Unconditional
// loads keep the wait counts exact (a guarded load would be a branch, and the
// compiler's vmcnt before the activation's LDS store would then wait for the
// whole weight stage).
template <int R, int CG>
struct GemvStage {
  u32x4 w[CG][R];

  __device__ __forceinline__ void load(const FusedGemv& a, const int8_t* const (&rows)[R], int c0, int lane) {
#pragma unroll
    for (int c = 0; c < CG; ++c) {
      const int k = (c0 + c) * kFChunk + lane * 16;
      const int kl = k < a.K ? k : 0;
#pragma unroll
      for (int r = 0; r < R; ++r) w[c][r] = ld16_stream(rows[r] + kl);
    }
  }
};

// Chunks per register stage: the largest divisor of NCH with at most 8 16-byte
// loads per lane (32 VGPRs) per stage; two stages are live at a time.
constexpr int stage_chunks(int R, int NCH) {
  int cg = NCH;
  while (cg > 1 && (R * cg > 8 || NCH % cg)) --cg;
  return cg;
}

// acc[r] += sum over the CG chunks of stage s (first chunk c0) of w * x, biased
// form; sx += sum of x. Columns past K have x = 0 in LDS.
template <int R, int CG>
__device__ __forceinline__ void stage_mac(const GemvStage<R, CG>& s, const uint16_t* hs, int c0, int lane,
                                          float (&acc)[R], float& sx) {
#pragma unroll
  for (int c = 0; c < CG; ++c) {
    const int k = (c0 + c) * kFChunk + lane * 16;
    float xf[16];
    unpack_bf16x16(*(const u32x4*)(hs + k), *(const u32x4*)(hs + k + 8), xf);
    float ts = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) ts += xf[e];
    sx += ts;
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = dot16_biased(s.w[c][r], xf, acc[r]);
  }
}

// Row totals of tile t (wave-uniform) and the epilogue: lane j < RH stores
// feature t * RH + j. Argmax keeps the lane's best (value, index) in best.
template <int R, int EPI>
__device__ __forceinline__ void tile_finish(const FusedGemv& a, int64_t t, int lane, const float (&acc)[R], float sx,
                                            const GemvEpi& ep, ArgBest& best) {
  constexpr int RH = EPI == kEpiSwiGLU ? R / 2 : R;
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
  const int64_t f = t * RH + lane;
  const bool own = lane < RH && f < a.N;
  if constexpr (EPI == kEpiStore) {
    if (own) a.y[f] = f32_to_bf16(mine * ep.sc);
  } else if constexpr (EPI == kEpiResid) {
    if (own) a.y[f] = f32_to_bf16(ep.res + bf16r(mine * ep.sc));
  } else if constexpr (EPI == kEpiSwiGLU) {
    if (own) {
      const float g = bf16r(mine * ep.sc);
      const float u = bf16r(mine_up * ep.sc_up);
      const float sg = bf16r(g / (1.0f + expf(-g)));
      a.y[f] = f32_to_bf16(sg * u);
    }
  } else {
    if (own) {
      const uint16_t lg = f32_to_bf16(mine * ep.sc);
      if (a.y) a.y[f] = lg;
      best = arg_better(best, ArgBest{bf16_to_f32(lg), (int)f});
    }
  }
}

// One int8 GEMV of a single activation row with a fused prologue / epilogue.
// A block is W wavefronts. A wavefront owns RH output features per tile (R
// weight rows: SwiGLU pairs each gate row with its up row): one tile per
// wavefront, except the capped lm_head grid, which walks tiles t, t + stride,
// ... Rows stream with 16-byte non-temporal loads in stages of CG chunks, in two
// ping-pong register buffers: stage s + 1 is issued before stage s is
// multiplied, and scheduling barriers keep the compiler from hoisting later
// stages (all of a K = 12288 row would not fit in registers). No buffer is
// copied, so the wait before each stage is for that stage alone. The activation is staged once per block in
// LDS (stage_load / stage_finish), its loads issued before the weights: vector
// loads retire in order. LDS hand-offs use lds_barrier(), which does not wait
// for the weight stream. Argmax: each lane keeps its best (value, index)
// across tiles; the block reduces once.
//
// The operands the first loads need lead the argument list as scalars, so the
// launch places them in registers (kernel-argument preload) and the loads go
// out without a read of the argument block first: w, ldw, K, N and the
// activation source (kXRow: x, x_token, norm_w; merge: ws_m, ws_l, ws_acc,
// nsplit, head_dim), copies of the same fields of `args`.
template <int R, int NCH, int EPI, bool NORM, int XSRC, int W>
__global__ __launch_bounds__(W * kWave) void fused_gemv_kernel(const int8_t* w, const void* src0, const void* src1,
                                                               const void* src2, int64_t ldw, int K, int N, int aux0,
                                                               int aux1, const FusedGemv args) {
  FusedGemv a = args;
  a.w = w;
  a.ldw = ldw;
  a.K = K;
  a.N = N;
  if constexpr (XSRC == kXRow) {
    a.x = (const uint16_t*)src0;
    a.x_token = (const int64_t*)src1;
    a.norm_w = (const uint16_t*)src2;
  } else {
    a.ws_m = (const float*)src0;
    a.ws_l = (const float*)src1;
    a.ws_acc = (const float*)src2;
    a.nsplit = aux0;
    a.head_dim = aux1;
  }
  constexpr int CG = stage_chunks(R, NCH);
  constexpr int NST = NCH / CG;
  constexpr bool kMulti = EPI == kEpiArgmax;
  static_assert(EPI != kEpiSwiGLU || R % 2 == 0, "SwiGLU pairs rows");
  using Stage = GemvStage<R, CG>;
  constexpr int RH = EPI == kEpiSwiGLU ? R / 2 : R;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t ntiles = (a.N + RH - 1) / RH;
  const int64_t stride = (int64_t)gridDim.x * W;
  int64_t t = (int64_t)blockIdx.x * W + wave;

  // Activation loads first (they retire first), then the weight stream.
  Staged<W * kWave, NCH, XSRC> stg;
  stage_load<W * kWave, NCH, NORM, XSRC>(a, stg);
  const int8_t* rows[R];
  tile_rows<R, EPI>(a, t, rows);
  Stage buf[2];
  buf[0].load(a, rows, 0, lane);
  GemvEpi ep = tile_epi<R, EPI>(a, t, lane);
  __shared__ __align__(16) uint16_t hs[NCH * kFChunk];
  stage_finish<W * kWave, NCH, NORM, XSRC>(a, stg, hs);

  ArgBest best{-INFINITY, 0x7fffffff};
  if constexpr (!kMulti || NST > 1) {
    // Stages of a tile over the ping-pong buffers (stage 0 in buf[0]).
    for (; t < ntiles; t += stride) {
      float acc[R];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = 0.f;
      float sx = 0.f;
      // Pairs of stages (A = buf[0], B = buf[1]) while two or more follow the
      // pair, then a tail of one or two stages. All loads in the loop body are
      // unconditional, so each wait covers exactly the stage about to be used.
      int st = 0;
#pragma unroll 1
      for (; st + 2 < NST; st += 2) {
        buf[1].load(a, rows, (st + 1) * CG, lane);
        __builtin_amdgcn_sched_barrier(0);
        stage_mac<R, CG>(buf[0], hs, st * CG, lane, acc, sx);
        __builtin_amdgcn_sched_barrier(0);
        buf[0].load(a, rows, (st + 2) * CG, lane);
        __builtin_amdgcn_sched_barrier(0);
        stage_mac<R, CG>(buf[1], hs, (st + 1) * CG, lane, acc, sx);
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (NST % 2 == 0) {
        buf[1].load(a, rows, (NST - 1) * CG, lane);
        __builtin_amdgcn_sched_barrier(0);
        stage_mac<R, CG>(buf[0], hs, (NST - 2) * CG, lane, acc, sx);
        __builtin_amdgcn_sched_barrier(0);
        stage_mac<R, CG>(buf[1], hs, (NST - 1) * CG, lane, acc, sx);
      } else {
        stage_mac<R, CG>(buf[0], hs, (NST - 1) * CG, lane, acc, sx);
      }
      tile_finish<R, EPI>(a, t, lane, acc, sx, ep, best);
      if (!kMulti || t + stride >= ntiles) break;
      tile_rows<R, EPI>(a, t + stride, rows);
      buf[0].load(a, rows, 0, lane);
      ep = tile_epi<R, EPI>(a, t + stride, lane);
    }
  } else {
    // One-stage rows over many tiles: the next tile's row is issued before this
    // one is multiplied, and the activation chunks (and their sum) stay in
    // registers across tiles.
    float xh[CG][16];
    float sxh = 0.f;
#pragma unroll
    for (int c = 0; c < CG; ++c) {
      const int k = c * kFChunk + lane * 16;
      unpack_bf16x16(*(const u32x4*)(hs + k), *(const u32x4*)(hs + k + 8), xh[c]);
#pragma unroll
      for (int e = 0; e < 16; ++e) sxh += xh[c][e];
    }
    Stage& cur = buf[0];
    for (; t < ntiles; t += stride) {
      const bool more = t + stride < ntiles;
      const int8_t* nrows[R];
      GemvEpi nep = ep;
      Stage nxt;
      if (more) {
        tile_rows<R, EPI>(a, t + stride, nrows);
        nxt.load(a, nrows, 0, lane);
        nep = tile_epi<R, EPI>(a, t + stride, lane);
      }
      float acc[R];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
      for (int c = 0; c < CG; ++c)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = dot16_biased(cur.w[c][r], xh[c], acc[r]);
      tile_finish<R, EPI>(a, t, lane, acc, sxh, ep, best);
      if (more) {
        cur = nxt;
        ep = nep;
      }
    }
  }
  if constexpr (kMulti) {
    best = block_argbest<W>(best);
    if (threadIdx.x == 0) {
      a.part_v[blockIdx.x] = best.v;
      a.part_i[blockIdx.x] = best.i;
    }
  }
}

// ---------------------------------------------------------------- 2-4 activation rows
//
// y[m, n] = bf16(scale[n] * sum_k x[m, k] w[n, k]) for m < M (2 to 4): the
// reference's decode contract (research/realmodel/int8_linear.py:26-38) at a
// few rows. The weights stream as in fused_gemv_kernel (stages of CG chunks in
// two ping-pong register buffers, unconditional loads, exact waits), the M
// activation rows are staged in LDS, and each weight byte is converted once and
// multiplied into every row. Per row, the chunk sums and the row reduction are
// the single-row kernel's in the same order, so each output row is bit-identical
// to a one-row call on that row.

// acc[m] += w * x[m] over one 16-byte weight load, biased form, in
// dot16_biased's order for each row.
template <int M>
__device__ __forceinline__ void dot16_biased_rows(const u32x4 wq, const float (&x)[M][16], float (&acc)[M]) {
  const uint32_t d[4] = {wq.x ^ 0x80808080u, wq.y ^ 0x80808080u, wq.z ^ 0x80808080u, wq.w ^ 0x80808080u};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const float wv = (float)((d[j] >> (8 * b)) & 0xffu);
#pragma unroll
      for (int m = 0; m < M; ++m) acc[m] = fmaf(wv, x[m][4 * j + b], acc[m]);
    }
  }
}

template <int M, int R, int CG>
__device__ __forceinline__ void stage_mac_rows(const GemvStage<R, CG>& s, const uint16_t* hs, int ldh, int c0,
                                               int lane, float (&acc)[R][M], float (&sx)[M]) {
#pragma unroll
  for (int c = 0; c < CG; ++c) {
    const int k = (c0 + c) * kFChunk + lane * 16;
    float x[M][16];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      unpack_bf16x16(*(const u32x4*)(hs + m * ldh + k), *(const u32x4*)(hs + m * ldh + k + 8), x[m]);
      float t = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) t += x[m][e];
      sx[m] += t;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) dot16_biased_rows<M>(s.w[c][r], x, acc[r]);
  }
}

// Stages of the few-rows kernel: the single-row kernel's, halved for two weight
// rows per wavefront over rows of 8 chunks or more (their full-size stages need
// more than 256 VGPRs with several activation rows and spill).
constexpr int rows_stage_chunks(int R, int NCH) { return stage_chunks(R >= 2 && NCH >= 8 ? 2 * R : R, NCH); }

template <int M, int R, int NCH, int W>
__global__ __launch_bounds__(W * kWave) void gemv_rows_kernel(const FusedGemv a) {
  constexpr int CG = rows_stage_chunks(R, NCH);
  constexpr int NST = NCH / CG;
  constexpr int NT = W * kWave;
  constexpr int KP = NCH * kFChunk;  // LDS row: K rounded up to whole chunks, zero past K
  constexpr int kPasses = (KP + NT * 8 - 1) / (NT * 8);
  using Stage = GemvStage<R, CG>;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int64_t t = (int64_t)blockIdx.x * W + tid / kWave;
  const u32x4 z{0u, 0u, 0u, 0u};

  // Activation loads first (they retire first), then the weight stream.
  u32x4 xv[M][kPasses];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int k8 = (p * NT + tid) * 8;
      xv[m][p] = k8 < a.K ? ld16(a.x + m * a.x_ld + k8) : z;
    }
  const int8_t* rows[R];
  tile_rows<R, kEpiStore>(a, t, rows);
  Stage buf[2];
  buf[0].load(a, rows, 0, lane);
  const GemvEpi ep = tile_epi<R, kEpiStore>(a, t, lane);
  __shared__ __align__(16) uint16_t hs[M * KP];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int k8 = (p * NT + tid) * 8;
      if (k8 < KP) *(u32x4*)(hs + m * KP + k8) = xv[m][p];
    }
  lds_barrier();
  if (t * R >= a.N) return;  // a wavefront past the last tile (no barrier follows)

  float acc[R][M], sx[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    sx[m] = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r][m] = 0.f;
  }
  int st = 0;
#pragma unroll 1
  for (; st + 2 < NST; st += 2) {
    buf[1].load(a, rows, (st + 1) * CG, lane);
    __builtin_amdgcn_sched_barrier(0);
    stage_mac_rows<M, R, CG>(buf[0], hs, KP, st * CG, lane, acc, sx);
    __builtin_amdgcn_sched_barrier(0);
    buf[0].load(a, rows, (st + 2) * CG, lane);
    __builtin_amdgcn_sched_barrier(0);
    stage_mac_rows<M, R, CG>(buf[1], hs, KP, (st + 1) * CG, lane, acc, sx);
    __builtin_amdgcn_sched_barrier(0);
  }
  if constexpr (NST % 2 == 0) {
    buf[1].load(a, rows, (NST - 1) * CG, lane);
    __builtin_amdgcn_sched_barrier(0);
    stage_mac_rows<M, R, CG>(buf[0], hs, KP, (NST - 2) * CG, lane, acc, sx);
    __builtin_amdgcn_sched_barrier(0);
    stage_mac_rows<M, R, CG>(buf[1], hs, KP, (NST - 1) * CG, lane, acc, sx);
  } else {
    stage_mac_rows<M, R, CG>(buf[0], hs, KP, (NST - 1) * CG, lane, acc, sx);
  }
  float mine[M];
#pragma unroll
  for (int m = 0; m < M; ++m) mine[m] = 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float v = wave_sum(acc[r][m] - 128.f * sx[m]);
      if (lane == r) mine[m] = v;
    }
  const int64_t f = t * R + lane;
  if (lane < R && f < a.N) {
#pragma unroll
    for (int m = 0; m < M; ++m) a.y[m * a.y_ld + f] = f32_to_bf16(mine[m] * ep.sc);
  }
}

// Greedy pick over the per-block maxima: token = first index of the largest
// logit (torch.argmax), position += 1, and (ring set) the token also to
// ring[new position % slots]. One block. Its arguments come as one struct,
// which the launch does not preload into registers: a one-block launch with
// preloaded arguments measured 0.12 us slower on the MI355X (launches of two
// blocks and more measured 0.03-0.05 us faster).
struct ArgmaxFinal {
  const float* part_v;
  const int* part_i;
  int parts;
  int64_t* token;
  int64_t* position;
  int64_t* ring;
  int slots;
};

__global__ __launch_bounds__(kFThreads) void argmax_final_kernel(const ArgmaxFinal a) {
  ArgBest best{-INFINITY, 0x7fffffff};
  for (int j = threadIdx.x; j < a.parts; j += kFThreads) best = arg_better(best, ArgBest{a.part_v[j], a.part_i[j]});
  best = block_argbest<kFWaves>(best);
  if (threadIdx.x == 0) {
    const int64_t tok = best.i == 0x7fffffff ? 0 : best.i;  // no logits at all: token 0
    *a.token = tok;
    if (a.position) {
      const int64_t p = *a.position + 1;
      *a.position = p;
      if (a.ring) a.ring[(p % a.slots + a.slots) % a.slots] = tok;
    }
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
  int group;  // query heads per kv head
  float eps, scale;
};

// A decode step's attention blocks serve one query head each while the cache
// holds at most this many slots, and a whole kv head's group of query heads
// (reading its K/V once) past it. Short caches are latency-bound: a block with
// one head finishes its loop and its merge sooner, and reading each K/V row once
// per query head costs little (the columns of one kv head share an XCD, so after
// the first the group's reads of a K/V row come from L2). Measured on the MI355X,
// with the split counts of egpt_qwen3_step_default_splits, against whole-group
// blocks: Qwen3-1.7B (2 query heads per kv head) 4.9% faster at 392 slots,
// 4.5-5.4% at 1264-1764 and 0.6-2.2% at 2264-3064, Qwen3-8B (4) 5.7%, 2.6-3.3% and
// 1.3-2.6% (at 2580-2980); at 3.8k slots the 1.7B 2.7% slower.
constexpr int kHeadBlockMaxSlots = 3072;

// Attention partials of one decode step: block (query heads hq0 .. hq0 + G - 1
// of one kv head, split). Every load that does not depend on arithmetic is
// issued first (queries, new key and value and norm weights, then, once the
// position is in, the RoPE rows and the first K/V rows of the split); the query
// and the new key are normalised and rotated while those are in flight. The
// blocks whose split holds slot p start their first softmax stream with the new
// token from registers (it is not read back from the cache), and the first of
// them for the kv head stores it to slot p for later steps; no block of the
// launch reads slot p from the cache, so no barrier orders the store.
//
// qkv, position, the norm weights, Hkv and group lead the argument list as
// scalars (copies of the same fields of `args`): the launch preloads them into
// registers, so the position and query loads go out without a read of the
// argument block first.
template <int D, int G>
__global__ __launch_bounds__(kAttnThreads) void attn_step_kernel(const uint16_t* qkv, const int64_t* position,
                                                                 const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                                                                 int Hkv, int group, const AttnStep args) {
  AttnStep a = args;
  a.qkv = qkv;
  a.position = position;
  a.q_norm_w = q_norm_w;
  a.k_norm_w = k_norm_w;
  a.Hkv = Hkv;
  a.group = group;
  using Geo = AttnGeom<__bf16, D, kAttnThreads, 1, 4>;
  constexpr int EPL = Geo::EPL;
  constexpr int LPS = Geo::LPS;
  const int tid = threadIdx.x;
  const int d0 = (tid % LPS) * EPL;
  // Block column x serves query heads hq0 .. hq0 + G - 1 of kv head x mod Hkv:
  // the columns of one kv head are x, x + Hkv, ..., so with Hkv a multiple of 8
  // they all run on one XCD (blocks go round-robin to the 8 XCDs) and the kv
  // head's K/V rows, read once per column, come from that XCD's L2 after the first.
  const int hk = (int)blockIdx.x % a.Hkv;
  const int hq0 = hk * a.group + ((int)blockIdx.x / a.Hkv) * G;
  const int split = blockIdx.y;
  const int Hq = a.Hkv * a.group;

  constexpr bool kMfma = kAttnMfma<__bf16, D, G>;
  // The MFMA form normalises and rotates each head once per block: lane group
  // grp (16 lanes, one 128-element row) takes query head hq0 + grp for grp < G
  // and the new key otherwise, and the block shares them through LDS. The vector
  // form keeps every head in every group's registers (its loop reads them there).
  const int grp = tid / LPS;
  constexpr int GQ = kMfma ? 1 : G;  // query rows each thread normalises

  // The rows that do not depend on the position go out before it is read.
  u32x4 qr[GQ], qw, kw, kr, vr, cr, sr;
  if constexpr (kMfma) {
    const bool qrow = grp < G;
    qr[0] = ld16(a.qkv + (int64_t)(qrow ? hq0 + grp : Hq + hk) * D + d0);
    qw = ld16((qrow ? a.q_norm_w : a.k_norm_w) + d0);
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g) qr[g] = ld16(a.qkv + (int64_t)(hq0 + g) * D + d0);
    qw = ld16(a.q_norm_w + d0);
    kw = ld16(a.k_norm_w + d0);
    kr = ld16(a.qkv + (int64_t)(Hq + hk) * D + d0);
  }
  vr = ld16(a.qkv + (int64_t)(Hq + a.Hkv + hk) * D + d0);
  __builtin_amdgcn_sched_barrier(0);

  // The position comes through the scalar cache: an earlier launch wrote it and
  // nothing writes it during this one. The scalar load has its own wait counter,
  // so waiting for it does not also wait for the rows above.
  int64_t pos = *(const __attribute__((address_space(4))) int64_t*)a.position;
  pos = pos < 0 ? 0 : (pos >= a.cap ? a.cap - 1 : pos);
  const int64_t len = pos + 1;
  int64_t start, end;
  attn_split_range(len, a.nsplit, split, start, end);
  const bool owner = start <= pos && pos < end;  // block-uniform
  const int64_t end_cached = owner ? pos : end;   // slot p comes from registers

  cr = ld16(a.cos_t + pos * D + d0);
  sr = ld16(a.sin_t + pos * D + d0);

  uint16_t* kc = a.k_cache + (int64_t)hk * a.c_sh;
  uint16_t* vc = a.v_cache + (int64_t)hk * a.c_sh;
  AttnPipe<1, 4> pp;
  MfmaKV t0;
  if constexpr (kMfma) {
    mfma_issue(t0, (const __bf16*)kc, a.c_sn, (const __bf16*)vc, a.c_sn, start + kMfmaSlots * (tid / kWave),
               end_cached);
    __builtin_amdgcn_sched_barrier(0);
  } else {
    attn_begin<Geo>(pp, (const __bf16*)kc, a.c_sn, (const __bf16*)vc, a.c_sn, start, end_cached);
  }

  float kn[EPL], vn[EPL];
  if constexpr (kMfma) {
    // This group's head (query hq0 + grp, or the new key) normalised and rotated,
    // then every head shared through LDS: rows 0..G-1 the queries, row G the key.
    const int lane = tid % kWave;
    float hv[EPL];
    head_norm_rope<D, EPL, LPS>(qr[0], qw, cr, sr, d0, a.eps, hv);
    __shared__ __align__(16) uint16_t qs[G + 1][D];
    if (grp <= G) {
      uint32_t pk[EPL / 2];
      pack_bf16<EPL>(hv, pk);
      *(u32x4*)&qs[grp][d0] = u32x4{pk[0], pk[1], pk[2], pk[3]};
    }
    lds_barrier();
    // B fragments of Q^T: column lane % 16 is query head lane % 16 (zero past G).
    const int h = lane & 15;
    bf16x8_mt qb[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const u32x4 z{0u, 0u, 0u, 0u};
      const u32x4 v = *(const u32x4*)&qs[h < G ? h : 0][32 * c + 8 * (lane >> 4)];
      qb[c] = __builtin_bit_cast(bf16x8_mt, h < G ? v : z);
    }
    // This lane's 8 elements of every query and of the key (the new token's
    // score and the cache write take them in that layout).
    float qf[G][EPL];
#pragma unroll
    for (int g = 0; g < G; ++g) Elem<__bf16>::unpack(*(const u32x4*)&qs[g][d0], qf[g]);
    const u32x4 kp = *(const u32x4*)&qs[G][d0];
    Elem<__bf16>::unpack(kp, kn);
    Elem<__bf16>::unpack(vr, vn);
    if (owner && tid < LPS && hq0 % a.group == 0) {  // one block of the kv head stores it
      *(u32x4*)(kc + pos * a.c_sn + d0) = kp;
      *(u32x4*)(vc + pos * a.c_sn + d0) = vr;
    }
    attn_partial_mfma<G>(qb, t0, (const __bf16*)kc, a.c_sn, (const __bf16*)vc, a.c_sn, start, end_cached, a.scale,
                         a.ws_m, a.ws_l, a.ws_acc, (int64_t)hq0 * a.nsplit + split, a.nsplit, owner, qf, kn, vn,
                         nullptr, 0);
  } else {
    float qf[G][EPL];
#pragma unroll
    for (int g = 0; g < G; ++g) head_norm_rope<D, EPL, LPS>(qr[g], qw, cr, sr, d0, a.eps, qf[g]);
    if (owner) {
      head_norm_rope<D, EPL, LPS>(kr, kw, cr, sr, d0, a.eps, kn);
      Elem<__bf16>::unpack(vr, vn);
      if (tid < LPS && hq0 % a.group == 0) {  // one block of the kv head stores it
        uint32_t packed[EPL / 2];
#pragma unroll
        for (int e = 0; e < EPL / 2; ++e)
          packed[e] = (uint32_t)f32_to_bf16(kn[2 * e]) | ((uint32_t)f32_to_bf16(kn[2 * e + 1]) << 16);
        *(u32x4*)(kc + pos * a.c_sn + d0) = u32x4{packed[0], packed[1], packed[2], packed[3]};
        *(u32x4*)(vc + pos * a.c_sn + d0) = vr;
      }
    }
    attn_partial<Geo, __bf16, G>(qf, pp, (const __bf16*)kc, a.c_sn, (const __bf16*)vc, a.c_sn, start, end_cached,
                               a.scale, a.ws_m, a.ws_l, a.ws_acc, (int64_t)hq0 * a.nsplit + split, a.nsplit,
                               owner, kn, vn);
  }
}

// Merge of the split partials: one block per query head. The attention launch's
// block column x (of X = Hq / G, G query heads per block) ran every split of its
// heads (from (x mod Hkv) group + (x / Hkv) G on) on one XCD (x mod 8, blocks
// being dispatched round-robin to the 8 XCDs) when X is a multiple of 8; merge
// block c takes head j = c / X of column c mod X, so it runs on that XCD and finds
// the partials in its L2.
constexpr int kMergeThreads = 256;

template <int D>
__global__ __launch_bounds__(kMergeThreads) void attn_merge_kernel(const float* __restrict__ ws_m,
                                                                   const float* __restrict__ ws_l,
                                                                   const float* __restrict__ ws_acc,
                                                                   uint16_t* __restrict__ out, int nsplit, int G,
                                                                   int Hkv) {
  const int X = (int)gridDim.x / G;
  const int x = (int)blockIdx.x % X;
  const int h = (x % Hkv) * (X / Hkv * G) + (x / Hkv) * G + (int)blockIdx.x / X;
  float r;
  if (attn_combine_block<D, kMergeThreads>(ws_m + (int64_t)h * nsplit, ws_l + (int64_t)h * nsplit,
                                           ws_acc + (int64_t)h * nsplit * D, nsplit, r))
    out[(int64_t)h * D + threadIdx.x] = f32_to_bf16(r);
}

// ------------------------------------------------------------------ host side

int chunks_for(int K) {
  const int n = (K + kFChunk - 1) / kFChunk;
  if (n <= 4) return n < 1 ? 1 : n;
  if (n <= 6) return 6;
  if (n <= 8) return 8;
  return 12;
}

// Launch shape, from a cold sweep of the Qwen3 shapes on the MI355X: 8
// wavefronts per block (the activation row is staged once per block), two rows
// per wavefront while that still leaves >= 256 blocks (fused QKV, lm_head;
// gate/up as one gate + one up row), else one (o_proj, down_proj): these small
// GEMVs are bound by latency, and more blocks start streaming sooner.
constexpr int kGemvWaves = 8;

int features_per_wave(int64_t n, bool pairs) {
  if (pairs) return 1;  // one gate row + one up row
  return (n + 2 * kGemvWaves - 1) / (2 * kGemvWaves) >= 256 ? 2 : 1;
}

template <int EPI, bool NORM, int XSRC, int R>
int launch_r(const FusedGemv& a, int nch, unsigned blocks, hipStream_t st) {
  constexpr int W = kGemvWaves;
  const bool row = XSRC == kXRow;
  const void* s0 = row ? (const void*)a.x : (const void*)a.ws_m;
  const void* s1 = row ? (const void*)a.x_token : (const void*)a.ws_l;
  const void* s2 = row ? (const void*)a.norm_w : (const void*)a.ws_acc;
  const int aux0 = row ? 0 : a.nsplit, aux1 = row ? 0 : a.head_dim;
  switch (nch) {
#define EGPT_CASE(C)                                                                                             \
  case C:                                                                                                        \
    hipLaunchKernelGGL((fused_gemv_kernel<R, C, EPI, NORM, XSRC, W>), dim3(blocks), dim3(W * kWave), 0, st, a.w, \
                       s0, s1, s2, a.ldw, a.K, a.N, aux0, aux1, a);                                             \
    break;
    EGPT_CASE(1) EGPT_CASE(2) EGPT_CASE(3) EGPT_CASE(4) EGPT_CASE(6) EGPT_CASE(8) EGPT_CASE(12)
#undef EGPT_CASE
    default: return EGPT_ERR_UNSUPPORTED;
  }
  return EGPT_LAUNCH_STATUS();
}

// Blocks of a fused GEMV launch: one tile per wavefront, except the lm_head,
// whose grid is capped (about four 8-wave blocks per CU) so each block stages
// the activation once and reduces its argmax once over many tiles.
constexpr unsigned kHeadMaxBlocks = 1024;

unsigned gemv_blocks(int64_t n, bool pairs, bool capped) {
  const int rh = features_per_wave(n, pairs);
  const int64_t tiles = (n + rh - 1) / rh;
  const unsigned b = (unsigned)((tiles + kGemvWaves - 1) / kGemvWaves);
  return capped && b > kHeadMaxBlocks ? kHeadMaxBlocks : b;
}

template <int EPI, bool NORM, int XSRC = kXRow>
int launch_fused(const FusedGemv& a, hipStream_t st) {
  const bool pairs = EPI == kEpiSwiGLU;
  const int rh = features_per_wave(a.N, pairs);
  const unsigned blocks = gemv_blocks(a.N, pairs, EPI == kEpiArgmax);
  const int nch = chunks_for(a.K);
  if constexpr (EPI == kEpiSwiGLU) {
    return launch_r<EPI, NORM, XSRC, 2>(a, nch, blocks, st);
  } else {
    if (rh >= 2) return launch_r<EPI, NORM, XSRC, 2>(a, nch, blocks, st);
    return launch_r<EPI, NORM, XSRC, 1>(a, nch, blocks, st);
  }
}

unsigned head_blocks(int vocab) { return gemv_blocks(vocab, false, true); }

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
  if (s->token_ring && s->token_ring_slots < 1) return EGPT_ERR_INVALID;
  return EGPT_OK;
}

// G: query heads per block (1, or the whole group a.group).
template <int D>
int launch_attn_step(const AttnStep& a, int G, uint16_t* out, bool merge, hipStream_t st) {
  dim3 grid((unsigned)(a.Hkv * a.group / G), (unsigned)a.nsplit);
#define EGPT_ATTN_ARGS a.qkv, a.position, a.q_norm_w, a.k_norm_w, a.Hkv, a.group, a
  switch (G) {
    case 1: hipLaunchKernelGGL((attn_step_kernel<D, 1>), grid, dim3(kAttnThreads), 0, st, EGPT_ATTN_ARGS); break;
    case 2: hipLaunchKernelGGL((attn_step_kernel<D, 2>), grid, dim3(kAttnThreads), 0, st, EGPT_ATTN_ARGS); break;
    case 4: hipLaunchKernelGGL((attn_step_kernel<D, 4>), grid, dim3(kAttnThreads), 0, st, EGPT_ATTN_ARGS); break;
    case 8: hipLaunchKernelGGL((attn_step_kernel<D, 8>), grid, dim3(kAttnThreads), 0, st, EGPT_ATTN_ARGS); break;
    default: return EGPT_ERR_UNSUPPORTED;
  }
#undef EGPT_ATTN_ARGS
  if (hipGetLastError() != hipSuccess) return EGPT_ERR_LAUNCH;
  if (merge)
    hipLaunchKernelGGL((attn_merge_kernel<D>), dim3((unsigned)(a.Hkv * a.group)), dim3(kMergeThreads), 0, st, a.ws_m,
                       a.ws_l, a.ws_acc, out, a.nsplit, G, a.Hkv);
  return EGPT_LAUNCH_STATUS();
}

// The public fused-GEMV description -> kernel arguments, validated; then the
// launch for its (epilogue, norm, source) combination.
int run_fused(const egpt_gemv_fused& p, hipStream_t st) {
  if (!p.w || !p.scale || p.N < 1 || p.K < 16 || p.K % 16 || p.K > kMaxChunks * kFChunk || p.ldw < p.K)
    return EGPT_ERR_INVALID;
  if (!aligned16(p.w) || p.ldw % 16) return EGPT_ERR_INVALID;
  const bool merge = p.merge_m != nullptr;
  const bool norm = p.norm_w != nullptr;
  if (merge) {
    if (!p.merge_l || !p.merge_acc || p.merge_splits < 1 || p.merge_splits > kMergeInGemvMaxSplits ||
        p.head_dim < 8 || p.head_dim % 8 || p.K % p.head_dim || p.K > kGemvWaves * kWave * 8 ||
        !aligned16(p.merge_acc))
      return EGPT_ERR_UNSUPPORTED;
  } else {
    if (!p.x || !aligned16(p.x) || (p.x_token && (p.x_rows < 1 || p.x_ld % 8))) return EGPT_ERR_INVALID;
  }
  if (norm && !aligned16(p.norm_w)) return EGPT_ERR_INVALID;
  FusedGemv a{};
  a.x = (const uint16_t*)p.x;
  a.x_token = p.x_token;
  a.x_ld = p.x_ld;
  a.x_rows = p.x_rows > 0 ? p.x_rows : 1;
  a.norm_w = (const uint16_t*)p.norm_w;
  a.eps = p.eps;
  a.w = p.w;
  a.ldw = p.ldw;
  a.scale = p.scale;
  a.N = p.N;
  a.K = p.K;
  a.y = (uint16_t*)p.y;
  a.resid = (const uint16_t*)p.resid;
  a.resid_token = p.resid_token;
  a.resid_ld = p.resid_ld;
  a.part_v = p.part_v;
  a.part_i = p.part_i;
  a.ws_m = p.merge_m;
  a.ws_l = p.merge_l;
  a.ws_acc = p.merge_acc;
  a.nsplit = p.merge_splits;
  a.head_dim = p.head_dim;
  switch (p.epilogue) {
    case EGPT_EPI_STORE:
      if (!p.y || merge) return merge ? EGPT_ERR_UNSUPPORTED : EGPT_ERR_INVALID;
      return norm ? launch_fused<kEpiStore, true>(a, st) : launch_fused<kEpiStore, false>(a, st);
    case EGPT_EPI_RESIDUAL:
      if (!p.y || !p.resid) return EGPT_ERR_INVALID;
      if (norm) return EGPT_ERR_UNSUPPORTED;
      if (!merge) return launch_fused<kEpiResid, false>(a, st);
      switch (merge_bound(a.nsplit)) {
        case 4: return launch_fused<kEpiResid, false, 4>(a, st);
        case 8: return launch_fused<kEpiResid, false, 8>(a, st);
        default: return launch_fused<kEpiResid, false, 16>(a, st);
      }
    case EGPT_EPI_SWIGLU:
      if (!p.y) return EGPT_ERR_INVALID;
      if (!norm || merge) return EGPT_ERR_UNSUPPORTED;
      return launch_fused<kEpiSwiGLU, true>(a, st);
    case EGPT_EPI_ARGMAX:
      if (!p.part_v || !p.part_i) return EGPT_ERR_INVALID;
      if (!norm || merge) return EGPT_ERR_UNSUPPORTED;
      return launch_fused<kEpiArgmax, true>(a, st);
    default:
      return EGPT_ERR_INVALID;
  }
}

// The four fused GEMVs of decode-step layer i, in launch order:
//   [0] RMSNorm(x; input_layernorm) -> QKV            (layer 0: x = embedding row of *token)
//   [1] o_proj(merge of the attention partials, or the merged row) + residual -> x
//   [2] RMSNorm(x; post_attention_layernorm) -> gate/up -> SwiGLU -> act
//   [3] down_proj(act) + residual -> x
void layer_gemvs(const egpt_qwen3_step* s, int i, egpt_gemv_fused* g) {
  const egpt_qwen3_layer& L = s->layer[i];
  const StepLayout lay = step_layout(s);
  char* ws = (char*)s->workspace;
  const bool first = i == 0;
  const int D = s->head_dim;
  for (int j = 0; j < 4; ++j) g[j] = egpt_gemv_fused{};
  g[0].epilogue = EGPT_EPI_STORE;
  g[0].N = (s->heads + 2 * s->kv_heads) * D;
  g[0].K = s->hidden;
  g[0].x = first ? s->embed : s->x;
  g[0].x_token = first ? s->token : nullptr;
  g[0].x_ld = s->hidden;
  g[0].x_rows = s->vocab;
  g[0].norm_w = L.in_norm;
  g[0].eps = s->eps;
  g[0].w = L.qkv_w;
  g[0].ldw = s->hidden;
  g[0].scale = L.qkv_s;
  g[0].y = s->qkv;

  g[1].epilogue = EGPT_EPI_RESIDUAL;
  g[1].N = s->hidden;
  g[1].K = s->heads * D;
  // the o_proj prologue merges the splits itself while each thread owns one
  // 8-element group of the attention row
  if (s->nsplit <= kMergeInGemvMaxSplits && s->heads * D <= kGemvWaves * kWave * 8) {
    g[1].merge_m = (const float*)ws;
    g[1].merge_l = (const float*)(ws + lay.ml);
    g[1].merge_acc = (const float*)(ws + 2 * lay.ml);
    g[1].merge_splits = s->nsplit;
    g[1].head_dim = D;
  } else {
    g[1].x = s->attn;
  }
  g[1].w = L.o_w;
  g[1].ldw = (int64_t)s->heads * D;
  g[1].scale = L.o_s;
  g[1].y = s->x;
  g[1].resid = first ? s->embed : s->x;
  g[1].resid_token = first ? s->token : nullptr;
  g[1].resid_ld = s->hidden;
  g[1].x_rows = s->vocab;

  g[2].epilogue = EGPT_EPI_SWIGLU;
  g[2].N = s->inter;
  g[2].K = s->hidden;
  g[2].x = s->x;
  g[2].norm_w = L.post_norm;
  g[2].eps = s->eps;
  g[2].w = L.gu_w;
  g[2].ldw = s->hidden;
  g[2].scale = L.gu_s;
  g[2].y = s->act;

  g[3].epilogue = EGPT_EPI_RESIDUAL;
  g[3].N = s->hidden;
  g[3].K = s->inter;
  g[3].x = s->act;
  g[3].w = L.down_w;
  g[3].ldw = s->inter;
  g[3].scale = L.down_s;
  g[3].y = s->x;
  g[3].resid = s->x;
}

// The head GEMV: RMSNorm(x; norm) -> lm_head -> logits and per-block maxima.
void head_gemv(const egpt_qwen3_step* s, egpt_gemv_fused* g) {
  const StepLayout lay = step_layout(s);
  char* ws = (char*)s->workspace;
  *g = egpt_gemv_fused{};
  g->epilogue = EGPT_EPI_ARGMAX;
  g->N = s->vocab;
  g->K = s->hidden;
  g->x = s->x;
  g->norm_w = s->final_norm;
  g->eps = s->eps;
  g->w = s->head_w;
  g->ldw = s->hidden;
  g->scale = s->head_s;
  g->y = s->logits;
  g->part_v = (float*)(ws + 2 * lay.ml + lay.acc);
  g->part_i = (int*)(ws + 2 * lay.ml + lay.acc + lay.part_v);
}

void step_gemvs(const egpt_qwen3_step* s, egpt_gemv_fused* out) {
  for (int i = 0; i < s->layers; ++i) layer_gemvs(s, i, out + 4 * i);
  head_gemv(s, out + 4 * s->layers);
}

}  // namespace

size_t fused_step_bytes(const egpt_qwen3_step* s) { return step_layout(s).total; }

int gemv_few_rows(const void* x, int64_t ldx, const int8_t* w, int64_t ldw, const float* scale, void* y, int64_t ldy,
                  int M, int N, int K, hipStream_t st) {
  if (!x || !w || !scale || !y || M < 2 || M > kGemvFewRowsMax || N < 1 || K < 16 || K % 16 ||
      K > kMaxChunks * kFChunk || ldw < K || ldx < K || ldy < N || ldw % 16 || ldx % 8 || !aligned16(x) ||
      !aligned16(w))
    return EGPT_ERR_UNSUPPORTED;
  FusedGemv a{};
  a.x = (const uint16_t*)x;
  a.x_ld = ldx;
  a.w = w;
  a.ldw = ldw;
  a.scale = scale;
  a.N = N;
  a.K = K;
  a.y = (uint16_t*)y;
  a.y_ld = ldy;
  const int r = features_per_wave(N, false);  // the single-row kernel's tiles
  const unsigned blocks = gemv_blocks(N, false, false);
  constexpr int W = kGemvWaves;
  const int nch = chunks_for(K);
#define EGPT_ROWS(MM, RR, C) hipLaunchKernelGGL((gemv_rows_kernel<MM, RR, C, W>), dim3(blocks), dim3(W * kWave), 0, st, a)
#define EGPT_CHUNKS(MM, RR)                                            \
  switch (nch) {                                                       \
    case 1: EGPT_ROWS(MM, RR, 1); break;                               \
    case 2: EGPT_ROWS(MM, RR, 2); break;                               \
    case 3: EGPT_ROWS(MM, RR, 3); break;                               \
    case 4: EGPT_ROWS(MM, RR, 4); break;                               \
    case 6: EGPT_ROWS(MM, RR, 6); break;                               \
    case 8: EGPT_ROWS(MM, RR, 8); break;                               \
    case 12: EGPT_ROWS(MM, RR, 12); break;                             \
    default: return EGPT_ERR_UNSUPPORTED;                              \
  }
  switch (M * 2 + (r >= 2 ? 1 : 0)) {
    case 4: EGPT_CHUNKS(2, 1) break;
    case 5: EGPT_CHUNKS(2, 2) break;
    case 6: EGPT_CHUNKS(3, 1) break;
    case 7: EGPT_CHUNKS(3, 2) break;
    case 8: EGPT_CHUNKS(4, 1) break;
    case 9: EGPT_CHUNKS(4, 2) break;
    default: return EGPT_ERR_UNSUPPORTED;
  }
#undef EGPT_CHUNKS
#undef EGPT_ROWS
  return EGPT_LAUNCH_STATUS();
}
int qwen3_check_step(const egpt_qwen3_step* s) { return check_step(s); }

}  // namespace egpt

using namespace egpt;

extern "C" int egpt_int8_gemv_fused_parts(const egpt_gemv_fused* g, int* parts) {
  if (!g || !parts || g->N < 1) return EGPT_ERR_INVALID;
  *parts = g->epilogue == EGPT_EPI_ARGMAX ? (int)gemv_blocks(g->N, false, true) : 0;
  return EGPT_OK;
}

extern "C" int egpt_int8_gemv_fused(const egpt_gemv_fused* g, hipStream_t stream) {
  if (!g) return EGPT_ERR_INVALID;
  return run_fused(*g, stream);
}

extern "C" int egpt_argmax_parts(const float* part_v, const int* part_i, int parts, int64_t* token,
                                 int64_t* position, hipStream_t stream) {
  if (!part_v || !part_i || !token || parts < 1) return EGPT_ERR_INVALID;
  const ArgmaxFinal f{part_v, part_i, parts, token, position, nullptr, 1};
  hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kFThreads), 0, stream, f);
  return EGPT_LAUNCH_STATUS();
}

extern "C" int egpt_qwen3_step_default_splits(int heads, int kv_heads, int head_dim, int cap) {
  if (heads < 1 || kv_heads < 1 || head_dim < 1 || cap < 1) return 1;
  const int by_len = (cap + 63) / 64;
  // Attention blocks of one query head (up to kHeadBlockMaxSlots): at most 4
  // splits up to 512 slots and 8 past that, so the o_proj prologue merges them at
  // its 4- or 8-split bound (16 splits past 2048 slots measured 1-6% slower). Measured on the MI355X against about one block per CU
  // (7, 11, 16 and 16 splits at 392, 664, 964 and 1764 slots): Qwen3-1.7B 1.9%,
  // 5.8%, 3% and 4.5% faster, Qwen3-8B 1.7%, 6% and 3.3% at 392, 964 and 1764.
  if (cap <= kHeadBlockMaxSlots) {
    const int lim = cap <= 512 ? 4 : 8;
    return by_len < lim ? by_len : lim;
  }
  // Past that, about one block per CU and at least 64 slots per split (more than
  // kMergeInGemvMaxSplits are merged by a launch of their own).
  int by_grid = (256 + kv_heads - 1) / kv_heads;
  if (by_grid < 1) by_grid = 1;
  int n = by_len < by_grid ? by_len : by_grid;
  if (n > 256) n = 256;
  return n < 1 ? 1 : n;
}

extern "C" int egpt_qwen3_step_workspace(const egpt_qwen3_step* s, size_t* bytes) {
  if (!s || !bytes || s->heads < 1 || s->kv_heads < 1 || s->nsplit < 1 || s->head_dim < 1 || s->vocab < 1)
    return EGPT_ERR_INVALID;
  *bytes = (step_layout(s).total + 255) / 256 * 256;
  return EGPT_OK;
}

extern "C" int egpt_qwen3_step_gemvs(const egpt_qwen3_step* s, egpt_gemv_fused* out, int capacity, int* count) {
  if (!count) return EGPT_ERR_INVALID;
  const int st = check_step(s);
  if (st != EGPT_OK) return st;
  *count = 4 * s->layers + 1;
  if (!out) return EGPT_OK;
  if (capacity < *count) return EGPT_ERR_INVALID;
  step_gemvs(s, out);
  return EGPT_OK;
}

extern "C" int egpt_qwen3_decode_step(const egpt_qwen3_step* s, hipStream_t stream) {
  int st = check_step(s);
  if (st != EGPT_OK) return st;
  const StepLayout lay = step_layout(s);
  char* ws = (char*)s->workspace;
  const int D = s->head_dim;
  const int G = s->heads / s->kv_heads;
  egpt_gemv_fused g[4];
  for (int i = 0; i < s->layers; ++i) {
    const egpt_qwen3_layer& L = s->layer[i];
    layer_gemvs(s, i, g);
    // 1. RMSNorm + QKV
    if ((st = run_fused(g[0], stream)) != EGPT_OK) return st;
    // 2. attention partials (and their merge, when the o_proj prologue does not merge)
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
    at.ws_m = (float*)ws;
    at.ws_l = (float*)(ws + lay.ml);
    at.ws_acc = (float*)(ws + 2 * lay.ml);
    at.Hkv = s->kv_heads;
    at.cap = s->cap;
    at.nsplit = s->nsplit;
    at.group = G;
    at.eps = s->eps;
    at.scale = 1.0f / sqrtf((float)D);
    uint16_t* attn_out = (uint16_t*)s->attn;
    const bool merge_in_gemv = g[1].merge_m != nullptr;
    const int hb = s->cap <= kHeadBlockMaxSlots ? 1 : G;  // query heads per attention block
    if (D == 128) st = launch_attn_step<128>(at, hb, attn_out, !merge_in_gemv, stream);
    else if (D == 64) st = launch_attn_step<64>(at, hb, attn_out, !merge_in_gemv, stream);
    else st = launch_attn_step<32>(at, hb, attn_out, !merge_in_gemv, stream);
    if (st != EGPT_OK) return st;
    // 3. o_proj + residual, 4. RMSNorm + gate/up + SwiGLU, 5. down + residual
    for (int j = 1; j < 4; ++j)
      if ((st = run_fused(g[j], stream)) != EGPT_OK) return st;
  }
  // head: final norm + lm_head + per-block maxima, then the greedy pick
  head_gemv(s, g);
  if ((st = run_fused(g[0], stream)) != EGPT_OK) return st;
  const ArgmaxFinal f{g[0].part_v, g[0].part_i, (int)head_blocks(s->vocab), s->token, s->position, s->token_ring,
                      s->token_ring ? s->token_ring_slots : 1};
  hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kFThreads), 0, stream, f);
  return EGPT_LAUNCH_STATUS();
}
