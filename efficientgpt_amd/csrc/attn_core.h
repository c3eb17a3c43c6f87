// Split-K decode attention core shared by the stand-alone attention kernels
// (decode_attn.hip) and the fused decode-step attention (qwen3_fused.hip).
//
// Semantics follow the reference's Triton pair (research/phase5/decode_attention.py:
// _split_kernel :22-56, _combine_kernel :59-71): scores (q . k) * scale in fp32,
// an fp32 online softmax per split keeping (max, sum, acc[D]), and the combine
//   w_i = exp(m_i - max_j m_j),  out = sum_i w_i acc_i / sum_i w_i l_i,
// where empty splits carry m = -inf and weight 0. Only slots inside the split's
// range are ever loaded. Exponentials are exp2((x - max) * log2 e): the same
// function as the reference's exp, rounded relative to the max-subtracted logit.
//
// Layout inside a block (256 threads, 4 wavefronts): one 16-byte load per lane
// covers EPL = 16 / sizeof(T) elements of a row, LPS = D / EPL lanes cover one
// slot (16 lanes for bf16 with D = 128), so a wavefront reads 64 / LPS
// consecutive slots (1 KiB) per load. Each LPS-lane group runs its own online
// softmax over every NG-th slot of the split (NG = 256 / LPS groups); the
// streams are merged through LDS against the block's largest running max.
#pragma once

#include "common.h"

namespace egpt {

constexpr int kAttnThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;

// Geometry of one attention block of NT threads over rows of D elements of T:
// a lane issues LPR 16-byte loads per K (and V) row, so it owns EPL contiguous
// elements; LPS lanes cover a row; the block runs NG independent softmax
// streams, each advancing U slots per iteration.
//   LPR 1: 16 lanes per 128-element bf16 row, every load instruction of a
//          wavefront reads 1 KiB of 4 consecutive rows (the layout used).
//   LPR > 1: fewer lanes per row, each owning LPR * 16 contiguous bytes: less
//          cross-lane reduction and softmax work per slot, but every load
//          instruction then touches 16 rows; measured slower on the MI355X
//          with non-temporal loads (41 vs 24 us at L = 32768), so kept only as
//          a tuning option.
// For bf16, q . k runs on packed bf16 pairs (v_dot2_f32_bf16) in either layout.
template <typename T, int D, int NT = kAttnThreads, int LPR = 1, int U = 4>
struct AttnGeom {
  static constexpr int EPV = 16 / Elem<T>::kBytes;  // elements per 16-byte load
  static constexpr int EPL = EPV * LPR;             // elements per lane
  static constexpr int LPS = D / EPL;               // lanes per slot
  static constexpr int NG = NT / LPS;               // independent softmax streams per block
  static constexpr int kUnroll = U;
  static_assert(LPS >= 1 && LPS <= 64 && (kWave % LPS) == 0 && D % EPL == 0, "unsupported head dim / layout");
};

template <typename T>
constexpr bool kAttnDot2 = __is_same(T, __bf16);  // q . k on packed bf16 pairs

// 2^x for softmax weights (x <= 0): the hardware v_exp_f32 alone. exp2f adds a
// range reduction (compare, select, add, ldexp) only so that results below
// 2^-126 come out as denormals instead of 0; a weight that small is below the
// fp32 resolution of the sums it joins (each holds a term of weight 1).
__device__ __forceinline__ float exp2_softmax(float x) { return __builtin_amdgcn_exp2f(x); }

// K/V rows in flight for one softmax stream: U slots, LPR 16-byte loads each.
template <int LPR, int U>
struct AttnPipe {
  u32x4 kr[U][LPR], vr[U][LPR];
};

// Loads of one iteration of a stream: slots n0 + u * NG. Every lane loads, so
// the wait counts stay exact: a slot at or past `end` reads slot 0 instead (in
// bounds and live for any position), and attn_mac() masks it out.
template <typename Geo, typename T, int LPR, int U>
__device__ __forceinline__ void attn_issue(AttnPipe<LPR, U>& pp, const T* __restrict__ kb, int64_t k_sn,
                                           const T* __restrict__ vb, int64_t v_sn, int64_t n0, int64_t end) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t n = n0 + (int64_t)u * Geo::NG;
    const int64_t nn = n < end ? n : 0;
#pragma unroll
    for (int j = 0; j < LPR; ++j) {
      // K and V are read once per call: non-temporal loads stream them past
      // the caches (measured 5.5 vs 4.9 TB/s at L = 32768, 16 q / 8 kv heads)
      pp.kr[u][j] = ld16_stream(kb + nn * k_sn + j * Geo::EPV);
      pp.vr[u][j] = ld16_stream(vb + nn * v_sn + j * Geo::EPV);
    }
  }
}

// Issue this thread's first K/V loads of slots [start, end); attn_partial()
// continues from them. Splitting the two lets a caller overlap the first round
// trip with work of its own (computing the query).
template <typename Geo, typename T, int LPR, int U>
__device__ __forceinline__ void attn_begin(AttnPipe<LPR, U>& pp, const T* __restrict__ kbase, int64_t k_sn,
                                           const T* __restrict__ vbase, int64_t v_sn, int64_t start, int64_t end) {
  const int tid = threadIdx.x;
  const int d0 = (tid % Geo::LPS) * Geo::EPL;
  attn_issue<Geo>(pp, kbase + d0, k_sn, vbase + d0, v_sn, start + tid / Geo::LPS, end);
  // Keep the caller's query arithmetic below the loads: left free, the scheduler
  // interleaves it with the address arithmetic, and its wait for the query rows
  // then holds the K/V loads back by one round trip.
  __builtin_amdgcn_sched_barrier(0);
}

// Packed bf16 pairs of EPL fp32 values that are exact bf16 (queries, new keys).
template <int EPL>
__device__ __forceinline__ void pack_bf16(const float (&x)[EPL], uint32_t (&p)[EPL / 2]) {
#pragma unroll
  for (int i = 0; i < EPL / 2; ++i) p[i] = (uint32_t)f32_to_bf16(x[2 * i]) | ((uint32_t)f32_to_bf16(x[2 * i + 1]) << 16);
}

// This lane's share of q . k for one slot: fp32 products and sums (bf16 pairs
// through v_dot2_f32_bf16 when T is bf16).
template <typename Geo, typename T, int LPR>
__device__ __forceinline__ float attn_qk(const u32x4 (&kr)[LPR], const float (&qf)[Geo::EPL],
                                         const uint32_t (&qp)[Geo::EPL / 2]) {
  float p = 0.f;
  if constexpr (kAttnDot2<T>) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int j = 0; j < LPR; ++j) {
      const uint32_t w[4] = {kr[j].x, kr[j].y, kr[j].z, kr[j].w};
#pragma unroll
      for (int i = 0; i < 4; ++i)
        p = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w[i]),
                                            __builtin_bit_cast(bf16x2_t, qp[4 * j + i]), p, false);
    }
  } else {
#pragma unroll
    for (int j = 0; j < LPR; ++j) {
      float kf[Geo::EPV];
      Elem<T>::unpack(kr[j], kf);
#pragma unroll
      for (int e = 0; e < Geo::EPV; ++e) p = fmaf(qf[j * Geo::EPV + e], kf[e], p);
    }
  }
  return p;
}

// One iteration of a softmax stream over the slots in pp (n0 + u * NG, those
// before `end` valid): scores (q . k) * scale in fp32, online-softmax update of
// (m, l, acc) for the G query heads.
template <typename Geo, typename T, int G, int LPR, int U>
__device__ __forceinline__ void attn_mac(const AttnPipe<LPR, U>& pp, const float (&qf)[G][Geo::EPL],
                                         const uint32_t (&qp)[G][Geo::EPL / 2], int64_t n0, int64_t end, float scale,
                                         float (&m)[G], float (&l)[G], float (&acc)[G][Geo::EPL]) {
  constexpr int EPL = Geo::EPL;
  constexpr int EPV = Geo::EPV;
  constexpr int LPS = Geo::LPS;
  constexpr int NG = Geo::NG;
  bool valid[U];
#pragma unroll
  for (int u = 0; u < U; ++u) valid[u] = n0 + (int64_t)u * NG < end;
  float s[U][G];
#pragma unroll
  for (int u = 0; u < U; ++u) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float p = group_sum<LPS>(attn_qk<Geo, T, LPR>(pp.kr[u], qf[g], qp[g])) * scale;
      s[u][g] = valid[u] ? p : -INFINITY;  // the reference's fp32 logit: (q . k) * scale
    }
  }
  float vf[U][EPL];
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int j = 0; j < LPR; ++j) {
      Elem<T>::unpack(pp.vr[u][j], &vf[u][j * EPV]);
#pragma unroll
      for (int e = 0; e < EPV; ++e) vf[u][j * EPV + e] = valid[u] ? vf[u][j * EPV + e] : 0.f;
    }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float mt = m[g];
#pragma unroll
    for (int u = 0; u < U; ++u) mt = fmaxf(mt, s[u][g]);
    // No valid slot yet in this stream (mt = -inf): exponents from 0 instead
    // give alpha = 0 and p = 0, so the state stays (-inf, 0, 0) with no branch.
    const float mref = mt == -INFINITY ? 0.f : mt;
    const float alpha = exp2_softmax((m[g] - mref) * kLog2e);
    float p[U];
    float psum = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      p[u] = exp2_softmax((s[u][g] - mref) * kLog2e);  // 0 for invalid slots
      psum += p[u];
    }
    l[g] = l[g] * alpha + psum;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      float a = acc[g][e] * alpha;
#pragma unroll
      for (int u = 0; u < U; ++u) a = fmaf(p[u], vf[u][e], a);
      acc[g][e] = a;
    }
    m[g] = mt;
  }
}

// One block's partial softmax state over slots [start, end) of one kv head, for
// the G query heads of its group (qf: this thread's EPL elements of each query,
// in fp32), continuing from attn_begin(). If xnew is set (block-uniform), one
// more slot with key xk / value xv (this thread's EPL elements, fp32) starts the
// first stream of the block: the new token of a decode step, taken from
// registers instead of being read back from the cache. The caller passes its
// arrays whatever xnew is: selecting between them and a null pointer would make
// the compiler keep them in scratch memory. Writes (m, l, acc[D]) of every query
// head to
//   ws_m[row + g * nsplit], ws_l[...], ws_acc[(row + g * nsplit) * D + d]
// where row = (b * Hq + hk * G) * nsplit + split. An empty range with no extra
// slot gives the empty state (m = -inf, l = 0, acc = 0). With `out` set (one
// split covering every live slot) the block writes the attention output itself,
// out[g * o_sh + d] = acc / l, instead of the partials: the value the combine
// would compute, whose single weight exp(m - m) is 1. Must be called by all NT
// threads of the block.
template <typename Geo, typename T, int G, int LPR, int U>
__device__ __forceinline__ void attn_partial(const float (&qf)[G][Geo::EPL], AttnPipe<LPR, U>& pp,
                                             const T* __restrict__ kbase, int64_t k_sn, const T* __restrict__ vbase,
                                             int64_t v_sn, int64_t start, int64_t end, float scale,
                                             float* __restrict__ ws_m, float* __restrict__ ws_l,
                                             float* __restrict__ ws_acc, int64_t row, int nsplit,
                                             bool xnew = false, const float* xk = nullptr, const float* xv = nullptr,
                                             T* __restrict__ out = nullptr, int64_t o_sh = 0) {
  constexpr int EPL = Geo::EPL;
  constexpr int EPV = Geo::EPV;
  constexpr int LPS = Geo::LPS;
  constexpr int NG = Geo::NG;
  constexpr int NT = NG * LPS;
  constexpr int D = EPL * LPS;
  const int tid = threadIdx.x;
  const int grp = tid / LPS;
  const int d0 = (tid % LPS) * EPL;
  kbase += d0;
  vbase += d0;

  uint32_t qp[G][EPL / 2];
#pragma unroll
  for (int g = 0; g < G; ++g) pack_bf16<EPL>(qf[g], qp[g]);

  float m[G], l[G], acc[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = 0.f;
  }

  // The extra slot starts stream 0 (block-uniform branch): its score and value
  // are in registers, so this runs while the first K/V rows are in flight and
  // the stream continues from the state (m, l, acc) = (s, 1, v).
  if (xnew) {
    uint32_t xkp[EPL / 2];
    float xkf[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) xkf[e] = xk[e];
    pack_bf16<EPL>(xkf, xkp);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float p = 0.f;
      if constexpr (kAttnDot2<T>) {
        typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
#pragma unroll
        for (int i = 0; i < EPL / 2; ++i)
          p = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, xkp[i]),
                                              __builtin_bit_cast(bf16x2_t, qp[g][i]), p, false);
      } else {
#pragma unroll
        for (int e = 0; e < EPL; ++e) p = fmaf(qf[g][e], xk[e], p);
      }
      const float sx = group_sum<LPS>(p) * scale;
      if (grp == 0) {
        m[g] = sx;
        l[g] = 1.f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] = xv[e];
      }
    }
  }

  constexpr int64_t kStep = (int64_t)NG * U;  // slots one stream advances per iteration
  // Iterations are block-uniform: stream grp handles slots start + grp + i * NG.
  // Two register buffers (pp = A, pb = B) in pairs of iterations: the loads of
  // iteration i + 1 are issued before iteration i is computed, no buffer is
  // copied, and all loads are unconditional, so each wait covers exactly the
  // iteration about to be used while the next one stays in flight.
  const int64_t n0 = start + grp;
  const int64_t nit = end > start ? (end - start + kStep - 1) / kStep : 0;
  AttnPipe<LPR, U> pb;
  int64_t it = 0;
#pragma unroll 1
  for (; it + 2 < nit; it += 2) {
    attn_issue<Geo>(pb, kbase, k_sn, vbase, v_sn, n0 + (it + 1) * kStep, end);
    __builtin_amdgcn_sched_barrier(0);
    attn_mac<Geo, T, G>(pp, qf, qp, n0 + it * kStep, end, scale, m, l, acc);
    __builtin_amdgcn_sched_barrier(0);
    attn_issue<Geo>(pp, kbase, k_sn, vbase, v_sn, n0 + (it + 2) * kStep, end);
    __builtin_amdgcn_sched_barrier(0);
    attn_mac<Geo, T, G>(pb, qf, qp, n0 + (it + 1) * kStep, end, scale, m, l, acc);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (it + 1 < nit) {
    attn_issue<Geo>(pb, kbase, k_sn, vbase, v_sn, n0 + (it + 1) * kStep, end);
    __builtin_amdgcn_sched_barrier(0);
    attn_mac<Geo, T, G>(pp, qf, qp, n0 + it * kStep, end, scale, m, l, acc);
    __builtin_amdgcn_sched_barrier(0);
    attn_mac<Geo, T, G>(pb, qf, qp, n0 + (it + 1) * kStep, end, scale, m, l, acc);
  } else if (it < nit) {
    attn_mac<Geo, T, G>(pp, qf, qp, n0 + it * kStep, end, scale, m, l, acc);
  }

  // Merge the block's NG streams against the block maximum M of their m: M
  // first (across the groups of a wavefront by lane exchanges, then across the
  // wavefronts through LDS), then every stream scales its state by
  // exp(m_s - M), one exponential per stream and query head, and the NG scaled
  // states are summed through LDS in a fixed order (reproducible results).
  constexpr int kWaves = NT / kWave;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  __shared__ float sm_max[kWaves][G];
  __shared__ float sm_l[NG][G];
  __shared__ float sm_acc[NG][G][D];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float v = m[g];  // uniform over the LPS lanes of a stream
#pragma unroll
    for (int off = LPS; off < kWave; off *= 2) {
      if (off == 8) {
        v = fmaxf(v, xor8(v));
      } else if (off == 16) {
        const LanePair p = pair16(v);
        v = fmaxf(p.lo, p.hi);
      } else if (off == 32) {
        const LanePair p = pair32(v);
        v = fmaxf(p.lo, p.hi);
      } else {
        v = fmaxf(v, __shfl_xor(v, off, kWave));
      }
    }
    if (lane == 0) sm_max[wave][g] = v;
  }
  lds_barrier();
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float mb = sm_max[0][g];
#pragma unroll
    for (int j = 1; j < kWaves; ++j) mb = fmaxf(mb, sm_max[j][g]);
    const float w = m[g] == -INFINITY ? 0.f : exp2f((m[g] - mb) * kLog2e);  // 0 for an empty stream
#pragma unroll
    for (int e = 0; e < EPL; ++e) sm_acc[grp][g][d0 + e] = acc[g][e] * w;
    if (tid % LPS == 0) sm_l[grp][g] = l[g] * w;
  }
  lds_barrier();
  for (int i = tid; i < G * D; i += NT) {
    const int g = i / D;
    const int d = i % D;
    float mx = sm_max[0][g];
#pragma unroll
    for (int j = 1; j < kWaves; ++j) mx = fmaxf(mx, sm_max[j][g]);
    float a = 0.f, ls = 0.f;
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      a += sm_acc[j][g][d];
      ls += sm_l[j][g];
    }
    if (out) {
      Elem<T>::store1(out + (int64_t)g * o_sh + d, a / ls);
      continue;
    }
    const int64_t slot = row + (int64_t)g * nsplit;
    ws_acc[slot * D + d] = a;
    if (d == 0) {
      ws_m[slot] = mx;
      ws_l[slot] = ls;
    }
  }
}

// ---------------------------------------------------------------- q . k on MFMA
//
// The whole-group form for bf16 caches, D = 128 and G = 4 query heads per kv head
// (attn_partial_mfma; written for G = 2 too, see kAttnMfma). A wavefront runs ONE softmax stream over tiles of 16
// slots, wavefront w of the block taking tiles w, w + 4, ... of the split:
//   * scores: S[16 slots x 16 cols] = K[16 x 128] . Q^T[128 x 16] by four
//     v_mfma_f32_16x16x32_bf16 (bf16 products exact, fp32 sums), query heads in
//     columns 0..G-1. K goes straight from memory into the A operand: lane l
//     loads 16 bytes of slot l % 16 at dims 32 c + 8 (l / 16), so a tile is four
//     16-byte loads per lane and every byte is read once. Lane l then holds the
//     scores of head l % 16 for slots 4 (l / 16) + r, r = 0..3.
//   * softmax: per head over the tile's 16 slots (own 4, then the lanes l ^ 16 and
//     l ^ 32), the online update in fp32 as in attn_mac; each lane keeps (m, l) of
//     head l % 16.
//   * p . v stays in fp32 FMAs (the reference's tl.sum(p * v)): the tile's p go
//     to a 16 x 16 LDS tile of the wavefront, and lane l, holding 8 dims
//     8 (l % 16) .. of V rows 4 t + l / 16 (t = 0..3, the row layout of
//     attn_issue), reads p of its row for the G heads. acc then sums a quarter of
//     the slots per lane group, all under the stream's one max, so the four groups
//     are added at the end with no rescaling.
// Per 16 slots this is 4 MFMAs and about 8 G + 70 VALU instructions per
// wavefront, against about 33 per slot for the vector form at G = 4 (16-lane
// reductions of every q . k). The four streams of a block merge as in attn_partial.
typedef __bf16 bf16x8_mt __attribute__((ext_vector_type(8)));
typedef float f32x4_mt __attribute__((ext_vector_type(4)));

// Whether a block of G query heads over D-element rows of T takes the MFMA form:
// at 4 query heads per kv head (Qwen3-8B's 32 / 8). Measured on the MI355X against
// the vector form, cold: stand-alone attention at 32 / 8 heads 32.4 -> 28.8 us at
// L = 32768 and 21.0 -> 18.3 us at 16384; the Qwen3-8B step after an 8192-token
// prompt 457 -> 471 tok/s. At 2 heads per kv head (16 / 8) the vector form's
// arithmetic is not what bounds it: the MFMA form was within noise at 4096-32768
// slots (27.4 against 28.1 us at 32768) and slower at 256 (6.5 against 5.7 us), and
// the Qwen3-1.7B step at a 3500-token prompt 0.4% slower; G = 2 keeps the vector form.
template <typename T, int D, int G>
constexpr bool kAttnMfma = __is_same(T, __bf16) && D == 128 && G == 4;

constexpr int kMfmaSlots = 16;  // slots of one wavefront tile
// The wavefront's p tile in LDS: p(slot s, head h) at (s % 4) * 68 + (s / 4) * 16 + h.
// Lanes store p of slots 4 (l / 16) + r (one r at a time: 64 consecutive words) and
// read the G heads of slot 4 t + l / 16 (the four lane groups 68 words apart: four
// distinct banks), so neither side conflicts on banks.
constexpr int kPTileStride = 68;
constexpr int kPTileWords = 4 * kPTileStride;

struct MfmaKV {
  u32x4 k[4];  // A operand: 16 slots x 32 dims per chunk
  u32x4 v[4];  // row layout: slot 4 t + l / 16, dims 8 (l % 16) ..
};

// Loads of the tile [n0, n0 + 16) of a wavefront. Slots at or past `end` read
// slot 0 instead (in bounds and live for any position) and are masked out of the
// softmax, so every load is unconditional and the wait counts stay exact.
__device__ __forceinline__ void mfma_issue(MfmaKV& t, const __bf16* __restrict__ kb, int64_t k_sn,
                                           const __bf16* __restrict__ vb, int64_t v_sn, int64_t n0, int64_t end) {
  const int lane = threadIdx.x % kWave;
  const int64_t nk = n0 + (lane & 15);
  const __bf16* kr = kb + (nk < end ? nk : 0) * k_sn + 8 * (lane >> 4);
#pragma unroll
  for (int c = 0; c < 4; ++c) t.k[c] = ld16_stream(kr + 32 * c);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t nv = n0 + 4 * r + (lane >> 4);
    t.v[r] = ld16_stream(vb + (nv < end ? nv : 0) * v_sn + 8 * (lane & 15));
  }
}

// One tile of a wavefront's stream: qb are the B fragments of Q^T (4 chunks of 32
// dims), (m, l) the state of head lane % 16, acc[g][e] the row-layout sums of head
// g at dim 8 (lane % 16) + e, lds_p the wavefront's 16 x 16 p tile.
template <int G>
__device__ __forceinline__ void mfma_mac(const MfmaKV& t, const bf16x8_mt (&qb)[4], int64_t n0, int64_t end,
                                         float scale, float& m, float& l, float (&acc)[G][8], float* lds_p) {
  const int lane = threadIdx.x % kWave;
  f32x4_mt sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < 4; ++c)
    sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_mt, t.k[c]), qb[c], sc, 0, 0, 0);
  float sv[4];
  float mx = -INFINITY;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t slot = n0 + 4 * (lane >> 4) + r;
    sv[r] = slot < end ? sc[r] * scale : -INFINITY;  // the reference's fp32 logit: (q . k) * scale
    mx = fmaxf(mx, sv[r]);
  }
  LanePair pr = pair16(mx);
  mx = fmaxf(pr.lo, pr.hi);
  pr = pair32(mx);
  mx = fmaxf(pr.lo, pr.hi);
  const float mt = fmaxf(m, mx);
  const float mref = mt == -INFINITY ? 0.f : mt;  // no valid slot yet: the state stays (-inf, 0, 0)
  const float alpha = exp2_softmax((m - mref) * kLog2e);
  float ps = 0.f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float p = exp2_softmax((sv[r] - mref) * kLog2e);  // 0 for masked slots
    ps += p;
    lds_p[r * kPTileStride + (lane >> 4) * 16 + (lane & 15)] = p;
  }
  pr = pair16(ps);
  ps = pr.lo + pr.hi;
  pr = pair32(ps);
  ps = pr.lo + pr.hi;
  l = l * alpha + ps;
  m = mt;
  // the p tile is read back across lanes of this wavefront only
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
  float ag[G];
  bool same = true;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    ag[g] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha), g));
    same = same && ag[g] == 1.f;
  }
  if (!same) {  // wave-uniform: once the running maxima settle, alpha is exactly 1 and acc needs no rescale
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] *= ag[g];
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float vf[8];
    Elem<__bf16>::unpack(t.v[r], vf);
    const float* prow = lds_p + (lane >> 4) * kPTileStride + r * 16;
    float pg[G];
#pragma unroll
    for (int g = 0; g < G; ++g) pg[g] = prow[g];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(pg[g], vf[e], acc[g][e]);
  }
  // the next tile's p must not overwrite this one before every lane has read it
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// The whole-group partial state over slots [start, end) for G query heads, a
// stream per wavefront (see above), continuing from the first tile `t0` that the
// caller issued at start + 16 * wave. qb: this lane's B fragments of Q^T (column
// lane % 16 is query head lane % 16 of the group; zero past G). If xnew is set,
// the new token (key xk, value xv: this lane's 8 dims 8 (lane % 16) .., fp32;
// qf: this lane's 8 dims of every query head) starts wavefront 0's stream. Output
// as attn_partial: partials at `row`, or `out` when one split covers every slot.
// Must be called by all kAttnThreads threads of the block.
template <int G>
__device__ __forceinline__ void attn_partial_mfma(const bf16x8_mt (&qb)[4], MfmaKV& t0, const __bf16* __restrict__ kb,
                                                  int64_t k_sn, const __bf16* __restrict__ vb, int64_t v_sn,
                                                  int64_t start, int64_t end, float scale, float* __restrict__ ws_m,
                                                  float* __restrict__ ws_l, float* __restrict__ ws_acc, int64_t row,
                                                  int nsplit, bool xnew, const float (&qf)[G][8],
                                                  const float (&xk)[8], const float (&xv)[8], __bf16* __restrict__ out,
                                                  int64_t o_sh) {
  constexpr int kW = kAttnThreads / kWave;
  constexpr int D = 128;
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  __shared__ float lds_p[kW][kPTileWords];

  float m = -INFINITY, l = 0.f, acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  if (xnew && wave == 0) {  // block-uniform: (s, 1, v) of the new token, v counted in lane group 0 only
    float sg[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float p = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) p = fmaf(qf[g][e], xk[e], p);
      sg[g] = group_sum<16>(p) * scale;
    }
    const int h = lane & 15;
#pragma unroll
    for (int g = 0; g < G; ++g)
      if (h == g) m = sg[g];
    l = h < G ? 1.f : 0.f;
    if (h >= G) m = -INFINITY;
    if ((lane >> 4) == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = xv[e];
    }
  }

  // Two register buffers in pairs of tiles, as attn_partial: the loads of the next
  // tile are issued before the current one is computed.
  const int64_t step = (int64_t)kMfmaSlots * kW;
  const int64_t n0 = start + (int64_t)kMfmaSlots * wave;
  const int64_t nit = end > n0 ? (end - n0 + step - 1) / step : 0;
  MfmaKV t1;
  int64_t it = 0;
#pragma unroll 1
  for (; it + 2 < nit; it += 2) {
    mfma_issue(t1, kb, k_sn, vb, v_sn, n0 + (it + 1) * step, end);
    __builtin_amdgcn_sched_barrier(0);
    mfma_mac<G>(t0, qb, n0 + it * step, end, scale, m, l, acc, lds_p[wave]);
    __builtin_amdgcn_sched_barrier(0);
    mfma_issue(t0, kb, k_sn, vb, v_sn, n0 + (it + 2) * step, end);
    __builtin_amdgcn_sched_barrier(0);
    mfma_mac<G>(t1, qb, n0 + (it + 1) * step, end, scale, m, l, acc, lds_p[wave]);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (it + 1 < nit) {
    mfma_issue(t1, kb, k_sn, vb, v_sn, n0 + (it + 1) * step, end);
    __builtin_amdgcn_sched_barrier(0);
    mfma_mac<G>(t0, qb, n0 + it * step, end, scale, m, l, acc, lds_p[wave]);
    __builtin_amdgcn_sched_barrier(0);
    mfma_mac<G>(t1, qb, n0 + (it + 1) * step, end, scale, m, l, acc, lds_p[wave]);
  } else if (it < nit) {
    mfma_mac<G>(t0, qb, n0 + it * step, end, scale, m, l, acc, lds_p[wave]);
  }

  // The four lane groups of a wavefront hold sums over disjoint slots under one max.
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      LanePair q2 = pair16(acc[g][e]);
      const float a2 = q2.lo + q2.hi;
      q2 = pair32(a2);
      acc[g][e] = q2.lo + q2.hi;
    }
  // Block merge of the kW streams against their largest max, in wavefront order.
  __shared__ float sm_max[kW][G];
  __shared__ float sm_l[kW][G];
  __shared__ float sm_acc[kW][G][D];
  float mg[G], lg[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    mg[g] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), g));
    lg[g] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(l), g));
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) sm_max[wave][g] = mg[g];
  }
  lds_barrier();
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float mb = sm_max[0][g];
#pragma unroll
    for (int j = 1; j < kW; ++j) mb = fmaxf(mb, sm_max[j][g]);
    const float w = mg[g] == -INFINITY ? 0.f : exp2f((mg[g] - mb) * kLog2e);
    if (lane < 16) {
#pragma unroll
      for (int e = 0; e < 8; ++e) sm_acc[wave][g][8 * lane + e] = acc[g][e] * w;
    }
    if (lane == 0) sm_l[wave][g] = lg[g] * w;
  }
  lds_barrier();
  for (int i = tid; i < G * D; i += kAttnThreads) {
    const int g = i / D;
    const int d = i % D;
    float mx = sm_max[0][g];
#pragma unroll
    for (int j = 1; j < kW; ++j) mx = fmaxf(mx, sm_max[j][g]);
    float a = 0.f, ls = 0.f;
#pragma unroll
    for (int j = 0; j < kW; ++j) {
      a += sm_acc[j][g][d];
      ls += sm_l[j][g];
    }
    if (out) {
      Elem<__bf16>::store1(out + (int64_t)g * o_sh + d, a / ls);
      continue;
    }
    const int64_t slot = row + (int64_t)g * nsplit;
    ws_acc[slot * D + d] = a;
    if (d == 0) {
      ws_m[slot] = mx;
      ws_l[slot] = ls;
    }
  }
}

// The partial-softmax reduce of one (row, query head),
//   out[d] = sum_s w_s acc_s[d] / sum_s w_s l_s,  w_s = exp(m_s - max_j m_j),
// for all D elements by a block of NT threads. The splits are dealt round-robin to NT / D thread groups (one thread
// per element d in each group); a group walks its splits 8 at a time with
// independent loads, and the groups' sums are added in group order, so the
// result is fixed for a given split count. Returns true on the threads of group
// 0, whose `out` holds element d = threadIdx.x. Empty splits carry m = -inf,
// l = 0 and acc = 0, so their weight and terms are 0. Call from all NT threads.
template <int D, int NT>
__device__ __forceinline__ bool attn_combine_block(const float* __restrict__ mrow, const float* __restrict__ lrow,
                                                   const float* __restrict__ arow, int nsplit, float& out) {
  static_assert(NT % D == 0 && NT % kWave == 0, "block must tile the head dimension");
  constexpr int kParts = NT / D;
  constexpr int kUn = 8;
  __shared__ float red[NT / kWave];
  __shared__ float part_a[kParts][D];
  __shared__ float part_l[kParts];
  const int tid = threadIdx.x;
  const int d = tid % D;
  const int part = tid / D;
  float mx = -INFINITY;
  for (int s = tid; s < nsplit; s += NT) mx = fmaxf(mx, mrow[s]);
  mx = wave_max(mx);
  if ((tid & (kWave - 1)) == 0) red[tid / kWave] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int j = 1; j < NT / kWave; ++j) mx = fmaxf(mx, red[j]);
  float a = 0.f, ls = 0.f;
  int s = part;
  for (; s + (kUn - 1) * kParts < nsplit; s += kUn * kParts) {
    float ms[kUn], lv[kUn], av[kUn];
#pragma unroll
    for (int u = 0; u < kUn; ++u) {
      const int su = s + u * kParts;
      ms[u] = mrow[su];
      lv[u] = lrow[su];
      av[u] = arow[(int64_t)su * D + d];
    }
#pragma unroll
    for (int u = 0; u < kUn; ++u) {
      const float wgt = ms[u] == -INFINITY ? 0.f : exp2f((ms[u] - mx) * kLog2e);
      a = fmaf(wgt, av[u], a);
      ls = fmaf(wgt, lv[u], ls);
    }
  }
  for (; s < nsplit; s += kParts) {
    const float msv = mrow[s];
    const float wgt = msv == -INFINITY ? 0.f : exp2f((msv - mx) * kLog2e);
    a = fmaf(wgt, arow[(int64_t)s * D + d], a);
    ls = fmaf(wgt, lrow[s], ls);
  }
  part_a[part][d] = a;
  if (d == 0) part_l[part] = ls;
  __syncthreads();
  if (part != 0) return false;
  float at = part_a[0][d], lt = part_l[0];
#pragma unroll
  for (int p = 1; p < kParts; ++p) {
    at += part_a[p][d];
    lt += part_l[p];
  }
  out = at / lt;
  return true;
}

// Split `len` live slots into `nsplit` contiguous pieces; piece `split` is [start, end).
__device__ __forceinline__ void attn_split_range(int64_t len, int nsplit, int split, int64_t& start, int64_t& end) {
  const int64_t chunk = (len + nsplit - 1) / nsplit;
  start = (int64_t)split * chunk;
  end = start + chunk < len ? start + chunk : len;
}

}  // namespace egpt
