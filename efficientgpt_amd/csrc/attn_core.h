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

// Workgroup barrier ordering LDS only. __syncthreads() also waits for every
// outstanding global load of the wavefront (s_waitcnt vmcnt(0)), which would
// stall the block behind loads still in flight at each LDS hand-off.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

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
