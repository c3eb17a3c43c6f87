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
// groups are merged by cross-lane butterflies within a wavefront, then the four
// wavefronts through LDS.
#pragma once

#include "common.h"

namespace egpt {

constexpr int kAttnThreads = 256;
constexpr int kAttnUnroll = 4;  // slots per group per iteration; double-buffered, so 2 x 4 K and V rows in flight
constexpr float kLog2e = 1.4426950408889634f;

template <typename T, int D>
struct AttnGeom {
  static constexpr int EPL = 16 / Elem<T>::kBytes;  // elements per 16-byte lane load
  static constexpr int LPS = D / EPL;               // lanes per slot
  static constexpr int NG = kAttnThreads / LPS;     // independent softmax streams per block
  static_assert(LPS >= 1 && LPS <= 64 && (kWave % LPS) == 0, "unsupported head dim / dtype");
};

// K/V rows in flight for one softmax stream (register double buffer).
struct AttnPipe {
  u32x4 kr[kAttnUnroll], vr[kAttnUnroll];
};

template <typename T, int D>
__device__ __forceinline__ void attn_issue(AttnPipe& pp, const T* __restrict__ kb, int64_t k_sn,
                                           const T* __restrict__ vb, int64_t v_sn, int64_t base, int64_t end) {
  constexpr int NG = AttnGeom<T, D>::NG;
#pragma unroll
  for (int u = 0; u < kAttnUnroll; ++u) {
    const int64_t n = base + (int64_t)u * NG;
    const int64_t nn = n < end ? n : base;  // never touch slots past the live range
    pp.kr[u] = ld16(kb + nn * k_sn);
    pp.vr[u] = ld16(vb + nn * v_sn);
  }
}

// Issue this thread's first K/V loads of slots [start, end); attn_partial()
// continues from them. Splitting the two lets a caller overlap the first round
// trip with work of its own (computing the query).
template <typename T, int D>
__device__ __forceinline__ void attn_begin(AttnPipe& pp, const T* __restrict__ kbase, int64_t k_sn,
                                           const T* __restrict__ vbase, int64_t v_sn, int64_t start, int64_t end) {
  constexpr int EPL = AttnGeom<T, D>::EPL;
  constexpr int LPS = AttnGeom<T, D>::LPS;
  const int tid = threadIdx.x;
  const int d0 = (tid % LPS) * EPL;
  const int64_t n0 = start + tid / LPS;
  if (n0 < end) attn_issue<T, D>(pp, kbase + d0, k_sn, vbase + d0, v_sn, n0, end);
}

// One block's partial softmax state over slots [start, end) of one kv head, for
// the G query heads of its group (qf: this thread's EPL elements of each query,
// in fp32), continuing from attn_begin(). If xk is non-null, one more slot with
// key xk / value xv (this thread's EPL elements, fp32) is folded in by the
// first stream of the block: the new token of a decode step, taken from
// registers instead of being read back from the cache. Writes (m, l, acc[D])
// of every query head to
//   ws_m[row + g * nsplit], ws_l[...], ws_acc[(row + g * nsplit) * D + d]
// where row = (b * Hq + hk * G) * nsplit + split. An empty range with no extra
// slot gives the empty state (m = -inf, l = 0, acc = 0). Must be called by all
// 256 threads.
template <typename T, int D, int G>
__device__ __forceinline__ void attn_partial(const float (&qf)[G][AttnGeom<T, D>::EPL], AttnPipe& pp,
                                             const T* __restrict__ kbase, int64_t k_sn, const T* __restrict__ vbase,
                                             int64_t v_sn, int64_t start, int64_t end, float scale,
                                             float* __restrict__ ws_m, float* __restrict__ ws_l,
                                             float* __restrict__ ws_acc, int64_t row, int nsplit,
                                             const float* xk = nullptr, const float* xv = nullptr) {
  constexpr int EPL = AttnGeom<T, D>::EPL;
  constexpr int LPS = AttnGeom<T, D>::LPS;
  constexpr int NG = AttnGeom<T, D>::NG;
  const int tid = threadIdx.x;
  const int grp = tid / LPS;
  const int d0 = (tid % LPS) * EPL;
  kbase += d0;
  vbase += d0;

  float m[G], l[G], acc[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = 0.f;
  }

  constexpr int64_t kStep = (int64_t)NG * kAttnUnroll;  // slots one group advances per iteration
  // Register double buffer: the loads of iteration i+1 are issued before the
  // arithmetic of iteration i, so each wavefront keeps 2 * kAttnUnroll K and V
  // rows in flight instead of waiting on every round trip.
  for (int64_t n0 = start + grp; n0 < end; n0 += kStep) {
    u32x4 kc[kAttnUnroll], vc[kAttnUnroll];
#pragma unroll
    for (int u = 0; u < kAttnUnroll; ++u) {
      kc[u] = pp.kr[u];
      vc[u] = pp.vr[u];
    }
    if (n0 + kStep < end) attn_issue<T, D>(pp, kbase, k_sn, vbase, v_sn, n0 + kStep, end);

    float s[kAttnUnroll][G];
#pragma unroll
    for (int u = 0; u < kAttnUnroll; ++u) {
      const bool valid = n0 + (int64_t)u * NG < end;
      float kf[EPL];
      Elem<T>::unpack(kc[u], kf);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float p = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) p = fmaf(qf[g][e], kf[e], p);
        p = group_sum<LPS>(p) * scale;  // the reference's fp32 logit: (q . k) * scale
        s[u][g] = valid ? p : -INFINITY;
      }
    }
    float vf[kAttnUnroll][EPL];
#pragma unroll
    for (int u = 0; u < kAttnUnroll; ++u) Elem<T>::unpack(vc[u], vf[u]);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mt = m[g];
#pragma unroll
      for (int u = 0; u < kAttnUnroll; ++u) mt = fmaxf(mt, s[u][g]);
      // slot n0 is always valid, so mt is finite
      const float alpha = exp2f((m[g] - mt) * kLog2e);
      float p[kAttnUnroll];
      float psum = 0.f;
#pragma unroll
      for (int u = 0; u < kAttnUnroll; ++u) {
        p[u] = exp2f((s[u][g] - mt) * kLog2e);  // 0 for invalid slots
        psum += p[u];
      }
      l[g] = l[g] * alpha + psum;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        float a = acc[g][e] * alpha;
#pragma unroll
        for (int u = 0; u < kAttnUnroll; ++u) a = fmaf(p[u], vf[u][e], a);
        acc[g][e] = a;
      }
      m[g] = mt;
    }
  }

  if (xk) {  // block-uniform: the extra slot goes to stream 0
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float p = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) p = fmaf(qf[g][e], xk[e], p);
      const float sx = group_sum<LPS>(p) * scale;
      if (grp == 0) {
        const float mt = fmaxf(m[g], sx);
        const float alpha = exp2f((m[g] - mt) * kLog2e);  // 0 when the stream was empty
        const float px = exp2f((sx - mt) * kLog2e);
        l[g] = l[g] * alpha + px;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] = fmaf(px, xv[e], acc[g][e] * alpha);
        m[g] = mt;
      }
    }
  }

  // Merge the groups of each wavefront: butterflies across groups (lane
  // distance LPS, 2*LPS, ...). Both partners end with the merged state.
#pragma unroll
  for (int off = LPS; off < kWave; off *= 2) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float mo = __shfl_xor(m[g], off, kWave);
      const float lo = __shfl_xor(l[g], off, kWave);
      const float mx = fmaxf(m[g], mo);
      const float ws = mx == -INFINITY ? 0.f : exp2f((m[g] - mx) * kLog2e);
      const float wo = mx == -INFINITY ? 0.f : exp2f((mo - mx) * kLog2e);
      l[g] = l[g] * ws + lo * wo;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float ao = __shfl_xor(acc[g][e], off, kWave);
        acc[g][e] = acc[g][e] * ws + ao * wo;
      }
      m[g] = mx;
    }
  }

  // Merge the 4 wavefronts through LDS and write this split's partial state.
  constexpr int kWaves = kAttnThreads / kWave;
  __shared__ float sm_m[kWaves][G];
  __shared__ float sm_l[kWaves][G];
  __shared__ float sm_acc[kWaves][G][D];
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  if (lane < LPS) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) sm_acc[wave][g][d0 + e] = acc[g][e];
      if (lane == 0) {
        sm_m[wave][g] = m[g];
        sm_l[wave][g] = l[g];
      }
    }
  }
  __syncthreads();
  for (int i = tid; i < G * D; i += kAttnThreads) {
    const int g = i / D;
    const int d = i % D;
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < kWaves; ++j) mx = fmaxf(mx, sm_m[j][g]);
    float a = 0.f, ls = 0.f;
    if (mx != -INFINITY) {
#pragma unroll
      for (int j = 0; j < kWaves; ++j) {
        const float wj = exp2f((sm_m[j][g] - mx) * kLog2e);
        a = fmaf(wj, sm_acc[j][g][d], a);
        ls = fmaf(wj, sm_l[j][g], ls);
      }
    }
    const int64_t slot = row + (int64_t)g * nsplit;
    ws_acc[slot * D + d] = a;
    if (d == 0) {
      ws_m[slot] = mx;
      ws_l[slot] = ls;
    }
  }
}

// The partial-softmax reduce of one (row, query head) at element d:
// out = sum_s w_s acc_s[d] / sum_s w_s l_s with w_s = exp(m_s - max m).
// Splits are visited in order, so the result does not depend on timing.
__device__ __forceinline__ float attn_combine_one(const float* __restrict__ mrow, const float* __restrict__ lrow,
                                                  const float* __restrict__ arow, int nsplit, int D, int d) {
  float mx = -INFINITY;
  for (int s = 0; s < nsplit; ++s) mx = fmaxf(mx, mrow[s]);
  float a = 0.f, ls = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    const float ms = mrow[s];
    if (ms == -INFINITY) continue;  // empty split: weight 0
    const float wgt = exp2f((ms - mx) * kLog2e);
    a = fmaf(wgt, arow[(int64_t)s * D + d], a);
    ls = fmaf(wgt, lrow[s], ls);
  }
  return a / ls;
}

// Split `len` live slots into `nsplit` contiguous pieces; piece `split` is [start, end).
__device__ __forceinline__ void attn_split_range(int64_t len, int nsplit, int split, int64_t& start, int64_t& end) {
  const int64_t chunk = (len + nsplit - 1) / nsplit;
  start = (int64_t)split * chunk;
  end = start + chunk < len ? start + chunk : len;
}

}  // namespace egpt
