// Split-K GQA decode attention (flash decoding) for gfx950 (MI355X).
//
// One query per (batch row, query head). Query head h reads kv head h / G,
// G = Hq / Hkv. The live key range of row b is slots 0..position[b]; it is cut
// into `nsplit` contiguous pieces at run time (the position is read on the
// device, so a captured graph keeps working as the sequence grows). Each block
// owns one (b, kv head, split) and serves all G query heads of the group, so
// every K/V byte is read once. A second kernel merges the per-split partial
// softmax states.
//
// Semantics follow the reference's Triton pair (research/phase5/decode_attention.py:
// _split_kernel :22-56, _combine_kernel :59-71): scores (q . k) * scale in fp32,
// an fp32 online softmax per split keeping (max, sum, acc[D]), and the combine
//   w_i = exp(m_i - max_j m_j),  out = sum_i w_i acc_i / sum_i w_i l_i,
// where empty splits carry m = -inf and weight 0. Only slots <= position[b] are
// ever loaded. Exponentials are exp2((x - max) * log2 e): the same function as
// the reference's exp, rounded relative to the max-subtracted logit; the
// summation order differs from SDPA, so results are not bit-exact against it.
//
// Layout inside a block (256 threads, 4 wavefronts): one 16-byte load per lane
// covers EPL = 16 / sizeof(T) elements of a row, LPS = D / EPL lanes cover one
// slot (16 lanes for bf16 with D = 128), so a wavefront reads 64 / LPS
// consecutive slots (1 KiB) per load. Each LPS-lane group runs its own online
// softmax over every NG-th slot of the split (NG = 256 / LPS groups); the
// groups are merged by cross-lane butterflies within a wavefront, then the four
// wavefronts through LDS.
#include "common.h"

namespace egpt {
namespace {

constexpr int kAttnThreads = 256;
constexpr int kUnroll = 4;  // slots per group per iteration; double-buffered, so 2 x 4 K and V rows in flight
constexpr float kLog2e = 1.4426950408889634f;

template <typename T, int D, int G>
__global__ __launch_bounds__(kAttnThreads) void attn_split_kernel(
    const T* __restrict__ q, int64_t q_sb, int64_t q_sh, const T* __restrict__ k, int64_t k_sb, int64_t k_sh,
    int64_t k_sn, const T* __restrict__ v, int64_t v_sb, int64_t v_sh, int64_t v_sn,
    const int64_t* __restrict__ position, int64_t pos_stride, float* __restrict__ ws_m, float* __restrict__ ws_l,
    float* __restrict__ ws_acc, int Hkv, int cap, int nsplit, float scale) {
  constexpr int EPL = 16 / Elem<T>::kBytes;  // elements per 16-byte lane load
  constexpr int LPS = D / EPL;               // lanes per slot
  constexpr int NG = kAttnThreads / LPS;     // independent softmax streams per block
  static_assert(LPS >= 1 && LPS <= 64 && (kWave % LPS) == 0, "unsupported head dim / dtype");

  const int tid = threadIdx.x;
  const int grp = tid / LPS;
  const int sub = tid % LPS;
  const int d0 = sub * EPL;
  const int bh = blockIdx.x;  // b * Hkv + kv head
  const int b = bh / Hkv;
  const int hk = bh % Hkv;
  const int split = blockIdx.y;
  const int Hq = Hkv * G;

  int64_t len = position[(int64_t)b * pos_stride] + 1;
  len = len < 1 ? 1 : (len > cap ? cap : len);
  const int64_t chunk = (len + nsplit - 1) / nsplit;
  const int64_t start = (int64_t)split * chunk;
  const int64_t end = start + chunk < len ? start + chunk : len;

  // Query heads of this group in fp32.
  float qf[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const T* qp = q + (int64_t)b * q_sb + (int64_t)(hk * G + g) * q_sh + d0;
    Elem<T>::unpack(ld16(qp), qf[g]);
  }

  float m[G], l[G], acc[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = 0.f;
  }

  const T* kbase = k + (int64_t)b * k_sb + (int64_t)hk * k_sh + d0;
  const T* vbase = v + (int64_t)b * v_sb + (int64_t)hk * v_sh + d0;
  constexpr int64_t kStep = (int64_t)NG * kUnroll;  // slots one group advances per iteration

  // Register double buffer: the loads of iteration i+1 are issued before the
  // arithmetic of iteration i, so each wavefront keeps 2 * kUnroll K and V rows
  // in flight instead of waiting on every round trip.
  u32x4 kr[kUnroll], vr[kUnroll];
  auto issue = [&](int64_t base, u32x4* kd, u32x4* vd) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t n = base + (int64_t)u * NG;
      const int64_t nn = n < end ? n : base;  // never touch slots past the live range
      kd[u] = ld16(kbase + nn * k_sn);
      vd[u] = ld16(vbase + nn * v_sn);
    }
  };
  int64_t n0 = start + grp;
  if (n0 < end) issue(n0, kr, vr);
  for (; n0 < end; n0 += kStep) {
    u32x4 kc[kUnroll], vc[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      kc[u] = kr[u];
      vc[u] = vr[u];
    }
    if (n0 + kStep < end) issue(n0 + kStep, kr, vr);

    float s[kUnroll][G];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
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
    float vf[kUnroll][EPL];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) Elem<T>::unpack(vc[u], vf[u]);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mt = m[g];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) mt = fmaxf(mt, s[u][g]);
      // slot n0 is always valid, so mt is finite; exp(x) = exp2(x * log2 e) after
      // the max is subtracted, so the rounding is relative to the small difference
      const float alpha = exp2f((m[g] - mt) * kLog2e);
      float p[kUnroll];
      float psum = 0.f;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        p[u] = exp2f((s[u][g] - mt) * kLog2e);  // 0 for invalid slots
        psum += p[u];
      }
      l[g] = l[g] * alpha + psum;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        float a = acc[g][e] * alpha;
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) a = fmaf(p[u], vf[u][e], a);
        acc[g][e] = a;
      }
      m[g] = mt;
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
    const int64_t slot = ((int64_t)b * Hq + hk * G + g) * nsplit + split;
    ws_acc[slot * D + d] = a;
    if (d == 0) {
      ws_m[slot] = mx;
      ws_l[slot] = ls;
    }
  }
}

// Partial-softmax reduce: one block per (b, query head), one thread per d.
template <typename T, int D>
__global__ __launch_bounds__(D) void attn_combine_kernel(const float* __restrict__ ws_m,
                                                         const float* __restrict__ ws_l,
                                                         const float* __restrict__ ws_acc, T* __restrict__ out,
                                                         int64_t o_sb, int64_t o_sh, int Hq, int nsplit) {
  const int bh = blockIdx.x;
  const int b = bh / Hq;
  const int h = bh % Hq;
  const int d = threadIdx.x;
  const float* mrow = ws_m + (int64_t)bh * nsplit;
  const float* lrow = ws_l + (int64_t)bh * nsplit;
  const float* arow = ws_acc + (int64_t)bh * nsplit * D;
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
  Elem<T>::store1(out + (int64_t)b * o_sb + (int64_t)h * o_sh + d, a / ls);
}

struct AttnArgs {
  const void *q, *k, *v;
  int64_t q_sb, q_sh, k_sb, k_sh, k_sn, v_sb, v_sh, v_sn;
  const int64_t* position;
  int64_t pos_stride;
  void* out;
  int64_t o_sb, o_sh;
  float *ws_m, *ws_l, *ws_acc;
  int B, Hq, Hkv, cap, nsplit;
  float scale;
};

template <typename T, int D, int G>
int launch_attn(const AttnArgs& a, hipStream_t st) {
  dim3 grid((unsigned)(a.B * a.Hkv), (unsigned)a.nsplit);
  hipLaunchKernelGGL((attn_split_kernel<T, D, G>), grid, dim3(kAttnThreads), 0, st, (const T*)a.q, a.q_sb, a.q_sh,
                     (const T*)a.k, a.k_sb, a.k_sh, a.k_sn, (const T*)a.v, a.v_sb, a.v_sh, a.v_sn, a.position,
                     a.pos_stride, a.ws_m, a.ws_l, a.ws_acc, a.Hkv, a.cap, a.nsplit, a.scale);
  if (hipGetLastError() != hipSuccess) return EGPT_ERR_LAUNCH;
  hipLaunchKernelGGL((attn_combine_kernel<T, D>), dim3((unsigned)(a.B * a.Hq)), dim3(D), 0, st, a.ws_m, a.ws_l,
                     a.ws_acc, (T*)a.out, a.o_sb, a.o_sh, a.Hq, a.nsplit);
  return EGPT_LAUNCH_STATUS();
}

template <typename T, int D>
int dispatch_group(const AttnArgs& a, hipStream_t st) {
  switch (a.Hq / a.Hkv) {
    case 1: return launch_attn<T, D, 1>(a, st);
    case 2: return launch_attn<T, D, 2>(a, st);
    case 4: return launch_attn<T, D, 4>(a, st);
    case 8: return launch_attn<T, D, 8>(a, st);
    default: return EGPT_ERR_UNSUPPORTED;
  }
}

template <typename T>
int dispatch_dim(const AttnArgs& a, int D, hipStream_t st) {
  if (D == 128) return dispatch_group<T, 128>(a, st);
  if (D == 64) return dispatch_group<T, 64>(a, st);
  if (D == 32) return dispatch_group<T, 32>(a, st);
  return EGPT_ERR_UNSUPPORTED;
}

size_t attn_workspace_bytes(int B, int Hq, int D, int nsplit) {
  const size_t rows = (size_t)B * (size_t)Hq * (size_t)nsplit;
  // m and l, each rounded up to 256 bytes so acc starts aligned
  const size_t ml = ((rows * sizeof(float) + 255) / 256) * 256;
  return 2 * ml + rows * (size_t)D * sizeof(float);
}

}  // namespace
}  // namespace egpt

using namespace egpt;

extern "C" int egpt_decode_attn_default_splits(int B, int Hkv, int cap) {
  if (B < 1 || Hkv < 1 || cap < 1) return 1;
  // At least one block-iteration (4 wavefronts x 16 slots) per split, below
  // which the per-split merge dominates; no more splits than needed to give the
  // 256 CUs about 1024 blocks.
  const int by_len = (cap + 63) / 64;
  int by_grid = (1024 + B * Hkv - 1) / (B * Hkv);
  if (by_grid < 1) by_grid = 1;
  int n = by_len < by_grid ? by_len : by_grid;
  if (n > 256) n = 256;
  return n < 1 ? 1 : n;
}

extern "C" int egpt_decode_attn_workspace(int B, int Hq, int Hkv, int cap, int D, int nsplit, size_t* bytes) {
  if (!bytes || B < 1 || Hq < 1 || Hkv < 1 || cap < 1 || D < 1) return EGPT_ERR_INVALID;
  if (nsplit <= 0) nsplit = egpt_decode_attn_default_splits(B, Hkv, cap);
  *bytes = attn_workspace_bytes(B, Hq, D, nsplit);
  return EGPT_OK;
}

extern "C" int egpt_decode_attn(int dtype, const void* q, int64_t q_sb, int64_t q_sh, const void* k, int64_t k_sb,
                                int64_t k_sh, int64_t k_sn, const void* v, int64_t v_sb, int64_t v_sh, int64_t v_sn,
                                const int64_t* position, int64_t pos_stride, void* out, int64_t o_sb, int64_t o_sh,
                                void* workspace, size_t workspace_bytes, int B, int Hq, int Hkv, int cap, int D,
                                int nsplit, float scale, hipStream_t stream) {
  if (!q || !k || !v || !position || !out) return EGPT_ERR_INVALID;
  if (B < 1 || Hq < 1 || Hkv < 1 || cap < 1 || D < 1) return EGPT_ERR_INVALID;
  if (Hq % Hkv != 0) return EGPT_ERR_INVALID;
  if (dtype != EGPT_F32 && dtype != EGPT_BF16 && dtype != EGPT_F16) return EGPT_ERR_UNSUPPORTED;
  if (nsplit <= 0) nsplit = egpt_decode_attn_default_splits(B, Hkv, cap);
  const size_t esz = dtype == EGPT_F32 ? 4 : 2;
  // 16-byte vector loads of every q/k/v row
  const int64_t strides[] = {q_sb, q_sh, k_sb, k_sh, k_sn, v_sb, v_sh, v_sn};
  for (int64_t s : strides)
    if (((size_t)s * esz) % 16 != 0) return EGPT_ERR_INVALID;
  if ((uintptr_t)q % 16 || (uintptr_t)k % 16 || (uintptr_t)v % 16) return EGPT_ERR_INVALID;
  const size_t need = attn_workspace_bytes(B, Hq, D, nsplit);
  if (!workspace || workspace_bytes < need || (uintptr_t)workspace % 256) return EGPT_ERR_WORKSPACE;
  const size_t rows = (size_t)B * Hq * nsplit;
  const size_t ml = ((rows * sizeof(float) + 255) / 256) * 256;
  AttnArgs a;
  a.q = q; a.k = k; a.v = v;
  a.q_sb = q_sb; a.q_sh = q_sh;
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_sn = k_sn;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_sn = v_sn;
  a.position = position; a.pos_stride = pos_stride;
  a.out = out; a.o_sb = o_sb; a.o_sh = o_sh;
  a.ws_m = (float*)workspace;
  a.ws_l = (float*)((char*)workspace + ml);
  a.ws_acc = (float*)((char*)workspace + 2 * ml);
  a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.cap = cap; a.nsplit = nsplit;
  a.scale = scale;
  switch (dtype) {
    case EGPT_BF16: return dispatch_dim<__bf16>(a, D, stream);
    case EGPT_F16: return dispatch_dim<_Float16>(a, D, stream);
    default: return dispatch_dim<float>(a, D, stream);
  }
}
