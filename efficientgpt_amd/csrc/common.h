// Device helpers shared by the gfx950 decode kernels: bf16/fp16 packing, DPP
// reductions over 64-wide wavefronts, 16-byte vector loads.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/egpt.h"

namespace egpt {

constexpr int kWave = 64;

// Native 4 x 32-bit vector: one 16-byte global load (global_load_dwordx4).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- conversions

__device__ __forceinline__ float bf16_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// fp32 -> bf16, round to nearest even (v_cvt_pk_bf16_f32 on gfx950; NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  __bf16 b = (__bf16)f;
  return __builtin_bit_cast(uint16_t, b);
}

// Two fp32 -> two bf16 in one word (lo in bits 0-15), round to nearest even: one
// v_cvt_pk_bf16_f32 where two scalar conversions take two and an OR.
typedef float f32x2_cvt __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_cvt __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack2_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_cvt{lo, hi}, bf16x2_cvt));
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// Element traits for the attention kernels: storage type -> fp32 and back.
template <typename T> struct Elem;
template <> struct Elem<float> {
  static constexpr int kBytes = 4;
  __device__ static __forceinline__ void unpack(const u32x4& v, float* out) {
    out[0] = __uint_as_float(v.x); out[1] = __uint_as_float(v.y);
    out[2] = __uint_as_float(v.z); out[3] = __uint_as_float(v.w);
  }
  __device__ static __forceinline__ float load1(const void* p) { return *(const float*)p; }
  __device__ static __forceinline__ void store1(void* p, float f) { *(float*)p = f; }
};
template <> struct Elem<__bf16> {
  static constexpr int kBytes = 2;
  __device__ static __forceinline__ void unpack(const u32x4& v, float* out) {
    out[0] = bf16_lo(v.x); out[1] = bf16_hi(v.x); out[2] = bf16_lo(v.y); out[3] = bf16_hi(v.y);
    out[4] = bf16_lo(v.z); out[5] = bf16_hi(v.z); out[6] = bf16_lo(v.w); out[7] = bf16_hi(v.w);
  }
  __device__ static __forceinline__ float load1(const void* p) { return bf16_to_f32(*(const uint16_t*)p); }
  __device__ static __forceinline__ void store1(void* p, float f) { *(uint16_t*)p = f32_to_bf16(f); }
};
template <> struct Elem<_Float16> {
  static constexpr int kBytes = 2;
  __device__ static __forceinline__ void unpack(const u32x4& v, float* out) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = f16_to_f32((uint16_t)(w[i] & 0xffffu));
      out[2 * i + 1] = f16_to_f32((uint16_t)(w[i] >> 16));
    }
  }
  __device__ static __forceinline__ float load1(const void* p) { return f16_to_f32(*(const uint16_t*)p); }
  __device__ static __forceinline__ void store1(void* p, float f) { *(uint16_t*)p = f32_to_f16(f); }
};

// ---------------------------------------------------------------- loads

// Global-memory accessors. Every pointer the kernels dereference through them is
// device (global) memory; the address-space cast makes the compiler emit global_*
// instructions even for pointers it cannot trace to a kernel argument (read from
// a table in memory, say). A generic pointer would give flat_* instructions, which
// also count against lgkmcnt, so every LDS wait would then wait for them too.
template <typename T>
using global_ptr = __attribute__((address_space(1))) T*;

template <typename T>
__device__ __forceinline__ T gload(const T* p) {
  return *(global_ptr<const T>)p;
}
template <typename T>
__device__ __forceinline__ void gstore(T* p, T v) {
  *(global_ptr<T>)p = v;
}

__device__ __forceinline__ u32x4 ld16(const void* p) { return *(global_ptr<const u32x4>)p; }

// Streaming load for data read exactly once (weights): non-temporal hint keeps it
// from evicting the small, re-read operands (activations, scales) from L2.
__device__ __forceinline__ u32x4 ld16_stream(const void* p) {
  return __builtin_nontemporal_load((global_ptr<const u32x4>)p);
}

// Workgroup barrier ordering LDS only. __syncthreads() also waits for every
// outstanding global load of the wavefront (s_waitcnt vmcnt(0)), which would
// stall the block behind loads still in flight at each LDS hand-off.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---------------------------------------------------------------- loads straight into LDS
// global_load_lds_dwordx4: lane i of the load writes the 16 bytes it reads to LDS bytes 16 i .. 16 i + 15 from the
// wave-uniform base in M0 (checked on the MI355X). The loads come from inline assembly, so the compiler neither
// tracks nor waits for them: the kernel waits itself (EGPT_WAIT_VMCNT counts every vector memory operation of the
// wavefront in issue order) and then publishes the data to the other wavefronts with a barrier.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p);
}
__device__ __forceinline__ void lds_load16(uint32_t lds_base, const void* g) {
  asm volatile("global_load_lds_dwordx4 %0, off" : : "v"(g), "{m0}"(lds_base) : "memory");
}
__device__ __forceinline__ void lds_load4(uint32_t lds_base, const void* g) {
  asm volatile("global_load_lds_dword %0, off" : : "v"(g), "{m0}"(lds_base) : "memory");
}
// s_waitcnt vmcnt(n) with the other counters left alone.
#define EGPT_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

// ---------------------------------------------------------------- DPP reductions

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i within 8 lanes
constexpr int kDppMirror = 0x140;     // lane i <-> 15-i within 16 lanes

constexpr int kDppRowRor8 = 0x128;    // lane i <- lane (i + 8) mod 16 within 16 lanes: xor 8

// The values of lanes l and l ^ 16 (resp. l ^ 32) as (lower partner, upper
// partner), the same pair on both lanes: one v_permlane16_swap / v_permlane32_swap
// (gfx950) instead of an LDS-crossbar shuffle. A symmetric combine of the two
// (sum, max, the softmax merge) computed as f(lo, hi) is then bit-identical on
// both partners.
struct LanePair {
  float lo, hi;
};
__device__ __forceinline__ LanePair pair16(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return LanePair{__uint_as_float(p[0]), __uint_as_float(p[1])};
}
__device__ __forceinline__ LanePair pair32(float v) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return LanePair{__uint_as_float(p[0]), __uint_as_float(p[1])};
}
// The value of lane l ^ 8 (16-lane rows: a DPP row rotation by 8).
__device__ __forceinline__ float xor8(float v) { return dpp<kDppRowRor8>(v); }

// Sum over aligned groups of N lanes (N in 1,2,4,8,16,32,64); every lane of a
// group receives the group's total. The summation order is fixed, so results
// are bitwise reproducible run to run.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (N >= 2) v += dpp<kDppXor1>(v);
  if constexpr (N >= 4) v += dpp<kDppXor2>(v);
  if constexpr (N >= 8) v += dpp<kDppHalfMirror>(v);
  if constexpr (N >= 16) v += dpp<kDppMirror>(v);
  if constexpr (N >= 32) {
    const LanePair p = pair16(v);
    v = p.lo + p.hi;
  }
  if constexpr (N >= 64) {
    const LanePair p = pair32(v);
    v = p.lo + p.hi;
  }
  return v;
}

template <int N>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (N >= 2) v = fmaxf(v, dpp<kDppXor1>(v));
  if constexpr (N >= 4) v = fmaxf(v, dpp<kDppXor2>(v));
  if constexpr (N >= 8) v = fmaxf(v, dpp<kDppHalfMirror>(v));
  if constexpr (N >= 16) v = fmaxf(v, dpp<kDppMirror>(v));
  if constexpr (N >= 32) {
    const LanePair p = pair16(v);
    v = fmaxf(p.lo, p.hi);
  }
  if constexpr (N >= 64) {
    const LanePair p = pair32(v);
    v = fmaxf(p.lo, p.hi);
  }
  return v;
}

// Whole-wavefront sum, returned as a wave-uniform value: 16-lane DPP butterflies
// then the four row totals read out of lanes 0/16/32/48.
__device__ __forceinline__ float wave_sum(float v) {
  v = group_sum<16>(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ float wave_max(float v) {
  v = group_max<16>(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// int8 GEMV of 2 to kGemvFewRowsMax rows (qwen3_fused.hip): y rows ldy apart
// from x rows ldx apart, each row bit-identical to a one-row egpt_int8_gemv.
// EGPT_ERR_UNSUPPORTED for shapes it does not take (K not a multiple of 16 or
// past 12288, unaligned rows).
constexpr int kGemvFewRowsMax = 4;
// egpt_int8_gemv gives 3-4 rows to gemv_few_rows below this many features, where
// a wavefront owns one weight row and the launch is latency-bound (Qwen3-1.7B's
// o_proj and down_proj at 4 rows: 3.9 / 7.0 us against 4.1 / 8.2 us on MFMA); at
// and above it the conversion and four FMAs per weight byte bound the vector
// kernel, and MFMA is faster (QKV 4.4 / gate_up 8.2 / lm_head 86 us against 4.9 /
// 9.2 / 89 us).
constexpr int kGemvFewRowsWideN = 4096;
int gemv_few_rows(const void* x, int64_t ldx, const int8_t* w, int64_t ldw, const float* scale, void* y, int64_t ldy,
                  int M, int N, int K, hipStream_t st);

// The split-K prefill GEMM's partials [splits][M][N] (fp32, in the workspace) added in split order and rounded
// as int8_gemm_reduce_kernel does, o = bf16(bf16(sum) * scale[n]), then the residual update and RMSNorm of each
// row as add_rmsnorm_kernel does: resid = bf16(resid + o) (written back), y = RMSNorm(resid) * norm_w. One block
// per row; the same per-thread element order and block sum as add_rmsnorm_kernel, so the result is bit-identical
// to the reduce launch followed by egpt_add_rmsnorm. Defined with the norm kernels (qwen3_step.hip).
int launch_reduce_add_rmsnorm(const float* part, int splits, const float* scale, void* resid, int64_t ld_resid,
                              const void* norm_w, void* y, int64_t ldy, int M, int N, float eps, hipStream_t st);

// The split-K prefill GEMM's partials of the fused QKV product ([splits][rows][(Hq + 2 Hkv) D], fp32) added in
// split order and rounded as int8_gemm_reduce_kernel does, then egpt_qk_norm_rope's 16-byte form on each
// (row, head): bit-identical to the reduce launch followed by egpt_qk_norm_rope, with the qkv rows never stored.
// check_ returns EGPT_OK when the operands take that form (D 32, 64 or 128, 16-byte aligned rows and strides,
// 2-16 splits), EGPT_ERR_UNSUPPORTED or EGPT_ERR_INVALID otherwise, launching nothing. Defined with the norm
// kernels (qwen3_step.hip).
int check_reduce_qk_norm_rope(int splits, const int64_t* positions, const void* q_norm_w, const void* k_norm_w,
                              const void* cos_t, const void* sin_t, const void* q_out, int64_t ld_q,
                              const void* k_cache, const void* v_cache, int64_t cache_head_stride,
                              int64_t cache_slot_stride, int rows, int Hq, int Hkv, int D, int cap);
int launch_reduce_qk_norm_rope(const float* part, int splits, const float* scale, const int64_t* positions,
                               const void* q_norm_w, const void* k_norm_w, const void* cos_t, const void* sin_t,
                               void* q_out, int64_t ld_q, void* k_cache, void* v_cache, int64_t cache_head_stride,
                               int64_t cache_slot_stride, int rows, int Hq, int Hkv, int D, int cap, float eps,
                               hipStream_t st);

}  // namespace egpt

// Map a HIP launch result to the library's status convention.
#define EGPT_LAUNCH_STATUS() (hipGetLastError() == hipSuccess ? EGPT_OK : EGPT_ERR_LAUNCH)
