// Per-output-channel symmetric int8 quantisation on the device: the int8 codes and
// fp32 steps of research/realmodel/int8_linear.py:106-117 (quantize_weight),
//   s[n]    = max(max_k |w[n, k]| / 127, 1e-12)              fp32, correctly rounded
//   q[n, k] = clamp(round_half_even(w[n, k] / s[n]), -127, 127)
// with the weight first converted exactly to fp32 (the reference's `.float()`).
//
// Every operation is one IEEE fp32 operation with a single correct rounding
// (max and abs are exact; __fdiv_rn is the round-to-nearest-even quotient,
// not a reciprocal times the dividend), so the codes and steps are the same
// bits as the formula evaluated on the CPU, whatever the order of the max.
#include "common.h"

namespace egpt {
namespace {

constexpr int kQuantWaves = 4;  // one row per wavefront

template <typename T>
__device__ __forceinline__ float load_as_f32(const T* p) {
  return Elem<T>::load1(p);
}

// NaN-propagating max (torch.amax and numpy's max both propagate NaN).
__device__ __forceinline__ float max_nan(float a, float b) { return (a > b || a != a) ? a : b; }

template <int CTRL>
__device__ __forceinline__ float dpp_max(float v) {
  return max_nan(v, dpp<CTRL>(v));
}

__device__ __forceinline__ float wave_max_nan(float v) {
  v = dpp_max<kDppXor1>(v);
  v = dpp_max<kDppXor2>(v);
  v = dpp_max<kDppHalfMirror>(v);
  v = dpp_max<kDppMirror>(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return max_nan(max_nan(r0, r1), max_nan(r2, r3));
}

// Wavefront w of block b quantises row b * kQuantWaves + w: one pass for the
// row's max |w|, one for the codes (the row is then in L1 / L2). Lanes read
// consecutive elements, so each load instruction covers 64 consecutive
// elements of the row.
template <typename T>
__global__ __launch_bounds__(kQuantWaves * kWave) void quantize_rows_kernel(const T* __restrict__ w, int64_t ldw,
                                                                              int N, int K, int8_t* __restrict__ q,
                                                                              int64_t ldq, float* __restrict__ s) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * kQuantWaves + threadIdx.x / kWave;
  if (row >= N) return;
  const T* wr = w + row * ldw;
  float amax = 0.f;
  for (int k = lane; k < K; k += kWave) amax = max_nan(amax, fabsf(load_as_f32(wr + k)));
  amax = wave_max_nan(amax);
  float step = __fdiv_rn(amax, 127.0f);
  step = step < 1e-12f ? 1e-12f : step;  // clamp_min; NaN stays NaN
  if (lane == 0) s[row] = step;
  int8_t* qr = q + row * ldq;
  for (int k = lane; k < K; k += kWave) {
    const float r = rintf(__fdiv_rn(load_as_f32(wr + k), step));  // round half to even
    qr[k] = (int8_t)(int)fminf(fmaxf(r, -127.f), 127.f);
  }
}

}  // namespace
}  // namespace egpt

using namespace egpt;

extern "C" int egpt_quantize_rows(int dtype, const void* w, int64_t ldw, int N, int K, int8_t* q, int64_t ldq,
                                  float* s, hipStream_t stream) {
  if (!w || !q || !s || N < 0 || K < 1 || ldw < K || ldq < K) return EGPT_ERR_INVALID;
  if (N == 0) return EGPT_OK;
  const dim3 grid((unsigned)((N + kQuantWaves - 1) / kQuantWaves));
  const dim3 block(kQuantWaves * kWave);
  switch (dtype) {
    case EGPT_F32:
      hipLaunchKernelGGL(quantize_rows_kernel<float>, grid, block, 0, stream, (const float*)w, ldw, N, K, q, ldq, s);
      break;
    case EGPT_BF16:
      hipLaunchKernelGGL(quantize_rows_kernel<__bf16>, grid, block, 0, stream, (const __bf16*)w, ldw, N, K, q, ldq,
                         s);
      break;
    case EGPT_F16:
      hipLaunchKernelGGL(quantize_rows_kernel<_Float16>, grid, block, 0, stream, (const _Float16*)w, ldw, N, K, q,
                         ldq, s);
      break;
    default:
      return EGPT_ERR_UNSUPPORTED;
  }
  return EGPT_LAUNCH_STATUS();
}
