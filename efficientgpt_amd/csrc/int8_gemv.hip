// Weight-only int8 GEMV for batch-1 decode on gfx950 (MI355X).
//
//   y[m, n] = bf16( scale[n] * sum_k x[m, k] * w[n, k] ),   M <= 16
//
// Same arithmetic contract as the reference's Triton _dot16 kernel
// (research/realmodel/int8_linear.py:26-38): int8 weights are exact in the
// multiplier's input format, products and sums are fp32, the per-channel scale
// multiplies the finished fp32 sum, and the result is rounded once to bf16.
//
// Design (memory-bound: ~1 byte of weight per 2 flops at M = 1):
//   * A block is 4 wavefronts; each wavefront owns R consecutive output rows and
//     streams them with 16-byte loads per lane, so one load instruction moves
//     1 KiB of a row (64 lanes x 16 int8). Rows are [N, K] row-major, the
//     nn.Linear layout, so a block reads one contiguous 4*R*K byte span.
//   * Dequantisation stays in registers: each int8 byte is biased to unsigned
//     (xor 0x80) and converted with one v_cvt_f32_ubyteN, multiplied by the fp32
//     activation with one FMA; the bias (128 * sum x) is removed once per lane.
//     Every product is exact in fp32 (8-bit x 8-bit significands).
//   * Activations are re-read per 1 KiB chunk from L1/L2 (a few KiB, shared by
//     every block), so register use does not grow with K.
//   * The row sum is a DPP butterfly over 16 lanes plus four readlanes: a fixed
//     summation order, so results are bitwise reproducible.
//   * The scale is applied after the reduction, then one bf16 rounding.
#include "common.h"

namespace egpt {
namespace {

constexpr int kGemvWaves = 4;
constexpr int kGemvThreads = kGemvWaves * kWave;
constexpr int kChunk = kWave * 16;  // int8 elements covered by one 16-byte load per lane
constexpr int kFusedMaxK = 12 * kChunk;  // the longest row egpt_int8_gemv_fused takes (include/egpt.h)

enum { kEpiStore = 0, kEpiPartial = 1 };

// 16 int8 weights (one 16-byte load) times 16 fp32 activations, biased form.
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

// Fast path. Preconditions (checked on the host): every K chunk boundary and
// every row start is 16-byte aligned (K % 16 == 0, kchunk % 16 == 0, ldw % 16 == 0,
// ldx % 8 == 0, aligned base pointers). NCH > 0 means each split covers exactly
// NCH * kChunk elements, so the chunk loop is fully unrolled with no K masking.
// Rows past N and x rows past m_rows are clamped to valid memory and discarded.
template <int M, int R, int NCH, int EPI>
__global__ __launch_bounds__(kGemvThreads) void gemv_i8_rows(
    const uint16_t* __restrict__ x, int64_t ldx, const int8_t* __restrict__ w, int64_t ldw,
    const float* __restrict__ scale, void* __restrict__ out, int64_t ldo, int m_rows, int N, int K,
    int kchunk) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t row0 = ((int64_t)blockIdx.x * kGemvWaves + wave) * R;
  if (row0 >= N) return;
  const int k_begin = blockIdx.y * kchunk;
  const int k_end = min(K, k_begin + kchunk);

  const int8_t* wrow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) wrow[r] = w + min(row0 + r, (int64_t)N - 1) * ldw;
  const uint16_t* xrow[M];
#pragma unroll
  for (int m = 0; m < M; ++m) xrow[m] = x + (int64_t)min(m, m_rows - 1) * ldx;

  float acc[M][R];
  float sx[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    sx[m] = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.f;
  }

  const int nch = NCH > 0 ? NCH : (k_end - k_begin + kChunk - 1) / kChunk;
#pragma unroll
  for (int c = 0; c < nch; ++c) {
    const int k = k_begin + c * kChunk + lane * 16;
    if (NCH > 0 || k < k_end) {
      u32x4 wv[R];
#pragma unroll
      for (int r = 0; r < R; ++r) wv[r] = ld16_stream(wrow[r] + k);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float xf[16];
        unpack_bf16x16(ld16(xrow[m] + k), ld16(xrow[m] + k + 8), xf);
        float t = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) t += xf[e];
        sx[m] += t;
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = dot16_biased(wv[r], xf, acc[m][r]);
      }
    }
  }

#pragma unroll
  for (int m = 0; m < M; ++m) {
    float mine = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float v = wave_sum(acc[m][r] - 128.f * sx[m]);
      if (lane == r) mine = v;
    }
    const int64_t n = row0 + lane;
    if (lane < R && m < m_rows && n < N) {
      if constexpr (EPI == kEpiStore) {
        ((uint16_t*)out)[(int64_t)m * ldo + n] = f32_to_bf16(mine * scale[n]);
      } else {
        ((float*)out)[((int64_t)blockIdx.y * m_rows + m) * ldo + n] = mine;
      }
    }
  }
}

// Any alignment, any K: one wavefront per output row, one element per lane step.
// Used for shapes the fast path does not take (odd K, unaligned rows).
__global__ __launch_bounds__(kGemvThreads) void gemv_i8_generic(
    const uint16_t* __restrict__ x, int64_t ldx, const int8_t* __restrict__ w, int64_t ldw,
    const float* __restrict__ scale, void* __restrict__ out, int64_t ldo, int m_rows, int N, int K,
    int kchunk, int epi) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t n = (int64_t)blockIdx.x * kGemvWaves + wave;
  if (n >= N) return;
  const int k_begin = blockIdx.y * kchunk;
  const int k_end = min(K, k_begin + kchunk);
  const int8_t* wr = w + n * ldw;
  for (int m = 0; m < m_rows; ++m) {
    const uint16_t* xr = x + (int64_t)m * ldx;
    float a = 0.f;
    for (int k = k_begin + lane; k < k_end; k += kWave) a = fmaf(bf16_to_f32(xr[k]), (float)wr[k], a);
    a = wave_sum(a);
    if (lane == 0) {
      if (epi == kEpiStore) {
        ((uint16_t*)out)[(int64_t)m * ldo + n] = f32_to_bf16(a * scale[n]);
      } else {
        ((float*)out)[((int64_t)blockIdx.y * m_rows + m) * ldo + n] = a;
      }
    }
  }
}

// Small batches (3 <= M <= 16 activation rows) on MFMA. At M rows a weight byte
// feeds M products; on the vector ALU that is M FMAs per byte and 8 rows already
// run at a fifth of the single-row bandwidth. v_mfma_f32_16x16x32_bf16 takes the
// activation rows as A (rows past M are clamped copies, never stored) and 16
// weight rows, converted exactly to bf16, as B. A dot product does not care
// about K order, so lane l owns 16 contiguous K of weight row n0 + l % 16 and of
// activation row l % 16 (K group l / 16); its two 8-element halves feed the two
// MFMAs of a 64-wide step. G wavefronts share 16 output features: wavefront j
// of the group takes the steps j, j + G, ... and the G partial tiles are summed
// through LDS in wavefront order (a fixed order: bitwise reproducible). Then
// y = bf16(scale * sum), the decode rounding.
// Layouts (checked on the MI355X): lane l holds A[l % 16][8 (l / 16) + e] and
// B[8 (l / 16) + e][l % 16]; accumulator register r is C[4 (l / 16) + r][l % 16].
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
constexpr int kMfmaWaves = 8;
constexpr int kMfmaStage = 4;  // 64-wide K steps whose loads are issued together

__device__ __forceinline__ bf16x8_t int8x8_bf16(uint32_t w0, uint32_t w1) {
  const uint32_t w[2] = {w0, w1};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float f0 = (float)(int)(int8_t)(w[i] & 0xffu);
    const float f1 = (float)(int)(int8_t)((w[i] >> 8) & 0xffu);
    const float f2 = (float)(int)(int8_t)((w[i] >> 16) & 0xffu);
    const float f3 = (float)(int)(int8_t)(w[i] >> 24);
    o[2 * i] = (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xffff0000u);
    o[2 * i + 1] = (__float_as_uint(f2) >> 16) | (__float_as_uint(f3) & 0xffff0000u);
  }
  return __builtin_bit_cast(bf16x8_t, u32x4{o[0], o[1], o[2], o[3]});
}

// G wavefronts share FG groups of 16 features (8 / G such sets per block); with
// G = 1 each wavefront would stream its rows over all of K and store its own
// outputs. Each activation fragment a wavefront loads feeds the FG groups' MFMAs,
// so wide outputs read the activations FG times less often per weight byte.
template <int G, int FG>
__global__ __launch_bounds__(kMfmaWaves * kWave) void gemv_i8_mfma(
    const uint16_t* __restrict__ x, int64_t ldx, const int8_t* __restrict__ w, int64_t ldw,
    const float* __restrict__ scale, uint16_t* __restrict__ y, int64_t ldy, int m_rows, int N, int K) {
  __shared__ float red[G > 1 ? kMfmaWaves : 1][FG * 256];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int group = wave / G, sub = wave % G;
  const int64_t n0 = ((int64_t)blockIdx.x * (kMfmaWaves / G) + group) * 16 * FG;
  const int8_t* wrow[FG];
#pragma unroll
  for (int f = 0; f < FG; ++f) wrow[f] = w + min(n0 + 16 * f + lane % 16, (int64_t)N - 1) * ldw + 16 * (lane / 16);
  const uint16_t* xrow = x + (int64_t)min(lane % 16, m_rows - 1) * ldx + 16 * (lane / 16);
  const int steps = K / 64;
  f32x4_t acc[FG];
#pragma unroll
  for (int f = 0; f < FG; ++f) acc[f] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int s0 = sub; s0 < steps; s0 += G * kMfmaStage) {
    u32x4 wv[kMfmaStage][FG], xa[kMfmaStage], xb[kMfmaStage];
#pragma unroll
    for (int j = 0; j < kMfmaStage; ++j) {
      const int st = min(s0 + j * G, steps - 1);  // past the end: a valid step, not accumulated
#pragma unroll
      for (int f = 0; f < FG; ++f) wv[j][f] = ld16_stream(wrow[f] + st * 64);
      xa[j] = ld16(xrow + st * 64);
      xb[j] = ld16(xrow + st * 64 + 8);
    }
#pragma unroll
    for (int j = 0; j < kMfmaStage; ++j) {
      if (s0 + j * G < steps) {
#pragma unroll
        for (int f = 0; f < FG; ++f) {
          acc[f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xa[j]),
                                                           int8x8_bf16(wv[j][f].x, wv[j][f].y), acc[f], 0, 0, 0);
          acc[f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xb[j]),
                                                           int8x8_bf16(wv[j][f].z, wv[j][f].w), acc[f], 0, 0, 0);
        }
      }
    }
  }
  if constexpr (G > 1) {
#pragma unroll
    for (int f = 0; f < FG; ++f)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave][f * 256 + (4 * (lane / 16) + r) * 16 + lane % 16] = acc[f][r];
    __syncthreads();
    // each set's G partials summed in wavefront order, one output per thread
    for (int e = threadIdx.x; e < (kMfmaWaves / G) * FG * 256; e += kMfmaWaves * kWave) {
      const int gi = e / (FG * 256), fe = e % (FG * 256);
      const int f = fe / 256, idx = fe % 256;
      float sum = red[gi * G][fe];
#pragma unroll
      for (int j = 1; j < G; ++j) sum += red[gi * G + j][fe];
      const int m = idx / 16;
      const int64_t nn = ((int64_t)blockIdx.x * (kMfmaWaves / G) + gi) * 16 * FG + 16 * f + idx % 16;
      if (m < m_rows && nn < N) y[(int64_t)m * ldy + nn] = f32_to_bf16(sum * scale[nn]);
    }
  } else {
#pragma unroll
    for (int f = 0; f < FG; ++f) {
      const int64_t n = n0 + 16 * f + lane % 16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 4 * (lane / 16) + r;
        if (m < m_rows && n < N) y[(int64_t)m * ldy + n] = f32_to_bf16(acc[f][r] * scale[n]);
      }
    }
  }
}

// The same contraction for wide outputs with short rows (K <= 64 * 8 * SPW): a
// capped grid whose blocks walk tiles of FG groups of 16 features. As in
// gemv_i8_mfma<8, FG>, the 8 wavefronts of a block split K (wavefront j takes
// the 64-wide steps j, j + 8, ...) and their tiles are summed through LDS in
// wavefront order, so the outputs are bit-identical to it. What differs: each
// wavefront loads its activation fragments once and keeps them in registers,
// and the next tile's weights (and scales) are issued before this tile is
// multiplied, in two fixed register buffers, so a block keeps streaming while it
// reduces instead of ending after one short burst of loads. Loads past the last
// tile re-read the block's own tile (unconditional loads keep the wait counts
// exact). The LDS tiles alternate between two buffers: one barrier per tile.
template <int SPW, int FG>
struct MfmaTile {
  u32x4 w[SPW][FG];
  float sc[(FG * 256 + kMfmaWaves * kWave - 1) / (kMfmaWaves * kWave)];
};

template <int SPW, int FG>
__device__ __forceinline__ void mfma_tile_load(MfmaTile<SPW, FG>& b, const int8_t* __restrict__ w, int64_t ldw,
                                               const float* __restrict__ scale, int N, int64_t tile, int steps,
                                               int lane, int wave) {
  constexpr int kE = (FG * 256 + kMfmaWaves * kWave - 1) / (kMfmaWaves * kWave);
  const int64_t n0 = tile * 16 * FG;
#pragma unroll
  for (int i = 0; i < kE; ++i) {
    const int e = min((int)threadIdx.x + i * kMfmaWaves * kWave, FG * 256 - 1);
    b.sc[i] = scale[min(n0 + 16 * (e / 256) + (e % 256) % 16, (int64_t)N - 1)];
  }
#pragma unroll
  for (int j = 0; j < SPW; ++j) {
    const int st = min(wave + kMfmaWaves * j, steps - 1);
#pragma unroll
    for (int f = 0; f < FG; ++f)
      b.w[j][f] = ld16_stream(w + min(n0 + 16 * f + lane % 16, (int64_t)N - 1) * ldw + 16 * (lane / 16) + st * 64);
  }
}

template <int SPW, int FG>
__device__ __forceinline__ void mfma_tile_finish(const MfmaTile<SPW, FG>& b, const u32x4 (&xa)[SPW],
                                                 const u32x4 (&xb)[SPW], float* red, uint16_t* __restrict__ y,
                                                 int64_t ldy, int m_rows, int N, int64_t tile, int steps, int lane,
                                                 int wave) {
  f32x4_t acc[FG];
#pragma unroll
  for (int f = 0; f < FG; ++f) acc[f] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < SPW; ++j) {
    if (wave + kMfmaWaves * j < steps) {
#pragma unroll
      for (int f = 0; f < FG; ++f) {
        acc[f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xa[j]),
                                                         int8x8_bf16(b.w[j][f].x, b.w[j][f].y), acc[f], 0, 0, 0);
        acc[f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xb[j]),
                                                         int8x8_bf16(b.w[j][f].z, b.w[j][f].w), acc[f], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int f = 0; f < FG; ++f)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave * FG * 256 + f * 256 + (4 * (lane / 16) + r) * 16 + lane % 16] = acc[f][r];
  lds_barrier();
  constexpr int kE = (FG * 256 + kMfmaWaves * kWave - 1) / (kMfmaWaves * kWave);
#pragma unroll
  for (int i = 0; i < kE; ++i) {
    const int e = (int)threadIdx.x + i * kMfmaWaves * kWave;
    if (e < FG * 256) {
      float sum = red[e];
#pragma unroll
      for (int j = 1; j < kMfmaWaves; ++j) sum += red[j * FG * 256 + e];
      const int m = (e % 256) / 16;
      const int64_t nn = tile * 16 * FG + 16 * (e / 256) + (e % 256) % 16;
      if (m < m_rows && nn < N) y[(int64_t)m * ldy + nn] = f32_to_bf16(sum * b.sc[i]);
    }
  }
}

template <int SPW, int FG>
__global__ __launch_bounds__(kMfmaWaves * kWave) void gemv_i8_mfma_walk(
    const uint16_t* __restrict__ x, int64_t ldx, const int8_t* __restrict__ w, int64_t ldw,
    const float* __restrict__ scale, uint16_t* __restrict__ y, int64_t ldy, int m_rows, int N, int K) {
  __shared__ float red[2][kMfmaWaves * FG * 256];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int steps = K / 64;
  const int64_t ntiles = ((int64_t)N + 16 * FG - 1) / (16 * FG);
  const int64_t stride = gridDim.x;
  // activation fragments of this wavefront's K steps (a step past the end is a
  // valid one, never accumulated)
  const uint16_t* xrow = x + (int64_t)min(lane % 16, m_rows - 1) * ldx + 16 * (lane / 16);
  u32x4 xa[SPW], xb[SPW];
#pragma unroll
  for (int j = 0; j < SPW; ++j) {
    const int st = min(wave + kMfmaWaves * j, steps - 1);
    xa[j] = ld16(xrow + st * 64);
    xb[j] = ld16(xrow + st * 64 + 8);
  }
  int64_t t = blockIdx.x;
  MfmaTile<SPW, FG> ta, tb;
  mfma_tile_load<SPW, FG>(ta, w, ldw, scale, N, t, steps, lane, wave);
#pragma unroll 1
  for (;;) {
    const int64_t u = t + stride;
    mfma_tile_load<SPW, FG>(tb, w, ldw, scale, N, u < ntiles ? u : t, steps, lane, wave);
    __builtin_amdgcn_sched_barrier(0);
    mfma_tile_finish<SPW, FG>(ta, xa, xb, red[0], y, ldy, m_rows, N, t, steps, lane, wave);
    __builtin_amdgcn_sched_barrier(0);
    if (u >= ntiles) break;
    const int64_t v = u + stride;
    mfma_tile_load<SPW, FG>(ta, w, ldw, scale, N, v < ntiles ? v : u, steps, lane, wave);
    __builtin_amdgcn_sched_barrier(0);
    mfma_tile_finish<SPW, FG>(tb, xa, xb, red[1], y, ldy, m_rows, N, u, steps, lane, wave);
    __builtin_amdgcn_sched_barrier(0);
    if (v >= ntiles) break;
    t = v;
  }
}

// LDS-staged form of the walking GEMV, for K of 2, 3, 4, 6, 8 or 12 chunks of 512 bytes. The
// MFMA operand layout puts 16 weight rows in every load instruction (64 bytes
// of each): streamed that way an int8 matrix moves at 4.2 TB/s on the MI355X,
// against 6.4 TB/s for loads that cover 1 KiB of consecutive bytes (a stream
// of 151936 x 2048, measured). Here the weights go straight from memory into
// LDS (global_load_lds_dwordx4: lane i of a load writes LDS bytes 16 i .. 16 i
// + 15 from the base in M0, checked on the MI355X), each load covering two
// 512-byte row slices, and the MFMA fragments are read from LDS. A tile of FG
// groups of 16 features is streamed in chunks of 512 K bytes; wavefront j
// loads rows 2 FG j .. 2 FG j + 2 FG - 1 of each chunk and multiplies the
// chunk's step j (K 64 j .. 64 j + 63), so over a tile it takes the steps j,
// j + 8, ... in order, as gemv_i8_mfma_walk does, with the same MFMAs and the
// same wavefront-order reduction: the outputs are bit-identical to it. The
// tile's scales come into LDS the same way. Three chunk buffers: the loads of
// chunk q + 2 are issued once every wavefront has passed chunk q's barrier (so
// none still reads that buffer), and each wait covers one chunk. In LDS a row's
// 16-byte unit u sits at unit u ^ (row % 16), so the 16 rows a fragment read
// touches fall on distinct banks.
//
// The LDS loads are issued from inline assembly, and the kernel waits for them
// itself (s_waitcnt vmcnt counts every vector memory operation in issue order):
// the compiler, seeing them, waits for all of them before any LDS read.
constexpr int kLdsChunk = 512;


template <int FG>
__device__ __forceinline__ void lds_chunk_issue(int8_t* buf, const int8_t* __restrict__ w, int64_t ldw, int N,
                                                int64_t tile, int c, int lane, int wave) {
#pragma unroll
  for (int i = 0; i < FG; ++i) {
    const int r = 2 * FG * wave + 2 * i + lane / 32;  // row within the tile
    const int64_t row = min(tile * 16 * FG + r, (int64_t)N - 1);
    const int u = (lane % 32) ^ (r % 16);  // the unit this lane's LDS slot holds
    lds_load16(lds_addr(buf + (2 * FG * wave + 2 * i) * kLdsChunk), w + row * ldw + c * kLdsChunk + 16 * u);
  }
}

template <int SPW, int FG>
__global__ __launch_bounds__(kMfmaWaves * kWave) void gemv_i8_mfma_lds(
    const uint16_t* __restrict__ x, int64_t ldx, const int8_t* __restrict__ w, int64_t ldw,
    const float* __restrict__ scale, uint16_t* __restrict__ y, int64_t ldy, int m_rows, int N, int K) {
  constexpr int kE = (FG * 256 + kMfmaWaves * kWave - 1) / (kMfmaWaves * kWave);
  constexpr int kBuf = 16 * FG * kLdsChunk;
  __shared__ __align__(16) int8_t wsm[3 * kBuf];
  __shared__ float red[kMfmaWaves * FG * 256];
  __shared__ float scs[3][kWave];  // the scales of a tile (16 FG used): slot = the block's tile index % 3
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t ntiles = ((int64_t)N + 16 * FG - 1) / (16 * FG);
  const int64_t stride = gridDim.x;
  // activation fragments of this wavefront's steps j + 8 c (all inside K = 512 SPW),
  // complete before the first weight load goes out
  const uint16_t* xrow = x + (int64_t)min(lane % 16, m_rows - 1) * ldx + 16 * (lane / 16);
  u32x4 xa[SPW], xb[SPW];
#pragma unroll
  for (int c = 0; c < SPW; ++c) {
    xa[c] = ld16(xrow + (wave + kMfmaWaves * c) * 64);
    xb[c] = ld16(xrow + (wave + kMfmaWaves * c) * 64 + 8);
  }
  // (the empty asm takes the fragments as inputs, so the compiler waits for them
  // here rather than moving the loads below the first weight loads)
#pragma unroll
  for (int c = 0; c < SPW; ++c) asm volatile("" : : "v"(xa[c]), "v"(xb[c]) : "memory");
  // Chunk position p: tile t0 + (p / SPW) stride, chunk p % SPW, buffer p % 3; a
  // position past the last tile re-reads that chunk of the block's first tile. A
  // tile's scales go out just before its first chunk, two tiles ahead at most.
  auto issue = [&](int64_t p) {
    int64_t tile = (int64_t)blockIdx.x + (p / SPW) * stride;
    const int c = (int)(p % SPW);
    if (tile >= ntiles) tile = blockIdx.x;
    if (c == 0)
      lds_load4(lds_addr(scs[(p / SPW) % 3]), scale + min(tile * 16 * FG + lane, (int64_t)N - 1));
    lds_chunk_issue<FG>(wsm + (int)(p % 3) * kBuf, w, ldw, N, tile, c, lane, wave);
  };
  issue(0);
  issue(1);
  int64_t p = 0;
  int slot = 0;
  f32x4_t acc[FG];
#pragma unroll 1
  for (int64_t t = blockIdx.x; t < ntiles; t += stride, slot = slot == 2 ? 0 : slot + 1) {
#pragma unroll
    for (int c = 0; c < SPW; ++c) {
      // Chunk p is in once no more than the operations issued after it are
      // outstanding: chunk p + 1 (FG loads), preceded by its tile's scales when
      // it starts one, and any stores since (more waiting, never less).
      __builtin_amdgcn_sched_barrier(0);
      if (c == SPW - 1) {
        EGPT_WAIT_VMCNT(FG + 1);
      } else {
        EGPT_WAIT_VMCNT(FG);
      }
      lds_barrier();
      __builtin_amdgcn_sched_barrier(0);
      // chunk p + 2 goes into the buffer chunk p - 1 used: every wavefront is past it
      issue(p + 2);
      if (c == 0) {
#pragma unroll
        for (int f = 0; f < FG; ++f) acc[f] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
      const int8_t* buf = wsm + (int)(p % 3) * kBuf;
#pragma unroll
      for (int f = 0; f < FG; ++f) {
        const int r = 16 * f + lane % 16;
        const int u = (4 * wave + lane / 16) ^ (r % 16);
        const u32x4 fr = *(const u32x4*)(buf + r * kLdsChunk + 16 * u);
        acc[f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xa[c]),
                                                         int8x8_bf16(fr.x, fr.y), acc[f], 0, 0, 0);
        acc[f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xb[c]),
                                                         int8x8_bf16(fr.z, fr.w), acc[f], 0, 0, 0);
      }
      ++p;
    }
    // wavefront-order reduction of the tile, scale, store (the chunk barriers of
    // the next tile separate these reads from its writes)
#pragma unroll
    for (int f = 0; f < FG; ++f)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave * FG * 256 + f * 256 + (4 * (lane / 16) + r) * 16 + lane % 16] = acc[f][r];
    lds_barrier();
#pragma unroll
    for (int i = 0; i < kE; ++i) {
      const int e = (int)threadIdx.x + i * kMfmaWaves * kWave;
      if (e < FG * 256) {
        float sum = red[e];
#pragma unroll
        for (int j = 1; j < kMfmaWaves; ++j) sum += red[j * FG * 256 + e];
        const int m = (e % 256) / 16;
        const int fi = 16 * (e / 256) + (e % 256) % 16;
        const int64_t nn = t * 16 * FG + fi;
        if (m < m_rows && nn < N) y[(int64_t)m * ldy + nn] = f32_to_bf16(sum * scs[slot][fi]);
      }
    }
  }
  // the two chunks issued past the last one land in this block's LDS: wait for them
  // before the block ends and its LDS goes to another
  EGPT_WAIT_VMCNT(0);
}

template <int G, int FG>
void launch_mfma(const uint16_t* x, int64_t ldx, const int8_t* w, int64_t ldw, const float* scale, uint16_t* y,
                 int64_t ldy, int M, int N, int K, hipStream_t st) {
  const int64_t per_block = 16 * FG * (kMfmaWaves / G);
  hipLaunchKernelGGL((gemv_i8_mfma<G, FG>), dim3((unsigned)((N + per_block - 1) / per_block)),
                     dim3(kMfmaWaves * kWave), 0, st, x, ldx, w, ldw, scale, y, ldy, M, N, K);
}

// Blocks of the tile-walking MFMA GEMV: one per CU (512 and 1024 measured
// slower: 10-30% at 151936 x 2048, 12288 x 2048 and 70001 x 1024).
constexpr int kMfmaWalkBlocks = 256;
// It takes outputs wider than this with rows of at most 2048 (K / 64 steps over
// 8 wavefronts, at most 4 each). Against gemv_i8_mfma (A/B on one box, cold,
// 3-16 rows): 151936 x 2048 72-78 -> 70-76 us, 12288 x 2048 9.1-11.5 ->
// 8.7-9.4, 70001 x 1024 30-35 -> 20-22; at 8192 and 4096 features, with two and
// one tiles per block, it is no faster.
constexpr int64_t kMfmaWalkMinN = 8192;

template <int FG>
int launch_mfma_walk(const uint16_t* x, int64_t ldx, const int8_t* w, int64_t ldw, const float* scale, uint16_t* y,
                     int64_t ldy, int M, int N, int K, hipStream_t st) {
  const int spw = (K / 64 + kMfmaWaves - 1) / kMfmaWaves;
  const int64_t tiles = ((int64_t)N + 16 * FG - 1) / (16 * FG);
  const dim3 grid((unsigned)(tiles < kMfmaWalkBlocks ? tiles : kMfmaWalkBlocks)), block(kMfmaWaves * kWave);
  switch (spw) {
    case 1: hipLaunchKernelGGL((gemv_i8_mfma_walk<1, FG>), grid, block, 0, st, x, ldx, w, ldw, scale, y, ldy, M, N, K); break;
    case 2: hipLaunchKernelGGL((gemv_i8_mfma_walk<2, FG>), grid, block, 0, st, x, ldx, w, ldw, scale, y, ldy, M, N, K); break;
    case 3:
    case 4: hipLaunchKernelGGL((gemv_i8_mfma_walk<4, FG>), grid, block, 0, st, x, ldx, w, ldw, scale, y, ldy, M, N, K); break;
    default: return EGPT_ERR_UNSUPPORTED;
  }
  return EGPT_LAUNCH_STATUS();
}

// Blocks of the LDS-staged GEMV: one per CU with four feature groups per tile
// (128.5 KiB of LDS), two with one. Measured against 512 / 256 (A/B on one box,
// cold, 3-16 rows): 151936 x 2048 56-60 against 57-61 us, 12288 x 2048 8.1-9.7
// against 9.2-10.1, 20000 x 1536 9.2-10.6 against 11.6-12.5.
template <int FG>
constexpr unsigned mfma_lds_blocks() { return FG == 4 ? 256 : 512; }

template <int FG>
int launch_mfma_lds(const uint16_t* x, int64_t ldx, const int8_t* w, int64_t ldw, const float* scale, uint16_t* y,
                    int64_t ldy, int M, int N, int K, hipStream_t st) {
  const int64_t tiles = ((int64_t)N + 16 * FG - 1) / (16 * FG);
  const dim3 grid((unsigned)(tiles < mfma_lds_blocks<FG>() ? tiles : mfma_lds_blocks<FG>())), block(kMfmaWaves * kWave);
  switch (K / kLdsChunk) {
    case 1: hipLaunchKernelGGL((gemv_i8_mfma_lds<1, FG>), grid, block, 0, st, x, ldx, w, ldw, scale, y, ldy, M, N, K); break;
    case 2: hipLaunchKernelGGL((gemv_i8_mfma_lds<2, FG>), grid, block, 0, st, x, ldx, w, ldw, scale, y, ldy, M, N, K); break;
    case 3: hipLaunchKernelGGL((gemv_i8_mfma_lds<3, FG>), grid, block, 0, st, x, ldx, w, ldw, scale, y, ldy, M, N, K); break;
    case 4: hipLaunchKernelGGL((gemv_i8_mfma_lds<4, FG>), grid, block, 0, st, x, ldx, w, ldw, scale, y, ldy, M, N, K); break;
    case 6: hipLaunchKernelGGL((gemv_i8_mfma_lds<6, FG>), grid, block, 0, st, x, ldx, w, ldw, scale, y, ldy, M, N, K); break;
    case 8: hipLaunchKernelGGL((gemv_i8_mfma_lds<8, FG>), grid, block, 0, st, x, ldx, w, ldw, scale, y, ldy, M, N, K); break;
    case 12: hipLaunchKernelGGL((gemv_i8_mfma_lds<12, FG>), grid, block, 0, st, x, ldx, w, ldw, scale, y, ldy, M, N, K); break;
    default: return EGPT_ERR_UNSUPPORTED;
  }
  return EGPT_LAUNCH_STATUS();
}

// Feature groups per MFMA wavefront: four for outputs of at least this many
// features (the lm_head: 151936 x 2048 at 8 rows 75 against 90-99 us, at 4 rows
// 72-75 against 80 us), one below it, where fewer, wider blocks lose more than the
// activation reads save (gate_up 12288 x 2048 at two groups: 9.3 against 8.2 us).
constexpr int64_t kMfmaWideN = 65536;

// Deterministic split-K reduction: fixed split order, then scale, one rounding.
__global__ __launch_bounds__(256) void gemv_splitk_reduce(const float* __restrict__ part, int splits, int m_rows,
                                                          int N, const float* __restrict__ scale,
                                                          uint16_t* __restrict__ y, int64_t ldy) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y;
  if (n >= N) return;
  float a = 0.f;
  for (int s = 0; s < splits; ++s) a += part[((int64_t)s * m_rows + m) * N + n];
  y[(int64_t)m * ldy + n] = f32_to_bf16(a * scale[n]);
}

struct GemvArgs {
  const uint16_t* x;
  int64_t ldx;
  const int8_t* w;
  int64_t ldw;
  const float* scale;
  void* out;
  int64_t ldo;
  int m_rows, N, K, kchunk, splits;
};

template <int M, int R, int NCH, int EPI>
void launch_rows(const GemvArgs& a, hipStream_t st) {
  const int rows_per_block = kGemvWaves * R;
  dim3 grid((unsigned)((a.N + rows_per_block - 1) / rows_per_block), (unsigned)a.splits);
  hipLaunchKernelGGL((gemv_i8_rows<M, R, NCH, EPI>), grid, dim3(kGemvThreads), 0, st, a.x, a.ldx, a.w, a.ldw,
                     a.scale, a.out, a.ldo, a.m_rows, a.N, a.K, a.kchunk);
}

// Rows per wavefront: enough blocks to cover the 256 CUs at least twice, capped
// by register budget (R * chunks of 16-byte loads in flight per lane).
int pick_rows(int N, int m_tile) {
  const int cap = m_tile == 1 ? 4 : (m_tile <= 4 ? 2 : 1);
  int r = 1;
  while (r < cap && (int64_t)N >= (int64_t)(2 * r) * kGemvWaves * 512) r *= 2;
  return r;
}

template <int M, int EPI>
void launch_fast_m(const GemvArgs& a, int nch_exact, hipStream_t st) {
  const int r = pick_rows(a.N, M);
  if constexpr (M == 1) {
    // Fully unrolled chunk loops for the common per-split lengths.
#define EGPT_NCH_CASE(NC)                                              \
  if (nch_exact == NC) {                                               \
    if (r == 4) return launch_rows<1, 4, NC, EPI>(a, st);              \
    if (r == 2) return launch_rows<1, 2, NC, EPI>(a, st);              \
    return launch_rows<1, 1, NC, EPI>(a, st);                          \
  }
    EGPT_NCH_CASE(1)
    EGPT_NCH_CASE(2)
    EGPT_NCH_CASE(3)
    EGPT_NCH_CASE(4)
    EGPT_NCH_CASE(6)
#undef EGPT_NCH_CASE
    if (r == 4) return launch_rows<1, 4, 0, EPI>(a, st);
    if (r == 2) return launch_rows<1, 2, 0, EPI>(a, st);
    return launch_rows<1, 1, 0, EPI>(a, st);
  } else {
    if (r >= 2) return launch_rows<M, 2, 0, EPI>(a, st);
    return launch_rows<M, 1, 0, EPI>(a, st);
  }
}

template <int EPI>
int launch_gemv(const GemvArgs& a, hipStream_t st) {
  const bool aligned = (a.K % 16 == 0) && (a.kchunk % 16 == 0) && (a.ldw % 16 == 0) &&
                       ((uintptr_t)a.w % 16 == 0) && ((uintptr_t)a.x % 16 == 0) &&
                       (a.m_rows == 1 || a.ldx % 8 == 0);
  if (!aligned || a.K == 0) {
    dim3 grid((unsigned)((a.N + kGemvWaves - 1) / kGemvWaves), (unsigned)a.splits);
    hipLaunchKernelGGL(gemv_i8_generic, grid, dim3(kGemvThreads), 0, st, a.x, a.ldx, a.w, a.ldw, a.scale, a.out,
                       a.ldo, a.m_rows, a.N, a.K, a.kchunk, EPI);
    return EGPT_LAUNCH_STATUS();
  }
  // Exact chunk count per split when every split has the same length.
  int nch_exact = 0;
  if (a.kchunk % kChunk == 0 && (int64_t)a.kchunk * a.splits == a.K) nch_exact = a.kchunk / kChunk;
  const int mt = a.m_rows;
  if (mt == 1) launch_fast_m<1, EPI>(a, nch_exact, st);
  else if (mt <= 2) launch_fast_m<2, EPI>(a, nch_exact, st);
  else if (mt <= 4) launch_fast_m<4, EPI>(a, nch_exact, st);
  else if (mt <= 8) launch_fast_m<8, EPI>(a, nch_exact, st);
  else launch_fast_m<16, EPI>(a, nch_exact, st);
  return EGPT_LAUNCH_STATUS();
}

int check_gemv_args(const void* x, int64_t ldx, const int8_t* w, int64_t ldw, const float* scale, const void* y,
                    int64_t ldy, int M, int N, int K) {
  if (!x || !w || !scale || !y) return EGPT_ERR_INVALID;
  if (M < 0 || N < 0 || K < 0) return EGPT_ERR_INVALID;
  if (M > EGPT_MAX_DECODE_ROWS) return EGPT_ERR_UNSUPPORTED;
  if (ldw < K || (M > 1 && (ldx < K || ldy < N))) return EGPT_ERR_INVALID;
  return EGPT_OK;
}

}  // namespace
}  // namespace egpt

using namespace egpt;

extern "C" int egpt_int8_gemv(const void* x, int64_t ldx, const int8_t* w, int64_t ldw, const float* scale,
                              void* y, int64_t ldy, int M, int N, int K, hipStream_t stream) {
  const int st = check_gemv_args(x, ldx, w, ldw, scale, y, ldy, M, N, K);
  if (st != EGPT_OK) return st;
  if (M == 0 || N == 0) return EGPT_OK;
  if (M == 1 && K >= 16 && K % 16 == 0 && K <= kFusedMaxK && ldw % 16 == 0 && (uintptr_t)w % 16 == 0 &&
      (uintptr_t)x % 16 == 0) {
    // One aligned row: the fused kernel's plain store variant. It computes the
    // same per-lane chunk sums in the same order and the same fixed row
    // reduction, so the result is bit-identical, and it streams the weights in
    // staged register buffers with exact wait counts.
    egpt_gemv_fused d{};
    d.epilogue = EGPT_EPI_STORE;
    d.N = N;
    d.K = K;
    d.x = x;
    d.x_ld = K;
    d.x_rows = 1;
    d.w = w;
    d.ldw = ldw;
    d.scale = scale;
    d.y = y;
    return egpt_int8_gemv_fused(&d, stream);
  }
  if ((M == 2 || (M <= kGemvFewRowsMax && N < kGemvFewRowsWideN)) && K >= 16 && K % 16 == 0 && K <= kFusedMaxK &&
      ldw % 16 == 0 && ldx % 8 == 0 && (uintptr_t)w % 16 == 0 && (uintptr_t)x % 16 == 0) {
    // 2 aligned rows, or 3-4 over narrow outputs: the single-row kernel's weight
    // stream with the rows in LDS, each weight converted once (each output row
    // bit-identical to a one-row call).
    return gemv_few_rows(x, ldx, w, ldw, scale, y, ldy, M, N, K, stream);
  }
  if (M >= 3 && K >= 64 && K % 64 == 0 && ldw % 16 == 0 && ldx % 8 == 0 && (uintptr_t)w % 16 == 0 &&
      (uintptr_t)x % 16 == 0) {
    // 3-16 rows (3-4 over wide outputs): MFMA
    const uint16_t* xx = (const uint16_t*)x;
    uint16_t* yy = (uint16_t*)y;
    // all 8 wavefronts on one 16-feature group: splitting K eight ways keeps the most
    // loads in flight (measured faster than 1, 2 or 4 wavefronts per group at every
    // Qwen3-1.7B shape, the 151936-row lm_head included)
    // Wide outputs, K of 1024-6144 in 512-byte chunks: the LDS-staged form (bit-identical to the walking one;
    // against it, A/B on one box, cold, 3-16 rows: 151936 x 2048 70-80 -> 56-60 us, 12288 x 2048 8.9-10.1 ->
    // 8.1-9.7, 70001 x 1024 20-22 -> 18-19, 20000 x 1536 11.7-12.9 -> 9.2-10.6; at K = 512 it was slower,
    // 7.3-7.9 against 7.0-7.6 us at 32768 outputs).
    // K of 3072-6144 (the Qwen3-8B rows) against gemv_i8_mfma: 151936 x 4096 152-163 -> 109-116 us, 24576 x 4096
    // 26-38 -> 23-27. At 8192 outputs and fewer (one tile per block) it was slower: 4096 x 4096 8.1-10.1 against
    // 7.3-8.7 us, 2048 x 6144 at 8-16 rows 11.8-13.8 against 9.3-11.2.
    {
      const int spw = K / kLdsChunk;
      if (K % kLdsChunk == 0 && (spw == 2 || spw == 3 || spw == 4 || spw == 6 || spw == 8 || spw == 12) &&
          N > kMfmaWalkMinN) {
        if (N >= kMfmaWideN) return launch_mfma_lds<4>(xx, ldx, w, ldw, scale, yy, ldy, M, N, K, stream);
        return launch_mfma_lds<1>(xx, ldx, w, ldw, scale, yy, ldy, M, N, K, stream);
      }
    }
    if (K <= 64 * kMfmaWaves * 4 && N > kMfmaWalkMinN) {
      if (N >= kMfmaWideN) return launch_mfma_walk<4>(xx, ldx, w, ldw, scale, yy, ldy, M, N, K, stream);
      return launch_mfma_walk<1>(xx, ldx, w, ldw, scale, yy, ldy, M, N, K, stream);
    }
    if (N >= kMfmaWideN) launch_mfma<kMfmaWaves, 4>(xx, ldx, w, ldw, scale, yy, ldy, M, N, K, stream);
    else launch_mfma<kMfmaWaves, 1>(xx, ldx, w, ldw, scale, yy, ldy, M, N, K, stream);
    return EGPT_LAUNCH_STATUS();
  }
  GemvArgs a{(const uint16_t*)x, ldx, w, ldw, scale, y, ldy, M, N, K, K > 0 ? K : 1, 1};
  return launch_gemv<kEpiStore>(a, stream);
}

extern "C" int egpt_int8_gemv_splitk_workspace(int M, int N, int K, int splits, size_t* bytes) {
  if (!bytes || M < 0 || N < 0 || K < 0 || splits < 1) return EGPT_ERR_INVALID;
  *bytes = (size_t)splits * (size_t)M * (size_t)N * sizeof(float);
  return EGPT_OK;
}

extern "C" int egpt_int8_gemv_splitk(const void* x, int64_t ldx, const int8_t* w, int64_t ldw, const float* scale,
                                     void* y, int64_t ldy, int M, int N, int K, int splits, void* workspace,
                                     size_t workspace_bytes, hipStream_t stream) {
  int st = check_gemv_args(x, ldx, w, ldw, scale, y, ldy, M, N, K);
  if (st != EGPT_OK) return st;
  if (splits < 1) return EGPT_ERR_INVALID;
  if (M == 0 || N == 0) return EGPT_OK;
  // K chunk per split: a multiple of 16 so the aligned fast path stays available;
  // the number of splits actually launched may shrink so no split is empty.
  int kchunk = (K + splits - 1) / splits;
  kchunk = ((kchunk + 15) / 16) * 16;
  if (kchunk == 0) kchunk = 16;
  const int used = (K + kchunk - 1) / kchunk > 0 ? (K + kchunk - 1) / kchunk : 1;
  size_t need = 0;
  egpt_int8_gemv_splitk_workspace(M, N, K, used, &need);
  if (!workspace || workspace_bytes < need) return EGPT_ERR_WORKSPACE;
  GemvArgs a{(const uint16_t*)x, ldx, w, ldw, scale, workspace, N, M, N, K, kchunk, used};
  st = launch_gemv<kEpiPartial>(a, stream);
  if (st != EGPT_OK) return st;
  dim3 grid((unsigned)((N + 255) / 256), (unsigned)M);
  hipLaunchKernelGGL(gemv_splitk_reduce, grid, dim3(256), 0, stream, (const float*)workspace, used, M, N, scale,
                     (uint16_t*)y, M > 1 ? ldy : (int64_t)N);
  return EGPT_LAUNCH_STATUS();
}
