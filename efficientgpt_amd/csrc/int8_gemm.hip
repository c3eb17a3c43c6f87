// Int8-weight GEMM for prefill (more than 16 activation rows) on gfx950 MFMA.
//
//   y[m, n] = bf16( fp32( bf16( sum_k x[m, k] * w[n, k] ) ) * scale[n] )
//
// The reference's prefill formula (research/realmodel/int8_linear.py:96-97): a bf16
// GEMM of x with the exact bf16 image of the int8 weights (fp32 accumulation,
// rounded once to bf16), then the per-row scale in fp32 and a second bf16
// rounding. The reference materialises w.to(bfloat16) and calls the library
// GEMM; here the int8 rows go through LDS as int8 and each wavefront converts
// its fragments to bf16 in registers, so the weights cross HBM once, as int8.
//
// Design:
//   * A block of 4 or 8 wavefronts computes a BM x BN tile of y; each wavefront
//     owns a grid of 32 x 32 tiles of v_mfma_f32_32x32x16_bf16 (fp32
//     accumulators, bf16 products exact).
//   * K advances 64 (128 in the split slices) at a time through two LDS buffers
//     and two register staging sets: the global loads of step k + 2 are issued
//     before the MFMAs of step k; one barrier per step.
//   * x rows sit in LDS as bf16 (BK + 8 padding). Weights are converted to bf16
//     once per block by the thread that loaded them, as it writes them to LDS (the
//     tiles with two wavefronts along M, which read the same fragments), or stay
//     int8 (BK + 16 padding) and each wavefront converts the 8-byte fragments it
//     reads (the 128 x 256 tile, whose wavefronts lie along N). The padding puts
//     the fragment reads of 16 consecutive rows on distinct banks.
//   * int8 -> bf16 is exact: every value in [-127, 127] is a bf16.
//   * Rows past M or N read a valid row and are never stored.
//   * Split-K (short M, long K: too few output tiles to give every CU a block):
//     block (split, tile) sums its K slice and stores the fp32 tile to a caller's
//     workspace [splits][M][N]; a second kernel adds the slices in split order and
//     applies the two roundings. The fp32 sum is the same product in another
//     order, as any GEMM blocking is.
// Operand layouts (checked on the MI355X): lane l holds A[l % 32][8 (l / 32) + e]
// and B[8 (l / 32) + e][l % 32], e = 0..7; accumulator register r of lane l is
// C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].
#include <algorithm>

#include "common.h"

namespace egpt {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 64;        // K per LDS stage of the one-pass kernel: K must be a multiple of it
constexpr int kBKSplit = 128;  // K per LDS stage of the split-K slices (half the dependent steps)

template <int BM, int BN, int BK, int WN, int NW>
struct GemmShape {
  static constexpr int NT = NW * kWave;      // threads of the block
  static constexpr int WM = NW / WN;          // wavefronts along M (the block's NW as WM x WN)
  static constexpr int TM = BM / (32 * WM);  // 32 x 32 tiles per wavefront along M
  static constexpr int TN = BN / (32 * WN);  // ... along N
  static constexpr int kLdsRow = BK + 8;    // bf16 elements per x row in LDS (16 bytes of padding)
  static constexpr int kLdsRowW = BK + 16;  // bytes per int8 weight row in LDS (16 bytes of padding)
  static constexpr int kALoads = BM * BK * 2 / (NT * 16);  // 16-byte x loads per thread per step
  static constexpr int kBLoads = BN * BK / (NT * 16);      // 16-byte int8 loads per thread per step
  static_assert(WM * WN == NW && TM >= 1 && TN >= 1 && kALoads >= 1 && kBLoads >= 1, "tile too small for the block");
};

// 8 int8 (one LDS fragment) -> 8 bf16, exact.
__device__ __forceinline__ bf16x8 int8x8_to_bf16(const uint32_t w0, const uint32_t w1) {
  const uint32_t w[2] = {w0, w1};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float f0 = (float)(int)(int8_t)(w[i] & 0xffu);
    const float f1 = (float)(int)(int8_t)((w[i] >> 8) & 0xffu);
    const float f2 = (float)(int)(int8_t)((w[i] >> 16) & 0xffu);
    const float f3 = (float)(int)(int8_t)(w[i] >> 24);
    // the upper halves of two floats in one v_perm_b32 (bytes 2, 3 of f0, then of f1)
    o[2 * i] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
    o[2 * i + 1] = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
  }
  return __builtin_bit_cast(bf16x8, u32x4{o[0], o[1], o[2], o[3]});
}

struct GemmArgs {
  const uint16_t* x;
  int64_t ldx;
  const int8_t* w;
  int64_t ldw;
  const float* scale;
  uint16_t* y;
  int64_t ldy;
  int M, N, K;
  int tiles_m, tiles_n;
  int splits, kchunk;  // K slices (1: no split) of kchunk columns each, the last one shorter
  float* part;         // splits > 1: fp32 partial tiles [splits][M][N]
  int inter;           // SwiGLU form: features (w holds inter gate rows, then inter up rows; N = 2 inter)
};

// SwiGLU form: block tile column j (of BN) -> weight row. Each wavefront's BN / WN columns hold half of its
// features' gate rows and then the same features' up rows, so gate and up of a feature land in the same lane
// and accumulator register of a wavefront's tiles tn and tn + TN / 2. Features past `inter` read the last one.
template <int BN, int WN>
__device__ __forceinline__ int64_t swiglu_row(int64_t pid_n, int j, int inter) {
  constexpr int kPerWave = BN / WN, kHalf = kPerWave / 2;
  const int wn = j / kPerWave, o = j % kPerWave;
  const int64_t f = min(pid_n * (BN / 2) + wn * kHalf + (o % kHalf), (int64_t)inter - 1);
  return o < kHalf ? f : inter + f;
}

// Wavefronts of the 128 x 256 and 128 x 128 tiles, and how many of them lie along N.
constexpr int kNW256 = 4;
constexpr int kWN256 = 4;
constexpr int kNW128 = 8;
constexpr int kWN128 = 4;

// Blocks per CU the register allocation must allow (launch bounds): two for the
// 128 x 256 tile.
template <int BM, int BN, int NW>
constexpr int kGemmMinBlocks = (BM == 128 && BN == 256 && NW == 4) ? 2 : 1;

constexpr int kXcds = 8;        // MI355X: 8 XCDs, each with its own L2
constexpr int kGroupM = 8;      // M tiles per group of the tile order

// Block -> output tile. Blocks are dispatched round-robin to the XCDs (block b on
// XCD b % 8), so XCD x is given the contiguous range of tile numbers
// [start_x, start_x + count_x); within a range, tiles go in groups of kGroupM
// M-tiles sweeping N. The blocks that run together on one XCD then share their x
// and weight slices in that XCD's L2 instead of each streaming its own from HBM.
// Both steps are bijections of [0, tiles), so every tile is computed once whatever
// the dispatch order.
__device__ __forceinline__ void gemm_tile(int b, int tiles_m, int tiles_n, int& pid_m, int& pid_n) {
  const int tiles = tiles_m * tiles_n;
  const int base = tiles / kXcds, extra = tiles % kXcds;
  const int x = b % kXcds, j = b / kXcds;
  const int t = x * base + min(x, extra) + j;
  const int group = kGroupM * tiles_n;
  const int first_m = (t / group) * kGroupM;
  const int gm = min(tiles_m - first_m, kGroupM);
  pid_m = first_m + (t % group) % gm;
  pid_n = (t % group) / gm;
}

// The store of a block's accumulators (TM x TN 32 x 32 tiles per wavefront, wavefront tile origin wm0, wn0 in the
// block tile m0, n0): y = bf16(bf16(acc) * scale), the reference's two roundings, or with SWIGLU the activation
// of each feature from its gate and up columns.
template <int BM, int BN, int TM, int TN, int WN, bool SWIGLU>
__device__ __forceinline__ void gemm_store(const GemmArgs& a, const f32x16 (&acc)[TM][TN], int64_t m0, int64_t n0,
                                           int wm0, int wn0, int pid_n, int lane, int wave) {
  // y = bf16(bf16(acc) * scale): the reference's two roundings. Stores address y
  // by 32-bit byte offsets from the row of this lane's first accumulator (the
  // host checks that y spans < 2 GiB); row r of a tile is a constant multiple of
  // the row pitch away.
  char* yb = (char*)a.y;
  const int64_t mrow0 = m0 + wm0 + 4 * (lane / 32);
  const uint32_t pitch = (uint32_t)(a.ldy * 2);
  if constexpr (SWIGLU && TN == 1) {
    // One 32-column tile per wavefront: its columns 0-15 are the gate rows of 16 features and 16-31 their up
    // rows (swiglu_row), so lane l (column l % 32 < 16) takes u from lane l ^ 16, the same rows one tile half
    // over. The arithmetic per element is the form below.
    const int c = lane % 32;
    const int64_t f = (int64_t)pid_n * (BN / 2) + (wave % WN) * (BN / WN / 2) + (c % 16);
    const int64_t fc = min(f, (int64_t)a.inter - 1);
    const float sg_scale = a.scale[fc], su_scale = a.scale[a.inter + fc];
    const uint32_t base = (uint32_t)((mrow0 * a.ldy + f) * 2);
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float up = __shfl_xor(acc[tm][0][r], 16);
        const int dm = tm * 32 + 8 * (r / 4) + r % 4;
        if (c < 16 && mrow0 + dm < a.M && f < a.inter) {
          const float g = bf16_to_f32(f32_to_bf16(bf16_to_f32(f32_to_bf16(acc[tm][0][r])) * sg_scale));
          const float u = bf16_to_f32(f32_to_bf16(bf16_to_f32(f32_to_bf16(up)) * su_scale));
          const float sg = bf16_to_f32(f32_to_bf16(g / (1.0f + expf(-g))));
          *(uint16_t*)(yb + (base + (uint32_t)dm * pitch)) = f32_to_bf16(sg * u);
        }
      }
    }
    return;
  } else if constexpr (SWIGLU) {
    // act = bf16(bf16(silu(g)) * u) with g and u the product's two roundings (the reference's prefill formula
    // for each), SwiGLU rounded as transformers' bf16 Qwen3MLP (models/qwen3/modeling_qwen3.py:49-62): the same
    // arithmetic per element as the GEMM followed by egpt_silu_mul.
#pragma unroll
    for (int tn = 0; tn < TN / 2; ++tn) {
      const int64_t f = (int64_t)pid_n * (BN / 2) + (wave % WN) * (BN / WN / 2) + tn * 32 + lane % 32;
      const int64_t fc = min(f, (int64_t)a.inter - 1);
      const float sg_scale = a.scale[fc], su_scale = a.scale[a.inter + fc];
      const uint32_t base = (uint32_t)((mrow0 * a.ldy + f) * 2);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dm = tm * 32 + 8 * (r / 4) + r % 4;
          if (mrow0 + dm < a.M && f < a.inter) {
            const float g = bf16_to_f32(f32_to_bf16(bf16_to_f32(f32_to_bf16(acc[tm][tn][r])) * sg_scale));
            const float u = bf16_to_f32(f32_to_bf16(bf16_to_f32(f32_to_bf16(acc[tm][tn + TN / 2][r])) * su_scale));
            const float sg = bf16_to_f32(f32_to_bf16(g / (1.0f + expf(-g))));
            *(uint16_t*)(yb + (base + (uint32_t)dm * pitch)) = f32_to_bf16(sg * u);
          }
        }
      }
    }
    return;
  }
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) {
    const int64_t n = n0 + wn0 + tn * 32 + lane % 32;
    const float sc = a.scale[min(n, (int64_t)a.N - 1)];
    const uint32_t base = (uint32_t)((mrow0 * a.ldy + n) * 2);
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int dm = tm * 32 + 8 * (r / 4) + r % 4;
        if (mrow0 + dm < a.M && n < a.N) {
          const float v = bf16_to_f32(f32_to_bf16(acc[tm][tn][r]));
          *(uint16_t*)(yb + (base + (uint32_t)dm * pitch)) = f32_to_bf16(v * sc);
        }
      }
    }
  }
}

// BF16B: the weights are converted to bf16 once, by the thread that loaded them,
// as they are written to LDS, and the wavefronts read bf16 fragments; otherwise
// they stay int8 in LDS and every wavefront converts the fragments it reads (the
// wavefronts along M convert the same fragment each). BF16B doubles the weights'
// LDS space and read bytes.
template <int BM, int BN, int BK, bool SPLIT, int WN, int NW, bool SWIGLU = false, bool BF16B = false>
__global__ __launch_bounds__(NW * kWave, (kGemmMinBlocks<BM, BN, NW>)) void int8_gemm_kernel(const GemmArgs a) {
  using S = GemmShape<BM, BN, BK, WN, NW>;
  constexpr int TM = S::TM, TN = S::TN;
  static_assert(!SWIGLU || (!SPLIT && (TN % 2 == 0 || TN == 1)),
                "the SwiGLU form pairs a wavefront's column tiles, or the two halves of its one tile");
  constexpr int kLdsRow = S::kLdsRow, kLdsRowW = S::kLdsRowW;
  // weight row pitch in LDS: bytes (int8) or bf16 elements (BF16B, the x rows' pitch)
  constexpr int kBRow = BF16B ? kLdsRow : kLdsRowW;
  __shared__ __align__(16) uint16_t As[2][BM * kLdsRow];
  __shared__ __align__(16) char Bsm[2][BF16B ? BN * kLdsRow * 2 : BN * kLdsRowW];
  int8_t(&Bs)[2][BN * kLdsRowW] = *reinterpret_cast<int8_t(*)[2][BN * kLdsRowW]>(&Bsm);
  uint16_t(&Bs16)[2][BN * kLdsRow] = *reinterpret_cast<uint16_t(*)[2][BN * kLdsRow]>(&Bsm);

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int wm0 = (wave / WN) * (BM / S::WM);  // wavefront tile origin in the block tile
  const int wn0 = (wave % WN) * (BN / WN);
  const int tiles = a.tiles_m * a.tiles_n;
  const int split = SPLIT ? (int)blockIdx.x / tiles : 0;
  int pid_m, pid_n;
  gemm_tile((int)blockIdx.x - split * tiles, a.tiles_m, a.tiles_n, pid_m, pid_n);
  const int64_t m0 = (int64_t)pid_m * BM;
  const int64_t n0 = (int64_t)pid_n * BN;
  const int kbeg = SPLIT ? split * a.kchunk : 0;  // this block's K slice [kbeg, kbeg + nk * BK)

  // global -> register staging of one K step: 32-bit byte offsets from the
  // operands' base pointers (the host checks that both operands span < 2 GiB)
  const char* xb = (const char*)a.x;
  const char* wb = (const char*)a.w;
  uint32_t xoff[S::kALoads];
  int a_lds[S::kALoads];
#pragma unroll
  for (int j = 0; j < S::kALoads; ++j) {
    const int i = tid + j * S::NT;
    const int row = i / (BK / 8), chunk = i % (BK / 8);
    xoff[j] = (uint32_t)((min(m0 + row, (int64_t)a.M - 1) * a.ldx + kbeg + chunk * 8) * 2);
    a_lds[j] = row * kLdsRow + chunk * 8;
  }
  uint32_t woff[S::kBLoads];
  int b_lds[S::kBLoads];
#pragma unroll
  for (int j = 0; j < S::kBLoads; ++j) {
    const int i = tid + j * S::NT;
    const int row = i / (BK / 16), chunk = i % (BK / 16);
    const int64_t wrow = SWIGLU ? swiglu_row<BN, WN>(pid_n, row, a.inter) : min(n0 + row, (int64_t)a.N - 1);
    woff[j] = (uint32_t)(wrow * a.ldw + kbeg + chunk * 16);
    b_lds[j] = row * kBRow + chunk * 16;
  }
  // Two register staging sets: the loads of step k + 2 are issued while step k is
  // multiplied and land in LDS among the MFMAs of step k + 1, one to two steps of
  // MFMA work later. Loads past the last step re-read the last K slice (in bounds, never
  // stored), so every load is unconditional and each wait is for one set only.
  const int nk = (SPLIT ? min(a.kchunk, a.K - kbeg) : a.K) / BK;
  u32x4 xr[2][S::kALoads], wr[2][S::kBLoads];
  auto load_step = [&](int kt, int set) {
    const uint32_t k0 = (uint32_t)(min(kt, nk - 1) * BK);
#pragma unroll
    for (int j = 0; j < S::kALoads; ++j) xr[set][j] = ld16(xb + (xoff[j] + 2 * k0));
#pragma unroll
    for (int j = 0; j < S::kBLoads; ++j) wr[set][j] = ld16_stream(wb + (woff[j] + k0));
  };
  // Part q of Q of the LDS stores of one K step (the staging loads j with j % Q == q).
  auto store_part = [&](int buf, int set, int q, int Q) {
#pragma unroll
    for (int j = 0; j < S::kALoads; ++j)
      if (j % Q == q) *(u32x4*)&As[buf][a_lds[j]] = xr[set][j];
#pragma unroll
    for (int j = 0; j < S::kBLoads; ++j) {
      if (j % Q != q) continue;
      if constexpr (BF16B) {
        *(bf16x8*)&Bs16[buf][b_lds[j]] = int8x8_to_bf16(wr[set][j].x, wr[set][j].y);
        *(bf16x8*)&Bs16[buf][b_lds[j] + 8] = int8x8_to_bf16(wr[set][j].z, wr[set][j].w);
      } else {
        *(u32x4*)&Bs[buf][b_lds[j]] = wr[set][j];
      }
    }
  };
  auto store_step = [&](int buf, int set) { store_part(buf, set, 0, 1); };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) acc[tm][tn] = f32x16{};

  // fragment offsets (elements) inside one LDS buffer
  const int frag_k = 8 * (lane / 32);
  int a_frag[TM], b_frag[TN];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) a_frag[tm] = (wm0 + tm * 32 + lane % 32) * kLdsRow + frag_k;
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) b_frag[tn] = (wn0 + tn * 32 + lane % 32) * kBRow + frag_k;

  // The MFMAs of one K step from LDS buffer `buf`, 16 K columns at a time. With
  // sbuf >= 0 (large tiles) the next step's LDS stores (staging set `set` into
  // buffer sbuf) are spread over the K sub-steps, after each one's MFMAs, so their
  // conversions and writes run while the MFMAs do instead of after them.
  auto mma_step = [&](int buf, int sbuf = -1, int set = 0) {
    if constexpr (TM * TN <= 2) {
      // Small tiles run one wavefront per SIMD with a short MFMA chain per K sub-step, so
      // nothing would cover an LDS read issued just before its MFMA: read every fragment
      // of the step first, then convert and multiply.
      bf16x8 af[BK / 16][TM];
      uint32_t bw[BK / 16][TN][2];
      bf16x8 bh[BK / 16][TN];
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) af[ks][tm] = *(const bf16x8*)&As[buf][a_frag[tm] + ks * 16];
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
          if constexpr (BF16B) {
            bh[ks][tn] = *(const bf16x8*)&Bs16[buf][b_frag[tn] + ks * 16];
          } else {
            const uint32_t* p = (const uint32_t*)&Bs[buf][b_frag[tn] + ks * 16];
            bw[ks][tn][0] = p[0];
            bw[ks][tn][1] = p[1];
          }
        }
      }
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        bf16x8 bfr[TN];
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
          bfr[tn] = BF16B ? bh[ks][tn] : int8x8_to_bf16(bw[ks][tn][0], bw[ks][tn][1]);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
          for (int tn = 0; tn < TN; ++tn)
            acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ks][tm], bfr[tn], acc[tm][tn], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        bf16x8 af[TM], bfr[TN];
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) af[tm] = *(const bf16x8*)&As[buf][a_frag[tm] + ks * 16];
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
          if constexpr (BF16B) {
            bfr[tn] = *(const bf16x8*)&Bs16[buf][b_frag[tn] + ks * 16];
          } else {
            const uint32_t* p = (const uint32_t*)&Bs[buf][b_frag[tn] + ks * 16];
            bfr[tn] = int8x8_to_bf16(p[0], p[1]);
          }
        }
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
          for (int tn = 0; tn < TN; ++tn)
            acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[tm], bfr[tn], acc[tm][tn], 0, 0, 0);
        if (sbuf >= 0) store_part(sbuf, set, ks, BK / 16);
      }
    }
    if constexpr (TM * TN <= 2) {
      if (sbuf >= 0) store_step(sbuf, set);
    }
  };

  load_step(0, 0);
  load_step(1, 1);
  store_step(0, 0);
  __syncthreads();
  // Pairs of steps so the staging sets are fixed registers: step kt computes LDS
  // buffer kt & 1, refills set kt & 1 with step kt + 2 and stores set (kt + 1) & 1
  // into the other buffer among its MFMAs; an odd last step runs after the loop. Scheduling barriers keep each phase in
  // place (hoisting the second step's fragment reads above the first step's MFMAs
  // would double the live registers).
  int kt = 0;
  for (; kt + 1 < nk; kt += 2) {
    load_step(kt + 2, 0);
    __builtin_amdgcn_sched_barrier(0);
    mma_step(0, 1, 1);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    load_step(kt + 3, 1);
    __builtin_amdgcn_sched_barrier(0);
    mma_step(1, kt + 2 < nk ? 0 : -1, 0);
    __builtin_amdgcn_sched_barrier(0);
    if (kt + 2 < nk) __syncthreads();
  }
  if (kt < nk) mma_step(0);

  if constexpr (SPLIT) {  // the fp32 tile of this K slice; the reduce kernel rounds
    float* part = a.part + (int64_t)split * a.M * a.N;
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int64_t n = n0 + wn0 + tn * 32 + lane % 32;
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t m = m0 + wm0 + tm * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
          if (m < a.M && n < a.N) part[m * a.N + n] = acc[tm][tn][r];
        }
    }
    return;
  }
  gemm_store<BM, BN, TM, TN, WN, SWIGLU>(a, acc, m0, n0, wm0, wn0, pid_n, lane, wave);
}

// The 256 x 256 tile with its operands loaded straight into LDS (global_load_lds_dwordx4), three K steps of 64
// in flight: the loads of step k + 2 are issued as step k starts, with no staging registers and no LDS stores by
// the wavefronts, and each step waits only for its own loads. A step's stage holds the x rows as bf16 (128
// bytes a row) and the weight rows as int8 (64 bytes a row), 48 KiB; every wavefront converts the weight
// fragments it reads. Rows carry no padding: the 16-byte chunks of x row r sit at chunk c ^ dma_aswz(r) and those
// of weight row n at c ^ dma_bswz(n), so the 16 lanes that a 16-byte LDS read serves together ({0-3, 12-15,
// 20-23, 24-27} or {4-7, 8-11, 16-19, 28-31} of a half wavefront, measured on the MI355X) fall on distinct banks.
// Each 16-byte weight read feeds two MFMAs: the MFMA k index 8 h + e of sub-step u of K pair p stands for the
// step's column 32 p + 16 h + 8 u + e in both operands (a permutation of the sum's terms within the step).
constexpr int kDmaBK = 64;
constexpr int kDmaWaves = 8;
constexpr int kDmaStages = 3;
constexpr int kDmaARow = kDmaBK * 2;                          // bytes per x row of a stage
constexpr int kDmaBRow = kDmaBK;                              // bytes per weight row of a stage
constexpr int kDmaAStage = 256 * kDmaARow;                    // 32 KiB
constexpr int kDmaStage = kDmaAStage + 256 * kDmaBRow;        // 48 KiB
constexpr int kDmaALoads = kDmaAStage / (kDmaWaves * 1024);   // 1 KiB loads per wavefront and step: 4
constexpr int kDmaBLoads = 256 * kDmaBRow / (kDmaWaves * 1024);  // 2

__device__ __forceinline__ int dma_aswz(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ int dma_bswz(int n) { return (n >> 2) & 3; }

template <bool SWIGLU>
__global__ __launch_bounds__(kDmaWaves * kWave, 1) void int8_gemm_dma_kernel(const GemmArgs a) {
  constexpr int BM = 256, BN = 256, WN = 4, WM = kDmaWaves / WN;
  constexpr int TM = BM / (32 * WM), TN = BN / (32 * WN);  // 4 x 2 tiles of 32 x 32 per wavefront
  __shared__ __align__(16) char smem[kDmaStages * kDmaStage];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int wm0 = (wave / WN) * (BM / WM);
  const int wn0 = (wave % WN) * (BN / WN);
  int pid_m, pid_n;
  gemm_tile((int)blockIdx.x, a.tiles_m, a.tiles_n, pid_m, pid_n);
  const int64_t m0 = (int64_t)pid_m * BM;
  const int64_t n0 = (int64_t)pid_n * BN;

  // Load q of a wavefront fills 1 KiB block wave * loads + q of its operand's stage: 8 x rows (lane i: row i / 8,
  // stored chunk i % 8) or 16 weight rows (lane i: row i / 4, stored chunk i % 4). 32-bit byte offsets from the
  // operands' bases (the host checks that both span < 2 GiB); rows past M or N read the last one.
  const char* xb = (const char*)a.x;
  const char* wb = (const char*)a.w;
  uint32_t xo[kDmaALoads], wo[kDmaBLoads];
#pragma unroll
  for (int q = 0; q < kDmaALoads; ++q) {
    const int row = (wave * kDmaALoads + q) * 8 + lane / 8;
    const int c = (lane % 8) ^ dma_aswz(row);
    xo[q] = (uint32_t)((min(m0 + row, (int64_t)a.M - 1) * a.ldx + 8 * c) * 2);
  }
#pragma unroll
  for (int q = 0; q < kDmaBLoads; ++q) {
    const int row = (wave * kDmaBLoads + q) * 16 + lane / 4;
    const int c = (lane % 4) ^ dma_bswz(row);
    const int64_t wrow = SWIGLU ? swiglu_row<BN, WN>(pid_n, row, a.inter) : min(n0 + row, (int64_t)a.N - 1);
    wo[q] = (uint32_t)(wrow * a.ldw + 16 * c);
  }
  const uint32_t sbase = lds_addr(smem);
  auto issue = [&](int kt, int stage) {
    const uint32_t k0 = (uint32_t)(kt * kDmaBK);
    const uint32_t abase = sbase + (uint32_t)(stage * kDmaStage);
#pragma unroll
    for (int q = 0; q < kDmaALoads; ++q)
      lds_load16(abase + (uint32_t)((wave * kDmaALoads + q) * 1024), xb + (xo[q] + 2 * k0));
#pragma unroll
    for (int q = 0; q < kDmaBLoads; ++q)
      lds_load16(abase + (uint32_t)(kDmaAStage + (wave * kDmaBLoads + q) * 1024), wb + (wo[q] + k0));
  };

  // Fragment reads: the swizzles depend on row bits that the wavefront and tile origins (multiples of 32) leave
  // alone, so each lane's chunk offsets are fixed.
  const int r32 = lane % 32, h = lane / 32;
  const int arow = (wm0 + r32) * kDmaARow;               // + tm * 32 rows
  const int brow = kDmaAStage + (wn0 + r32) * kDmaBRow;  // + tn * 32 rows
  int ach[2][2], bch[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    bch[p] = 16 * ((2 * p + h) ^ dma_bswz(r32));
#pragma unroll
    for (int u = 0; u < 2; ++u) ach[p][u] = 16 * ((4 * p + 2 * h + u) ^ dma_aswz(r32));
  }

  f32x16 acc[TM][TN];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) acc[tm][tn] = f32x16{};

  auto compute = [&](int stage) {
    const char* sm = smem + stage * kDmaStage;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      bf16x8 bl[TN][2];
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const u32x4 w16 = *(const u32x4*)(sm + brow + tn * 32 * kDmaBRow + bch[p]);
        bl[tn][0] = int8x8_to_bf16(w16.x, w16.y);
        bl[tn][1] = int8x8_to_bf16(w16.z, w16.w);
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        bf16x8 af[TM];
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) af[tm] = *(const bf16x8*)(sm + arow + tm * 32 * kDmaARow + ach[p][u]);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
          for (int tn = 0; tn < TN; ++tn)
            acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[tm], bl[tn][u], acc[tm][tn], 0, 0, 0);
      }
    }
  };

  // Step kt: wait for this wavefront's loads of step kt (those of step kt + 1 may stay in flight), publish them
  // with the barrier (which also retires every wavefront's reads of step kt - 1's stage), refill that stage with
  // step kt + 2, multiply step kt.
  const int nk = a.K / kDmaBK;
  issue(0, 0);
  if (nk > 1) issue(1, 1);
  int stage = 0;
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk)
      EGPT_WAIT_VMCNT(kDmaALoads + kDmaBLoads);
    else
      EGPT_WAIT_VMCNT(0);
    lds_barrier();
    if (kt + 2 < nk) issue(kt + 2, stage == 0 ? 2 : stage - 1);
    compute(stage);
    stage = stage == 2 ? 0 : stage + 1;
  }
  gemm_store<BM, BN, TM, TN, WN, SWIGLU>(a, acc, m0, n0, wm0, wn0, pid_n, lane, wave);
}

// Split-K reduce: y[m, n] = bf16(bf16(sum_s part[s][m][n]) * scale[n]), splits added in order. The split
// count is a template argument so that every slice's load is issued before the first addition.
constexpr int kReduceThreads = 256;

template <int S>
__global__ __launch_bounds__(kReduceThreads) void int8_gemm_reduce_kernel(const float* __restrict__ part,
                                                                          const float* __restrict__ scale,
                                                                          uint16_t* __restrict__ y, int64_t ldy, int M,
                                                                          int N) {
  const int64_t mn = (int64_t)M * N;
  for (int64_t i = (int64_t)blockIdx.x * kReduceThreads + threadIdx.x; i < mn;
       i += (int64_t)gridDim.x * kReduceThreads) {
    float v[S];
#pragma unroll
    for (int sp = 0; sp < S; ++sp) v[sp] = part[sp * mn + i];
    float acc = v[0];
#pragma unroll
    for (int sp = 1; sp < S; ++sp) acc += v[sp];
    const int64_t m = i / N, n = i - m * N;
    y[m * ldy + n] = f32_to_bf16(bf16_to_f32(f32_to_bf16(acc)) * scale[n]);
  }
}

template <int BM, int BN>
unsigned gemm_blocks(const GemmArgs& a) {
  return (unsigned)(((int64_t)a.N + BN - 1) / BN) * (unsigned)(((int64_t)a.M + BM - 1) / BM);
}

constexpr int kMaxSplits = 16;

// Tiles whose weights go to LDS as bf16 (converted once per block, int8_gemm_kernel's BF16B).
template <int BM, int BN>
constexpr bool kBf16B = (BM == 64 && BN == 64) || (BM == 128 && BN == 64) || (BM == 128 && BN == 128);

// The reduce for a.splits (2 ... S) slices; false for a count outside that range.
template <int S>
bool launch_reduce(const GemmArgs& a, unsigned blocks, hipStream_t st) {
  if constexpr (S < 2) {
    return false;
  } else {
    if (a.splits != S) return launch_reduce<S - 1>(a, blocks, st);
    hipLaunchKernelGGL(int8_gemm_reduce_kernel<S>, dim3(blocks), dim3(kReduceThreads), 0, st, a.part, a.scale, a.y,
                       a.ldy, a.M, a.N);
    return true;
  }
}

// The split slices' fp32 tiles into a.part (64 x 64 tiles, a.splits > 1); no reduce.
int launch_split_partials(GemmArgs a, hipStream_t st) {
  a.tiles_m = (int)(((int64_t)a.M + 63) / 64);
  a.tiles_n = (int)(((int64_t)a.N + 63) / 64);
  const unsigned tiles = (unsigned)a.tiles_m * (unsigned)a.tiles_n;
  hipLaunchKernelGGL((int8_gemm_kernel<64, 64, kBKSplit, true, 2, 4, false, kBf16B<64, 64>>),
                     dim3(tiles * (unsigned)a.splits), dim3(4 * kWave), 0, st, a);
  return EGPT_LAUNCH_STATUS();
}

template <int BM, int BN, int WN = 2, int NW = 4>
int launch_gemm(GemmArgs a, hipStream_t st) {
  a.tiles_m = (int)(((int64_t)a.M + BM - 1) / BM);
  a.tiles_n = (int)(((int64_t)a.N + BN - 1) / BN);
  const unsigned tiles = (unsigned)a.tiles_m * (unsigned)a.tiles_n;
  if constexpr (BM == 64 && BN == 64 && WN == 2 && NW == 4) {  // split-K runs 64 x 64 tiles
    if (a.splits > 1) {
      if (launch_split_partials(a, st) != EGPT_OK) return EGPT_ERR_LAUNCH;
      const int64_t mn = (int64_t)a.M * a.N;
      const unsigned blocks = (unsigned)std::min<int64_t>((mn + kReduceThreads - 1) / kReduceThreads, 4096);
      if (!launch_reduce<kMaxSplits>(a, blocks, st)) return EGPT_ERR_INVALID;
      return EGPT_LAUNCH_STATUS();
    }
  }
  if constexpr (BM == 64 && BN == 64 && WN == 2 && NW == 4) {
    // Fewer tiles than CUs: each block's chain of dependent K steps is the time,
    // and a 128-wide step halves it (measured on the MI355X: 200 x 2048 -> 2048
    // 16.5 -> 12.5 us, 160 x 2048 -> 4096 16.8 -> 13.2; with 320 tiles, 300 x 2048
    // -> 4096, 1.7% slower).
    if (a.K % kBKSplit == 0 && tiles < 256) {
      hipLaunchKernelGGL((int8_gemm_kernel<64, 64, kBKSplit, false, 2, 4, false, kBf16B<64, 64>>), dim3(tiles),
                         dim3(4 * kWave), 0, st, a);
      return EGPT_LAUNCH_STATUS();
    }
  }
  hipLaunchKernelGGL((int8_gemm_kernel<BM, BN, kBK, false, WN, NW, false, kBf16B<BM, BN>>), dim3(tiles),
                     dim3(NW * kWave), 0, st, a);
  return EGPT_LAUNCH_STATUS();
}

// The 256 x 256 LDS-direct tiles (K a multiple of 64); with SWIGLU each block covers 128 features.
template <bool SWIGLU>
int launch_gemm_dma(GemmArgs a, hipStream_t st) {
  a.tiles_m = (int)(((int64_t)a.M + 255) / 256);
  a.tiles_n = SWIGLU ? (int)(((int64_t)a.inter + 127) / 128) : (int)(((int64_t)a.N + 255) / 256);
  hipLaunchKernelGGL((int8_gemm_dma_kernel<SWIGLU>), dim3((unsigned)a.tiles_m * (unsigned)a.tiles_n),
                     dim3(kDmaWaves * kWave), 0, st, a);
  return EGPT_LAUNCH_STATUS();
}

// The same product for shapes the MFMA kernel does not take (K not a multiple of
// 64, rows not 16-byte aligned, operands past its 32-bit offsets): one wavefront
// per output feature n and group of kGenericRows rows, lanes striding K with
// element loads (any alignment, 64-bit indexing), fp32 sums reduced across the
// wavefront in a fixed order, then the two roundings of the prefill formula,
// y = bf16(bf16(sum) * scale[n]). No MFMA and no LDS: a correct form for the
// odd shapes, not a fast one.
constexpr int kGenericRows = 4;
constexpr int kGenericWaves = 4;

__global__ __launch_bounds__(kGenericWaves * kWave) void int8_gemm_generic_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const int8_t* __restrict__ w, int64_t ldw,
    const float* __restrict__ scale, uint16_t* __restrict__ y, int64_t ldy, int M, int N, int K) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t mgroups = ((int64_t)M + kGenericRows - 1) / kGenericRows;
  const int64_t wv = (int64_t)blockIdx.x * kGenericWaves + threadIdx.x / kWave;
  if (wv >= mgroups * N) return;  // wave-uniform
  const int64_t n = wv / mgroups;  // neighbouring wavefronts share a weight row
  const int64_t m0 = (wv - n * mgroups) * kGenericRows;
  const int8_t* wr = w + n * ldw;
  float acc[kGenericRows] = {};
  for (int64_t k = lane; k < K; k += kWave) {
    const float wk = (float)gload(wr + k);
#pragma unroll
    for (int r = 0; r < kGenericRows; ++r)
      if (m0 + r < M) acc[r] = fmaf(bf16_to_f32(gload(x + (m0 + r) * ldx + k)), wk, acc[r]);
  }
#pragma unroll
  for (int r = 0; r < kGenericRows; ++r) {
    const float sum = wave_sum(acc[r]);
    if (lane == r && m0 + r < M) gstore(y + (m0 + r) * ldy + n, f32_to_bf16(bf16_to_f32(f32_to_bf16(sum)) * scale[n]));
  }
}

int launch_generic(const uint16_t* x, int64_t ldx, const int8_t* w, int64_t ldw, const float* scale, uint16_t* y,
                   int64_t ldy, int M, int N, int K, hipStream_t st) {
  const int64_t waves = ((int64_t)M + kGenericRows - 1) / kGenericRows * N;
  const int64_t blocks = (waves + kGenericWaves - 1) / kGenericWaves;
  if (blocks > (int64_t)UINT32_MAX) return EGPT_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(int8_gemm_generic_kernel, dim3((unsigned)blocks), dim3(kGenericWaves * kWave), 0, st, x, ldx, w,
                     ldw, scale, y, ldy, M, N, K);
  return EGPT_LAUNCH_STATUS();
}

// K slices for a short-M GEMM (at most 256 rows) whose 64 x 64 tiles leave CUs
// idle: the fewest (a power of two, at most 16) that give every CU a block, each
// slice a multiple of kBKSplit and at least 256 wide. 1 when the tiles already fill
// the chip, or K is short or not a multiple of kBKSplit.
constexpr int kMinSliceSteps = 4;
constexpr int kSplitTargetBlocks = 256;

void gemm_split(int64_t M, int64_t N, int64_t K, int& splits, int& kchunk) {
  const int64_t tiles = ((M + 63) / 64) * ((N + 63) / 64);
  splits = 1;
  kchunk = (int)K;
  if (M > 256 || K % kBKSplit) return;  // taller blocks take the larger tiles below
  // Past 128 rows only grids that fill at most half the CUs split (measured on the
  // MI355X: 200 x 2048 -> 2048, 128 tiles, 12.6 -> 10.1 us with 2 splits; 160 x 2048
  // -> 4096, 192 tiles, 13.4 -> 16.2 us with 2)
  if (M > 128 && tiles > kSplitTargetBlocks / 2) return;
  while (tiles * splits < kSplitTargetBlocks && splits < kMaxSplits && K / (2 * splits) >= kMinSliceSteps * kBK) splits *= 2;
  if (splits == 1) return;
  kchunk = (int)(((K + splits - 1) / splits + kBKSplit - 1) / kBKSplit * kBKSplit);
  splits = (int)((K + kchunk - 1) / kchunk);
}

}  // namespace
}  // namespace egpt

using namespace egpt;

extern "C" int egpt_int8_gemm_workspace(int M, int N, int K, size_t* bytes) {
  if (!bytes || M < 0 || N < 0 || K < 0) return EGPT_ERR_INVALID;
  int splits, kchunk;
  gemm_split(M, N, K, splits, kchunk);
  *bytes = splits > 1 ? (size_t)splits * (size_t)M * (size_t)N * sizeof(float) : 0;
  return EGPT_OK;
}

extern "C" int egpt_int8_gemm_ws(const void* x, int64_t ldx, const int8_t* w, int64_t ldw, const float* scale,
                                 void* y, int64_t ldy, int M, int N, int K, void* workspace, size_t workspace_bytes,
                                 hipStream_t stream) {
  if (!x || !w || !scale || !y || M < 0 || N < 0 || K < 0) return EGPT_ERR_INVALID;
  if (ldx < K || ldw < K || ldy < N) return EGPT_ERR_INVALID;
  if (M == 0 || N == 0) return EGPT_OK;
  // The MFMA kernel takes K a multiple of 64, 16-byte aligned rows and operands its
  // 32-bit byte offsets reach; every other shape runs the generic kernel.
  if (K == 0 || K % kBK || ldx % 8 || ldw % 16 || (uintptr_t)x % 16 || (uintptr_t)w % 16 ||
      (int64_t)M * ldx * 2 >= ((int64_t)1 << 31) || (int64_t)N * ldw >= ((int64_t)1 << 31) ||
      (int64_t)M * ldy * 2 >= ((int64_t)1 << 31) ||
      ((int64_t)M + 63) / 64 * (((int64_t)N + 63) / 64) > (int64_t)INT32_MAX / kMaxSplits)
    return launch_generic((const uint16_t*)x, ldx, w, ldw, scale, (uint16_t*)y, ldy, M, N, K, stream);
  GemmArgs a{(const uint16_t*)x, ldx, w, ldw, scale, (uint16_t*)y, ldy, M, N, K, 0, 0, 1, K, nullptr, 0};
  if (workspace) {  // a workspace lets short-M shapes split K
    int splits, kchunk;
    gemm_split(M, N, K, splits, kchunk);
    if (splits > 1) {
      if (workspace_bytes < (size_t)splits * (size_t)M * (size_t)N * sizeof(float) || (uintptr_t)workspace % 16)
        return EGPT_ERR_WORKSPACE;
      a.splits = splits;
      a.kchunk = kchunk;
      a.part = (float*)workspace;
      return launch_gemm<64, 64>(a, stream);
    }
  }
// The largest tile that still gives every CU a block; small M keeps more, narrower tiles.
  if (M > 128 && gemm_blocks<256, 256>(a) >= 256) return launch_gemm_dma<false>(a, stream);
  if (M > 64 && gemm_blocks<128, 256>(a) >= 256) return launch_gemm<128, 256, kWN256, kNW256>(a, stream);
  if (M > 64 && gemm_blocks<128, 128>(a) >= 256) return launch_gemm<128, 128, kWN128, kNW128>(a, stream);
  if (M > 64 && gemm_blocks<128, 64>(a) >= 256) return launch_gemm<128, 64>(a, stream);
  return launch_gemm<64, 64>(a, stream);
}

extern "C" int egpt_int8_gemm_swiglu(const void* x, int64_t ldx, const int8_t* w, int64_t ldw, const float* scale,
                                     void* act, int64_t ld_act, int M, int inter, int K, hipStream_t stream) {
  if (!x || !w || !scale || !act || M < 0 || inter < 0 || K < 0) return EGPT_ERR_INVALID;
  if (ldx < K || ldw < K || ld_act < inter) return EGPT_ERR_INVALID;
  if (M == 0 || inter == 0) return EGPT_OK;
  const int64_t N = 2 * (int64_t)inter;
  if (K == 0 || K % kBK || ldx % 8 || ldw % 16 || (uintptr_t)x % 16 || (uintptr_t)w % 16 ||
      (int64_t)M * ldx * 2 >= ((int64_t)1 << 31) || N * ldw >= ((int64_t)1 << 31) ||
      (int64_t)M * ld_act * 2 >= ((int64_t)1 << 31) || N > INT32_MAX)
    return EGPT_ERR_UNSUPPORTED;
  GemmArgs a{(const uint16_t*)x, ldx, w, ldw, scale, (uint16_t*)act, ld_act, M, (int)N, K, 0, 0, 1, K, nullptr,
             inter};
  // The tiles whose wavefronts own two column tiles (a feature's gate and up in one lane), where the plain
  // product would take them: 256 x 256 and 128 x 256 (each block covers BN / 2 features).
  auto blocks = [&](int bm, int bn) {
    return (int64_t)((M + bm - 1) / bm) * ((inter + bn / 2 - 1) / (bn / 2));
  };
  if (M > 128 && blocks(256, 256) >= 256) return launch_gemm_dma<true>(a, stream);
  if (M > 64 && blocks(128, 256) >= 256) {
    a.tiles_m = (M + 127) / 128;
    a.tiles_n = (inter + 127) / 128;
    hipLaunchKernelGGL((int8_gemm_kernel<128, 256, kBK, false, kWN256, kNW256, true>),
                       dim3((unsigned)(a.tiles_m * a.tiles_n)), dim3(kNW256 * kWave), 0, stream, a);
    return EGPT_LAUNCH_STATUS();
  }
  // 64 x 64 tiles (32 features each, gate and up in the two halves of a wavefront's tile) where the plain
  // product would run them too: not where it would split K, which this form cannot.
  int splits, kchunk;
  gemm_split(M, N, K, splits, kchunk);
  if (splits > 1 || N > INT32_MAX / 2) return EGPT_ERR_UNSUPPORTED;
  a.tiles_m = (M + 63) / 64;
  a.tiles_n = (inter + 31) / 32;
  const unsigned tiles = (unsigned)a.tiles_m * (unsigned)a.tiles_n;
  if (K % kBKSplit == 0 && tiles < 256)
    hipLaunchKernelGGL((int8_gemm_kernel<64, 64, kBKSplit, false, 2, 4, true, kBf16B<64, 64>>), dim3(tiles),
                       dim3(4 * kWave), 0, stream, a);
  else
    hipLaunchKernelGGL((int8_gemm_kernel<64, 64, kBK, false, 2, 4, true, kBf16B<64, 64>>), dim3(tiles),
                       dim3(4 * kWave), 0, stream, a);
  return EGPT_LAUNCH_STATUS();
}

extern "C" int egpt_int8_gemm_add_rmsnorm(const void* x, int64_t ldx, const int8_t* w, int64_t ldw,
                                          const float* scale, void* resid, int64_t ld_resid, const void* norm_w,
                                          void* y, int64_t ldy, int M, int N, int K, float eps, void* workspace,
                                          size_t workspace_bytes, hipStream_t stream) {
  if (!x || !w || !scale || !resid || !norm_w || !y || M < 0 || N < 0 || K < 0) return EGPT_ERR_INVALID;
  if (ldx < K || ldw < K || ld_resid < N || ldy < N) return EGPT_ERR_INVALID;
  if (M == 0 || N == 0) return EGPT_OK;
  if (K == 0 || K % kBK || ldx % 8 || ldw % 16 || (uintptr_t)x % 16 || (uintptr_t)w % 16)
    return EGPT_ERR_UNSUPPORTED;
  if ((int64_t)M * ldx * 2 >= ((int64_t)1 << 31) || (int64_t)N * ldw >= ((int64_t)1 << 31)) return EGPT_ERR_UNSUPPORTED;
  if ((size_t)N * sizeof(float) > 64 * 1024) return EGPT_ERR_UNSUPPORTED;  // the row kernel stages a row in LDS
  int splits, kchunk;
  gemm_split(M, N, K, splits, kchunk);
  if (splits < 2) return EGPT_ERR_UNSUPPORTED;  // nothing to fold: egpt_int8_gemm_ws, then egpt_add_rmsnorm
  if (!workspace || workspace_bytes < (size_t)splits * (size_t)M * (size_t)N * sizeof(float) ||
      (uintptr_t)workspace % 16)
    return EGPT_ERR_WORKSPACE;
  GemmArgs a{(const uint16_t*)x, ldx, w, ldw, scale, nullptr, N, M, N, K, 0, 0, splits, kchunk, (float*)workspace,
             0};
  const int st = launch_split_partials(a, stream);
  if (st != EGPT_OK) return st;
  return launch_reduce_add_rmsnorm((const float*)workspace, splits, scale, resid, ld_resid, norm_w, y, ldy, M, N,
                                   eps, stream);
}

extern "C" int egpt_int8_gemm_qk_norm_rope(const void* x, int64_t ldx, const int8_t* w, int64_t ldw,
                                           const float* scale, const int64_t* positions, const void* q_norm_w,
                                           const void* k_norm_w, const void* cos_t, const void* sin_t, void* q_out,
                                           int64_t ld_q, void* k_cache, void* v_cache, int64_t cache_head_stride,
                                           int64_t cache_slot_stride, int M, int Hq, int Hkv, int D, int K, int cap,
                                           float eps, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!x || !w || !scale || M < 0 || K < 0 || Hq < 1 || Hkv < 1 || D < 1) return EGPT_ERR_INVALID;
  const int64_t N = (int64_t)(Hq + 2 * Hkv) * D;
  if (ldx < K || ldw < K || N > INT32_MAX) return EGPT_ERR_INVALID;
  if (M == 0) return EGPT_OK;
  if (K == 0 || K % kBK || ldx % 8 || ldw % 16 || (uintptr_t)x % 16 || (uintptr_t)w % 16)
    return EGPT_ERR_UNSUPPORTED;
  if ((int64_t)M * ldx * 2 >= ((int64_t)1 << 31) || N * ldw >= ((int64_t)1 << 31)) return EGPT_ERR_UNSUPPORTED;
  int splits, kchunk;
  gemm_split(M, N, K, splits, kchunk);
  if (splits < 2) return EGPT_ERR_UNSUPPORTED;  // nothing to fold: egpt_int8_gemm_ws, then egpt_qk_norm_rope
  const int c = check_reduce_qk_norm_rope(splits, positions, q_norm_w, k_norm_w, cos_t, sin_t, q_out, ld_q, k_cache,
                                          v_cache, cache_head_stride, cache_slot_stride, M, Hq, Hkv, D, cap);
  if (c != EGPT_OK) return c;
  if (!workspace || workspace_bytes < (size_t)splits * (size_t)M * (size_t)N * sizeof(float) ||
      (uintptr_t)workspace % 16)
    return EGPT_ERR_WORKSPACE;
  GemmArgs a{(const uint16_t*)x, ldx, w, ldw, scale, nullptr, N, M, (int)N, K, 0, 0, splits, kchunk,
             (float*)workspace, 0};
  const int st = launch_split_partials(a, stream);
  if (st != EGPT_OK) return st;
  return launch_reduce_qk_norm_rope((const float*)workspace, splits, scale, positions, q_norm_w, k_norm_w, cos_t,
                                    sin_t, q_out, ld_q, k_cache, v_cache, cache_head_stride, cache_slot_stride, M, Hq,
                                    Hkv, D, cap, eps, stream);
}

extern "C" int egpt_int8_gemm(const void* x, int64_t ldx, const int8_t* w, int64_t ldw, const float* scale, void* y,
                              int64_t ldy, int M, int N, int K, hipStream_t stream) {
  return egpt_int8_gemm_ws(x, ldx, w, ldw, scale, y, ldy, M, N, K, nullptr, 0, stream);
}
