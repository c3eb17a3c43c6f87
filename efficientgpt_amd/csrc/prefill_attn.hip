// Causal GQA attention over a prompt (prefill), flash form on gfx950 MFMA.
//
//   out[t, hq, :] = sum_{s <= pos0 + t} softmax_s((q[t, hq] . k[hk, s]) * scale) v[hk, s]
//
// for query rows t = 0 .. rows - 1 at positions pos0 + t, query head hq of kv
// head hk = hq / group. This is the attention of the reference's prompt pass (the
// transformers Qwen3 forward over the prompt: SDPA with a causal mask over the
// static cache, HF models/qwen3/modeling_qwen3.py), for which the decode kernels
// would rescan the prefix once per query row. bf16 q, k, v and output; the logits
// (q . k) * scale and the online softmax in fp32; the probabilities enter the
// p . v products as bf16, as in SDPA's bf16 flash path; the softmax runs in the
// units of the raw scores, p = 2^((q.k - max) * scale * log2 e), the flash form's
// folded scale.
//
// A block is 8 wavefronts over one kv head; each wavefront owns 32 consecutive
// query rows of one query head, so a block covers min(group, 4) query heads and
// 32 * 8 / min(group, 4) positions, and every head of the block shares the K/V
// tiles it stages. K/V advance 64 slots at a time through three LDS buffers (the
// global loads of tile j + 1 are issued before tile j is multiplied; wavefronts
// 4-7 run a phase behind 0-3 and read tile j - 1's V during tile j).
//
// Per tile and wavefront, with v_mfma_f32_32x32x16_bf16 (lane l holds A[l % 32]
// [8 (l / 32) + e] and B[8 (l / 32) + e][l % 32]; accumulator register r of lane
// l is C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32]):
//   * S^T = K Q^T: K rows from LDS as A, the wavefront's queries as B (held in
//     registers for the whole kernel). Lane l's accumulators then hold 16 slots
//     of ONE query, l % 32 (its other 16 are in lane l ^ 32), so the softmax
//     statistics of a query are per lane: the row max and sum need one lane swap.
//   * O^T += V^T P^T: the probabilities go from those accumulators straight into
//     the B operand (no LDS round trip). That operand's k index 8 (l / 32) + e
//     then stands for slot 8 (e / 4) + 4 (l / 32) + e % 4 of a 16-slot step
//     (bits 2 and 3 of the slot swapped), so V^T is staged in LDS with its slots
//     in that order. The output accumulators also hold one query per lane, so the
//     online-softmax rescale is per lane too.
// Padding query rows (past `rows`) read a valid row and are never stored; slots
// past the block's last position read the last one and are masked.
#include "common.h"

namespace egpt {
namespace {

typedef __bf16 bf16x8_pf __attribute__((ext_vector_type(8)));
typedef float f32x16_pf __attribute__((ext_vector_type(16)));

constexpr int kPfSlots = 64;           // K/V slots per tile
constexpr int kPfWaves = 8;
constexpr int kPfThreads = kPfWaves * 64;
constexpr int kPfStage = kPfThreads / 2;  // threads staging K (and as many staging V)
constexpr int kPfVRow = kPfSlots + 8;  // bf16 per V^T row in LDS
constexpr float kPfLog2e = 1.4426950408889634f;

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_ld;
  const uint16_t* k;
  const uint16_t* v;
  int64_t c_sh, c_sn;
  uint16_t* out;
  int64_t o_ld;
  int rows, group, pos0;
  int hb;      // query heads per block
  int bt;      // query positions per block
  int ntiles;  // position tiles
  float scale;
};

// Position of slot s (0..15 of a 16-slot step) in the staged V^T row: bits 2 and 3 swapped.
__device__ __forceinline__ int vperm(int s) { return (s & 3) | ((s >> 2 & 1) << 3) | ((s >> 3 & 1) << 2); }

// The 8-slot (16-byte) chunks of V^T row r sit at chunk index c ^ vswz(r): bit 0 of vswz is row bit 6, bit 1 row
// bit 5, bit 2 the parity of row bits 2-4. Unswizzled rows are 36 banks apart, so the 16 lanes of an 8-byte
// store pass (rows 8 apart, one per chunk of dims) all hit the same banks; with it they pair up two to a bank.
// A 16-byte read pass serves the lanes {0-3, 12-15, 20-23, 24-27} (or {4-7, 8-11, 16-19, 28-31}) of a half
// wavefront over 64 banks; the p . v reads of those 16 rows (one chunk each) still fall on distinct banks.
__device__ __forceinline__ int vswz(int r) { return ((r >> 6) & 1) | ((r >> 4) & 2) | ((((r >> 2) ^ (r >> 3) ^ (r >> 4)) & 1) << 2); }

// D: head dim (32, 64 or 128), a multiple of the MFMA's 32 output rows.
template <int D>
__global__ __launch_bounds__(kPfThreads, 1) void prefill_attn_kernel(const PrefillArgs a) {
  constexpr int kPfD = D;
  constexpr int kPfKRow = kPfD + 8;     // bf16 per K row in LDS (16 bytes of padding)
  constexpr int kChunks = kPfD / 8;     // 16-byte chunks per K/V row
  constexpr int kLoads = kChunks / 4;   // 16-byte loads per staging thread and tile: 64 slots x kChunks / 256
  __shared__ __align__(16) uint16_t Ks[3][kPfSlots * kPfKRow];
  __shared__ __align__(16) uint16_t Vs[3][kPfD * kPfVRow];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int half = lane >> 5;
  const int col = lane & 31;
  // Block -> (kv head, subset of its query heads, position tile). The first
  // blocks dispatched take the last position tiles, whose causal ranges are the
  // longest.
  const int subsets = a.group / a.hb;
  const int hk = (int)blockIdx.x / subsets;
  const int sub = (int)blockIdx.x % subsets;
  const int ptile = a.ntiles - 1 - (int)blockIdx.y;
  const int t0 = ptile * a.bt;
  const int wph = a.bt / 32;  // wavefronts per query head
  const int hq = hk * a.group + sub * a.hb + wave / wph;
  const int tw = t0 + (wave % wph) * 32;  // the wavefront's first query row
  const int tq = tw + col;                // this lane's query row
  const int64_t qpos = (int64_t)a.pos0 + tq;
  // Slots this block visits: 0 .. its last query's position.
  const int64_t last = (int64_t)a.pos0 + min(t0 + a.bt, a.rows) - 1;
  const int nt = (int)(last / kPfSlots) + 1;

  // B fragments of Q^T: this lane's query, dims 16 kk + 8 half .. + 7.
  u32x4 qf[kPfD / 16];
  {
    const uint16_t* qrow = a.q + (int64_t)min(tq, a.rows - 1) * a.q_ld + (int64_t)hq * kPfD + 8 * half;
#pragma unroll
    for (int kk = 0; kk < kPfD / 16; ++kk) qf[kk] = ld16(qrow + 16 * kk);
  }

  // Staging of one K/V tile: 64 slots x kChunks chunks of 8 dims each for K and V.
  // The first 4 wavefronts stage V, the other 4 K, so every thread keeps kLoads
  // 16-byte loads in flight (4 at D 128). A K thread t takes chunks (slot c /
  // kChunks, chunk c % kChunks) for c = t + 256 i; a V thread t < 64 kChunks / 4
  // takes chunk vc = t % kChunks of the four consecutive slots 4 vg .. 4 vg + 3 (vg
  // = t / kChunks), whose staged positions are consecutive too (vperm keeps bits 0
  // and 1), so each of its 8 dims is one 8-byte LDS store; at D < 128 the other V
  // threads stage nothing.
  const uint16_t* kb = a.k + (int64_t)hk * a.c_sh;
  const uint16_t* vb = a.v + (int64_t)hk * a.c_sh;
  const int stid = tid % kPfStage;
  const bool do_k = tid >= kPfStage;  // wave-uniform
  const int vg = stid / kChunks, vc = stid % kChunks;
  const bool v_stager = vg < kPfSlots / 4;
  u32x4 sr[4];
  auto gload = [&](int j) {
    if (do_k) {
#pragma unroll
      for (int i = 0; i < kLoads; ++i) {
        const int c = stid + kPfStage * i;
        const int64_t s = min((int64_t)j * kPfSlots + c / kChunks, last);
        sr[i] = ld16(kb + s * a.c_sn + (c % kChunks) * 8);
      }
    } else if (v_stager) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t s = min((int64_t)j * kPfSlots + 4 * vg + i, last);
        sr[i] = ld16(vb + s * a.c_sn + vc * 8);
      }
    }
  };
  auto lstore = [&](int buf) {
    if (do_k) {
#pragma unroll
      for (int i = 0; i < kLoads; ++i) {
        const int c = stid + kPfStage * i;
        *(u32x4*)&Ks[buf][(c / kChunks) * kPfKRow + (c % kChunks) * 8] = sr[i];
      }
    } else if (v_stager) {
      // V^T: dim vc * 8 + e of slots 4 vg .. 4 vg + 3 at their staged positions, in chunk order vswz
      const int p0 = (4 * vg) & ~15;
      const int p = p0 + vperm((4 * vg) & 15);
      // dim 2 w + h of the four slots: the 16-bit half h of word w of each row,
      // two slots per v_perm_b32 (bytes 0-1 or 2-3 of each source)
      const uint32_t r0[4] = {sr[0].x, sr[0].y, sr[0].z, sr[0].w};
      const uint32_t r1[4] = {sr[1].x, sr[1].y, sr[1].z, sr[1].w};
      const uint32_t r2[4] = {sr[2].x, sr[2].y, sr[2].z, sr[2].w};
      const uint32_t r3[4] = {sr[3].x, sr[3].y, sr[3].z, sr[3].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
        const int w = e / 2;
        const int row = vc * 8 + e;
        *(uint2*)&Vs[buf][row * kPfVRow + (p ^ (vswz(row) * 8))] =
            make_uint2(__builtin_amdgcn_perm(r1[w], r0[w], sel), __builtin_amdgcn_perm(r3[w], r2[w], sel));
      }
    }
  };

  f32x16_pf o[kPfD / 32];
#pragma unroll
  for (int dt = 0; dt < kPfD / 32; ++dt) o[dt] = f32x16_pf{};
  float m = -INFINITY, l = 0.f;

  // S^T for slots 64 j + 32 mt + (8 (r / 4) + 4 half + r % 4), query col, from
  // the K tile in LDS buffer b (the two 32-slot halves are independent chains:
  // interleaved, each MFMA's accumulator was written two MFMAs earlier).
  auto qk = [&](int b, f32x16_pf (&st)[2]) {
    st[0] = f32x16_pf{};
    st[1] = f32x16_pf{};
#pragma unroll
    for (int kk = 0; kk < kPfD / 16; ++kk)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const u32x4 av = *(const u32x4*)&Ks[b][(32 * mt + col) * kPfKRow + 8 * half + 16 * kk];
        st[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_pf, av),
                                                         __builtin_bit_cast(bf16x8_pf, qf[kk]), st[mt], 0, 0, 0);
      }
  };
  // Online softmax of this lane's query over tile j's 64 slots (32 here, 32 in
  // lane ^ 32), in the units of the raw scores q . k: the scale is positive, so
  // the maximum commutes with it, and p = 2^((s - m) * scale * log2 e) takes one
  // FMA and one exp2 per slot. Tiles wholly at or before the wavefront's first
  // position need no causal mask (wave-uniform). The output is rescaled here; the
  // probabilities leave as the bf16 B operands of the four 16-slot p . v steps.
  auto softmax = [&](int j, f32x16_pf (&st)[2], u32x4 (&pb)[4]) {
    if ((int64_t)j * kPfSlots + kPfSlots - 1 > (int64_t)a.pos0 + tw) {
      // slots of the tile this lane's query sees: those at most lim past the tile's first
      const int lim = (int)min((int64_t)kPfSlots, max((int64_t)-1, qpos - (int64_t)j * kPfSlots));
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int sl = 32 * mt + 8 * (r / 4) + 4 * half + r % 4;
          st[mt][r] = sl <= lim ? st[mt][r] : -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, st[mt][r]);
    LanePair pr = pair32(mx);
    mx = fmaxf(pr.lo, pr.hi);
    const float mn = fmaxf(m, mx);
    const float mref = mn == -INFINITY ? 0.f : mn;
    const float c = a.scale * kPfLog2e;
    const float alpha = __builtin_amdgcn_exp2f((m - mref) * c);
    const float off = -mref * c;
    float ps = 0.f;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(fmaf(st[mt][r], c, off));  // 0 for masked slots
        st[mt][r] = p;
        ps += p;
      }
    pr = pair32(ps);
    ps = pr.lo + pr.hi;
    l = l * alpha + ps;
    m = mn;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {  // once the maxima settle alpha is exactly 1
#pragma unroll
      for (int dt = 0; dt < kPfD / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
    }
#pragma unroll
    for (int js = 0; js < 4; ++js) {
      const f32x16_pf& pt = st[js / 2];
      const int r0 = 8 * (js % 2);
      pb[js] = u32x4{pack2_bf16(pt[r0], pt[r0 + 1]), pack2_bf16(pt[r0 + 2], pt[r0 + 3]),
                     pack2_bf16(pt[r0 + 4], pt[r0 + 5]), pack2_bf16(pt[r0 + 6], pt[r0 + 7])};
    }
  };
  // O^T += V^T P^T over the four 16-slot steps of the V tile in LDS buffer b.
  auto pv = [&](int b, const u32x4 (&pb)[4]) {
#pragma unroll
    for (int js = 0; js < 4; ++js) {
#pragma unroll
      for (int dt = 0; dt < kPfD / 32; ++dt) {
        const int row = col + 32 * dt;
        const u32x4 av = *(const u32x4*)&Vs[b][row * kPfVRow + (((2 * js + half) ^ vswz(row)) * 8)];
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_pf, av),
                                                        __builtin_bit_cast(bf16x8_pf, pb[js]), o[dt], 0, 0, 0);
      }
    }
  };

  // Wavefronts 4-7 run a phase behind 0-3: in the iteration of tile j they
  // multiply tile j - 1's p . v first, then tile j's q . k and softmax, so while
  // the wavefront beside them on their SIMD is in its softmax (VALU) they are in
  // q . k, and in their softmax it is in p . v (MFMA). V tiles stay for one more
  // iteration, so the tiles rotate through three LDS buffers. Every output
  // accumulator takes the same operations in the same order either way.
  const bool lag = wave >= kPfWaves / 2;  // wave-uniform
  u32x4 pprev[4];
  gload(0);
  lstore(0);
  __syncthreads();
  int b = 0;  // LDS buffer of tile j (j mod 3)
#pragma unroll 1
  for (int j = 0; j < nt; ++j) {
    const int bn = b == 2 ? 0 : b + 1;
    if (j + 1 < nt) gload(j + 1);
    f32x16_pf st[2];
    if (!lag) {
      u32x4 pb[4];
      qk(b, st);
      softmax(j, st, pb);
      pv(b, pb);
    } else {
      if (j > 0) pv(b == 0 ? 2 : b - 1, pprev);
      qk(b, st);
      softmax(j, st, pprev);
    }
    if (j + 1 < nt) lstore(bn);
    __syncthreads();
    b = bn;
  }
  if (lag) pv(b == 0 ? 2 : b - 1, pprev);  // tile nt - 1

  // out[tq, hq, 32 dt + 8 (r / 4) + 4 half + r % 4] = o / l, four dims per 8-byte store
  if (tq < a.rows) {
    const float inv = 1.f / l;
    uint16_t* orow = a.out + (int64_t)tq * a.o_ld + (int64_t)hq * kPfD + 4 * half;
#pragma unroll
    for (int dt = 0; dt < kPfD / 32; ++dt)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const uint32_t lo = pack2_bf16(o[dt][4 * r4] * inv, o[dt][4 * r4 + 1] * inv);
        const uint32_t hi = pack2_bf16(o[dt][4 * r4 + 2] * inv, o[dt][4 * r4 + 3] * inv);
        *(uint2*)(orow + 32 * dt + 8 * r4) = make_uint2(lo, hi);
      }
  }
}

}  // namespace
}  // namespace egpt

using namespace egpt;

extern "C" int egpt_prefill_attn(const void* q, int64_t q_ld, const void* k, const void* v, int64_t c_sh,
                                 int64_t c_sn, void* out, int64_t o_ld, int rows, int Hq, int Hkv, int D, int cap,
                                 int pos0, float scale, hipStream_t stream) {
  if (!q || !k || !v || !out || rows < 0 || Hq < 1 || Hkv < 1 || Hq % Hkv || cap < 1 || pos0 < 0 || !(scale > 0.f))
    return EGPT_ERR_INVALID;
  if (rows == 0) return EGPT_OK;
  if ((int64_t)pos0 + rows > cap) return EGPT_ERR_INVALID;
  if (D != 32 && D != 64 && D != 128) return EGPT_ERR_UNSUPPORTED;
  const int group = Hq / Hkv;
  if (q_ld < (int64_t)Hq * D || o_ld < (int64_t)Hq * D || c_sn < D || c_sh < (int64_t)cap * c_sn) return EGPT_ERR_INVALID;
  if (q_ld % 8 || o_ld % 4 || c_sn % 8 || c_sh % 8 || ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v) % 16 ||
      (uintptr_t)out % 8)
    return EGPT_ERR_UNSUPPORTED;
  PrefillArgs a{};
  a.q = (const uint16_t*)q;
  a.q_ld = q_ld;
  a.k = (const uint16_t*)k;
  a.v = (const uint16_t*)v;
  a.c_sh = c_sh;
  a.c_sn = c_sn;
  a.out = (uint16_t*)out;
  a.o_ld = o_ld;
  a.rows = rows;
  a.group = group;
  a.pos0 = pos0;
  // query heads per block: the largest of 4, 2, 1 that divides the group
  a.hb = group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1;
  a.bt = 32 * kPfWaves / a.hb;
  a.ntiles = (rows + a.bt - 1) / a.bt;
  a.scale = scale;
  const dim3 grid((unsigned)(Hkv * (group / a.hb)), (unsigned)a.ntiles);
  switch (D) {
    case 32: hipLaunchKernelGGL(prefill_attn_kernel<32>, grid, dim3(kPfThreads), 0, stream, a); break;
    case 64: hipLaunchKernelGGL(prefill_attn_kernel<64>, grid, dim3(kPfThreads), 0, stream, a); break;
    default: hipLaunchKernelGGL(prefill_attn_kernel<128>, grid, dim3(kPfThreads), 0, stream, a); break;
  }
  return EGPT_LAUNCH_STATUS();
}
