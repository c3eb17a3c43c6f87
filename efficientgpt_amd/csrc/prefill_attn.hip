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
// units of the raw scores, p = 2^((q.k - m) * scale * log2 e), the flash form's
// folded scale, with a reference maximum m that moves only when a tile's maximum
// passes it by more than 8 in the exponent (so p < 2^8 and the output is rescaled
// on few tiles).
//
// A block is 8 wavefronts over one kv head; each wavefront owns 32 consecutive
// query rows of one query head, so a block covers min(group, 4) query heads and
// 32 * 8 / min(group, 4) positions, and every head of the block shares the K/V
// tiles it stages. K/V advance 64 slots at a time, loaded straight into LDS
// (global_load_lds_dwordx4) two tiles ahead, through three K and four V buffers
// (wavefronts 4-7 run a phase behind 0-3 and read tile j - 1's V during tile j).
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
//     (bits 2 and 3 of the slot swapped). V stays slot-major in LDS; the A operand
//     V^T takes two transposing reads (ds_read_b64_tr_b16) per MFMA, slots
//     4 (l / 32) + 0..3 and 8 + 4 (l / 32) + 0..3 of the step. The output
//     accumulators also hold one query per lane, so the online-softmax rescale is
//     per lane too.
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
constexpr float kPfLog2e = 1.4426950408889634f;
constexpr float kPfLazy = 8.f;  // exponent by which a score may pass the softmax's reference maximum (p < 2^8)

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

typedef short v4i16_pf __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16 (gfx950): within each group of 16 lanes, lane l receives element l % 4 of the four
// 16-bit elements at the addresses of lanes (l % 16) / 4 + 4 i, i = 0..3 (checked on the MI355X).
__device__ __forceinline__ uint2 lds_read_tr16(const char* p) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                       (__attribute__((address_space(3))) v4i16_pf*)(const void*)p));
}

// D: head dim (32, 64 or 128), a multiple of the MFMA's 32 output rows.
template <int D>
__global__ __launch_bounds__(kPfThreads, 1) void prefill_attn_kernel(const PrefillArgs a) {
  constexpr int kPfD = D;
  constexpr int kChunks = kPfD / 8;     // 16-byte chunks per K/V row (slot)
  constexpr int kLogC = kPfD == 128 ? 4 : kPfD == 64 ? 3 : 2;
  constexpr int kRow = 2 * kPfD;        // bytes per slot row in LDS (no padding: chunks swizzled)
  constexpr int kTile = kPfSlots * kRow;
  constexpr int kTileLoads = 2 * kTile / (kPfWaves * 1024);  // 1 KiB LDS-direct loads per wavefront and tile
  // K row r keeps chunk c at c ^ kswz(r), so the 16 rows a 16-byte read pass serves ({0-3, 12-15, 20-23,
  // 24-27} or {4-7, 8-11, 16-19, 28-31} of a half wavefront) land on distinct banks; V row r at c ^ vswz(r),
  // so the four rows x 64 bytes of a transposing read pass do.
  auto kswz = [](int r) { return (r >> (4 - kLogC)) & (kChunks - 1); };
  auto vswz = [](int r) { return 4 * ((r & 3) >> (4 - kLogC)); };
  __shared__ __align__(16) char Ks[3][kTile];
  __shared__ __align__(16) char Vs[4][kTile];

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

  // Loads of one K/V tile (64 slots x kChunks chunks of 8 dims each, K then V): 1 KiB blocks t = wave + 8 q;
  // lane i of a block fills row i / kChunks, stored chunk i % kChunks. Slots past the block's last position read
  // the last one.
  const uint16_t* kb = a.k + (int64_t)hk * a.c_sh;
  const uint16_t* vb = a.v + (int64_t)hk * a.c_sh;
  const uint32_t kbase = lds_addr(&Ks[0][0]), vbase = lds_addr(&Vs[0][0]);
  auto issue = [&](int j) {
#pragma unroll
    for (int q = 0; q < kTileLoads; ++q) {
      const int t = wave + kPfWaves * q;
      const bool isk = t < kTile / 1024;  // wave-uniform
      const int blk = isk ? t : t - kTile / 1024;
      const int row = blk * (1024 / kRow) + lane / kChunks;
      const int c = (lane % kChunks) ^ (isk ? kswz(row) : vswz(row));
      const int64_t sl = min((int64_t)j * kPfSlots + row, last);
      const uint32_t dst = isk ? kbase + (uint32_t)((j % 3) * kTile + blk * 1024)
                               : vbase + (uint32_t)((j % 4) * kTile + blk * 1024);
      lds_load16(dst, (isk ? kb : vb) + sl * a.c_sn + 8 * c);
    }
  };

  // B fragments of Q^T: this lane's query, dims 16 kk + 8 half .. + 7, loaded while tile 0 is, and waited for
  // before the loop: the compiler does not see the LDS-direct loads, so a load of its own still pending in the
  // loop would make it wait for every load in flight before each q . k.
  issue(0);
  u32x4 qf[kPfD / 16];
  {
    const uint16_t* qrow = a.q + (int64_t)min(tq, a.rows - 1) * a.q_ld + (int64_t)hq * kPfD + 8 * half;
#pragma unroll
    for (int kk = 0; kk < kPfD / 16; ++kk) qf[kk] = ld16(qrow + 16 * kk);
  }
  EGPT_WAIT_VMCNT(0);
  if (nt > 1) issue(1);

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
        const u32x4 av = *(const u32x4*)&Ks[b][(32 * mt + col) * kRow + 16 * ((2 * kk + half) ^ kswz(col))];
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
    // The reference maximum m moves only when the tile's maximum passes it by more than kPfLazy in the exponent,
    // so the probabilities stay below 2^kPfLazy (the output is o / l whichever maximum they are taken against)
    // and the output is rescaled only on those tiles. m starts at -inf: the first tile with a visible slot sets
    // it (mx - m is then +inf), a tile with none leaves it (NaN or -inf compare false).
    const float c = a.scale * kPfLog2e;
    const bool move = (mx - m) * c > kPfLazy;
    const float mn = move ? mx : m;
    const float mref = mn == -INFINITY ? 0.f : mn;
    const float alpha = move ? __builtin_amdgcn_exp2f((m - mref) * c) : 1.f;
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
    if (__builtin_amdgcn_ballot_w64(move)) {
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
  // O^T += V^T P^T over the four 16-slot steps of the V tile in LDS buffer b. Lane s points its two transposing
  // reads at slot 4 (s / 32) + (s % 16) / 4 (and 8 slots on) of the step, dims 32 dt + 16 ((s / 16) % 2) +
  // 4 (s % 4) .. + 3, so lane l receives V^T[32 dt + l % 32][the step's slots 4 (l / 32) + 0..3, then + 8].
  const int vrow = 4 * half + (lane % 16) / 4;
  int voff[kPfD / 32];
#pragma unroll
  for (int dt = 0; dt < kPfD / 32; ++dt)
    voff[dt] = vrow * kRow + 16 * ((4 * dt + 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1)) ^ vswz(vrow)) + 8 * (lane & 1);
  auto pv = [&](int b, const u32x4 (&pb)[4]) {
#pragma unroll
    for (int js = 0; js < 4; ++js) {
#pragma unroll
      for (int dt = 0; dt < kPfD / 32; ++dt) {
        const char* vp = &Vs[b][16 * js * kRow + voff[dt]];
        const uint2 lo = lds_read_tr16(vp), hi = lds_read_tr16(vp + 8 * kRow);
        const u32x4 av{lo.x, lo.y, hi.x, hi.y};
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_pf, av),
                                                        __builtin_bit_cast(bf16x8_pf, pb[js]), o[dt], 0, 0, 0);
      }
    }
  };

  // Wavefronts 4-7 run a phase behind 0-3: in the iteration of tile j they
  // multiply tile j - 1's p . v first, then tile j's q . k and softmax, so while
  // the wavefront beside them on their SIMD is in its softmax (VALU) they are in
  // q . k, and in their softmax it is in p . v (MFMA). V tiles stay for one more
  // iteration, so V rotates through four LDS buffers and K through three. Every
  // output accumulator takes the same operations in the same order either way.
  const bool lag = wave >= kPfWaves / 2;  // wave-uniform
  u32x4 pprev[4];
  // Tile j: wait for this wavefront's loads of tile j (tile j + 1's stay in flight), publish them with the
  // barrier, which also retires every wavefront's reads of K tile j - 1 and V tile j - 2, load tile j + 2 into
  // those buffers, multiply tile j.
#pragma unroll 1
  for (int j = 0; j < nt; ++j) {
    if (j + 1 < nt)
      EGPT_WAIT_VMCNT(kTileLoads);
    else
      EGPT_WAIT_VMCNT(0);
    lds_barrier();
    if (j + 2 < nt) issue(j + 2);
    const int kbuf = j % 3, vbuf = j % 4;
    f32x16_pf st[2];
    // A wavefront raises its issue priority for its MFMA phases, so that where both wavefronts of a SIMD are
    // ready the one feeding the matrix core goes first and the other's softmax fills in behind it.
    if (!lag) {
      u32x4 pb[4];
      __builtin_amdgcn_s_setprio(1);
      qk(kbuf, st);
      __builtin_amdgcn_s_setprio(0);
      softmax(j, st, pb);
      __builtin_amdgcn_s_setprio(1);
      pv(vbuf, pb);
      __builtin_amdgcn_s_setprio(0);
    } else {
      __builtin_amdgcn_s_setprio(1);
      if (j > 0) pv(vbuf == 0 ? 3 : vbuf - 1, pprev);
      qk(kbuf, st);
      __builtin_amdgcn_s_setprio(0);
      softmax(j, st, pprev);
    }
  }
  if (lag) pv((nt - 1) % 4, pprev);  // tile nt - 1

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
