// Split-K GQA decode attention (flash decoding) for gfx950 (MI355X).
//
// One query per (batch row, query head). Query head h reads kv head h / G,
// G = Hq / Hkv. The live key range of row b is slots 0..position[b]; it is cut
// into `nsplit` contiguous pieces at run time (the position is read on the
// device, so a captured graph keeps working as the sequence grows). Each block
// owns one (b, kv head, split) and serves all G query heads of the group, so
// every K/V byte is read once. A second kernel merges the per-split partial
// softmax states. The arithmetic lives in attn_core.h; its summation order
// differs from SDPA, so results are not bit-exact against it.
#include <mutex>

#include "attn_core.h"

namespace egpt {
namespace {

// One 16-byte load per lane per K/V row, 4 slots per stream per iteration: the
// fastest layout of a cold sweep (L 4096 / 32768, 16 q / 8 kv heads, D 128).
template <typename T>
constexpr int kSplitLPR = 1;
template <typename T>
constexpr int kSplitUnroll = 4;

// Caches up to this many slots run the single-pass form by default.
constexpr int kOnePassMaxSlots = 256;

template <typename T, int D, int G, int NT = kAttnThreads>
__global__ __launch_bounds__(NT) void attn_split_kernel(
    const T* __restrict__ q, int64_t q_sb, int64_t q_sh, const T* __restrict__ k, int64_t k_sb, int64_t k_sh,
    int64_t k_sn, const T* __restrict__ v, int64_t v_sb, int64_t v_sh, int64_t v_sn,
    const int64_t* __restrict__ position, int64_t pos_stride, float* __restrict__ ws_m, float* __restrict__ ws_l,
    float* __restrict__ ws_acc, int Hkv, int cap, int nsplit, float scale, T* __restrict__ out, int64_t o_sb,
    int64_t o_sh) {
  constexpr int LPR = kSplitLPR<T>;
  constexpr int U = G >= 8 ? 2 : kSplitUnroll<T>;  // G >= 8: two buffers of 4 slots spill
  using Geo = AttnGeom<T, D, NT, LPR, U>;
  constexpr int EPL = Geo::EPL;
  constexpr int EPV = Geo::EPV;
  const int d0 = (threadIdx.x % Geo::LPS) * EPL;
  const int bh = blockIdx.x;  // b * Hkv + kv head
  const int b = bh / Hkv;
  const int hk = bh % Hkv;
  const int split = blockIdx.y;
  const int Hq = Hkv * G;

  int64_t len = position[(int64_t)b * pos_stride] + 1;
  len = len < 1 ? 1 : (len > cap ? cap : len);
  int64_t start, end;
  attn_split_range(len, nsplit, split, start, end);

  if constexpr (kAttnMfma<T, D, G>) {
    // q . k on MFMA: the B fragments of Q^T straight from q (column h = lane % 16 is
    // query head hk * G + h; zero past the group), then the first K/V tile.
    const int lane = threadIdx.x % kWave;
    const int h = lane & 15;
    bf16x8_mt qb[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const u32x4 z{0u, 0u, 0u, 0u};
      const u32x4 v = ld16(q + (int64_t)b * q_sb + (int64_t)(hk * G + (h < G ? h : 0)) * q_sh + 32 * c + 8 * (lane >> 4));
      qb[c] = __builtin_bit_cast(bf16x8_mt, h < G ? v : z);
    }
    const __bf16* kbb = (const __bf16*)(k + (int64_t)b * k_sb + (int64_t)hk * k_sh);
    const __bf16* vbb = (const __bf16*)(v + (int64_t)b * v_sb + (int64_t)hk * v_sh);
    MfmaKV t0;
    mfma_issue(t0, kbb, k_sn, vbb, v_sn, start + kMfmaSlots * (int)(threadIdx.x / kWave), end);
    const float none[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float qnone[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) qnone[g][e] = 0.f;
    __bf16* o = nsplit == 1 ? (__bf16*)out + (int64_t)b * o_sb + (int64_t)(hk * G) * o_sh : nullptr;
    attn_partial_mfma<G>(qb, t0, kbb, k_sn, vbb, v_sn, start, end, scale, ws_m, ws_l, ws_acc,
                         ((int64_t)b * Hq + hk * G) * nsplit + split, nsplit, false, qnone, none, none, o, o_sh);
    return;
  }

  u32x4 qr[G][LPR];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < LPR; ++j) qr[g][j] = ld16(q + (int64_t)b * q_sb + (int64_t)(hk * G + g) * q_sh + d0 + j * EPV);
  const T* kb = k + (int64_t)b * k_sb + (int64_t)hk * k_sh;
  const T* vb = v + (int64_t)b * v_sb + (int64_t)hk * v_sh;
  AttnPipe<LPR, U> pp;
  attn_begin<Geo>(pp, kb, k_sn, vb, v_sn, start, end);
  float qf[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < LPR; ++j) Elem<T>::unpack(qr[g][j], &qf[g][j * EPV]);
  // One split: the block writes the output rows of its G query heads (no combine launch).
  T* o = nsplit == 1 ? out + (int64_t)b * o_sb + (int64_t)(hk * G) * o_sh : nullptr;
  attn_partial<Geo, T, G>(qf, pp, kb, k_sn, vb, v_sn, start, end, scale, ws_m, ws_l, ws_acc,
                          ((int64_t)b * Hq + hk * G) * nsplit + split, nsplit, false, nullptr, nullptr, o, o_sh);
}

// Partial-softmax reduce: one block of kCombineThreads per (b, query head).
// Block c takes (row, kv head) group p = c % P (P = B * Hkv groups) and query
// head c / P of that group's G: blocks are dispatched round-robin to the 8 XCDs,
// so with P a multiple of 8 it runs on the XCD whose L2 took the group's partials
// (split block (p, split) has linear index split * P + p).
constexpr int kCombineThreads = 256;

template <typename T, int D>
__global__ __launch_bounds__(kCombineThreads) void attn_combine_kernel(const float* __restrict__ ws_m,
                                                                       const float* __restrict__ ws_l,
                                                                       const float* __restrict__ ws_acc,
                                                                       T* __restrict__ out, int64_t o_sb, int64_t o_sh,
                                                                       int Hq, int Hkv, int nsplit) {
  const int G = Hq / Hkv;
  const int P = (int)gridDim.x / G;
  const int p = (int)blockIdx.x % P;
  const int b = p / Hkv;
  const int h = (p % Hkv) * G + (int)blockIdx.x / P;
  const int bh = b * Hq + h;
  float r;
  if (attn_combine_block<D, kCombineThreads>(ws_m + (int64_t)bh * nsplit, ws_l + (int64_t)bh * nsplit,
                                             ws_acc + (int64_t)bh * nsplit * D, nsplit, r))
    Elem<T>::store1(out + (int64_t)b * o_sb + (int64_t)h * o_sh + threadIdx.x, r);
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
                     a.pos_stride, a.ws_m, a.ws_l, a.ws_acc, a.Hkv, a.cap, a.nsplit, a.scale, (T*)a.out, a.o_sb,
                     a.o_sh);
  if (hipGetLastError() != hipSuccess) return EGPT_ERR_LAUNCH;
  if (a.nsplit == 1) return EGPT_OK;  // the split kernel wrote the output
  hipLaunchKernelGGL((attn_combine_kernel<T, D>), dim3((unsigned)(a.B * a.Hq)), dim3(kCombineThreads), 0, st,
                     a.ws_m, a.ws_l, a.ws_acc, (T*)a.out, a.o_sb, a.o_sh, a.Hq, a.Hkv, a.nsplit);
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
  // Up to 256 slots one pass: the combine launch that splitting adds costs
  // more than it saves there (single pass 1.1-1.8x faster at 6 / 8 kv heads and
  // 8-128 (row, kv head) programs, caches of 128 and 256 slots, graph replays).
  if (cap <= kOnePassMaxSlots) return 1;
  // About one block per CU (256): a split block streams at the rate its
  // instruction issue allows, and more, shorter splits add merge work without
  // adding bandwidth (cold sweep at 16 q / 8 kv heads, L 4096 and 32768). At
  // least 64 slots per split below that, where the per-split merge dominates.
  const int by_len = (cap + 63) / 64;
  int by_grid = (256 + B * Hkv - 1) / (B * Hkv);
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

// ---------------------------------------------------------------------------
// The same attention with no allocation at all: the split partials live in a
// file-scope device array instead of a caller's workspace. Each device holds its
// own copy of the array at its own address; the host learns that address once per
// device (hipGetSymbolAddress, with the device current) and passes it to the
// kernels like any workspace. The array's name is never used as a device address
// on the host. Every split writes its own partial before the combine reads it, so
// nothing in the array has to start at zero; calls that overlap on one device
// share the array and race.
namespace egpt {
namespace {

static __device__ __align__(256) unsigned char scratch[EGPT_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex[kMaxDevices];
void* g_scratch_ptr[kMaxDevices];  // set only by a lookup that succeeded

// The scratch array's address on the current device, looked up on its first
// successful use there. A failed lookup is not kept: the next call tries again.
// The first lookup on a device is refused while the stream is being captured
// (the lookup is a runtime call that a capture may not allow); once the address
// is known, captured calls need no runtime call at all.
int scratch_on_current_device(hipStream_t stream, void** ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return EGPT_ERR_LAUNCH;
  if (dev < 0 || dev >= kMaxDevices) return EGPT_ERR_UNSUPPORTED;
  if (stream) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess) return EGPT_ERR_INVALID;
    if (sdev != dev) return EGPT_ERR_INVALID;  // the array's address is per device: launch with its device current
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex[dev]);
  if (!g_scratch_ptr[dev]) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) != hipSuccess) return EGPT_ERR_LAUNCH;
    if (cap != hipStreamCaptureStatusNone) return EGPT_ERR_INVALID;  // make one call outside the capture first
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return EGPT_ERR_LAUNCH;
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return EGPT_OK;
}

}  // namespace
}  // namespace egpt

extern "C" int egpt_decode_attn_noalloc(int dtype, const void* q, int64_t q_sb, int64_t q_sh, const void* k,
                                        int64_t k_sb, int64_t k_sh, int64_t k_sn, const void* v, int64_t v_sb,
                                        int64_t v_sh, int64_t v_sn, const int64_t* position, int64_t pos_stride,
                                        void* out, int64_t o_sb, int64_t o_sh, int B, int Hq, int Hkv, int cap, int D,
                                        int nsplit, float scale, hipStream_t stream) {
  if (B < 1 || Hq < 1 || Hkv < 1 || cap < 1 || D < 1) return EGPT_ERR_INVALID;
  if (nsplit <= 0) nsplit = egpt_decode_attn_default_splits(B, Hkv, cap);
  if (attn_workspace_bytes(B, Hq, D, nsplit) > EGPT_NOALLOC_SCRATCH_BYTES) return EGPT_ERR_WORKSPACE;
  void* ws = nullptr;
  const int st = scratch_on_current_device(stream, &ws);
  if (st != EGPT_OK) return st;
  return egpt_decode_attn(dtype, q, q_sb, q_sh, k, k_sb, k_sh, k_sn, v, v_sb, v_sh, v_sn, position, pos_stride, out,
                          o_sb, o_sh, ws, EGPT_NOALLOC_SCRATCH_BYTES, B, Hq, Hkv, cap, D, nsplit, scale, stream);
}
