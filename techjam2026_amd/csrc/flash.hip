// Entry points of the gfx950 FlashAttention forward and its operand preparation
// (mask extents, K / V^T planes). The attention kernel itself is in flash_kernels.h;
// each MFMA mode's launches are compiled in their own translation unit.
#include <mutex>

#include "flash_kernels.h"

namespace kf {

// kv_len[b] = 1 + last valid position (0 if none); prefix[b] = all of [0, kv_len) valid.
__global__ __launch_bounds__(256) void mask_prep_kernel(const void* keep, int dtype, int64_t ld,
                                                        int S, int32_t* kv_len, int32_t* prefix) {
  __shared__ int smax[4], scnt[4];
  const int b = blockIdx.x;
  int last = -1, cnt = 0;
  int s0 = 0;                          // positions below s0 are done by the 16-byte path
  if (dtype == KF_U8 && ld % 16 == 0 && ((uintptr_t)keep & 15) == 0) {
    // byte masks: 16 positions per load (a 65536-key row is 16 loads per thread, not 256)
    const uint8_t* row = (const uint8_t*)keep + (int64_t)b * ld;
    const int nv = S / 16;
    for (int i = threadIdx.x; i < nv; i += blockDim.x) {
      const uint4 w = *(const uint4*)(row + 16 * i);
      const uint32_t q[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if ((q[j >> 2] >> (8 * (j & 3))) & 0xffu) { last = max(last, 16 * i + j); ++cnt; }
    }
    s0 = 16 * nv;
  }
  for (int s = s0 + threadIdx.x; s < S; s += blockDim.x) {
    if (ld_elem(keep, dtype, (int64_t)b * ld + s) != 0.0f) { last = max(last, s); ++cnt; }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    last = max(last, __shfl_xor(last, off));
    cnt += __shfl_xor(cnt, off);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) { smax[wave] = last; scnt[wave] = cnt; }
  __syncthreads();
  if (threadIdx.x == 0) {
    int L = -1, C = 0;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) { L = max(L, smax[i]); C += scnt[i]; }
    kv_len[b] = L + 1;
    if (prefix) prefix[b] = (C == L + 1) ? 1 : 0;
  }
}

// k, v [B, H, S, hd] (any strides, unit d) -> K planes (layout of ko strides) and V^T
// planes [.., hd, keys]. One thread per 8-element chunk of one (b, h, s) row.
template <int IT>
__global__ __launch_bounds__(256) void attn_prep_kernel(
    const void* k, int64_t ks0, int64_t ks1, int64_t ks2,
    const void* v, int64_t vs0, int64_t vs1, int64_t vs2,
    void* k_hi, void* k_lo, int64_t os0, int64_t os1, int64_t os2,
    void* vt_hi, void* vt_lo, int64_t ts0, int64_t ts1, int64_t ts2,
    int B, int H, int S, int hd, int kv_dtype) {
  const int cpr = hd / 8;
  const int64_t total = (int64_t)B * H * S * cpr;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(i % cpr);
    int64_t rest = i / cpr;
    const int s = (int)(rest % S); rest /= S;
    const int h = (int)(rest % H);
    const int b = (int)(rest / H);
    const int d = c * 8;
    float x[8];
    if (k_hi) {                 // null: the caller's K already has the kernel's layout
      ld8<IT>(k, b * ks0 + h * ks1 + s * ks2 + d, x);
      const int64_t ko = b * os0 + h * os1 + s * os2 + d;
      store4_any(k_hi, k_lo, kv_dtype, ko, x);
      store4_any(k_hi, k_lo, kv_dtype, ko + 4, x + 4);
    }
    ld8<IT>(v, b * vs0 + h * vs1 + s * vs2 + d, x);
    const int64_t vo = b * ts0 + h * ts1 + s;
#pragma unroll
    for (int e = 0; e < 8; ++e) st_elem(vt_hi, kv_dtype, vo + (int64_t)(d + e) * ts2, x[e], vt_lo);
    if (s == S - 1) {     // zero the V^T pad columns [S, roundup(S, 8)) that attention reads
      for (int sp = S; sp < ((S + 7) & ~7); ++sp)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          st_elem(vt_hi, kv_dtype, vo + (sp - s) + (int64_t)(d + e) * ts2, 0.0f, vt_lo);
    }
  }
}

static int kv_code(int mode) {
  return mode == KF_MMA_F16X3 ? KF_F16X2 : mode == KF_MMA_BF16X3 ? KF_BF16X2
       : mode == KF_MMA_F16 ? KF_F16 : KF_BF16;
}

}  // namespace kf

using namespace kf;

// Check hook (declared in kf950.h; host only, launches nothing): writes (b, h, qb) of
// every block of a B x H x nqb attention grid as the kernel maps them, for tests of the
// mapping's bijectivity and per-XCD balance without a device.
extern "C" int kf_flash_block_map(int B, int H, int nqb, int causal, int* out) {
  if (B < 1 || H < 1 || nqb < 1 || out == nullptr) return KF_EINVAL;
  const int n = B * H * nqb;
  for (int bid = 0; bid < n; ++bid) {
    const FlashBlock m = flash_block_map(bid, n, B, H, nqb, causal != 0);
    out[3 * bid] = m.b;
    out[3 * bid + 1] = m.h;
    out[3 * bid + 2] = m.qb;
  }
  return KF_OK;
}

static bool hd_ok(int64_t hd) {
  return hd == 8 || hd == 16 || hd == 32 || hd == 64 || hd == 128 || hd == 256;
}

// Host-only query of the tile the attention kernel uses at head_dim `hd` in MFMA `mode`
// (`p16`: KF_FLASH_P16 single-plane probabilities, which do not change the tile):
// info[0..5] = BLOCK_M (query rows per block), BLOCK_N (keys per LDS stage), wavefronts
// per block, LDS stages, 16-row query groups per wavefront, LDS bytes per block.
template <int HDP, int P> static void tile_info(int* info) {
  if constexpr (P == 1 && HDP == 64) {
    // single-pass fp16 / bf16 at hd 64 run the two-tile pipelined kernel (unless
    // KF_FLASH_NO_PIPE / KF_FLASH_ONE_TILE): 64 query rows (four 16-row groups) per
    // wavefront; LDS bytes of its K / V^T stages
    info[0] = PairTile::BM; info[1] = PairTile::BN; info[2] = PairTile::NW;
    info[3] = PairTile::STAGES; info[4] = 4; info[5] = PairTile::STAGES * PairTile::STAGE_BYTES;
  } else if constexpr (P == 1 && HDP == 128) {
    // single-pass fp16 / bf16 at hd 128 run the pipelined kernel (unless
    // KF_FLASH_NO_PIPE): 32 query rows (two 16-row groups) per wavefront
    using PT = PipeTile<HDP>;
    info[0] = PT::BM; info[1] = PT::BN; info[2] = PT::NW; info[3] = PT::STAGES; info[4] = 2;
    info[5] = PT::STAGES * PT::STAGE_BYTES;
  } else {
    using FT = FlashTile<HDP, P>;
    info[0] = FT::BM; info[1] = FT::BN; info[2] = FT::NW; info[3] = FT::STAGES; info[4] = FT::QG;
    info[5] = FT::STAGES * FT::STAGE_BYTES;
  }
}

extern "C" int kf_flash_tile_info(int hd, int mode, int* info) {
  if (!info || !hd_ok(hd) || mode < KF_MMA_F16 || mode > KF_MMA_BF16X3) return KF_EINVAL;
  const bool split = mode == KF_MMA_F16X3 || mode == KF_MMA_BF16X3;
  if (split && hd == SmallTile::HD) {
    // head_dim 8 in the split modes runs the packed-contraction kernel (unless
    // KF_FLASH_NO_PIPE): 32 query rows (two 16-row groups) per wavefront
    info[0] = SmallTile::BM; info[1] = SmallTile::BN; info[2] = SmallTile::NW;
    info[3] = SmallTile::STAGES; info[4] = 2; info[5] = SmallTile::STAGES * SmallTile::STAGE_BYTES;
    return KF_OK;
  }
  const int hdp = hd < 32 ? 32 : hd;
  switch (hdp) {
    case 32: split ? tile_info<32, 2>(info) : tile_info<32, 1>(info); break;
    case 64: split ? tile_info<64, 2>(info) : tile_info<64, 1>(info); break;
    case 128: split ? tile_info<128, 2>(info) : tile_info<128, 1>(info); break;
    default: split ? tile_info<256, 2>(info) : tile_info<256, 1>(info); break;
  }
  return KF_OK;
}

extern "C" int kf_mask_prep(const void* keep, int keep_dtype, int64_t ld_keep, int64_t B, int64_t S,
                            int32_t* kv_len, int32_t* prefix, void* stream) {
  if (!keep || !kv_len || B < 0 || S <= 0 || ld_keep < S || keep_dtype < KF_F32 || keep_dtype > KF_U8 ||
      S > 0x7fffffff || B > 0x7fffffff) {
    kf_set_error("kf_mask_prep: bad arguments");
    return KF_EINVAL;
  }
  if (B == 0) return KF_OK;
  hipLaunchKernelGGL(mask_prep_kernel, dim3((unsigned)B), dim3(256), 0, (hipStream_t)stream, keep,
                     keep_dtype, ld_keep, (int)S, kv_len, prefix);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { kf_set_error("kf_mask_prep: launch failed: %s", hipGetErrorString(e)); return KF_ELAUNCH; }
  return KF_OK;
}


extern "C" int kf_attn_prep(const void* k, const int64_t* ks, const void* v, const int64_t* vs,
                            int in_dtype, void* k_hi, void* k_lo, const int64_t* kos,
                            void* vt_hi, void* vt_lo, const int64_t* vts,
                            int64_t B, int64_t H, int64_t S, int64_t hd, int mode, void* stream) {
  const bool split = mode == KF_MMA_F16X3 || mode == KF_MMA_BF16X3;
  const bool with_k = k != nullptr;          // k and k_hi null: write V^T only
  if (with_k != (k_hi != nullptr) || !v || !vs || !vts || !vt_hi ||
      (with_k && (!ks || !kos || (split && !k_lo))) || (split && !vt_lo) ||
      B < 0 || H <= 0 || S < 0 || in_dtype < KF_F32 || in_dtype > KF_BF16 ||
      mode < KF_MMA_F16 || mode > KF_MMA_BF16X3) {
    kf_set_error("kf_attn_prep: bad arguments");
    return KF_EINVAL;
  }
  if (!hd_ok(hd) || (with_k && (ks[3] != 1 || kos[3] != 1)) || vs[3] != 1 || vts[3] != 1) {
    kf_set_error("kf_attn_prep: unsupported head_dim %lld or non-unit inner stride", (long long)hd);
    return KF_EUNSUPPORTED;
  }
  if (vts[2] < ((S + 7) & ~7LL)) {
    kf_set_error("kf_attn_prep: V^T row stride %lld below roundup(S, 8)", (long long)vts[2]);
    return KF_EINVAL;
  }
  const int64_t vec = in_dtype == KF_F32 ? 4 : 8;
  for (int i = 0; i < 3; ++i)
    if ((with_k && (ks[i] % vec || kos[i] % 4)) || vs[i] % vec) {
      kf_set_error("kf_attn_prep: strides must be multiples of the vector width");
      return KF_EUNSUPPORTED;
    }
  if (((uintptr_t)k | (uintptr_t)v) & 15 || ((uintptr_t)k_hi & 7) || (k_lo && ((uintptr_t)k_lo & 7))) {
    kf_set_error("kf_attn_prep: misaligned pointers");
    return KF_EUNSUPPORTED;
  }
  if (B == 0 || S == 0) return KF_OK;
  const int64_t total = B * H * S * (hd / 8);
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipStream_t st = (hipStream_t)stream;
  const int kvd = kv_code(mode);
  static const int64_t zero4[4] = {0, 0, 0, 1};
  const int64_t* kst = with_k ? ks : zero4;
  const int64_t* kost = with_k ? kos : zero4;
#define KF_PREP(IT)                                                                            \
  hipLaunchKernelGGL(attn_prep_kernel<IT>, dim3((unsigned)blocks), dim3(256), 0, st, k, kst[0], \
                     kst[1], kst[2], v, vs[0], vs[1], vs[2], k_hi, k_lo, kost[0], kost[1], kost[2], \
                     vt_hi, vt_lo, vts[0], vts[1], vts[2], (int)B, (int)H, (int)S, (int)hd, kvd)
  switch (in_dtype) {
    case KF_F32: KF_PREP(KF_F32); break;
    case KF_F16: KF_PREP(KF_F16); break;
    default: KF_PREP(KF_BF16); break;
  }
#undef KF_PREP
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { kf_set_error("kf_attn_prep: launch failed: %s", hipGetErrorString(e)); return KF_ELAUNCH; }
  return KF_OK;
}

extern "C" int kf_flash_fwd(const void* q, const int64_t* qs, int q_dtype,
                            const void* k_hi, const void* k_lo, const int64_t* ks,
                            const void* vt_hi, const void* vt_lo, const int64_t* vs,
                            void* o, void* o_lo, const int64_t* os, int o_dtype,
                            const void* keep, int keep_dtype, int64_t ld_keep,
                            const int32_t* kv_len, const int32_t* prefix,
                            int64_t B, int64_t H, int64_t S, int64_t hd,
                            float sm_scale, int mode, int flags, void* stream) {
  const bool split = mode == KF_MMA_F16X3 || mode == KF_MMA_BF16X3;
  if (!q || !k_hi || !vt_hi || !o || !qs || !ks || !vs || !os || B < 0 || H <= 0 || S < 0 ||
      (split && (!k_lo || !vt_lo)) || mode < KF_MMA_F16 || mode > KF_MMA_BF16X3) {
    kf_set_error("kf_flash_fwd: bad arguments");
    return KF_EINVAL;
  }
  if (!hd_ok(hd)) {
    kf_set_error("kf_flash_fwd: unsupported head_dim %lld (8, 16, 32, 64, 128, 256)", (long long)hd);
    return KF_EUNSUPPORTED;
  }
  if (qs[3] != 1 || ks[3] != 1 || vs[3] != 1 || os[3] != 1) {
    kf_set_error("kf_flash_fwd: innermost strides must be 1");
    return KF_EINVAL;
  }
  if ((flags & KF_FLASH_ROUND_SCORES) && mode != KF_MMA_F16 && mode != KF_MMA_BF16) {
    kf_set_error("kf_flash_fwd: KF_FLASH_ROUND_SCORES needs KF_MMA_F16 or KF_MMA_BF16");
    return KF_EINVAL;
  }
  if (keep && (keep_dtype < KF_F32 || keep_dtype > KF_U8 || ld_keep < S)) {
    kf_set_error("kf_flash_fwd: bad keep mask");
    return KF_EINVAL;
  }
  const bool o_planes = o_dtype == KF_F16X2 || o_dtype == KF_BF16X2;
  if (q_dtype < KF_F32 || q_dtype > KF_BF16 || o_dtype < KF_F32 || o_dtype == KF_U8 ||
      o_dtype > KF_BF16X2 || (o_planes && !o_lo)) {
    kf_set_error("kf_flash_fwd: bad dtype (or missing output lo plane)");
    return KF_EINVAL;
  }
  const int64_t qvec = q_dtype == KF_F32 ? 4 : 8;
  for (int i = 0; i < 3; ++i) {
    if (qs[i] % qvec || ks[i] % 8 || os[i] % 4) {
      kf_set_error("kf_flash_fwd: strides must be multiples of the vector width");
      return KF_EUNSUPPORTED;
    }
  }
  if (vs[2] % 8 || vs[0] % 8 || vs[1] % 8) {
    kf_set_error("kf_flash_fwd: V^T strides must be multiples of 8");
    return KF_EUNSUPPORTED;
  }
  if (vs[2] < S) {
    kf_set_error("kf_flash_fwd: V^T row stride %lld below S %lld", (long long)vs[2], (long long)S);
    return KF_EINVAL;
  }
  if (((uintptr_t)q | (uintptr_t)k_hi | (uintptr_t)vt_hi) & 15 || (k_lo && ((uintptr_t)k_lo & 15)) ||
      (vt_lo && ((uintptr_t)vt_lo & 15)) || ((uintptr_t)o & (o_dtype == KF_F32 ? 15 : 7)) ||
      (o_planes && ((uintptr_t)o_lo & 7))) {
    kf_set_error("kf_flash_fwd: pointers must be 16-byte aligned");
    return KF_EUNSUPPORTED;
  }
  if (S > (1 << 30) || B * H > (1LL << 31)) { kf_set_error("kf_flash_fwd: problem too large"); return KF_EUNSUPPORTED; }
  if (B == 0 || S == 0) return KF_OK;
  FlashArgs a{q, qs[0], qs[1], qs[2], k_hi, k_lo, ks[0], ks[1], ks[2],
              vt_hi, vt_lo, vs[0], vs[1], vs[2],
              o, o_lo, os[0], os[1], os[2], o_dtype, keep, keep_dtype, ld_keep, kv_len, prefix,
              (int)B, (int)H, (int)S, (int)hd, sm_scale * kLog2e, sm_scale, flags};
  const int hdp = hd < 32 ? 32 : (int)hd;
  const int64_t nqb = (S + FlashTile<32>::BM - 1) / FlashTile<32>::BM;   // smallest BM
  if (nqb * B * H * 2 > 0x7fffffffLL) { kf_set_error("kf_flash_fwd: grid too large"); return KF_EUNSUPPORTED; }
  hipStream_t st = (hipStream_t)stream;
  switch (mode) {
    case KF_MMA_F16: flash_launch_f16(a, q_dtype, hdp, st); break;
    case KF_MMA_BF16: flash_launch_bf16(a, q_dtype, hdp, st); break;
    case KF_MMA_F16X3: flash_launch_f16x3(a, q_dtype, hdp, st); break;
    default: flash_launch_bf16x3(a, q_dtype, hdp, st); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { kf_set_error("kf_flash_fwd: launch failed: %s", hipGetErrorString(e)); return KF_ELAUNCH; }
  return KF_OK;
}

// ---------------------------------------------------------------- no-allocation variant
// kf_flash_attention_static: the op-level attention (k, v into the attention layout,
// mask extents, attention) with its staging -- the K / V^T planes and kv_len / prefix --
// in a file-scope device array instead of caller-allocated buffers, for callers that
// cannot allocate. Every GPU holds its own copy of the array until the process ends; its
// address on each device is looked up once (hipGetSymbolAddress, with that device
// current) and only that address is handed to kernels. All calls on one GPU share it:
// calls that overlap on one GPU (different streams, or host threads) race.
constexpr size_t kStaticScratchBytes = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_of_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    kf_set_error("kf_flash_attention_static: no usable current device (%s)",
                 e != hipSuccess ? hipGetErrorString(e) : "device ordinal out of range");
    return KF_EDEVICE;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      kf_set_error("kf_flash_attention_static: hipGetSymbolAddress(scratch) failed on device "
                   "%d: %s", dev, hipGetErrorString(e));
      return KF_EDEVICE;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return KF_OK;
}

size_t round256(size_t n) { return (n + 255) & ~size_t(255); }
}  // namespace

extern "C" int kf_flash_attention_static(const void* q, const int64_t* qs,
                                         const void* k, const int64_t* ks,
                                         const void* v, const int64_t* vs, int in_dtype,
                                         void* o, void* o_lo, const int64_t* os, int o_dtype,
                                         const void* keep, int keep_dtype, int64_t ld_keep,
                                         int64_t B, int64_t H, int64_t S, int64_t hd,
                                         float sm_scale, int mode, int flags, void* stream) {
  if (!q || !k || !v || !qs || !ks || !vs || !o || !os || B < 0 || H <= 0 || S < 0 ||
      mode < KF_MMA_F16 || mode > KF_MMA_BF16X3 || in_dtype < KF_F32 || in_dtype > KF_BF16) {
    kf_set_error("kf_flash_attention_static: bad arguments");
    return KF_EINVAL;
  }
  if (!hd_ok(hd)) {
    kf_set_error("kf_flash_attention_static: unsupported head_dim %lld", (long long)hd);
    return KF_EUNSUPPORTED;
  }
  if (B == 0 || S == 0) return KF_OK;
  if (B > (1 << 20) || S > (1 << 26) || H > (1 << 16)) {
    kf_set_error("kf_flash_attention_static: problem too large");
    return KF_EINVAL;
  }
  // scratch layout: [kv_len: B][prefix: B] (with a keep mask), K planes [B, H, S, hd],
  // V^T planes [B, H, hd, roundup(S, 8)]; each piece 256-byte aligned
  const bool split = mode == KF_MMA_F16X3 || mode == KF_MMA_BF16X3;
  const int planes = split ? 2 : 1;
  const int64_t S8 = (S + 7) & ~7LL;
  // bound B * H by division before any product of all four extents is formed: one (b, h)
  // slice's K and V^T planes take per_bh <= 2 * 2 * 256 * 2^27 bytes and B * H <= 2^36,
  // neither of which overflows, while B * H * S * hd * 2 could wrap and pass the check
  const size_t per_bh = size_t(planes) * 2 * size_t(hd) * size_t(S + S8);
  if (size_t(B) * size_t(H) > kStaticScratchBytes / per_bh) {
    kf_set_error("kf_flash_attention_static: B=%lld H=%lld S=%lld hd=%lld needs more staging "
                 "than the static scratch holds (%zu bytes; use kf_attn_prep + kf_mask_prep + "
                 "kf_flash_fwd with caller buffers)", (long long)B, (long long)H, (long long)S,
                 (long long)hd, kStaticScratchBytes);
    return KF_EINVAL;
  }
  const size_t mask_bytes = keep ? round256(size_t(2 * B) * sizeof(int32_t)) : 0;
  const size_t k_bytes = round256(size_t(B) * H * S * hd * 2);
  const size_t v_bytes = round256(size_t(B) * H * hd * S8 * 2);
  const size_t need = mask_bytes + planes * (k_bytes + v_bytes);
  if (need > kStaticScratchBytes) {
    kf_set_error("kf_flash_attention_static: B=%lld H=%lld S=%lld hd=%lld needs %zu bytes of "
                 "staging; the static scratch holds %zu (use kf_attn_prep + kf_mask_prep + "
                 "kf_flash_fwd with caller buffers)", (long long)B, (long long)H, (long long)S,
                 (long long)hd, need, kStaticScratchBytes);
    return KF_EINVAL;
  }
  void* base = nullptr;
  int st = scratch_of_current_device(&base);
  if (st != KF_OK) return st;
  unsigned char* p = (unsigned char*)base;
  int32_t* kv_len = keep ? (int32_t*)p : nullptr;
  int32_t* prefix = keep ? (int32_t*)p + B : nullptr;
  p += mask_bytes;
  void* k_hi = p;
  void* k_lo = split ? p + k_bytes : nullptr;
  p += planes * k_bytes;
  void* vt_hi = p;
  void* vt_lo = split ? p + v_bytes : nullptr;
  const int64_t kos[4] = {H * S * hd, S * hd, hd, 1};
  const int64_t vts[4] = {H * hd * S8, hd * S8, S8, 1};
  // every scratch byte a kernel reads is written first in stream order (attn_prep writes
  // the planes and zeroes the V^T pad columns, mask_prep writes kv_len and prefix), so
  // nothing is cleared
  st = kf_attn_prep(k, ks, v, vs, in_dtype, k_hi, k_lo, kos, vt_hi, vt_lo, vts, B, H, S, hd,
                    mode, stream);
  if (st != KF_OK) return st;
  if (keep) {
    st = kf_mask_prep(keep, keep_dtype, ld_keep, B, S, kv_len, prefix, stream);
    if (st != KF_OK) return st;
  }
  return kf_flash_fwd(q, qs, in_dtype, k_hi, k_lo, kos, vt_hi, vt_lo, vts, o, o_lo, os, o_dtype,
                      keep, keep_dtype, ld_keep, kv_len, prefix, B, H, S, hd, sm_scale, mode,
                      flags, stream);
}
