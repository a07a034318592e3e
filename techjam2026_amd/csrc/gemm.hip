// Entry points of the gfx950 GEMM: argument checks, tile choice, weight preparation.
// The kernels are in gemm_kernels.h; each MFMA mode's launches are compiled in their own
// translation unit (gemm_<mode>.hip).
#include "gemm_kernels.h"

namespace kf {

template <typename E>
__global__ void split_kernel(const float* src, int64_t n, E* hi, E* lo) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float x = src[i];
    const E h = (E)x;
    hi[i] = h;
    if (lo) lo[i] = (E)(x - (float)h);
  }
}

// Automatic choice for 16-bit operands, from per-call sweeps of the layer's GEMM shapes
// on MI355X at the precisions the plans use (C2, C4, C5). Short K (head-sized) takes small
// tiles (128 x 64 for the QKV epilogue), N <= 64 the 128 x 64 x 64 tile. Where K is a
// multiple of 64 a stage carries 64 k (two 32-k sub-tiles, both halves of each 128-byte
// line copied back to back): 128 x 128 x 64 in two stages is the best or within 4 % of
// it everywhere (C2 QKV 56.7 -> 49.8 us, ffn_in 45.4 -> 35.0, C4 out_proj 110.7 -> 92.5,
// C5 ffn_in 1080 -> 976) except on large grids where the weight has more planes than the
// activation (f16x2: 256 x 128, C4 QKV 542 -> 473), carries split planes on both sides
// (f16x3: 128 x 256 x 32; for both, 256 x 256 x 32 in two stages with single-buffered
// fragments where N >= 512: C5 QKV 4477 -> 4069 us, ffn_out 1580 -> 1427, C4 QKV 596 -> 536,
// out_proj 231 -> 194, an f16x3 ffn_in with GELU 887 -> 790, C5 out_proj (f16x2) 1067 ->
// 1004; one-round grids such as C2's run it 1.5-2.6x slower), or K is long (fp16,
// K >= 4096: 256 x 256 x 64 in two stages, 64 x 128 per wavefront, C4 ffn_out 331 -> 320
// with 128 x 256 x 64 in three stages, then 324 -> 258 with 256 x 256).
static int pick_dma(int64_t M, int64_t N, int64_t K, int mode, bool qkv) {
  const int64_t t128 = ((M + 127) / 128) * ((N + 127) / 128);
  const bool split = mode == KF_MMA_F16X3 || mode == KF_MMA_BF16X3;
  if (K < 128) return qkv ? DMA_128x64k32s3w4 : DMA_64x64k32s3w4;
  if (N <= 64 && K % 64 == 0) return DMA_128x64k64s3w8;
  if (K % 64 == 0) {
    if (t128 >= 1024) {
      if (mode == KF_MMA_F16X2) return N >= 512 ? DMA_256x256k32s2w8 : DMA_256x128k64s2w8;
      if (split) return N >= 512 ? DMA_256x256k32s2w8 : DMA_128x256k32s3w8;
      if (K >= 4096) return qkv ? DMA_128x256k64s3w8 : DMA_256x256k64s2w8;
    }
    return DMA_128x128k64s2w8;
  }
  if (t128 >= 1024) return mode == KF_MMA_F16X2 ? DMA_256x128k32s3w8 : DMA_128x256k32s3w8;
  if (N <= 512) return DMA_128x128k32s3w8;
  return DMA_128x128k32s4w8;
}

// The tile a call runs: the caller's explicit choice where it applies to the operands
// (an LDS-DMA tile needs 16-bit A and K a multiple of its BK; f16x2 runs on LDS-DMA tiles
// only), else the automatic one.
static int pick_tile(int requested, int64_t M, int64_t N, int64_t K, bool a16, int mode, bool qkv) {
  int t = requested;
  if (t >= DMA_FIRST && (!a16 || K % kTileInfo[t].bk)) t = TILE_AUTO;
  if (mode == KF_MMA_F16X2 && t != TILE_AUTO && t < DMA_FIRST) t = TILE_AUTO;
  if (t == TILE_AUTO && a16 && K % 32 == 0) t = pick_dma(M, N, K, mode, qkv);
  if (t == TILE_AUTO) {
    const int64_t blocks128 = ((M + 127) / 128) * ((N + 127) / 128);
    if (blocks128 >= 512) t = TILE_128x128k32;
    else t = K >= 1024 ? TILE_128x128k64 : TILE_64x64k64;
  }
  return t;
}

static inline bool is_dma_tile(int tile) { return tile >= DMA_FIRST; }

static inline bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

static void launch_mode_any(const GemmArgs& g, int mode, int a_dtype, int tile, int epi,
                            hipStream_t st) {
  switch (mode) {
    case KF_MMA_F16X2: gemm_launch_f16x2(g, a_dtype, tile, epi, st); break;
    case KF_MMA_F16: gemm_launch_f16(g, a_dtype, tile, epi, st); break;
    case KF_MMA_BF16: gemm_launch_bf16(g, a_dtype, tile, epi, st); break;
    case KF_MMA_F16X3: gemm_launch_f16x3(g, a_dtype, tile, epi, st); break;
    case KF_MMA_BF16X3: gemm_launch_bf16x3(g, a_dtype, tile, epi, st); break;
    default: gemm_launch_f32(g, a_dtype, st); break;
  }
}

}  // namespace kf

using namespace kf;

extern "C" int kf_gemm_tile_info(int tile, int* info) {
  if (tile < TILE_AUTO || tile > TILE_LAST || info == nullptr) return KF_EINVAL;
  const TileInfo& t = kTileInfo[tile];
  info[0] = t.bm; info[1] = t.bn; info[2] = t.bk; info[3] = t.stages; info[4] = t.waves;
  info[5] = t.dma;
  return KF_OK;
}

extern "C" int kf_gemm_tiled(const void* a, const void* a_lo, int a_dtype, int64_t lda,
                             const void* w_hi, const void* w_lo, int64_t ldw,
                             const float* bias,
                             void* c, void* c_lo, int c_dtype, int64_t ldc,
                             int64_t M, int64_t N, int64_t K, int mode, int act, int tile,
                             void* stream) {
  if (!a || !w_hi || !c || M < 0 || N <= 0 || K <= 0) {
    kf_set_error("kf_gemm: bad arguments (M=%lld N=%lld K=%lld)", (long long)M, (long long)N,
                 (long long)K);
    return KF_EINVAL;
  }
  if (tile < TILE_AUTO || tile > TILE_LAST) {
    kf_set_error("kf_gemm: unknown tile id %d", tile);
    return KF_EINVAL;
  }
  const bool split = mode == KF_MMA_F16X3 || mode == KF_MMA_BF16X3 || mode == KF_MMA_F16X2;
  if (mode < KF_MMA_F32 || mode > KF_MMA_F16X2 || c_dtype < KF_F32 || c_dtype == KF_U8 ||
      c_dtype > KF_BF16X2 || (act != KF_ACT_NONE && act != KF_ACT_GELU_ERF)) {
    kf_set_error("kf_gemm: bad mode/c_dtype/act (%d/%d/%d)", mode, c_dtype, act);
    return KF_EINVAL;
  }
  // operand formats each mode accepts
  bool a_ok;
  switch (mode) {
    case KF_MMA_F16: a_ok = a_dtype == KF_F32 || a_dtype == KF_F16; break;
    case KF_MMA_BF16: a_ok = a_dtype == KF_F32 || a_dtype == KF_BF16; break;
    case KF_MMA_F16X3: a_ok = a_dtype == KF_F32 || a_dtype == KF_F16X2; break;
    case KF_MMA_BF16X3: a_ok = a_dtype == KF_F32 || a_dtype == KF_BF16X2; break;
    case KF_MMA_F16X2: a_ok = a_dtype == KF_F16; break;
    default: a_ok = a_dtype == KF_F32 || a_dtype == KF_F16 || a_dtype == KF_BF16; break;
  }
  if (!a_ok) {
    kf_set_error("kf_gemm: A dtype %d is not an operand format of MFMA mode %d", a_dtype, mode);
    return KF_EUNSUPPORTED;
  }
  const bool a_planes = a_dtype == KF_F16X2 || a_dtype == KF_BF16X2;
  const bool c_planes = c_dtype == KF_F16X2 || c_dtype == KF_BF16X2;
  if ((split && !w_lo) || (a_planes && !a_lo) || (c_planes && !c_lo)) {
    kf_set_error("kf_gemm: missing lo plane");
    return KF_EINVAL;
  }
  if (K % 8 || N % 4 || lda % 8 || ldw % 8 || ldc % 4 || lda < K || ldw < K || ldc < N ||
      !al16(a) || (a_planes && !al16(a_lo)) || !al16(w_hi) || (w_lo && !al16(w_lo)) ||
      !al16(c) || (c_planes && !al16(c_lo)) || (bias && !al16(bias))) {
    kf_set_error("kf_gemm: unsupported shape/alignment (M=%lld N=%lld K=%lld lda=%lld "
                 "ldw=%lld ldc=%lld): needs K%%8 == 0, N%%4 == 0 and 16-byte aligned rows",
                 (long long)M, (long long)N, (long long)K, (long long)lda, (long long)ldw,
                 (long long)ldc);
    return KF_EUNSUPPORTED;
  }
  if (M > (1LL << 30) || N > (1LL << 30) || K > (1LL << 30) ||
      ((M + 63) / 64) * ((N + 63) / 64) > 0x7fffffffLL) {
    kf_set_error("kf_gemm: problem too large");
    return KF_EUNSUPPORTED;
  }
  if (M == 0) return KF_OK;
  const bool c16 = c_dtype != KF_F32;
  const int wide16 = c16 && ldc % 8 == 0 && N % 8 == 0 && al16(c) && (!c_planes || al16(c_lo));
  GemmArgs g{a, a_lo, lda, w_hi, w_lo, ldw, bias, c, c_lo, c_dtype, ldc,
             (int)M, (int)N, (int)K, act,
             nullptr, nullptr, nullptr, nullptr, nullptr, 0, 0, 0, 0, 0, wide16};
  hipStream_t st = (hipStream_t)stream;
  const int t = pick_tile(tile, M, N, K, a_dtype != KF_F32, mode, false);
  if (mode == KF_MMA_F16X2 && !is_dma_tile(t)) {
    kf_set_error("kf_gemm: f16x2 needs the LDS-DMA path (fp16 A, K %% 32 == 0; K=%lld)",
                 (long long)K);
    return KF_EUNSUPPORTED;
  }
  // compile-time epilogues for the output type / activation pairs the layer uses
  const bool f16fam = mode == KF_MMA_F16 || mode == KF_MMA_F16X3 || mode == KF_MMA_F16X2;
  int epi = 0;
  if (c_dtype == KF_F32 && act == KF_ACT_NONE) epi = 2;
  else if (act == KF_ACT_GELU_ERF && c_dtype == (f16fam ? KF_F16 : KF_BF16)) epi = 3;
  else if (act == KF_ACT_GELU_ERF && c_dtype == (f16fam ? KF_F16X2 : KF_BF16X2)) epi = 4;
  launch_mode_any(g, mode, a_dtype, t, epi, st);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    kf_set_error("kf_gemm: launch failed: %s", hipGetErrorString(e));
    return KF_ELAUNCH;
  }
  return KF_OK;
}

extern "C" int kf_gemm(const void* a, const void* a_lo, int a_dtype, int64_t lda,
                       const void* w_hi, const void* w_lo, int64_t ldw,
                       const float* bias,
                       void* c, void* c_lo, int c_dtype, int64_t ldc,
                       int64_t M, int64_t N, int64_t K, int mode, int act, void* stream) {
  return kf_gemm_tiled(a, a_lo, a_dtype, lda, w_hi, w_lo, ldw, bias, c, c_lo, c_dtype, ldc,
                       M, N, K, mode, act, TILE_AUTO, stream);
}

extern "C" int kf_gemm_qkv_tiled(const void* a, const void* a_lo, int a_dtype, int64_t lda,
                                 const void* w_hi, const void* w_lo, int64_t ldw, const float* bias,
                                 float* q_out, void* k_hi, void* k_lo, void* vt_hi, void* vt_lo,
                                 int64_t sp, int64_t B, int64_t S, int64_t H, int64_t hd, int mode,
                                 int tile, void* stream) {
  const int64_t d = H * hd, M = B * S;
  const bool split = mode == KF_MMA_F16X3 || mode == KF_MMA_BF16X3 || mode == KF_MMA_F16X2;
  if (!a || !w_hi || !bias || !q_out || !k_hi || !vt_hi || B < 0 || S <= 0 || H <= 0 ||
      hd <= 0 || hd % 4 || sp < S || sp % 8 || (split && !w_lo) ||
      tile < TILE_AUTO || tile > TILE_LAST) {
    kf_set_error("kf_gemm_qkv: bad arguments");
    return KF_EINVAL;
  }
  bool a_ok;
  switch (mode) {
    case KF_MMA_F16: a_ok = a_dtype == KF_F32 || a_dtype == KF_F16; break;
    case KF_MMA_BF16: a_ok = a_dtype == KF_F32 || a_dtype == KF_BF16; break;
    case KF_MMA_F16X3: a_ok = a_dtype == KF_F32 || a_dtype == KF_F16X2; break;
    case KF_MMA_BF16X3: a_ok = a_dtype == KF_F32 || a_dtype == KF_BF16X2; break;
    case KF_MMA_F16X2: a_ok = a_dtype == KF_F16; break;
    default: a_ok = false;
  }
  const bool a_planes = a_dtype == KF_F16X2 || a_dtype == KF_BF16X2;
  if (!a_ok || (a_planes && !a_lo)) {
    kf_set_error("kf_gemm_qkv: A dtype %d / MFMA mode %d not supported", a_dtype, mode);
    return KF_EUNSUPPORTED;
  }
  if (d % 8 || lda % 8 || ldw % 8 || lda < d || ldw < d || !al16(a) || (a_planes && !al16(a_lo)) ||
      !al16(w_hi) || (w_lo && !al16(w_lo)) || !al16(bias) || !al16(q_out) || ((uintptr_t)k_hi & 7) ||
      (k_lo && ((uintptr_t)k_lo & 7)) || M > (1LL << 30) || d > (1 << 20)) {
    kf_set_error("kf_gemm_qkv: unsupported shape/alignment (d=%lld)", (long long)d);
    return KF_EUNSUPPORTED;
  }
  // f16x2 writes K and V^T as f16 planes like f16x3 (attention then runs f16x3); a split
  // mode called with no lo planes writes one plane of each, the values rounded to nearest
  // (its attention reads single-pass operands)
  const bool split_kv = mode == KF_MMA_F16X3 || mode == KF_MMA_F16X2 || mode == KF_MMA_BF16X3;
  const bool single_kv = split_kv && !k_lo && !vt_lo;
  if (split_kv && !single_kv && (!k_lo || !vt_lo)) {
    kf_set_error("kf_gemm_qkv: a split mode takes both lo planes (k and v^T) or neither");
    return KF_EINVAL;
  }
  if (mode == KF_MMA_F16X2 && single_kv) {
    kf_set_error("kf_gemm_qkv: f16x2 writes split k / v^T planes");
    return KF_EUNSUPPORTED;
  }
  if (M == 0) return KF_OK;
  const int kv_dtype = single_kv ? (mode == KF_MMA_BF16X3 ? KF_BF16 : KF_F16)
                     : (mode == KF_MMA_F16X3 || mode == KF_MMA_F16X2) ? KF_F16X2
                     : mode == KF_MMA_BF16X3 ? KF_BF16X2 : mode == KF_MMA_F16 ? KF_F16 : KF_BF16;
  // 8-column stores: q (fp32) needs 16-byte alignment, k (16-bit) 16-byte alignment
  const int wide16 = hd % 8 == 0 && al16(k_hi) && (!k_lo || al16(k_lo));
  auto log2_or_neg = [](int64_t v) -> int {
    if (v <= 0 || (v & (v - 1))) return -1;
    int l = 0;
    while ((1LL << l) < v) ++l;
    return l;
  };
  GemmArgs g{a, a_lo, lda, w_hi, w_lo, ldw, bias, nullptr, nullptr, KF_F32, 0,
             (int)M, (int)(3 * d), (int)d, KF_ACT_NONE,
             q_out, k_hi, k_lo, vt_hi, vt_lo, kv_dtype, sp, (int)S, (int)H, (int)hd, wide16,
             log2_or_neg(S), log2_or_neg(hd)};
  hipStream_t st = (hipStream_t)stream;
  const int t = pick_tile(tile, M, 3 * d, d, a_dtype != KF_F32, mode, true);
  if (mode == KF_MMA_F16X2 && !is_dma_tile(t)) {
    kf_set_error("kf_gemm_qkv: f16x2 needs the LDS-DMA path (fp16 A, d %% 32 == 0; d=%lld)",
                 (long long)d);
    return KF_EUNSUPPORTED;
  }
  launch_mode_any(g, mode, a_dtype, t, single_kv ? 5 : 1, st);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { kf_set_error("kf_gemm_qkv: launch failed: %s", hipGetErrorString(e)); return KF_ELAUNCH; }
  return KF_OK;
}

extern "C" int kf_gemm_qkv(const void* a, const void* a_lo, int a_dtype, int64_t lda,
                           const void* w_hi, const void* w_lo, int64_t ldw, const float* bias,
                           float* q_out, void* k_hi, void* k_lo, void* vt_hi, void* vt_lo,
                           int64_t sp, int64_t B, int64_t S, int64_t H, int64_t hd, int mode,
                           void* stream) {
  return kf_gemm_qkv_tiled(a, a_lo, a_dtype, lda, w_hi, w_lo, ldw, bias, q_out, k_hi, k_lo,
                           vt_hi, vt_lo, sp, B, S, H, hd, mode, TILE_AUTO, stream);
}

extern "C" int kf_split(const float* src, int64_t n, int mode, void* hi, void* lo, void* stream) {
  if (!src || !hi || n < 0) { kf_set_error("kf_split: bad arguments"); return KF_EINVAL; }
  const bool split = mode == KF_MMA_F16X3 || mode == KF_MMA_BF16X3 || mode == KF_MMA_F16X2;
  if (split && !lo) { kf_set_error("kf_split: split mode needs lo"); return KF_EINVAL; }
  if (n == 0) return KF_OK;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipStream_t st = (hipStream_t)stream;
  switch (mode) {
    case KF_MMA_F16: case KF_MMA_F16X3: case KF_MMA_F16X2:
      hipLaunchKernelGGL(split_kernel<_Float16>, dim3(blocks), dim3(256), 0, st, src, n,
                         (_Float16*)hi, split ? (_Float16*)lo : nullptr);
      break;
    case KF_MMA_BF16: case KF_MMA_BF16X3:
      hipLaunchKernelGGL(split_kernel<__bf16>, dim3(blocks), dim3(256), 0, st, src, n,
                         (__bf16*)hi, split ? (__bf16*)lo : nullptr);
      break;
    default:
      kf_set_error("kf_split: mode %d has no 16-bit planes", mode);
      return KF_EINVAL;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { kf_set_error("kf_split: launch failed: %s", hipGetErrorString(e)); return KF_ELAUNCH; }
  return KF_OK;
}
