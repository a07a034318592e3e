// Kernels of the gfx950 FlashAttention forward (shared by the per-mode translation units
// flash_<mode>.hip).
//
// FlashAttention forward for gfx950 with causal and key-padding masks in registers.
//
// Semantics of kernelforge/ops/flash.py:42-249: for each (batch, head) and query row,
// softmax over keys of (q . k) * sm_scale with -inf on masked keys (key > query under the
// causal mask, keep[b, key] == 0 under the padding mask), online in fp32 with exp2 and the
// two NaN guards (an all-masked block rescales against 0; a row with no valid key emits 0),
// then P (in the MFMA input format) times V.
//
// Operands (the "attention layout", produced by the fused QKV GEMM epilogue or by
// kf_attn_prep): q in fp32 / fp16 / bf16, any strides; k as 16-bit planes (hi, lo for the
// split modes) with rows of head_dim; v already transposed, V^T planes with rows of keys.
// Staging a K or V^T tile is therefore a plain 16-byte copy into LDS -- no conversion
// and no transpose inside the loop. V^T columns [S, roundup(S, 8)) must hold finite
// values (the producers zero them).
//
// Data flow per block (NW = 8 wavefronts for hd >= 128, else 4; 16 * QG query rows each,
// BM = 16 * QG * NW):
//  * K [key][d] and V^T [d][key] tiles of BN keys are copied global -> LDS by DMA
//    (global_load_lds_dwordx4) into two or three buffers (three where they fit in LDS) with
//    XOR-swizzled rows: the copies of the next one or two tiles run while tile t is
//    computed. Eight wavefronts share each tile, halving the copy traffic per flop.
//  * Scores are formed transposed, S^T = K . Q^T (v_mfma_f32_16x16x32), with sm_scale *
//    log2(e) folded into the query fragments, so scores arrive in log2 units. The two
//    16-key S^T tiles of a 32-key chunk use permuted K rows (tile t, row p -> key
//    (p/4)*8 + 4t + p%4), so lane (r, g) ends with the 8 consecutive keys 8g..8g+7 of
//    query r -- exactly the "B" operand layout of P^T in O^T = V^T . P^T. Softmax state
//    and the output accumulator of a query live in the same lane; the row maximum crosses
//    the four 16-lane groups with two v_permlane{16,32}_swap, and the row sum is reduced
//    once at the end.
//  * P is split with packed conversions (v_cvt_pkrtz_f16_f32 / v_cvt_pk_bf16_f32); the
//    accumulator rescale is skipped when no row maximum moved (alpha == 1 exactly).
//  * Key blocks past the last valid key are skipped (kv_len from kf_mask_prep): masked
//    keys contribute p = 0 and alpha = 1 there, so skipping is exact. Masks are evaluated
//    only on tiles that touch the diagonal or the padding.

#pragma once

#include <type_traits>

#include "kf_common.h"

namespace kf {

struct FlashArgs {
  const void* q; int64_t qs0, qs1, qs2;
  const void* k_hi; const void* k_lo; int64_t ks0, ks1, ks2;
  const void* vt_hi; const void* vt_lo; int64_t vs0, vs1, vs2;
  void* o; void* o_lo; int64_t os0, os1, os2; int o_dtype;
  const void* keep; int keep_dtype; int64_t ld_keep;
  const int32_t* kv_len; const int32_t* prefix;
  int B, H, S, hd;
  float scale_log2;
  float scale;           // sm_scale itself (score-rounding variant)
  int flags;
};

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.0f;     // log2 units: probabilities stay <= 256

// GMT: the general-mask instantiation's tile (same block height, so one grid serves both)
template <int HDP, int P = 2, bool GMT = false> struct FlashTile {
  // hd 64 in the split modes, prefix masks: eight wavefronts of one 16-row group (the same
  // 128-row block as four of two groups) at ~100-126 VGPRs, so two blocks give each SIMD
  // four wavefronts instead of two (C2-shape f16x3 attention 28.0 -> 25.3 us, outputs
  // bit-identical: each row takes the same MFMAs and softmax steps in the same order). The
  // general-mask launch, empty on prefix masks, keeps 256-thread blocks: with 512 its empty
  // launch over C5's 32768 blocks took 75.5 instead of 44.7 us.
  static constexpr bool kWide64 = HDP == 64 && P == 2 && !GMT;
  static constexpr int BN = HDP >= 256 ? 32 : 64;   // keys per LDS stage
  static constexpr int QG = HDP >= 256 || kWide64 ? 1 : 2;   // 16-row query groups per wavefront
  // Measured on MI355X (B4 H16 S8192 causal): hd >= 128 gains from eight wavefronts
  // sharing each K/V tile and three stages in flight (hd 128 f16x3: 198 -> 309 TF); hd <= 64
  // runs best with two stages (two blocks per CU).
  static constexpr int NW = HDP >= 128 || kWide64 ? 8 : 4;   // wavefronts per block (share K/V tiles)
  static constexpr int NTH = 64 * NW;
  static constexpr int BM = NW * 16 * QG;
  static constexpr int STAGE_BYTES = 2 * P * BN * HDP * 2;              // K and V^T planes
  // hd 256 single-pass (32-key stages of 32 KB): four stages, two tiles of copies in flight
  // (C4-shape attention 0.416 -> 0.405 ms, measured on MI355X)
  static constexpr int STAGES = (HDP >= 256 && P == 1) ? 4 : (HDP >= 128 && 3 * STAGE_BYTES <= 160 * 1024) ? 3 : 2;
  static_assert(BM == (HDP >= 256 ? 128 : HDP >= 128 ? 256 : 128), "one block height per head dim");
};

// keep[row + key0 + e] for e < 8 (keys past S clamped to S - 1), one dtype dispatch.
template <typename T>
__device__ __forceinline__ void keep8_t(const T* p, int key0, int S, float* out) {
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = (float)p[min(key0 + e, S - 1)];
}
__device__ __forceinline__ void load_keep8(const FlashArgs& a, int64_t row, int key0, float* out) {
  switch (a.keep_dtype) {
    case KF_U8: keep8_t((const uint8_t*)a.keep + row, key0, a.S, out); break;
    case KF_F32: keep8_t((const float*)a.keep + row, key0, a.S, out); break;
    case KF_F16: keep8_t((const _Float16*)a.keep + row, key0, a.S, out); break;
    default: keep8_t((const __bf16*)a.keep + row, key0, a.S, out); break;
  }
}

__device__ __forceinline__ void store_o4(const FlashArgs& a, int64_t off, const float* v) {
  store4_any(a.o, a.o_lo, a.o_dtype, off, v);
}

// Lane l and lane l ^ 16 (resp. l ^ 32) exchange a value with one VALU swap: each lane of
// the returned pair is either itself or its partner, so max / sum of the pair is the
// two-lane reduction.
__device__ __forceinline__ float xmax16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xmax32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xsum16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xsum32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Probabilities p (in [0, 1]) to the MFMA "B" operand: split modes hi + lo, single-pass
// rounded to nearest (the reference's cast of P to the value dtype). f16x3 uses the
// packed round-toward-zero convert, whose error the lo plane absorbs (hi + lo still
// represents p to 2^-20 relative); bf16 converts are packed round-to-nearest already.
template <int MODE, typename V>
__device__ __forceinline__ void p_operand(const float* p, V& hi, V& lo) {
  using TR = ModeTraits<MODE>;
  if constexpr (MODE == MODE_F16) {
    round8<_Float16, V>(p, hi);
  } else if constexpr (MODE == MODE_F16X3) {
    typedef __fp16 fp16x2 __attribute__((ext_vector_type(2)));
    uint32_t h[4], l[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const fp16x2 hv = __builtin_amdgcn_cvt_pkrtz(p[2 * j], p[2 * j + 1]);
      h[j] = __builtin_bit_cast(uint32_t, hv);
      // residuals p - hi with the fp16 halves read in place (v_fma_mix_f32: -1 * f16 + f32)
      float r0, r1;
      asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[0,0,0] op_sel_hi:[1,0,0]"
          : "=v"(r0) : "v"(h[j]), "v"(p[2 * j]));
      asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
          : "=v"(r1) : "v"(h[j]), "v"(p[2 * j + 1]));
      const fp16x2 lv = __builtin_amdgcn_cvt_pkrtz(r0, r1);
      l[j] = __builtin_bit_cast(uint32_t, lv);
    }
    hi = from_u4<V>(U4{h[0], h[1], h[2], h[3]});
    lo = from_u4<V>(U4{l[0], l[1], l[2], l[3]});
  } else {
    if constexpr (TR::split) split8<__bf16, V>(p, hi, lo);
    else round8<__bf16, V>(p, hi);
  }
}

// Chunk swizzles of the K tile ([key][d], HDP / 8 chunks per row) and the V^T tile
// ([d][key], BN / 8 chunks per row) in LDS. Fragment reads go to K rows
// (r / 4) * 8 + r % 4 (+ 4 tt + 32 c) and V^T rows 16 j + r, so each swizzle was chosen by
// measuring the ds_read_b128 throughput of that exact read sequence over every
// bit-select of the row index on MI355X (e.g. hd 64 K: 119 -> 274, hd 128 K: 32 -> 193,
// hd 128 V^T: 63 -> 187 B/clk/CU relative units, unswizzled -> swizzled).
template <int HDP> __host__ __device__ constexpr int kswz(int row) {
  const int b0 = row & 1, b1 = (row >> 1) & 1, b2 = (row >> 2) & 1, b4 = (row >> 4) & 1, b5 = (row >> 5) & 1;
  if constexpr (HDP == 32) return b5 | (b4 << 1);
  else if constexpr (HDP == 64) return b5 | (b1 << 1) | (b4 << 2);
  else if constexpr (HDP == 128) return b5 | (b1 << 1) | (b0 << 2) | (b4 << 3);
  else return b2 | (b1 << 1) | (b0 << 2) | (b4 << 3);
}
template <int HDP> __host__ __device__ constexpr int vswz(int row) {
  const int b1 = (row >> 1) & 1, b2 = (row >> 2) & 1, b3 = (row >> 3) & 1, b4 = (row >> 4) & 1, b5 = (row >> 5) & 1;
  if constexpr (HDP >= 256) return b4 | (b3 << 1);              // BN = 32: 4 chunks per row
  else if constexpr (HDP == 128) return b5 | (b2 << 1) | (b1 << 2);
  else return b5 | (b3 << 1) | (b1 << 2);
}

// GM: general key masks (keep read per key) or prefix masks (validity from kv_len alone).
// VAR: kVarP16 -- split modes carry P as one rounded plane instead of hi + lo
// (KF_FLASH_P16); kVarRoundScores -- q.k is rounded to the mode's 16-bit type, scaled,
// and rounded again before the softmax, as the reference's narrow forward computes
// `matmul(q, k^T) * scale` (KF_FLASH_ROUND_SCORES).
// The host launches the prefix instantiation and, when a keep mask is given, the general
// one; each block serves only the batch rows of its kind, so the common path carries no
// per-key mask loads.
constexpr int kVarNone = 0, kVarP16 = 1, kVarRoundScores = 2;

template <typename E> __device__ __forceinline__ float round_to(float v) { return (float)(E)v; }

// Block -> (batch row, head, query block) of the attention grid. Blocks reach the XCDs
// round-robin (block i runs on XCD i % 8) and each XCD is given a contiguous range of
// `lin`, so the blocks an XCD holds at one time share their K / V^T tiles in its L2.
// Inside that order the slots cycle through the batch rows before the heads, and with
// fewer than 8 heads a head's query blocks are dealt out in NP parts, so every XCD gets
// the same share of every batch row: causal work grows as the square of a row's valid
// length, and an XCD range of whole batch rows left the XCDs holding short rows idle
// while the others finished (max / mean XCD work 1.69 on a B4 S65536 input with lengths
// uniform in [S/2, S]). Causal query blocks come in light/heavy pairs (q-block k and
// nqb - 1 - k), part p taking the pairs k = p (mod NP), except on grids of longer rows and
// more than one round, which order a head's blocks heavy to light. A bijection for any B, H,
// nqb.
struct FlashBlock { int b, h, qb; };
__host__ __device__ inline FlashBlock flash_block_map(int bid, int nblocks, int B, int H,
                                                      int nqb, bool causal) {
  int lin = bid, j = bid, per = nblocks;
  if (nblocks % kXcds == 0) {
    per = nblocks / kXcds;
    j = bid / kXcds;
    lin = (bid % kXcds) * per + j;
  }
  int np = 1;
  while (np * H < kXcds && nqb % (4 * np) == 0) np *= 2;
  const int per_part = nqb / np;
  const int vslot = lin / per_part, i = lin % per_part;
  const int rest = vslot / B;
  FlashBlock m;
  m.b = vslot % B;
  m.h = rest % H;
  const int part = rest / H;
  if (causal && nqb >= 8 && per >= 128) {
    // Causal rows of 8+ query blocks on a grid of more blocks than the chip holds at once
    // (>= 1024): a head's query blocks heavy to light, so the blocks an XCD holds at one time
    // cover neighbouring query ranges, walk the same K / V^T tiles at about the same time
    // (out of its L2), and the light blocks make the tail. Measured on MI355X (outputs
    // unchanged): C5 attention 17.4 -> 15.4 ms, C4 0.48 -> 0.42 ms, C3 67 -> 61 us. Grids the
    // chip holds at once keep the light/heavy pairs below, which give each CU one of each.
    m.qb = nqb - 1 - (i * np + part);
  } else if (causal) {
    const int k = (i >> 1) * np + part;
    // The second half of an XCD's range takes each pair heavy block first: where the
    // whole grid is resident at once (two blocks per CU), a CU's two blocks then hold
    // one light and one heavy block whether the dispatcher gives a CU blocks j and j + 1
    // or j and j + per / 2. A pair (i, i + 1) lies in one half when per % 4 == 0 and
    // per_part is even, which keeps the swap a bijection.
    const bool swap = nblocks % kXcds == 0 && per % 4 == 0 && per_part % 2 == 0 &&
                      2 * j >= per;
    m.qb = ((i & 1) != swap) ? nqb - 1 - k : k;
  } else {
    m.qb = i * np + part;
  }
  return m;
}

template <int MODE, int QT, int HDP, bool GM, int VAR = kVarNone>
__global__ __launch_bounds__((FlashTile<HDP, ModeTraits<MODE>::split ? 2 : 1, GM>::NTH))
void flash_fwd_kernel(FlashArgs a) {
  using TR = ModeTraits<MODE>;
  static_assert(VAR != kVarP16 || MODE == MODE_F16X3, "single-plane P is an f16x3 option");
  static_assert(VAR != kVarRoundScores || MODE == MODE_F16 || MODE == MODE_BF16,
                "score rounding follows a single-pass 16-bit mode");
  constexpr bool PS = VAR != kVarP16;         // P as hi + lo in split modes
  // two query groups pipelined within a tile (their K and V^T fragments held in registers
  // for both): where those fit beside the rest -- head_dim <= 64 with prefix masks (the
  // general-mask variant would fall to one wavefront per SIMD)
  constexpr bool kPipe = FlashTile<HDP, TR::split ? 2 : 1, GM>::QG == 2 && HDP <= 64 && !GM;
  constexpr bool RS = VAR == kVarRoundScores;
  using V = typename TR::vec;
  using E = typename TR::elem;
  constexpr int P = TR::split ? 2 : 1;
  using FT = FlashTile<HDP, P, GM>;
  static_assert(FT::BM == FlashTile<HDP, P, !GM>::BM, "one grid for both mask instantiations");
  constexpr int BN = FT::BN, QG = FT::QG, BM = FT::BM, NTH = FT::NTH, STAGES = FT::STAGES;
  constexpr int NC = BN / 32;          // 32-key chunks per tile
  constexpr int ND = HDP / 32;         // 32-wide contraction chunks of q . k
  constexpr int NT = HDP / 16;         // 16-row d tiles of O^T
  constexpr int CK = HDP / 8, CV = BN / 8;     // 16-byte chunks per K row / V^T row
  constexpr int TILE = BN * HDP;               // elements of one K (or V^T) plane tile
  constexpr int STG = 2 * P * TILE;            // K planes then V^T planes
  constexpr int NCH = TILE / 8 / NTH;          // chunks per thread per plane tile
  constexpr int NL = NCH * 2 * P;              // copies per thread per tile
  static_assert(NCH >= 1 && (TILE / 8) % NTH == 0, "staging must tile the block");
  // the swizzles permute chunks within a row: their largest value must stay below the
  // chunks per row (vswz yields up to 3 at hd >= 256, else up to 7; kswz up to 15)
  static_assert(CV >= (HDP >= 256 ? 4 : 8) && CK >= (HDP == 32 ? 4 : HDP == 64 ? 8 : 16),
                "K / V^T swizzle wider than a tile row");

  __shared__ __attribute__((aligned(1024))) E smem[STAGES * STG];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, grp = lane >> 4;

  const int nqb = (a.S + BM - 1) / BM;
  const bool causal = a.flags & KF_FLASH_CAUSAL;
  const FlashBlock blk = flash_block_map(blockIdx.x, gridDim.x, a.B, a.H, nqb, causal);
  const int b = blk.b, h = blk.h, qb = blk.qb;

  const int kvlen = a.kv_len ? a.kv_len[b] : a.S;
  // prefix: keys [0, kvlen) are all valid, so kvlen alone decides validity (keep unread)
  const bool prefix = a.keep == nullptr || (a.kv_len && a.prefix && a.prefix[b] != 0);
  if (prefix == GM) return;            // the other instantiation serves this batch row
  const bool skip_pad = (a.flags & KF_FLASH_SKIP_PAD_ROWS) && a.kv_len;

  const int q_lo = qb * BM;
  const int qw0 = q_lo + wave * 16 * QG;         // first query row of this wavefront
  const int64_t obase = (int64_t)b * a.os0 + (int64_t)h * a.os1;

  auto write_zero_rows = [&](int q0) KF_INLINE {
#pragma unroll
    for (int qg = 0; qg < QG; ++qg) {
      const int qi = q0 + qg * 16 + r;
      if (qi >= a.S) continue;
      const float z[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int d = 16 * j + 4 * grp;
        if (d < a.hd) store_o4(a, obase + (int64_t)qi * a.os2 + d, z);
      }
    }
  };

  if (skip_pad && q_lo >= kvlen) {        // whole block is padding rows
    write_zero_rows(qw0);
    return;
  }

  const int kend_blk = causal ? min(kvlen, q_lo + BM) : kvlen;
  const int kend_w = causal ? min(kvlen, qw0 + 16 * QG) : kvlen;
  const bool wave_active = qw0 < a.S && !(skip_pad && qw0 >= kvlen);

  // ---- K / V^T staging: LDS DMA from clamped source addresses. Keys past S re-read key
  // S - 1, d chunks past hd re-read the last chunk, V^T columns past S8 = roundup(S, 8)
  // re-read [S8 - 8, S8): all finite, and each lands where it is multiplied by an exact
  // zero (a masked probability, a zero-padded query column) or feeds an output row d >= hd
  // that is never stored. No branch, no register staging.
  const int64_t kbase = (int64_t)b * a.ks0 + (int64_t)h * a.ks1;
  const int64_t vbase = (int64_t)b * a.vs0 + (int64_t)h * a.vs1;
  const int S8 = (a.S + 7) & ~7;
  const E* kpl[P];
  const E* vpl[P];
  kpl[0] = (const E*)a.k_hi;
  vpl[0] = (const E*)a.vt_hi;
  if constexpr (P == 2) {
    kpl[1] = (const E*)a.k_lo;
    vpl[1] = (const E*)a.vt_lo;
  }
  // chunk i of this thread: K row (key) p / CK, d chunk p % CK; V^T row (d) p / CV, key
  // chunk p % CV, with p = i * NTH + tid and the swizzles applied on the source side
  auto k_src = [&](int i, int k0) KF_INLINE -> int64_t {
    const int p = i * NTH + tid, row = p / CK;
    const int col = min((p % CK) ^ kswz<HDP>(row), a.hd / 8 - 1) * 8;
    return kbase + (int64_t)min(k0 + row, a.S - 1) * a.ks2 + col;
  };
  auto v_src = [&](int i, int k0) KF_INLINE -> int64_t {
    const int p = i * NTH + tid, row = p / CV;
    const int col = ((p % CV) ^ vswz<HDP>(row)) * 8;
    return vbase + (int64_t)min(row, a.hd - 1) * a.vs2 + min(k0 + col, S8 - 8);
  };
  // tiles that end inside S advance the tile-0 offsets by a uniform step; the tail tile
  // recomputes them with the clamps
  int64_t ko0[NCH], vo0[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    ko0[i] = k_src(i, 0);
    vo0[i] = v_src(i, 0);
  }
  const int64_t kstep = (int64_t)BN * a.ks2;
  auto issue = [&](int t) KF_INLINE {
    E* dst = smem + (t % STAGES) * STG;
    const int k0 = t * BN;
    const bool inside = k0 + BN <= a.S;          // uniform: no clamp can bind
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int64_t ko = inside ? ko0[i] + t * kstep : k_src(i, k0);
      const int64_t vo = inside ? vo0[i] + k0 : v_src(i, k0);
#pragma unroll
      for (int p = 0; p < P; ++p) {
        dma16(kpl[p] + ko, dst + p * TILE + (i * NTH + wave * 64) * 8);
        dma16(vpl[p] + vo, dst + (P + p) * TILE + (i * NTH + wave * 64) * 8);
      }
    }
  };

  const int ntiles = (kend_blk + BN - 1) / BN;
#pragma unroll
  for (int t = 0; t < STAGES - 1; ++t)
    if (t < ntiles) issue(t);

  // ---- query fragments (MFMA "B" operand of S^T), pre-scaled by sm_scale * log2(e)
  // (unscaled when the scores are rounded: the scale is applied after the rounding)
  V qf[QG][ND][P];
  {
    const int64_t qbase = (int64_t)b * a.qs0 + (int64_t)h * a.qs1;
#pragma unroll
    for (int qg = 0; qg < QG; ++qg)
#pragma unroll
      for (int dc = 0; dc < ND; ++dc) {
        const int qi = qw0 + qg * 16 + r, d = dc * 32 + grp * 8;
        float x[8];
        if (qi < a.S && d < a.hd) {
          ld8<QT>(a.q, qbase + (int64_t)qi * a.qs2 + d, x);
          if constexpr (!RS) {
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] *= a.scale_log2;
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = 0.0f;
        }
        if constexpr (TR::split) split8<E, V>(x, qf[qg][dc][0], qf[qg][dc][P - 1]);
        else round8<E, V>(x, qf[qg][dc][0]);
      }
  }

  // fragment offsets (elements within a stage)
  int koff[NC][2][ND], voff[NC][NT];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int krow = 32 * c + (r >> 2) * 8 + 4 * tt + (r & 3);
#pragma unroll
      for (int dc = 0; dc < ND; ++dc) koff[c][tt][dc] = krow * HDP + (((dc * 4 + grp) ^ kswz<HDP>(krow)) << 3);
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int vrow = 16 * j + r;
      voff[c][j] = P * TILE + vrow * BN + (((4 * c + grp) ^ vswz<HDP>(vrow)) << 3);
    }
  }

  float m_ref[QG], l_i[QG];
  bool m_set[QG];
  f32x4 acc[QG][NT];
#pragma unroll
  for (int qg = 0; qg < QG; ++qg) {
    m_ref[qg] = 0.0f;
    m_set[qg] = false;
    l_i[qg] = 0.0f;
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[qg][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  for (int t = 0; t < ntiles; ++t) {
    // this wavefront's copies of tile t have landed once at most the later tiles' copies
    // are pending (loads complete in issue order; keep reads issued later only make the
    // wait longer)
    if constexpr (STAGES == 4) {
      const int later = min(2, ntiles - 1 - t);
      if (later >= 2) wait_vmcnt<2 * NL>();
      else if (later == 1) wait_vmcnt<NL>();
      else wait_vmcnt<0>();
    } else if constexpr (STAGES == 3) {
      if (t + 1 < ntiles) wait_vmcnt<NL>();
      else wait_vmcnt<0>();
    } else {
      wait_vmcnt<0>();
    }
    lds_barrier();                   // everyone's copies landed; tile t-1 no longer read
    if (t + STAGES - 1 < ntiles) issue(t + STAGES - 1);
    const E* st = smem + (t % STAGES) * STG;
    const int k0 = t * BN;

    if (wave_active && k0 < kend_w) {
      if constexpr (kPipe) {
        // Two query groups in flight: the second group's S MFMAs run under the first
        // group's exponentials, and the first group's P.V MFMAs under the second group's.
        // The K (then V^T) fragments of the tile are read once into registers for both.
        f32x4 s[QG][NC][2];
#pragma unroll
        for (int qg = 0; qg < QG; ++qg)
#pragma unroll
          for (int c = 0; c < NC; ++c) {    // scores arrive relative to the row's reference max
            const float nm = RS ? 0.0f : -m_ref[qg];
            s[qg][c][0] = s[qg][c][1] = f32x4{nm, nm, nm, nm};
          }
        auto s_mma = [&](int qg, int c, int tt, int dc, const V* kf) KF_INLINE {
          if constexpr (TR::split) {
            s[qg][c][tt] = mma16(kf[0], qf[qg][dc][1], s[qg][c][tt]);
            s[qg][c][tt] = mma16(kf[1], qf[qg][dc][0], s[qg][c][tt]);
          }
          s[qg][c][tt] = mma16(kf[0], qf[qg][dc][0], s[qg][c][tt]);
        };
        V pf[QG][NC][P];
        float x[QG][NC][8];
        // softmax part 1: scores relative to the row's reference maximum, masked; the
        // reference moves (rarely) here -- see the lazy rescaling note below
        auto soft1 = [&](int qg) KF_INLINE {
          const int qg0 = qw0 + qg * 16;
          const int qi = qg0 + r;
          const bool full = !GM && k0 + BN <= kvlen && (!causal || k0 + BN - 1 <= qg0);
#pragma unroll
          for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) x[qg][c][jj] = s[qg][c][jj >> 2][jj & 3];
          if constexpr (RS) {
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
              for (int jj = 0; jj < 8; ++jj)
                x[qg][c][jj] = round_to<E>(round_to<E>(x[qg][c][jj]) * a.scale) * kLog2e - m_ref[qg];
          }
          if (__builtin_expect(!full, 0)) {
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
              for (int jj = 0; jj < 8; ++jj) {
                const int key = k0 + 32 * c + 8 * grp + jj;
                const bool ok = key < kvlen && (!causal || key <= qi);
                x[qg][c][jj] = ok ? x[qg][c][jj] : kNegInf;
              }
            if constexpr (GM) {
#pragma unroll
              for (int c = 0; c < NC; ++c) {
                float kv[8];
                load_keep8(a, (int64_t)b * a.ld_keep, k0 + 32 * c + 8 * grp, kv);
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) x[qg][c][jj] = kv[jj] != 0.0f ? x[qg][c][jj] : kNegInf;
              }
            }
          }
          float mloc = kNegInf;
#pragma unroll
          for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) mloc = fmaxf(mloc, x[qg][c][jj]);
          mloc = xmax32(xmax16(mloc));
          const bool move = mloc > kLazy || (!m_set[qg] && mloc != kNegInf);
          if (__builtin_expect(__any(move), 0)) {
            const float delta = move ? mloc : 0.0f;
            const float alpha = __builtin_amdgcn_exp2f(-delta);
            m_ref[qg] += delta;
            m_set[qg] = m_set[qg] || move;
            l_i[qg] *= alpha;
#pragma unroll
            for (int j = 0; j < NT; ++j) acc[qg][j] *= alpha;
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
              for (int jj = 0; jj < 8; ++jj) x[qg][c][jj] -= delta;
          }
        };
        // softmax part 2: the probabilities, their row sum and the P operand of P.V
        auto soft2 = [&](int qg) KF_INLINE {
          float psum = 0.0f;
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            float pv[8];
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
              pv[jj] = __builtin_amdgcn_exp2f(x[qg][c][jj]);
              psum += pv[jj];
            }
            if constexpr (PS) p_operand<MODE, V>(pv, pf[qg][c][0], pf[qg][c][P - 1]);
            else round8<_Float16, V>(pv, pf[qg][c][0]);
          }
          l_i[qg] += psum;
        };
        auto pv_mma = [&](int qg, int c, int j, const V* vf) KF_INLINE {
          if constexpr (TR::split) {
            if constexpr (PS) acc[qg][j] = mma16(vf[0], pf[qg][c][1], acc[qg][j]);
            acc[qg][j] = mma16(vf[1], pf[qg][c][0], acc[qg][j]);
          }
          acc[qg][j] = mma16(vf[0], pf[qg][c][0], acc[qg][j]);
        };
        constexpr int NMS = NC * 2 * ND * (TR::split ? 3 : 1);             // S MFMAs per group
        constexpr int NMP = NC * NT * (TR::split ? (PS ? 3 : 2) : 1);      // P.V MFMAs per group

        V kf[NC][2][ND][P];
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int dc = 0; dc < ND; ++dc)
#pragma unroll
              for (int p = 0; p < P; ++p)
                kf[c][tt][dc][p] = from_u4<V>(*(const U4*)&st[koff[c][tt][dc] + p * TILE]);
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int dc = 0; dc < ND; ++dc) s_mma(0, c, tt, dc, kf[c][tt][dc]);
        soft1(0);
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int dc = 0; dc < ND; ++dc) s_mma(1, c, tt, dc, kf[c][tt][dc]);
        soft2(0);
#pragma unroll
        for (int i = 0; i < NMS; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);   // VALU
        }
        V vf[NC][NT][P];
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int p = 0; p < P; ++p)
              vf[c][j][p] = (HDP == 32 && 16 * j >= a.hd) ? V{} : from_u4<V>(*(const U4*)&st[voff[c][j] + p * TILE]);
        soft1(1);
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int j = 0; j < NT; ++j)
            if (!(HDP == 32 && 16 * j >= a.hd)) pv_mma(0, c, j, vf[c][j]);
        soft2(1);
#pragma unroll
        for (int i = 0; i < NMP; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);   // VALU
        }
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int j = 0; j < NT; ++j)
            if (!(HDP == 32 && 16 * j >= a.hd)) pv_mma(1, c, j, vf[c][j]);
      } else {
        // ---- S^T = K . Q^T (log2 units) for BN keys and every query group of this wavefront
        f32x4 s[QG][NC][2];
#pragma unroll
        for (int qg = 0; qg < QG; ++qg)
#pragma unroll
          for (int c = 0; c < NC; ++c) {      // scores arrive relative to the row's reference max
            const float nm = RS ? 0.0f : -m_ref[qg];
            s[qg][c][0] = s[qg][c][1] = f32x4{nm, nm, nm, nm};
          }
        // Single pass at hd 256 (one group, one MFMA per fragment): every K fragment of the
        // tile is read before the S MFMAs and every V^T fragment right after them, so the
        // reads wait once per phase and V^T lands under the softmax. (The copies are
        // FLAT-encoded LDS writes, so each LDS-read wait is a wait for all reads: read
        // one fragment ahead, the MFMAs had waited for each read in turn.)
        constexpr bool kBatch = !TR::split && QG == 1 && HDP == 256 && !GM;
        V kall[kBatch ? NC : 1][2][kBatch ? ND : 1];
        V vall[kBatch ? NC : 1][kBatch ? NT : 1];
        if constexpr (kBatch) {
#pragma unroll
          for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
              for (int dc = 0; dc < ND; ++dc)
                kall[c][tt][dc] = from_u4<V>(*(const U4*)&st[koff[c][tt][dc]]);
        }
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int dc = 0; dc < ND; ++dc) {
              V kf[P];
              if constexpr (kBatch) {
                kf[0] = kall[c][tt][dc];
              } else {
#pragma unroll
                for (int p = 0; p < P; ++p) kf[p] = from_u4<V>(*(const U4*)&st[koff[c][tt][dc] + p * TILE]);
              }
#pragma unroll
              for (int qg = 0; qg < QG; ++qg) {
                if constexpr (TR::split) {
                  s[qg][c][tt] = mma16(kf[0], qf[qg][dc][1], s[qg][c][tt]);
                  s[qg][c][tt] = mma16(kf[1], qf[qg][dc][0], s[qg][c][tt]);
                }
                s[qg][c][tt] = mma16(kf[0], qf[qg][dc][0], s[qg][c][tt]);
              }
            }

        if constexpr (kBatch) {
#pragma unroll
          for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int j = 0; j < NT; ++j) vall[c][j] = from_u4<V>(*(const U4*)&st[voff[c][j]]);
          __builtin_amdgcn_sched_group_barrier(0x100, NC * 2 * ND, 0);   // K reads
          __builtin_amdgcn_sched_group_barrier(0x008, NC * 2 * ND, 0);   // S MFMAs
          __builtin_amdgcn_sched_group_barrier(0x100, NC * NT, 0);       // V^T reads
        }
        // ---- online softmax per query group; lane holds keys k0 + 32c + 8grp + (4tt + i)
        V pf[QG][NC][P];
#pragma unroll
        for (int qg = 0; qg < QG; ++qg) {
          const int qg0 = qw0 + qg * 16;
          const int qi = qg0 + r;
          const bool full = !GM && k0 + BN <= kvlen && (!causal || k0 + BN - 1 <= qg0);
          float x[NC][8];
#pragma unroll
          for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) x[c][jj] = s[qg][c][jj >> 2][jj & 3];
          if constexpr (RS) {            // E(E(q.k) * scale), then log2 units relative to m_ref
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
              for (int jj = 0; jj < 8; ++jj)
                x[c][jj] = round_to<E>(round_to<E>(x[c][jj]) * a.scale) * kLog2e - m_ref[qg];
          }
          if (__builtin_expect(!full, 0)) {
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
              for (int jj = 0; jj < 8; ++jj) {
                const int key = k0 + 32 * c + 8 * grp + jj;
                const bool ok = key < kvlen && (!causal || key <= qi);
                x[c][jj] = ok ? x[c][jj] : kNegInf;
              }
            if constexpr (GM) {
#pragma unroll
              for (int c = 0; c < NC; ++c) {
                float kv[8];
                load_keep8(a, (int64_t)b * a.ld_keep, k0 + 32 * c + 8 * grp, kv);
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) x[c][jj] = kv[jj] != 0.0f ? x[c][jj] : kNegInf;
              }
            }
          }
          // Lazy rescaling: p = exp2(s - m_ref) with a reference maximum that moves only
          // when the tile maximum exceeds it by more than kLazy (p stays <= 2^kLazy, well
          // inside fp16 range) or on the row's first tile with a valid key. Any reference
          // gives the same softmax (it cancels in acc / l); moving it rarely removes the
          // per-tile subtraction and the per-tile accumulator rescale.
          float mloc = kNegInf;
#pragma unroll
          for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) mloc = fmaxf(mloc, x[c][jj]);
          mloc = xmax32(xmax16(mloc));
          const bool move = mloc > kLazy || (!m_set[qg] && mloc != kNegInf);
          if (__builtin_expect(__any(move), 0)) {
            const float delta = move ? mloc : 0.0f;
            const float alpha = __builtin_amdgcn_exp2f(-delta);
            m_ref[qg] += delta;
            m_set[qg] = m_set[qg] || move;
            l_i[qg] *= alpha;
#pragma unroll
            for (int j = 0; j < NT; ++j) acc[qg][j] *= alpha;
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
              for (int jj = 0; jj < 8; ++jj) x[c][jj] -= delta;
          }
          float psum = 0.0f;
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            float pv[8];
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
              pv[jj] = __builtin_amdgcn_exp2f(x[c][jj]);
              psum += pv[jj];
            }
            if constexpr (PS) {
              p_operand<MODE, V>(pv, pf[qg][c][0], pf[qg][c][P - 1]);
            } else {                     // one fp16 plane, rounded to nearest (v_cvt_pk_f16_f32)
              round8<_Float16, V>(pv, pf[qg][c][0]);
            }
          }
          l_i[qg] += psum;
        }

        // ---- O^T += V^T . P^T
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int j = 0; j < NT; ++j) {
            if (HDP == 32 && 16 * j >= a.hd) continue;     // hd 8 / 16: only the first d tile
            V vf[P];
            if constexpr (kBatch) {
              vf[0] = vall[c][j];
            } else {
#pragma unroll
              for (int p = 0; p < P; ++p) vf[p] = from_u4<V>(*(const U4*)&st[voff[c][j] + p * TILE]);
            }
#pragma unroll
            for (int qg = 0; qg < QG; ++qg) {
              if constexpr (TR::split) {
                if constexpr (PS) acc[qg][j] = mma16(vf[0], pf[qg][c][1], acc[qg][j]);
                acc[qg][j] = mma16(vf[1], pf[qg][c][0], acc[qg][j]);
              }
              acc[qg][j] = mma16(vf[0], pf[qg][c][0], acc[qg][j]);
            }
          }
      }
    }
  }


  // ---- finalize: reduce the row sum over the four lane groups, normalise, store
  if (!wave_active) {
    if (qw0 < a.S) write_zero_rows(qw0);
    return;
  }
#pragma unroll
  for (int qg = 0; qg < QG; ++qg) {
    const float l = xsum32(xsum16(l_i[qg]));
    const int qi = qw0 + qg * 16 + r;
    if (qi >= a.S) continue;
    // padding rows of a partly valid wavefront: zeros, as for wholly padded blocks
    const float inv = (skip_pad && qi >= kvlen) ? 0.0f : 1.0f / (l == 0.0f ? 1.0f : l);
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int d = 16 * j + 4 * grp;
      if (d >= a.hd) continue;
      float o[4] = {acc[qg][j][0] * inv, acc[qg][j][1] * inv, acc[qg][j][2] * inv, acc[qg][j][3] * inv};
      store_o4(a, obase + (int64_t)qi * a.os2 + d, o);
    }
  }
}

// ------------------------------------------------------------ pipelined single-pass kernel
// Single-pass fp16 / bf16 attention at head_dim 64 and 128 with prefix masks, on the
// 32x32x16 MFMA and software-pipelined over 32-key chunks.
//
// Why 32x32: on MI355X an MFMA holds the SIMD's VALU issue for part of its run, and the
// softmax is VALU work. Measured: v_mfma_f32_16x16x32_f16 (16 matrix cycles) hides ~2
// plain VALU instructions and no v_exp_f32 (~9.4 cycles each); v_mfma_f32_32x32x16_f16
// (the same flops in 32 cycles) hides ~5 plain VALU instructions or 2 exponentials. With
// 16x16 tiles the softmax (exponentials, maxima, sums, conversions, LDS addresses) sets
// the time; with 32x32 most of it runs under the MFMAs.
//
// Layout. Each wavefront owns 32 query rows (one 32-column MFMA tile); BM = 32 x waves.
// Per 32-key chunk, S^T (keys x queries) = K . Q^T takes HDP / 16 MFMAs with K rows as the
// "A" operand in a permuted order -- operand row m holds chunk key m with bits 2 and 3
// swapped -- so that lane l (query l % 32, half h = l / 32) ends with keys 8h .. 8h + 7 in
// registers 0-7 and 16 + 8h .. 16 + 8h + 7 in registers 8-15: exactly the "B" operand
// (P^T, 8 consecutive keys per lane) of the two 16-key steps of O^T += V^T . P^T. Softmax
// state and the output of a query sit in the lane pair (l, l ^ 32); the row maximum
// crosses the pair with one v_permlane32_swap.
//
// Pipeline: the q.k MFMAs of chunk k + 1 are issued among the exponentials of chunk k,
// then the P.V MFMAs of chunk k; LDS stages of 64 keys (two chunks), three or four deep, the
// barrier that frees a stage between a tile's two chunks. Lazy rescaling as in
// flash_fwd_kernel (the reference maximum moves on a row's first valid key or when a score
// exceeds it by more than kLazy, in log2 units). A wave's first chunk and masked chunks
// check it before the next chunk's scores start; steady chunks check their largest
// probability afterwards and re-form the scores where it moved (chunk_steady), with the
// same results.
//
// LDS rows: K [64 keys][HDP], V^T [HDP][64 keys], 16-byte chunks XOR-swizzled so that the
// 16 lanes of each ds_read_b128 phase (16 consecutive operand rows, one logical chunk)
// land on 16 distinct 16-byte bank slots: K at hd 128 (256-byte rows) by row & 15; K at
// hd 64 and V^T (128-byte rows, two per bank period) by (row >> 1) & 7.
template <int HDP> struct PipeTile {
  static constexpr int BN = 64;
  static constexpr int NW = HDP >= 128 ? 8 : 4;
  static constexpr int NTH = 64 * NW, BM = 32 * NW;
  // hd 128: four 32 KB stages (copies two tiles ahead); hd 64: three 16 KB stages, which
  // keep three blocks per CU (measured: four stages at hd 64 cost a block per CU, -8 %)
  static constexpr int STAGES = HDP >= 128 ? 4 : 3;
  static constexpr int STAGE_BYTES = 2 * BN * HDP * 2;
  static_assert(STAGES * STAGE_BYTES <= 160 * 1024, "LDS");
  static_assert(STAGES >= 3, "two tiles in flight while one is computed");
};

// Wait until a wavefront's tile has landed while `later` tiles issued after it (at most N)
// may stay in flight: copies complete in issue order, PER copies per tile.
template <int N, int PER> __device__ __forceinline__ void wait_tile_landed(int later) {
  if constexpr (N > 0) {
    if (later >= N) {
      wait_vmcnt<N * PER>();
      return;
    }
    wait_tile_landed<N - 1, PER>(later);
  } else {
    wait_vmcnt<0>();
  }
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 mma32(const half8& a, const half8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mma32(const bhalf8& a, const bhalf8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

template <int HDP> __host__ __device__ constexpr int pk_swz(int row) {
  return HDP >= 128 ? (row & 15) : ((row >> 1) & 7);
}
__host__ __device__ constexpr int pv_swz(int row) { return (row >> 1) & 7; }
// operand row m of a 32-key S^T tile holds chunk key m with bits 2 and 3 swapped
__host__ __device__ constexpr int pkey(int m) {
  return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1);
}

template <int MODE, int QT, int HDP>
__global__ __launch_bounds__(PipeTile<HDP>::NTH) void flash_pipe_kernel(FlashArgs a) {
  using TR = ModeTraits<MODE>;
  static_assert(!TR::split, "single-pass modes only");
  using V = typename TR::vec;
  using E = typename TR::elem;
  using FT = PipeTile<HDP>;
  constexpr int BN = FT::BN, BM = FT::BM, NTH = FT::NTH, STAGES = FT::STAGES;
  constexpr int NDS = HDP / 16;        // 16-wide contraction steps of q . k
  constexpr int NJ = HDP / 32;         // 32-row d tiles of O^T
  constexpr int CK = HDP / 8, CV = BN / 8;
  constexpr int TILE = BN * HDP;
  constexpr int STG = 2 * TILE;        // K then V^T
  constexpr int NCH = TILE / 8 / NTH;
  static_assert(NCH >= 1 && (TILE / 8) % NTH == 0, "staging must tile the block");

  __shared__ __attribute__((aligned(1024))) E smem[STAGES * STG];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, hh = lane >> 5;       // query column of the tile, lane half

  const int nqb = (a.S + BM - 1) / BM;
  const bool causal = a.flags & KF_FLASH_CAUSAL;
  const FlashBlock blk = flash_block_map(blockIdx.x, gridDim.x, a.B, a.H, nqb, causal);
  const int b = blk.b, h = blk.h, qb = blk.qb;

  const int kvlen = a.kv_len ? a.kv_len[b] : a.S;
  const bool prefix = a.keep == nullptr || (a.kv_len && a.prefix && a.prefix[b] != 0);
  if (!prefix) return;                 // the general-mask kernel serves this batch row
  const bool skip_pad = (a.flags & KF_FLASH_SKIP_PAD_ROWS) && a.kv_len;

  const int q_lo = qb * BM;
  const int qw0 = q_lo + wave * 32;    // first query row of this wavefront
  const int qi = qw0 + n;              // this lane's query row
  const int64_t obase = (int64_t)b * a.os0 + (int64_t)h * a.os1;

  // output of this lane: query qi, d = 32 j + 8 (r / 4) + 4 hh + r % 4 for register r
  auto store_rows = [&](const f32x16* o, float scale) KF_INLINE {
    if (qi >= a.S) return;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * j + 8 * g + 4 * hh;
        if (d >= a.hd) continue;
        const float v[4] = {o[j][4 * g] * scale, o[j][4 * g + 1] * scale, o[j][4 * g + 2] * scale,
                            o[j][4 * g + 3] * scale};
        store_o4(a, obase + (int64_t)qi * a.os2 + d, v);
      }
  };
  auto write_zero_rows = [&]() KF_INLINE {
    f32x16 z[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) z[j] = f32x16{};
    store_rows(z, 0.0f);
  };
  if (skip_pad && q_lo >= kvlen) {
    write_zero_rows();
    return;
  }

  const int kend_blk = causal ? min(kvlen, q_lo + BM) : kvlen;
  const int kend_w = causal ? min(kvlen, qw0 + 32) : kvlen;
  const bool wave_active = qw0 < a.S && !(skip_pad && qw0 >= kvlen);
  const int nch = wave_active ? (kend_w + 31) / 32 : 0;      // 32-key chunks this wave computes

  // ---- staging: one (batch, head) slice of K and V^T from block-uniform bases with
  // 32-bit lane offsets (the host checks the slice spans fit); swizzle on the source side
  const E* kblk = (const E*)a.k_hi + ((int64_t)b * a.ks0 + (int64_t)h * a.ks1);
  const E* vblk = (const E*)a.vt_hi + ((int64_t)b * a.vs0 + (int64_t)h * a.vs1);
  const int S8 = (a.S + 7) & ~7;
  const int ks2 = (int)a.ks2, vs2 = (int)a.vs2;
  auto k_src = [&](int i, int k0) KF_INLINE -> int {
    const int p = i * NTH + tid, row = p / CK;
    const int col = min((p % CK) ^ pk_swz<HDP>(row), a.hd / 8 - 1) * 8;
    return min(k0 + row, a.S - 1) * ks2 + col;
  };
  auto v_src = [&](int i, int k0) KF_INLINE -> int {
    const int p = i * NTH + tid, row = p / CV;
    const int col = ((p % CV) ^ pv_swz(row)) * 8;
    return min(row, a.hd - 1) * vs2 + min(k0 + col, S8 - 8);
  };
  // Copies go through buffer resources on the slice bases with byte offsets (dma16_buf: the
  // LDS-read waits stay exact while copies are in flight; the host keeps the slices' byte
  // spans below 2^31). Tiles that end inside S pass the tile-0 offsets and a uniform tile
  // step; only the tail tile recomputes them with the clamps. A uniform branch, not a
  // select, so the common path carries none of the clamp arithmetic.
  const __amdgpu_buffer_rsrc_t krs = buffer_rsrc(kblk), vrs = buffer_rsrc(vblk);
  constexpr int EC = (int)sizeof(E);
  int ko0[NCH], vo0[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    ko0[i] = k_src(i, 0) * EC;
    vo0[i] = v_src(i, 0) * EC;
  }
  const int kstep = BN * ks2 * EC;
  auto issue = [&](int t) KF_INLINE {
    E* dst = smem + (t % STAGES) * STG;
    const int k0 = t * BN;
    if (__builtin_expect(k0 + BN <= a.S, 1)) {
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        dma16_buf(krs, ko0[i], t * kstep, dst + (i * NTH + wave * 64) * 8);
        dma16_buf(vrs, vo0[i], k0 * EC, dst + TILE + (i * NTH + wave * 64) * 8);
      }
    } else {
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        dma16_buf(krs, k_src(i, k0) * EC, 0, dst + (i * NTH + wave * 64) * 8);
        dma16_buf(vrs, v_src(i, k0) * EC, 0, dst + TILE + (i * NTH + wave * 64) * 8);
      }
    }
  };

  const int ntiles = (kend_blk + BN - 1) / BN;
#pragma unroll
  for (int t = 0; t < STAGES - 1; ++t)
    if (t < ntiles) issue(t);

  // ---- query fragments ("B" of S^T = K . Q^T): d 16 ds + 8 hh .. + 7 of query qi,
  // pre-scaled by sm_scale * log2(e)
  V qf[NDS];
  {
    const int64_t qbase = (int64_t)b * a.qs0 + (int64_t)h * a.qs1;
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) {
      const int d = ds * 16 + hh * 8;
      float x[8];
      if (qi < a.S && d < a.hd) {
        ld8<QT>(a.q, qbase + (int64_t)qi * a.qs2 + d, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= a.scale_log2;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = 0.0f;
      }
      round8<E, V>(x, qf[ds]);
    }
  }

  // fragment bases (elements within a stage). K: operand row m = n is key pkey(n) of the
  // chunk; chunk c adds 32 rows (an immediate); the swizzle does not read row bit 5.
  // V^T: rows 32 j + n; d tile j adds 32 rows (an immediate); the swizzle reads bits 1-3.
  static_assert(pk_swz<HDP>(5) == pk_swz<HDP>(5 + 32) && pv_swz(7) == pv_swz(7 + 32),
                "fragment bases assume the swizzles ignore row bit 5");
  int kb[NDS], vb[2][2];
  {
    const int krow = pkey(n);
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) kb[ds] = krow * HDP + (((2 * ds + hh) ^ pk_swz<HDP>(krow)) << 3);
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int st = 0; st < 2; ++st)
        vb[c][st] = TILE + n * BN + (((4 * c + 2 * st + hh) ^ pv_swz(n)) << 3);
  }

  float m_ref = 0.0f, l_i = 0.0f;
  bool m_set = false;
  f32x16 acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = f32x16{};
  // The reference maximum enters the scores as the C operand of a chunk's first S^T
  // MFMA: negm holds -m_ref in all 16 accumulator slots (every one of them belongs to this
  // lane's query), so S^T arrives relative to the reference with no per-chunk
  // initialisation and no extra MFMA. m_ref is kept representable in the 16-bit type
  // (rounded when it moves, clamped to its finite range): scores and rescaling use the
  // same value.
  f32x16 negm = f32x16{};
  constexpr float kRefMax = MODE == MODE_F16 ? 60000.0f : 1.0e30f;

  // Fragment byte offsets carry their stage: kbs for the stage S^T reads K from, vbs for
  // the stage P.V reads V^T from; moving to the next stage adds a block-uniform step.
  constexpr int EB = (int)sizeof(E);
  int kbs[NDS], vbs[2][2];
#pragma unroll
  for (int ds = 0; ds < NDS; ++ds) kbs[ds] = kb[ds] * EB;
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int st = 0; st < 2; ++st) vbs[c][st] = vb[c][st] * EB;
  auto stage_step = [&](int t) KF_INLINE {
    return ((t % STAGES) == STAGES - 1 ? -(STAGES - 1) * STG : STG) * EB;
  };
  const char* sbase = (const char*)smem;

  // S^T of chunk c of the stage kbs points at (koff: a block-uniform byte offset to
  // another stage)
  auto s_chunk = [&](int c, f32x16& s, int koff = 0) KF_INLINE {
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) {
      const V kf = from_u4<V>(*(const U4*)(sbase + kbs[ds] + koff + 32 * c * HDP * EB));
      s = mma32(kf, qf[ds], ds == 0 ? negm : s);
    }
  };
  // P.V with the two 16-key steps of one d tile NJ MFMAs apart
  auto pv_chunk = [&](int c, const V* pf, int voff = 0) KF_INLINE {
#pragma unroll
    for (int ps = 0; ps < 2; ++ps)
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const V vf = from_u4<V>(*(const U4*)(sbase + vbs[c][ps] + voff + 32 * j * BN * EB));
        acc[j] = mma32(vf, pf[ps], acc[j]);
      }
  };
  // The moving step of the lazy reference for a chunk whose scores are x (relative to
  // m_ref): the row maximum mx over the lane pair; rows past the bound (or at their
  // first valid key) take the rounded, clamped maximum as the new reference.
  auto move_ref = [&](float (&x)[16], float mx) KF_INLINE {
    const bool move = mx > kLazy || (!m_set && mx != kNegInf);
    if (__builtin_expect(__any(move), 0)) {
      const float target = fminf(fmaxf(m_ref + mx, -kRefMax), kRefMax);
      const float m_new = move ? (float)(E)target : m_ref;
      const float delta = m_new - m_ref;          // exact: both are 16-bit values
      const float alpha = __builtin_amdgcn_exp2f(-delta);
      m_ref = m_new;
      m_set = m_set || move;
      l_i *= alpha;
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[j] *= alpha;
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] -= delta;
      negm = f32x16{} - m_ref;
    }
  };
  auto row_max = [&](const float (&x)[16]) KF_INLINE {
    float mx = kNegInf;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, x[r]);
    return xmax32(mx);
  };
  auto probs = [&](const float (&x)[16], float (&p)[16], V (&pf)[2]) KF_INLINE {
    float psum = 0.0f;
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        p[8 * ps + e] = __builtin_amdgcn_exp2f(x[8 * ps + e]);
        psum += p[8 * ps + e];
      }
      if constexpr (MODE == MODE_F16) round8<_Float16, V>(&p[8 * ps], pf[ps]);
      else round8<__bf16, V>(&p[8 * ps], pf[ps]);
    }
    return psum;
  };
  // P.V runs one chunk behind the softmax: chunk k's probabilities (`pend`) enter acc
  // during chunk k + 1's step, so a steady step interleaves all of its MFMAs -- S^T of
  // chunk k + 1 and P.V of chunk k - 1, NM of them -- with the exponentials, row sums and
  // packing of chunk k (a 32x32x16 MFMA covers about two exponentials and a few other
  // VALU instructions of its own wavefront). Chunk k - 1's P.V is issued before chunk k's
  // reference can move (the move scales acc), so the additions into acc and its rescales
  // come in the order of the undeferred loop: the results are the same, bit for bit.
  constexpr int NM = NDS + 2 * NJ;            // MFMAs of a steady step
  constexpr int TPM = (16 + NM - 1) / NM;     // exponentials per MFMA
  constexpr int VPM = (28 + NM - 1) / NM;     // other VALU per MFMA
  V pend[2];
  // fragment reads PF MFMAs ahead of their MFMA (two at hd 64: the registers of a third
  // wavefront per SIMD; hd 128 runs two wavefronts per SIMD, its LDS allows no more)
  auto sched_step = [&]() KF_INLINE {
    constexpr int PF = FT::NW >= 8 ? 4 : 2;
    __builtin_amdgcn_sched_group_barrier(0x100, PF, 0);
#pragma unroll
    for (int i = 0; i < NM; ++i) {
      if (i + PF < NM) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x400, TPM, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);
    }
  };
  // Steady chunk k (`cur`, chunk c_cur of its tile): wholly valid, chunk k + 1 computed
  // (`nxt`, chunk c_nxt), every row of the wave has its reference (a wholly valid chunk
  // of the wave came before), and chunk k - 1's P.V pending (chunk c_pend of its tile).
  // The next chunk's S^T and the pending P.V are issued at once among this chunk's
  // exponentials, with no row maximum in front: every p <= 2^kLazy is the common case,
  // and a row sum below 2^kLazy proves it for the lane. Otherwise (rare) the largest p
  // decides; where some score did pass the bound, this chunk's scores are formed again
  // from LDS against the old reference (the same MFMAs, the same values), the reference
  // moves exactly as in the other chunk kinds, and the next chunk's scores are formed again
  // against the moved reference -- the results are those of checking the maximum first.
  // kback: byte offset from the stage kbs points at to this chunk's stage; knxt: offset
  // added to kbs for the next chunk's S^T; voff: offset added to vbs for the pending P.V
  // (zero where kbs / vbs already point at those stages; immediates in the unrolled loop)
  auto chunk_steady = [&](f32x16& cur, int c_cur, f32x16& nxt, int c_nxt, int kback,
                          int knxt, int c_pend, int voff) KF_INLINE {
    constexpr float kTrig = 256.0f;   // 2^kLazy
    static_assert(kLazy == 8.0f, "kTrig is 2^kLazy");
    float x[16], p[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = cur[r];
    s_chunk(c_nxt, nxt, knxt);
    pv_chunk(c_pend, pend, voff);
    V pf[2];
    float psum = probs(x, p, pf);
    sched_step();
    if (__builtin_expect(__any(psum >= kTrig || !m_set), 0)) {
      float pm = 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) pm = fmaxf(pm, p[r]);
      if (__any(pm >= kTrig || !m_set)) {
        f32x16 s;
        s_chunk(c_cur, s, kback);
#pragma unroll
        for (int r = 0; r < 16; ++r) x[r] = s[r];
        move_ref(x, row_max(x));
        s_chunk(c_nxt, nxt, knxt);
        psum = probs(x, p, pf);
      }
    }
    l_i += psum;
    pend[0] = pf[0];
    pend[1] = pf[1];
  };
  // chunk k: (a) chunk k - 1's pending P.V (k > 0); (b) the row maximum and the rare move
  // of the reference; (c) the next chunk's S^T among this chunk's exponentials; the
  // probabilities are left pending. FAST: the chunk is wholly valid and the next one is
  // computed (the first chunk of the fast loop), so (c) is one branch-free block.
  auto chunk = [&](auto fast, int k, f32x16& cur, int c_cur, f32x16& nxt, int c_nxt,
                   int c_pend) KF_INLINE {
    constexpr bool FAST = decltype(fast)::value;
    if (k > 0) pv_chunk(c_pend, pend);
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = cur[r];
    if constexpr (!FAST) {
      const int k0 = k * 32;
      const bool full = k0 + 32 <= kvlen && (!causal || k0 + 31 <= qw0);
      if (!full) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + 16 * (r >> 3) + 8 * hh + (r & 7);
          const bool ok = key < kvlen && (!causal || key <= qi);
          x[r] = ok ? x[r] : kNegInf;
        }
      }
    }
    float mx = kNegInf;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, x[r]);
    mx = xmax32(mx);
    const bool move = mx > kLazy || (!m_set && mx != kNegInf);
    if (__builtin_expect(__any(move), 0)) {
      const float target = fminf(fmaxf(m_ref + mx, -kRefMax), kRefMax);
      const float m_new = move ? (float)(E)target : m_ref;
      const float delta = m_new - m_ref;          // exact: both are 16-bit values
      const float alpha = __builtin_amdgcn_exp2f(-delta);
      m_ref = m_new;
      m_set = m_set || move;
      l_i *= alpha;
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[j] *= alpha;
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] -= delta;
      negm = f32x16{} - m_ref;
    }
    if constexpr (FAST) {
      s_chunk(c_nxt, nxt);
    } else {
      if (k + 1 < nch) s_chunk(c_nxt, nxt);
    }
    float psum = 0.0f;
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pv[e] = __builtin_amdgcn_exp2f(x[8 * ps + e]);
        psum += pv[e];
      }
      if constexpr (MODE == MODE_F16) round8<_Float16, V>(pv, pend[ps]);
      else round8<__bf16, V>(pv, pend[ps]);
    }
    l_i += psum;
    if constexpr (FAST) {
      // K fragment reads PF steps ahead; two exponentials and a few VALU per MFMA
      constexpr int PF = 4;
      __builtin_amdgcn_sched_group_barrier(0x100, PF, 0);
#pragma unroll
      for (int i = 0; i < NDS; ++i) {
        if (i + PF < NDS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x400, 16 / NDS, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
      }
    }
  };

  // Copies complete in issue order: with n later tiles issued, tile t has landed once at
  // most n * 2 * NCH copies are outstanding. Tiles 0 .. STAGES - 2 are issued up front and
  // next_stage(t) issues tile t + STAGES - 1 once tile t + 1 has landed.
  f32x16 sa, sb;
  if (ntiles > 0) {
    wait_tile_landed<STAGES - 2, 2 * NCH>(min(STAGES - 2, ntiles - 1));
    lds_barrier();
    if (nch > 0) s_chunk(0, sa);
  }
  const std::integral_constant<bool, true> kFast;
  const std::integral_constant<bool, false> kSlow;
  // the next stage's copies landed in every wavefront, and stage t - 1 is no longer read;
  // S^T reads move on to stage t + 1
  // (move false: the fragment offsets stay put; the unrolled loop names the stage)
  auto next_stage = [&](int t, bool move = true) KF_INLINE {
    if (t + 1 < ntiles) {
      wait_tile_landed<STAGES - 3, 2 * NCH>(min(STAGES - 3, ntiles - 2 - t));   // tile t + 1
      lds_barrier();
      if (t + STAGES - 1 < ntiles) issue(t + STAGES - 1);
      if (move) {
        const int step = stage_step(t);
#pragma unroll
        for (int ds = 0; ds < NDS; ++ds) kbs[ds] += step;
      }
    }
  };
  // P.V reads move on from tile t to tile t + 1 (called once the even chunk of tile t + 1
  // has issued the pending P.V of tile t's odd chunk)
  auto next_v = [&](int t) KF_INLINE {
    const int step = stage_step(t);
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int st = 0; st < 2; ++st) vbs[c][st] += step;
  };
  // Two loops per wavefront: first the tiles whose chunks 2t, 2t + 1 and 2t + 2 are all
  // computed (2t + 2 < nch: the fast path), then the rest. Each tile passes one barrier in
  // either loop, so every wavefront of the block passes the same number of barriers.
  // (One loop branching between the paths made the allocator keep both paths' registers.)
  // The first chunk of the fast loop checks its row maximum (it sets every row's
  // reference); the rest are steady chunks. A steady chunk that re-forms its scores
  // reads them from stage t: the second chunk of a tile runs after next_stage(t) moved
  // kbs on (always, in the fast loop: tile t + 1 exists). vbs points at the tile of the
  // pending chunk: tile t - 1 in the even chunk of tile t, tile t in the odd one.
  const int t_fast = (nch - 1) / 2 > 0 ? (nch - 1) / 2 : 0;
  int t = 0;
  if (t_fast > 0) {
    chunk(kFast, 0, sa, 0, sb, 1, 0);
    next_stage(0);
    chunk_steady(sb, 1, sa, 0, -stage_step(0), 0, 0, 0);
    t = 1;
  }
  if constexpr (STAGES == 3) {
    // Unrolled over the three stages (tile t = 1 + 3i + j sits in stage (1 + j) % 3):
    // fragment offsets are stage-0 bases plus immediates (the three stages fit the
    // ds_read offset field), so no per-tile offset adds or stage arithmetic.
    if (t == 1 && t + 2 < t_fast) {
      constexpr int SB = STG * EB;       // bytes per stage
      // kbs points at tile 1 (stage 1), vbs at tile 0 (stage 0): both to stage 0
#pragma unroll
      for (int ds = 0; ds < NDS; ++ds) kbs[ds] -= SB;
      auto tile_u = [&](auto st_c, int tt) KF_INLINE {
        constexpr int ST = decltype(st_c)::value, NX = (ST + 1) % 3, PR = (ST + 2) % 3;
        chunk_steady(sa, 0, sb, 1, ST * SB, ST * SB, 1, PR * SB);
        next_stage(tt, false);
        chunk_steady(sb, 1, sa, 0, ST * SB, NX * SB, 0, ST * SB);
      };
      for (; t + 2 < t_fast; t += 3) {
        tile_u(std::integral_constant<int, 1>{}, t);
        tile_u(std::integral_constant<int, 2>{}, t + 1);
        tile_u(std::integral_constant<int, 0>{}, t + 2);
      }
      // t = 1 (mod 3) again: kbs back to tile t's stage (1); vbs stays at stage 0, the
      // stage of tile t - 1, which holds the pending chunk
#pragma unroll
      for (int ds = 0; ds < NDS; ++ds) kbs[ds] += SB;
    }
  }
  for (; t < t_fast; ++t) {
    chunk_steady(sa, 0, sb, 1, 0, 0, 1, 0);
    next_stage(t);
    next_v(t - 1);
    chunk_steady(sb, 1, sa, 0, -stage_step(t), 0, 0, 0);
  }
  // the last chunk's P.V, with vbs at its tile
  auto flush = [&](int c_last) KF_INLINE { pv_chunk(c_last, pend); };
  for (; t < ntiles; ++t) {
    const int k0 = 2 * t;
    if (k0 < nch) chunk(kSlow, k0, sa, 0, sb, 1, 1);
    next_stage(t);
    if (t > 0) next_v(t - 1);
    if (k0 + 1 == nch) flush(0);
    if (k0 + 1 < nch) chunk(kSlow, k0 + 1, sb, 1, sa, 0, 0);
    if (k0 + 2 == nch) flush(1);
  }

  // ---- finalize: the row sum over the lane pair, normalise, store
  if (!wave_active) {
    if (qw0 < a.S) write_zero_rows();
    return;
  }
  const float l = xsum32(l_i);
  const float inv = (skip_pad && qi >= kvlen) ? 0.0f : 1.0f / (l == 0.0f ? 1.0f : l);
  store_rows(acc, inv);
}

// ---------------------------------------------------------------------------------------
// Head dim 64, single-pass fp16 / bf16, prefix masks: two 32-row query tiles per wavefront.
// Tile A holds query rows qw0 .. qw0 + 31, tile B rows qw0 + 32 .. qw0 + 63 (BM = 64 x 4
// wavefronts), so every K and V^T fragment read from LDS feeds the MFMAs of both tiles and
// every K/V copy into LDS serves 256 query rows: half the fragment reads and half the
// global -> LDS copies per flop of flash_pipe_kernel (one tile per wavefront), whose
// fragment reads and copies, not the MFMA or VALU issue rates, set its time at long
// sequences.
//
// The tiles alternate between the MFMA and the VALU. A steady step pair of chunk j:
//   step 1: MFMAs S^T_B(j) and tile A's pending P.V of chunk j - 1; the VALU computes tile
//           A's probabilities of chunk j (from S^T_A(j), formed in the previous step 2);
//   step 2: MFMAs S^T_A(j + 1) and tile B's pending P.V of chunk j - 1; the VALU computes
//           tile B's probabilities of chunk j.
// K(j + 1) is read into the K fragment registers after S^T_B(j) has issued and V^T(j) into
// the V^T registers after tile B's P.V has issued, four MFMAs ahead of their first use.
// Each tile takes the MFMAs and softmax steps of flash_pipe_kernel in the same order -- the
// reference maximum enters through the first S^T MFMA (negm), the lazy reference moves on
// a row's first valid key or beyond kLazy, P.V is added one chunk late and before any move
// of the reference -- so the outputs equal flash_pipe_kernel's bit for bit. A tile's next
// scores are formed after its check, so a move never re-forms them; a steady chunk whose row
// sum reaches 2^kLazy re-forms its own scores from LDS and decides on them (a score above
// kLazy gives a probability above 2^kLazy, so this takes the same moves as checking the
// largest probability first).
//
// Chunks 0 .. F - 1 are wholly valid for both tiles (F from the causal diagonal of tile A
// and kv_len). Chunk 0 is checked for both tiles, then steady step pairs run in passes of
// 2 x STAGES chunks (LDS offsets as ds_read immediates); the remaining chunks -- the rest of
// the wholly valid ones, the diagonal and the padding edge -- run checked, one tile after the
// other, with their fragments read per use. The LDS ring is that of flash_pipe_kernel: tiles
// of 64 keys (two chunks), one barrier per tile, before the odd chunk of each tile.
struct PairTile {
  static constexpr int HDP = 64, BN = 64, NW = 4, NTH = 64 * NW, BM = 64 * NW;
  static constexpr int STAGES = 3;
  static constexpr int STAGE_BYTES = 2 * BN * HDP * 2;
  static_assert(STAGES >= 3, "two tiles in flight while one is computed");
};

template <int MODE, int QT>
__global__ __launch_bounds__(PairTile::NTH) __attribute__((amdgpu_waves_per_eu(2))) void flash_pair_kernel(FlashArgs a) {
  using TR = ModeTraits<MODE>;
  static_assert(!TR::split, "single-pass modes only");
  using V = typename TR::vec;
  using E = typename TR::elem;
  using FT = PairTile;
  constexpr int HDP = FT::HDP, BN = FT::BN, BM = FT::BM, NTH = FT::NTH, STAGES = FT::STAGES;
  constexpr int NDS = HDP / 16;        // 16-wide contraction steps of q . k
  constexpr int NJ = HDP / 32;         // 32-row d tiles of O^T
  constexpr int CK = HDP / 8, CV = BN / 8;
  constexpr int TILE = BN * HDP;
  constexpr int STG = 2 * TILE;        // K then V^T
  constexpr int NCH = TILE / 8 / NTH;
  constexpr int EB = (int)sizeof(E);
  constexpr int SB = STG * EB;         // bytes per stage
  constexpr int PER = 2 * STAGES;      // chunks per pass of the unrolled steady loop
  // sched_barrier mask: VALU, SALU, transcendental and LDS reads may cross, MFMAs may not
  constexpr int kSchedNoMfma = 0x0002 | 0x0004 | 0x0400 | 0x0100;
  static_assert(NCH >= 1 && (TILE / 8) % NTH == 0, "staging must tile the block");
  static_assert(STAGES * SB <= 65536, "fragment offsets fit the ds_read offset field");

  __shared__ __attribute__((aligned(1024))) E smem[STAGES * STG];
  __shared__ int src_off[2 * NCH][NTH];   // this lane's copy source offsets (kept out of registers)

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, hh = lane >> 5;       // query column of a tile, lane half

  const int nqb = (a.S + BM - 1) / BM;
  const bool causal = a.flags & KF_FLASH_CAUSAL;
  const FlashBlock blk = flash_block_map(blockIdx.x, gridDim.x, a.B, a.H, nqb, causal);
  const int b = blk.b, h = blk.h, qb = blk.qb;

  const int kvlen = a.kv_len ? a.kv_len[b] : a.S;
  const bool prefix = a.keep == nullptr || (a.kv_len && a.prefix && a.prefix[b] != 0);
  if (!prefix) return;                 // the general-mask kernel serves this batch row
  const bool skip_pad = (a.flags & KF_FLASH_SKIP_PAD_ROWS) && a.kv_len;

  const int q_lo = qb * BM;
  const int qw0 = q_lo + wave * 64;    // tile A's first query row; tile B's is qw0 + 32
  const int64_t obase = (int64_t)b * a.os0 + (int64_t)h * a.os1;

  // output of query qi: d = 32 j + 8 (r / 4) + 4 hh + r % 4 for register r of o[j]
  auto store_rows = [&](int qi, const f32x16* o, float scale) KF_INLINE {
    if (qi >= a.S) return;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * j + 8 * g + 4 * hh;
        if (d >= a.hd) continue;
        const float v[4] = {o[j][4 * g] * scale, o[j][4 * g + 1] * scale, o[j][4 * g + 2] * scale,
                            o[j][4 * g + 3] * scale};
        store_o4(a, obase + (int64_t)qi * a.os2 + d, v);
      }
  };
  auto write_zero_rows = [&](int qi) KF_INLINE {
    f32x16 z[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) z[j] = f32x16{};
    store_rows(qi, z, 0.0f);
  };
  if (skip_pad && q_lo >= kvlen) {
    write_zero_rows(qw0 + n);
    write_zero_rows(qw0 + 32 + n);
    return;
  }

  const int kend_blk = causal ? min(kvlen, q_lo + BM) : kvlen;
  auto tile_active = [&](int q0) KF_INLINE { return q0 < a.S && !(skip_pad && q0 >= kvlen); };
  const bool actA = tile_active(qw0), actB = tile_active(qw0 + 32);
  const int nchA = actA ? ((causal ? min(kvlen, qw0 + 32) : kvlen) + 31) / 32 : 0;
  const int nchB = actB ? ((causal ? min(kvlen, qw0 + 64) : kvlen) + 31) / 32 : 0;
  // chunks wholly valid for tile A, hence for B (its rows come later); 0 unless both run
  const int F = actB ? (causal ? min(kvlen / 32, qw0 / 32) : kvlen / 32) : 0;

  // ---- staging (as flash_pipe_kernel): one (batch, head) slice of K and V^T from
  // block-uniform bases with 32-bit lane offsets; swizzle on the source side
  const E* kblk = (const E*)a.k_hi + ((int64_t)b * a.ks0 + (int64_t)h * a.ks1);
  const E* vblk = (const E*)a.vt_hi + ((int64_t)b * a.vs0 + (int64_t)h * a.vs1);
  const int S8 = (a.S + 7) & ~7;
  const int ks2 = (int)a.ks2, vs2 = (int)a.vs2;
  auto k_src = [&](int i, int k0) KF_INLINE -> int {
    const int p = i * NTH + tid, row = p / CK;
    const int col = min((p % CK) ^ pk_swz<HDP>(row), a.hd / 8 - 1) * 8;
    return min(k0 + row, a.S - 1) * ks2 + col;
  };
  auto v_src = [&](int i, int k0) KF_INLINE -> int {
    const int p = i * NTH + tid, row = p / CV;
    const int col = ((p % CV) ^ pv_swz(row)) * 8;
    return min(row, a.hd - 1) * vs2 + min(k0 + col, S8 - 8);
  };
  // Copies go through buffer resources on the slice bases (dma16_buf: the LDS-read waits
  // of the loop stay exact while copies are in flight). Tiles that end inside S copy from
  // tile 0's byte offsets plus a uniform step; each lane's offsets wait in LDS (written and
  // read by that lane only) between the copies. Byte offsets stay below 2^31: the host
  // checks S * ks2 and hd * vs2 against it.
  const __amdgpu_buffer_rsrc_t krs = buffer_rsrc(kblk), vrs = buffer_rsrc(vblk);
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    src_off[i][tid] = k_src(i, 0) * EB;
    src_off[NCH + i][tid] = v_src(i, 0) * EB;
  }
  const int kstep = BN * ks2 * EB;
  auto issue = [&](int t) KF_INLINE {
    E* dst = smem + (t % STAGES) * STG;
    const int k0 = t * BN;
    if (__builtin_expect(k0 + BN <= a.S, 1)) {
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        dma16_buf(krs, src_off[i][tid], t * kstep, dst + (i * NTH + wave * 64) * 8);
        dma16_buf(vrs, src_off[NCH + i][tid], k0 * EB, dst + TILE + (i * NTH + wave * 64) * 8);
      }
    } else {
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        dma16_buf(krs, k_src(i, k0) * EB, 0, dst + (i * NTH + wave * 64) * 8);
        dma16_buf(vrs, v_src(i, k0) * EB, 0, dst + TILE + (i * NTH + wave * 64) * 8);
      }
    }
  };

  const int ntiles = (kend_blk + BN - 1) / BN;
#pragma unroll
  for (int t = 0; t < STAGES - 1; ++t)
    if (t < ntiles) issue(t);

  // ---- query fragments of both tiles ("B" of S^T = K . Q^T), pre-scaled by
  // sm_scale * log2(e)
  auto load_q = [&](int qi, V (&qf)[NDS]) KF_INLINE {
    const int64_t qbase = (int64_t)b * a.qs0 + (int64_t)h * a.qs1;
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) {
      const int d = ds * 16 + hh * 8;
      float x[8];
      if (qi < a.S && d < a.hd) {
        ld8<QT>(a.q, qbase + (int64_t)qi * a.qs2 + d, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= a.scale_log2;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = 0.0f;
      }
      round8<E, V>(x, qf[ds]);
    }
  };
  V qfA[NDS], qfB[NDS];
  load_q(qw0 + n, qfA);
  load_q(qw0 + 32 + n, qfB);

  // fragment byte offsets within stage 0 (flash_pipe_kernel's layout): K operand row m = n
  // is key pkey(n) of the chunk, the chunk's parity adds 32 rows; V^T rows 32 j + n
  int kb[NDS], vb[2][2];
  {
    const int krow = pkey(n);
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds)
      kb[ds] = (krow * HDP + (((2 * ds + hh) ^ pk_swz<HDP>(krow)) << 3)) * EB;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int st = 0; st < 2; ++st)
        vb[c][st] = (TILE + n * BN + (((4 * c + 2 * st + hh) ^ pv_swz(n)) << 3)) * EB;
  }
  const char* sbase = (const char*)smem;
  // chunk j's K fragments / V^T fragments (its tile's stage and its parity); a compile-time
  // residue of j makes every offset an immediate
  auto ld_k = [&](V (&kf)[NDS], int j) KF_INLINE {
    const int off = ((j >> 1) % STAGES) * SB + (j & 1) * (32 * HDP * EB);
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) kf[ds] = from_u4<V>(*(const U4*)(sbase + kb[ds] + off));
  };
  auto ld_v = [&](V (&vf)[2][NJ], int j) KF_INLINE {
    // (the parity's bases formed here: a runtime index into vb would put vb in memory)
    const int off = ((j >> 1) % STAGES) * SB;
    const int c = j & 1;
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
      const int base = (TILE + n * BN + (((4 * c + 2 * ps + hh) ^ pv_swz(n)) << 3)) * EB;
#pragma unroll
      for (int jd = 0; jd < NJ; ++jd)
        vf[ps][jd] = from_u4<V>(*(const U4*)(sbase + base + off + jd * (32 * BN * EB)));
    }
  };
  auto ld_k_r = [&](auto rc, V (&kf)[NDS]) KF_INLINE {
    constexpr int R = decltype(rc)::value;
    constexpr int off = ((R >> 1) % STAGES) * SB + (R & 1) * (32 * HDP * EB);
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) kf[ds] = from_u4<V>(*(const U4*)(sbase + kb[ds] + off));
  };
  auto ld_v_r = [&](auto rc, V (&vf)[2][NJ]) KF_INLINE {
    constexpr int R = decltype(rc)::value;
    constexpr int off = ((R >> 1) % STAGES) * SB;
#pragma unroll
    for (int ps = 0; ps < 2; ++ps)
#pragma unroll
      for (int jd = 0; jd < NJ; ++jd)
        vf[ps][jd] = from_u4<V>(*(const U4*)(sbase + vb[R & 1][ps] + off + jd * (32 * BN * EB)));
  };

  // per-tile softmax state (flash_pipe_kernel's, once per tile)
  struct Rows {
    f32x16 acc[NJ];
    f32x16 negm;           // -m_ref in every slot: the C operand of a chunk's first S^T MFMA
                           // (m_ref itself is read back from it: -(0 - m) == m)
    V pend[2];             // probabilities whose P.V is pending
    float l;
    bool m_set;
  };
  Rows tA, tB;
#pragma unroll
  for (int j = 0; j < NJ; ++j) tA.acc[j] = tB.acc[j] = f32x16{};
  tA.negm = tB.negm = f32x16{};
  tA.l = tB.l = 0.0f;
  tA.m_set = tB.m_set = false;
  constexpr float kRefMax = MODE == MODE_F16 ? 60000.0f : 1.0e30f;

  auto s_mma = [&](const V (&kf)[NDS], const V (&qf)[NDS], const f32x16& negm, f32x16& s) KF_INLINE {
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) s = mma32(kf[ds], qf[ds], ds == 0 ? negm : s);
  };
  auto pv_mma = [&](const V (&vf)[2][NJ], Rows& t) KF_INLINE {
#pragma unroll
    for (int ps = 0; ps < 2; ++ps)
#pragma unroll
      for (int jd = 0; jd < NJ; ++jd) t.acc[jd] = mma32(vf[ps][jd], t.pend[ps], t.acc[jd]);
  };
  auto move_ref = [&](Rows& t, float (&x)[16], float mx) KF_INLINE {
    const bool move = mx > kLazy || (!t.m_set && mx != kNegInf);
    if (__builtin_expect(__any(move), 0)) {
      const float m_ref = -t.negm[0];
      const float target = fminf(fmaxf(m_ref + mx, -kRefMax), kRefMax);
      const float m_new = move ? (float)(E)target : m_ref;
      const float delta = m_new - m_ref;          // exact: both are 16-bit values
      const float alpha = __builtin_amdgcn_exp2f(-delta);
      t.m_set = t.m_set || move;
      t.l *= alpha;
#pragma unroll
      for (int j = 0; j < NJ; ++j) t.acc[j] *= alpha;
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] -= delta;
      t.negm = f32x16{} - m_new;
    }
  };
  auto row_max = [&](const float (&x)[16]) KF_INLINE {
    float mx = kNegInf;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, x[r]);
    return xmax32(mx);
  };
  auto probs = [&](const float (&x)[16], V (&pf)[2]) KF_INLINE {
    float psum = 0.0f;
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
      float p[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        p[e] = __builtin_amdgcn_exp2f(x[8 * ps + e]);
        psum += p[e];
      }
      if constexpr (MODE == MODE_F16) round8<_Float16, V>(p, pf[ps]);
      else round8<__bf16, V>(p, pf[ps]);
    }
    return psum;
  };
  // A checked chunk j of a tile whose first row is q0 (scores in s, its pending P.V
  // already added): the mask where the chunk is not wholly valid, the row maximum and the
  // move of the reference, then the probabilities become the pending ones.
  auto checked = [&](Rows& t, const f32x16& s, int j, int q0) KF_INLINE {
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = s[r];
    const int k0 = j * 32;
    const bool full = k0 + 32 <= kvlen && (!causal || k0 + 31 <= q0);
    if (!full) {
      const int qi = q0 + n;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + 16 * (r >> 3) + 8 * hh + (r & 7);
        const bool ok = key < kvlen && (!causal || key <= qi);
        x[r] = ok ? x[r] : kNegInf;
      }
    }
    move_ref(t, x, row_max(x));
    t.l += probs(x, t.pend);
  };
  // A steady chunk (wholly valid, every row's reference set): probabilities first; where a
  // row sum reaches 2^kLazy, the chunk's scores are formed again (into s, whose scores the
  // probabilities have consumed) from its K fragments in LDS (byte offset koff; the same
  // MFMAs, the same values) and checked.
  constexpr float kTrig = 256.0f;     // 2^kLazy
  static_assert(kLazy == 8.0f, "kTrig is 2^kLazy");
  auto steady_rare = [&](Rows& t, const V (&qf)[NDS], int koff, f32x16& s, float& psum, V (&pf)[2]) KF_INLINE {
    // the packing stays in this step (otherwise sunk past the branch, where the next step's
    // P.V MFMAs would wait for it)
    asm volatile("" :: "v"(pf[0]), "v"(pf[1]));
    if (__builtin_expect(__any(psum >= kTrig || !t.m_set), 0)) {
#pragma unroll
      for (int ds = 0; ds < NDS; ++ds) {
        const V k1 = from_u4<V>(*(const U4*)(sbase + kb[ds] + koff));
        s = mma32(k1, qf[ds], ds == 0 ? t.negm : s);
      }
      float x[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] = s[r];
      move_ref(t, x, row_max(x));
      psum = probs(x, pf);
    }
  };

  // the next stage's copies landed in every wavefront and stage t - 1 is no longer read
  // (the barrier before chunk 2t + 1)
  auto next_stage = [&](int t) KF_INLINE {
    if (t + 1 < ntiles) {
      wait_tile_landed<STAGES - 3, 2 * NCH>(min(STAGES - 3, ntiles - 2 - t));   // tile t + 1
      lds_barrier();
      if (t + STAGES - 1 < ntiles) issue(t + STAGES - 1);
    }
  };

  f32x16 sA, sB;
  V kf[NDS], vf[2][NJ];
  if (ntiles > 0) {
    wait_tile_landed<STAGES - 2, 2 * NCH>(min(STAGES - 2, ntiles - 1));
    lds_barrier();
  }

  // Steady step pair of chunk j (residue R = j mod PER, a compile-time constant): kf holds
  // K(j), vf V^T(j - 1), sA S^T_A(j); tile A has no P.V pending, tile B that of chunk j - 1.
  auto pair_step = [&](auto rc, int j) KF_INLINE {
    constexpr int R = decltype(rc)::value;
    constexpr int KOFF = ((R >> 1) % STAGES) * SB + (R & 1) * (32 * HDP * EB);
    if constexpr (R & 1) next_stage(j >> 1);
    // step 1: S^T_B(j) and tile B's P.V of chunk j - 1; tile A's probabilities of chunk j.
    // K(j + 1) and V^T(j) are read into kf / vf once their MFMAs have issued.
    s_mma(kf, qfB, tB.negm, sB);
    ld_k_r(std::integral_constant<int, R + 1>{}, kf);
    __builtin_amdgcn_sched_barrier(kSchedNoMfma);      // S^T MFMAs first, then P.V
    pv_mma(vf, tB);
    ld_v_r(rc, vf);
    V pf[2];
    float psum;
    {
      float x[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] = sA[r];
      psum = probs(x, pf);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i == 4) __builtin_amdgcn_sched_group_barrier(0x100, NDS, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x400, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * NJ, 0);
    steady_rare(tA, qfA, KOFF, sA, psum, pf);
    tA.l += psum;
    tA.pend[0] = pf[0];
    tA.pend[1] = pf[1];
    // step 2: S^T_A(j + 1) and tile A's P.V of chunk j; tile B's probabilities of chunk j
    s_mma(kf, qfA, tA.negm, sA);
    __builtin_amdgcn_sched_barrier(kSchedNoMfma);      // K(j + 1) landed first, V^T(j) later
    pv_mma(vf, tA);
    {
      float x[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] = sB[r];
      psum = probs(x, pf);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x400, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
    }
    steady_rare(tB, qfB, KOFF, sB, psum, pf);
    tB.l += psum;
    tB.pend[0] = pf[0];
    tB.pend[1] = pf[1];
  };

  int c0 = 0;              // first chunk of the checked loop
  bool sa_ready = false;   // sA holds S^T_A(c0)
  bool pendA = false, pendB = false;   // a tile's P.V of chunk c0 - 1 is pending
  if (F >= 2) {
    // chunk 0, both tiles checked (it sets every row's reference), and tile A's P.V of it:
    // the state a steady step pair of chunk 1 starts from
    ld_k(kf, 0);
    s_mma(kf, qfA, tA.negm, sA);
    s_mma(kf, qfB, tB.negm, sB);
    ld_k(kf, 1);
    checked(tA, sA, 0, qw0);
    s_mma(kf, qfA, tA.negm, sA);
    ld_v(vf, 0);
    pv_mma(vf, tA);
    checked(tB, sB, 0, qw0 + 32);
    // steady step pairs of chunks 1 .. nit, whole passes of PER chunks (chunk j + U - 1 of a
    // pass has residue U)
    auto pass = [&](auto self, auto uc, int j) KF_INLINE {
      constexpr int U = decltype(uc)::value;
      if constexpr (U <= PER) {
        pair_step(std::integral_constant<int, U>{}, j + U - 1);
        self(self, std::integral_constant<int, U + 1>{}, j);
      }
    };
    const int nit = ((F - 2) / PER) * PER;
    for (int j = 1; j <= nit; j += PER) pass(pass, std::integral_constant<int, 1>{}, j);
    c0 = nit + 1;
    sa_ready = true;
    pendB = true;
  }

  // checked chunks c0 .. : each tile adds its pending P.V, forms and checks its scores, and
  // adds its last chunk's P.V at once; fragments are read per use
  const int nch = max(nchA, nchB);
  auto checked_tile = [&](Rows& t, const V (&qf)[NDS], int c, int q0, int nch_t, bool use_sa,
                          bool pending) KF_INLINE {
    V kt[NDS], vt[2][NJ];
    if (pending) {
      ld_v(vt, c - 1);
      pv_mma(vt, t);
    }
    f32x16 s;
    if (use_sa) {
      s = sA;
    } else {
      ld_k(kt, c);
      s_mma(kt, qf, t.negm, s);
    }
    checked(t, s, c, q0);
    if (c == nch_t - 1) {
      ld_v(vt, c);
      pv_mma(vt, t);
    }
  };
  int c = c0;
  for (; c < nch; ++c) {
    if (c & 1) next_stage(c >> 1);
    if (c < nchA) checked_tile(tA, qfA, c, qw0, nchA, sa_ready && c == c0, c > c0 || pendA);
    if (c < nchB) checked_tile(tB, qfB, c, qw0 + 32, nchB, false, c > c0 || pendB);
  }
  // every wavefront passes the block's remaining barriers
  for (; c < 2 * ntiles; ++c)
    if (c & 1) next_stage(c >> 1);

  // ---- finalize: the row sum over the lane pair, normalise, store
  auto finish = [&](Rows& t, int q0, bool act) KF_INLINE {
    const int qi = q0 + n;
    if (!act) {
      if (q0 < a.S) write_zero_rows(qi);
      return;
    }
    const float l = xsum32(t.l);
    const float inv = (skip_pad && qi >= kvlen) ? 0.0f : 1.0f / (l == 0.0f ? 1.0f : l);
    store_rows(qi, t.acc, inv);
  };
  finish(tA, qw0, actA);
  finish(tB, qw0 + 32, actB);
}

// ---------------------------------------------------------------------------------------
// Head dim 8 in the split modes (f16x3 / bf16x3; P as hi + lo planes, or with
// KF_FLASH_P16 one rounded plane), pipelined on the 32x32x16 MFMA like flash_pipe_kernel,
// with the split products packed into the contraction instead of zero padding it:
//   S^T = K . Q^T in two 16-slot steps, [k_hi | k_hi] . [q_hi | q_lo] then
//         [k_lo | e0] . [q_hi | -m_ref e0]  (e0 = (1, 0, ..., 0)),
// i.e. k_hi q_hi + k_hi q_lo + k_lo q_hi relative to the lazy reference, two MFMAs per 32
// keys x 32 queries where the 16x16x32 kernel pads 8 to 32 and issues six; and
//   O^T = [V^T_hi; V^T_lo; 1; 0] . (P_hi + P_lo)
// whose rows 0-7 and 8-15 add to the output and whose row 16 is the softmax row sum, so
// the row sum costs no VALU. One wavefront holds 32 query rows (lane pair (l, l ^ 32) per
// query, as in flash_pipe_kernel).
//
// LDS stage (16-bit elements): K_hi [64 keys][8] | K_lo [64][8] | V^T_hi [8][64 keys] |
// pad | V^T_lo [8][64] | e0, ones, zeros (8 each, written once, never copied over). V^T
// rows hold their eight 16-byte key chunks XOR-swizzled by the row (chunk j at j ^ row),
// and the 128-byte pad puts row r of V^T_lo in the other half of the 256-byte bank period
// from row r of V^T_hi, so the 16 rows one ds_read_b128 phase reads hit 16 distinct bank
// slots. Each wavefront copies one plane per stage (K_hi, K_lo, V^T_hi, V^T_lo).
struct SmallTile {
  static constexpr int HD = 8, BN = 64, NW = 4, NTH = 64 * NW, BM = 32 * NW, STAGES = 3;
  static constexpr int KH = 0, KL = 512, VH = 1024, VL = VH + 512 + 64, CST = VL + 512;
  static constexpr int STG = 2176;                    // elements per stage (4352 bytes)
  static constexpr int STAGE_BYTES = STG * 2;
  static_assert(STG >= CST + 24 && STG % 64 == 0, "stage layout");
  static_assert(BM == FlashTile<32, 2>::BM, "one grid for both mask instantiations");
};

template <int MODE, int QT, int VAR>
__global__ __launch_bounds__(SmallTile::NTH) void flash_small_kernel(FlashArgs a) {
  using TR = ModeTraits<MODE>;
  static_assert(TR::split, "split modes only");
  static_assert(VAR == kVarNone || (VAR == kVarP16 && MODE == MODE_F16X3), "variant");
  using V = typename TR::vec;
  using E = typename TR::elem;
  using ST = SmallTile;
  constexpr int BN = ST::BN, BM = ST::BM, STAGES = ST::STAGES, STG = ST::STG;
  constexpr bool P16 = VAR == kVarP16;
  constexpr int EB = (int)sizeof(E);

  __shared__ __attribute__((aligned(1024))) E smem[STAGES * STG];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, hh = lane >> 5;

  const int nqb = (a.S + BM - 1) / BM;
  const bool causal = a.flags & KF_FLASH_CAUSAL;
  const FlashBlock blk = flash_block_map(blockIdx.x, gridDim.x, a.B, a.H, nqb, causal);
  const int b = blk.b, h = blk.h, qb = blk.qb;

  const int kvlen = a.kv_len ? a.kv_len[b] : a.S;
  const bool prefix = a.keep == nullptr || (a.kv_len && a.prefix && a.prefix[b] != 0);
  if (!prefix) return;                 // the general-mask kernel serves this batch row
  const bool skip_pad = (a.flags & KF_FLASH_SKIP_PAD_ROWS) && a.kv_len;

  const int q_lo = qb * BM;
  const int qw0 = q_lo + wave * 32;
  const int qi = qw0 + n;
  const int64_t obase = (int64_t)b * a.os0 + (int64_t)h * a.os1;
  // output of this lane: query qi, d = 4 hh .. 4 hh + 3
  auto store_out = [&](const float* v4) KF_INLINE {
    if (qi < a.S) store_o4(a, obase + (int64_t)qi * a.os2 + 4 * hh, v4);
  };
  if (skip_pad && q_lo >= kvlen) {
    const float z[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    store_out(z);
    return;
  }

  const int kend_blk = causal ? min(kvlen, q_lo + BM) : kvlen;
  const int kend_w = causal ? min(kvlen, qw0 + 32) : kvlen;
  const bool wave_active = qw0 < a.S && !(skip_pad && qw0 >= kvlen);
  const int nch = wave_active ? (kend_w + 31) / 32 : 0;

  // ---- staging: wavefront w copies plane w of each stage (K_hi, K_lo, V^T_hi, V^T_lo)
  // from a block-uniform slice base with a 32-bit lane offset (the host checks the slice
  // spans fit); the V^T swizzle is applied on the source side
  const bool wk = wave < 2;
  const E* src = (const E*)(wave == 0 ? a.k_hi : wave == 1 ? a.k_lo : wave == 2 ? a.vt_hi : a.vt_lo) +
                 (wk ? (int64_t)b * a.ks0 + (int64_t)h * a.ks1 : (int64_t)b * a.vs0 + (int64_t)h * a.vs1);
  const int dst_off = wave == 0 ? ST::KH : wave == 1 ? ST::KL : wave == 2 ? ST::VH : ST::VL;
  const int S8 = (a.S + 7) & ~7;
  const int ks2 = (int)a.ks2, vs2 = (int)a.vs2;
  const int vr = lane >> 3, vj = (lane & 7) ^ vr;     // V^T row, logical chunk of this copy
  const int off0 = wk ? lane * ks2 : vr * vs2 + 8 * vj;
  const int tstep = wk ? BN * ks2 : BN;
  auto issue = [&](int t) KF_INLINE {
    E* dst = smem + (t % STAGES) * STG + dst_off;
    const int k0 = t * BN;
    if (__builtin_expect(k0 + BN <= a.S, 1)) {
      dma16(src + t * tstep + off0, dst);
    } else {
      const int o = wk ? min(k0 + lane, a.S - 1) * ks2 : vr * vs2 + min(k0 + 8 * vj, S8 - 8);
      dma16(src + o, dst);
    }
  };

  const int ntiles = (kend_blk + BN - 1) / BN;
#pragma unroll
  for (int t = 0; t < STAGES - 1; ++t)
    if (t < ntiles) issue(t);
  // constant blocks of every stage (visible after the first barrier, which waits lgkmcnt)
  if (tid < STAGES * 24) {
    const int s = tid / 24, e = tid % 24;
    smem[s * STG + ST::CST + e] = (E)((e == 0 || (e >= 8 && e < 16)) ? 1.0f : 0.0f);
  }

  // ---- query fragments ("B" of S^T): step 0 q_hi | q_lo, step 1 q_hi | -m_ref e0, of query
  // qi pre-scaled by sm_scale * log2(e) and split hi + lo
  V qf0, qf1;
  {
    float x[8];
    if (qi < a.S) {
      ld8<QT>(a.q, (int64_t)b * a.qs0 + (int64_t)h * a.qs1 + (int64_t)qi * a.qs2, x);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] *= a.scale_log2;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = 0.0f;
    }
    V qh, ql;
    split8<E, V>(x, qh, ql);
    qf0 = hh ? ql : qh;
    qf1 = hh ? V{} : qh;
  }

  // ---- fragment byte offsets within a stage. K: operand row m = n is key pkey(n) of the
  // chunk; chunk c adds 32 rows (an immediate) to the K_hi read; the K_lo | e0 read has a
  // base per chunk (the e0 lanes stay on the constant). V^T: operand row n is V^T_hi row n
  // (n < 8), V^T_lo row n - 8 (n < 16), ones (16) or zeros, key chunk 4 c + 2 ps + hh.
  int kb0, kb1[2], vb[2][2];
  {
    const int krow = pkey(n);
    kb0 = (ST::KH + krow * 8) * EB;
#pragma unroll
    for (int c = 0; c < 2; ++c) kb1[c] = (hh ? ST::CST : ST::KL + (krow + 32 * c) * 8) * EB;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int ps = 0; ps < 2; ++ps) {
        const int j = 4 * c + 2 * ps + hh;
        int e;
        if (n < 8) e = ST::VH + n * BN + ((j ^ n) << 3);
        else if (n < 16) e = ST::VL + (n - 8) * BN + ((j ^ (n - 8)) << 3);
        else e = ST::CST + (n == 16 ? 8 : 16);
        vb[c][ps] = e * EB;
      }
  }
  auto stage_step = [&](int t) KF_INLINE {
    return ((t % STAGES) == STAGES - 1 ? -(STAGES - 1) * STG : STG) * EB;
  };
  const char* sbase = (const char*)smem;

  float m_ref = 0.0f;
  bool m_set = false;
  f32x16 acc = f32x16{};               // rows 0-7 V_hi.P, 8-15 V_lo.P, 16 the row sum
  constexpr float kRefMax = MODE == MODE_F16X3 ? 60000.0f : 1.0e30f;

  auto s_chunk = [&](int c, f32x16& s, int koff = 0) KF_INLINE {
    const V k0f = from_u4<V>(*(const U4*)(sbase + kb0 + koff + 32 * c * 8 * EB));
    const V k1f = from_u4<V>(*(const U4*)(sbase + kb1[c] + koff));
    s = mma32(k0f, qf0, f32x16{});
    s = mma32(k1f, qf1, s);
  };
  auto pv_chunk = [&](int c, const V* ph, const V* pl, int voff = 0) KF_INLINE {
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
      const V vf = from_u4<V>(*(const U4*)(sbase + vb[c][ps] + voff));
      acc = mma32(vf, ph[ps], acc);
      if constexpr (!P16) acc = mma32(vf, pl[ps], acc);
    }
  };
  auto probs = [&](const float (&x)[16], V (&ph)[2], V (&pl)[2]) KF_INLINE {
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
      float p[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) p[e] = __builtin_amdgcn_exp2f(x[8 * ps + e]);
      if constexpr (P16) round8<_Float16, V>(p, ph[ps]);
      else p_operand<MODE, V>(p, ph[ps], pl[ps]);
    }
  };
  auto row_max = [&](const float (&x)[16]) KF_INLINE {
    float mx = kNegInf;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, x[r]);
    return xmax32(mx);
  };
  auto move_ref = [&](float (&x)[16], float mx) KF_INLINE {
    const bool move = mx > kLazy || (!m_set && mx != kNegInf);
    if (__builtin_expect(__any(move), 0)) {
      const float target = fminf(fmaxf(m_ref + mx, -kRefMax), kRefMax);
      const float m_new = move ? (float)(E)target : m_ref;
      const float delta = m_new - m_ref;          // exact: both are 16-bit values
      const float alpha = __builtin_amdgcn_exp2f(-delta);
      m_ref = m_new;
      m_set = m_set || move;
      acc *= alpha;
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] -= delta;
      if (hh) qf1[0] = (E)(-m_ref);
    }
  };
  // first or masked chunk k: row maximum (and masks) first, then the next chunk's S^T
  auto chunk = [&](auto fast, int k, f32x16& cur, int c_cur, f32x16& nxt, int c_nxt) KF_INLINE {
    constexpr bool FAST = decltype(fast)::value;
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = cur[r];
    if constexpr (!FAST) {
      const int k0 = k * 32;
      const bool full = k0 + 32 <= kvlen && (!causal || k0 + 31 <= qw0);
      if (!full) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + 16 * (r >> 3) + 8 * hh + (r & 7);
          const bool ok = key < kvlen && (!causal || key <= qi);
          x[r] = ok ? x[r] : kNegInf;
        }
      }
    }
    move_ref(x, row_max(x));
    if constexpr (FAST) {
      s_chunk(c_nxt, nxt);
    } else {
      if (k + 1 < nch) s_chunk(c_nxt, nxt);
    }
    V ph[2], pl[2];
    probs(x, ph, pl);
    pv_chunk(c_cur, ph, pl);
  };
  // steady chunk (wholly valid, the next one computed, every row's reference set): the
  // next chunk's S^T at once among this chunk's exponentials; the largest p decides
  // whether some score passed the lazy bound, and only then are this chunk's scores
  // formed again from LDS against the old reference (the same MFMAs, the same values),
  // the reference moved, and the next chunk's scores formed again against it -- the
  // results of checking the maximum first (flash_pipe_kernel's steady chunks).
  // (kback, knxt, voff: as in flash_pipe_kernel's steady chunks)
  auto chunk_steady = [&](f32x16& cur, int c_cur, f32x16& nxt, int c_nxt, int kback,
                          int knxt = 0, int voff = 0) KF_INLINE {
    constexpr float kTrig = 256.0f;   // 2^kLazy
    static_assert(kLazy == 8.0f, "kTrig is 2^kLazy");
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = cur[r];
    s_chunk(c_nxt, nxt, knxt);
    V ph[2], pl[2];
    float pm = 0.0f;
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
      float p[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        p[e] = __builtin_amdgcn_exp2f(x[8 * ps + e]);
        pm = fmaxf(pm, p[e]);
      }
      if constexpr (P16) round8<_Float16, V>(p, ph[ps]);
      else p_operand<MODE, V>(p, ph[ps], pl[ps]);
    }
    if (__builtin_expect(__any(pm >= kTrig || !m_set), 0)) {
      f32x16 s;
      s_chunk(c_cur, s, kback);
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] = s[r];
      move_ref(x, row_max(x));
      s_chunk(c_nxt, nxt, knxt);
      probs(x, ph, pl);
    }
    pv_chunk(c_cur, ph, pl, voff);
  };

  // Copies complete in issue order, one per wavefront per tile: with n later tiles
  // issued, tile t has landed once at most n copies are outstanding.
  static_assert(STAGES == 3, "the waits below are written for 3 stages");
  f32x16 sa, sb;
  if (ntiles > 0) {
    if (ntiles > 1) wait_vmcnt<1>();
    else wait_vmcnt<0>();
    lds_barrier();
    if (nch > 0) s_chunk(0, sa);
  }
  const std::integral_constant<bool, true> kFast;
  const std::integral_constant<bool, false> kSlow;
  auto next_stage = [&](int t, bool move = true) KF_INLINE {
    if (t + 1 < ntiles) {
      wait_vmcnt<0>();
      lds_barrier();
      if (t + STAGES - 1 < ntiles) issue(t + STAGES - 1);
      if (move) {
        const int step = stage_step(t);
        kb0 += step;
        kb1[0] += step;
        kb1[1] += step;
      }
    }
  };
  auto next_v = [&](int t) KF_INLINE {
    const int step = stage_step(t);
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int ps = 0; ps < 2; ++ps) vb[c][ps] += step;
  };
  // the loops of flash_pipe_kernel: tiles whose chunks 2t, 2t + 1, 2t + 2 are all computed
  // (the first of them checks its maximum, the rest are steady), then the masked rest;
  // every wavefront passes one barrier per tile
  const int t_fast = (nch - 1) / 2 > 0 ? (nch - 1) / 2 : 0;
  int t = 0;
  if (t_fast > 0) {
    chunk(kFast, 0, sa, 0, sb, 1);
    next_stage(0);
    chunk_steady(sb, 1, sa, 0, -stage_step(0));
    next_v(0);
    t = 1;
  }
  {
    // unrolled over the three stages, offsets as immediates (flash_pipe_kernel's loop)
    if (t == 1 && t + 2 < t_fast) {
      constexpr int SB = STG * EB;       // bytes per stage
      kb0 -= SB;
      kb1[0] -= SB;
      kb1[1] -= SB;
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int ps = 0; ps < 2; ++ps) vb[c][ps] -= SB;
      auto tile_u = [&](auto st_c, int tt) KF_INLINE {
        constexpr int S0 = decltype(st_c)::value, NX = (S0 + 1) % 3;
        chunk_steady(sa, 0, sb, 1, S0 * SB, S0 * SB, S0 * SB);
        next_stage(tt, false);
        chunk_steady(sb, 1, sa, 0, S0 * SB, NX * SB, S0 * SB);
      };
      for (; t + 2 < t_fast; t += 3) {
        tile_u(std::integral_constant<int, 1>{}, t);
        tile_u(std::integral_constant<int, 2>{}, t + 1);
        tile_u(std::integral_constant<int, 0>{}, t + 2);
      }
      kb0 += SB;
      kb1[0] += SB;
      kb1[1] += SB;
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int ps = 0; ps < 2; ++ps) vb[c][ps] += SB;
    }
  }
  for (; t < t_fast; ++t) {
    chunk_steady(sa, 0, sb, 1, 0);
    next_stage(t);
    chunk_steady(sb, 1, sa, 0, -stage_step(t));
    next_v(t);
  }
  for (; t < ntiles; ++t) {
    if (2 * t < nch) chunk(kSlow, 2 * t, sa, 0, sb, 1);
    next_stage(t);
    if (2 * t + 1 < nch) chunk(kSlow, 2 * t + 1, sb, 1, sa, 0);
    next_v(t);
  }

  // ---- finalize: row sum from accumulator row 16 (lane n, register 8; zero on the
  // partner lane), V_hi.P + V_lo.P, normalise, store
  if (!wave_active) {
    if (qw0 < a.S) {
      const float z[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      store_out(z);
    }
    return;
  }
  const float l = xsum32(acc[8]);
  const float inv = (skip_pad && qi >= kvlen) ? 0.0f : 1.0f / (l == 0.0f ? 1.0f : l);
  const float o4[4] = {(acc[0] + acc[4]) * inv, (acc[1] + acc[5]) * inv, (acc[2] + acc[6]) * inv,
                       (acc[3] + acc[7]) * inv};
  store_out(o4);
}

template <int MODE, int QT, int HDP>
static void launch_flash(const FlashArgs& a, hipStream_t st) {
  using FT = FlashTile<HDP, ModeTraits<MODE>::split ? 2 : 1>;
  using FTG = FlashTile<HDP, ModeTraits<MODE>::split ? 2 : 1, true>;   // general-mask launch
  const int nqb = (a.S + FT::BM - 1) / FT::BM;
  const int64_t blocks = (int64_t)nqb * a.B * a.H;
  const bool any_prefix = a.keep == nullptr || (a.kv_len && a.prefix);
  const bool any_general = a.keep != nullptr;
  if constexpr (HDP == 32 && ModeTraits<MODE>::split) {
    // head_dim 8 in the split modes: the packed-contraction kernel for prefix-mask rows
    // (32-bit slice offsets, as the pipelined kernel), unless KF_FLASH_NO_PIPE
    const bool fits = (int64_t)a.S * a.ks2 < (1LL << 31) && (int64_t)a.hd * a.vs2 < (1LL << 31);
    if (a.hd == SmallTile::HD && fits && !(a.flags & KF_FLASH_NO_PIPE)) {
      if constexpr (MODE == MODE_F16X3) {
        if (a.flags & KF_FLASH_P16) {
          if (any_prefix)
            hipLaunchKernelGGL((flash_small_kernel<MODE, QT, kVarP16>), dim3((unsigned)blocks),
                               dim3(SmallTile::NTH), 0, st, a);
          if (any_general)
            hipLaunchKernelGGL((flash_fwd_kernel<MODE, QT, HDP, true, kVarP16>), dim3((unsigned)blocks), dim3(FTG::NTH), 0, st, a);
          return;
        }
      }
      if (any_prefix)
        hipLaunchKernelGGL((flash_small_kernel<MODE, QT, kVarNone>), dim3((unsigned)blocks),
                           dim3(SmallTile::NTH), 0, st, a);
      if (any_general)
        hipLaunchKernelGGL((flash_fwd_kernel<MODE, QT, HDP, true>), dim3((unsigned)blocks), dim3(FTG::NTH), 0, st, a);
      return;
    }
  }
  if constexpr (MODE == MODE_F16X3) {
    if (a.flags & KF_FLASH_P16) {
      if (any_prefix)
        hipLaunchKernelGGL((flash_fwd_kernel<MODE, QT, HDP, false, kVarP16>), dim3((unsigned)blocks), dim3(FT::NTH), 0, st, a);
      if (any_general)
        hipLaunchKernelGGL((flash_fwd_kernel<MODE, QT, HDP, true, kVarP16>), dim3((unsigned)blocks), dim3(FTG::NTH), 0, st, a);
      return;
    }
  }
  if constexpr (MODE == MODE_F16 || MODE == MODE_BF16) {
    if (a.flags & KF_FLASH_ROUND_SCORES) {
      if (any_prefix)
        hipLaunchKernelGGL((flash_fwd_kernel<MODE, QT, HDP, false, kVarRoundScores>), dim3((unsigned)blocks), dim3(FT::NTH), 0, st, a);
      if (any_general)
        hipLaunchKernelGGL((flash_fwd_kernel<MODE, QT, HDP, true, kVarRoundScores>), dim3((unsigned)blocks), dim3(FTG::NTH), 0, st, a);
      return;
    }
  }
  if constexpr ((MODE == MODE_F16 || MODE == MODE_BF16) && (HDP == 64 || HDP == 128)) {
    // the pipelined kernels copy from one (batch, head) slice of K and V^T with 32-bit byte
    // offsets
    const bool fits = (int64_t)a.S * a.ks2 * 2 < (1LL << 31) && (int64_t)a.hd * a.vs2 * 2 < (1LL << 31);
    const int64_t pipe_blocks = (int64_t)((a.S + PipeTile<HDP>::BM - 1) / PipeTile<HDP>::BM) * a.B * a.H;
    const int64_t pair_blocks = (int64_t)((a.S + PairTile::BM - 1) / PairTile::BM) * a.B * a.H;
    const bool pair = HDP == 64 && !(a.flags & KF_FLASH_ONE_TILE);
    if (any_prefix && fits && !(a.flags & KF_FLASH_NO_PIPE)) {
      if (pair)
        hipLaunchKernelGGL((flash_pair_kernel<MODE, QT>), dim3((unsigned)pair_blocks),
                           dim3(PairTile::NTH), 0, st, a);
      else
        hipLaunchKernelGGL((flash_pipe_kernel<MODE, QT, HDP>), dim3((unsigned)pipe_blocks),
                           dim3(PipeTile<HDP>::NTH), 0, st, a);
    } else if (any_prefix)
      hipLaunchKernelGGL((flash_fwd_kernel<MODE, QT, HDP, false>), dim3((unsigned)blocks), dim3(FT::NTH), 0, st, a);
  } else {
    if (any_prefix)
      hipLaunchKernelGGL((flash_fwd_kernel<MODE, QT, HDP, false>), dim3((unsigned)blocks), dim3(FT::NTH), 0, st, a);
  }
  if (any_general)
    hipLaunchKernelGGL((flash_fwd_kernel<MODE, QT, HDP, true>), dim3((unsigned)blocks), dim3(FTG::NTH), 0, st, a);
}

template <int MODE, int QT>
static void launch_hd(const FlashArgs& a, int hdp, hipStream_t st) {
  switch (hdp) {
    case 32: launch_flash<MODE, QT, 32>(a, st); break;
    case 64: launch_flash<MODE, QT, 64>(a, st); break;
    case 128: launch_flash<MODE, QT, 128>(a, st); break;
    default: launch_flash<MODE, QT, 256>(a, st); break;
  }
}

template <int MODE>
static void launch_q(const FlashArgs& a, int q_dtype, int hdp, hipStream_t st) {
  switch (q_dtype) {
    case KF_F32: launch_hd<MODE, KF_F32>(a, hdp, st); break;
    case KF_F16: launch_hd<MODE, KF_F16>(a, hdp, st); break;
    default: launch_hd<MODE, KF_BF16>(a, hdp, st); break;
  }
}

void flash_launch_f16(const FlashArgs& a, int q_dtype, int hdp, hipStream_t st);
void flash_launch_bf16(const FlashArgs& a, int q_dtype, int hdp, hipStream_t st);
void flash_launch_f16x3(const FlashArgs& a, int q_dtype, int hdp, hipStream_t st);
void flash_launch_bf16x3(const FlashArgs& a, int q_dtype, int hdp, hipStream_t st);

}  // namespace kf
