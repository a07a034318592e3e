// FlashAttention forward for gfx950 with causal and key-padding masks in registers.
//
// Semantics of kernelforge/ops/flash.py:42-249: for each (batch, head) and query row,
// softmax over keys of (q . k) * sm_scale with -inf on masked keys (key > query under the
// causal mask, keep[b, key] == 0 under the padding mask), online in fp32 with exp2 and the
// two NaN guards (an all-masked block rescales against 0; a row with no valid key emits 0),
// then P (cast to the MFMA input format) times V.
//
// Data flow per 256-thread block (4 wavefronts, 16 * QG query rows each, BM = 64 * QG):
//  * K and V tiles of BN keys are staged through double-buffered LDS: K as [key][d]
//    (d contiguous), V transposed to [d][key] while it is written, so that both MFMA
//    operands read 16 contiguous bytes per lane. fp32 inputs are split (or rounded) to the
//    16-bit MFMA format once, while they are staged.
//  * Scores are formed transposed, S^T = K . Q^T (v_mfma_f32_16x16x32): K rows are the
//    MFMA "A" operand and a lane's query fragment is the "B" operand. The two 16-key S^T
//    tiles of a 32-key chunk use permuted K rows (tile t, row p -> key (p/4)*8 + 4t + p%4),
//    so lane (r, g) ends with the 8 consecutive keys 8g..8g+7 of query r -- exactly the
//    "B" operand layout of P^T in O^T = V^T . P^T. Softmax statistics and the output
//    accumulator of a query therefore live in the same lane; only the row maximum crosses
//    lanes (two xor-shuffles over the four 16-lane groups), the row sum is reduced once at
//    the end.
//  * Blocks past the last valid key are skipped (kv_len from kf_mask_prep): masked keys
//    contribute p = 0 and alpha = 1 there, so skipping them is exact. Masks are evaluated
//    only on tiles that touch the diagonal or the padding.
#include "kf_common.h"

namespace kf {

struct FlashArgs {
  const void* q; int64_t qs0, qs1, qs2;
  const void* k; int64_t ks0, ks1, ks2;
  const void* v; int64_t vs0, vs1, vs2;
  void* o; void* o_lo; int64_t os0, os1, os2; int o_dtype;
  const void* keep; int keep_dtype; int64_t ld_keep;
  const int32_t* kv_len; const int32_t* prefix;
  int B, H, S, hd;
  float scale_log2;
  int flags;
};

constexpr float kNegInf = -__builtin_huge_valf();

template <int HDP> struct FlashTile {
  static constexpr int BN = HDP >= 256 ? 32 : 64;   // keys per LDS stage
  static constexpr int QG = HDP >= 256 ? 1 : 2;     // 16-row query groups per wavefront
  static constexpr int BM = 4 * 16 * QG;
};

__device__ __forceinline__ void store_o4(const FlashArgs& a, int64_t off, const float* v) {
  store4_any(a.o, a.o_lo, a.o_dtype, off, v);
}

template <int MODE, int IT, int HDP>
__global__ __launch_bounds__(256) void flash_fwd_kernel(FlashArgs a) {
  using TR = ModeTraits<MODE>;
  using V = typename TR::vec;
  using E = typename TR::elem;
  constexpr int P = TR::split ? 2 : 1;
  constexpr int BN = FlashTile<HDP>::BN, QG = FlashTile<HDP>::QG, BM = FlashTile<HDP>::BM;
  constexpr int NC = BN / 32;          // 32-key chunks per tile
  constexpr int ND = HDP / 32;         // 32-wide contraction chunks of q . k
  constexpr int NT = HDP / 16;         // 16-row d tiles of O^T
  constexpr int KLD = HDP + 8, VLD = BN + 8;   // padded LDS rows (16-byte skew)
  constexpr int NCHUNK = BN * HDP / 8 / 256;   // 8-element staging chunks per thread
  static_assert(NCHUNK >= 1 && (BN * HDP / 8) % 256 == 0, "staging must tile the block");

  __shared__ __attribute__((aligned(16))) E Ks[2][P][BN][KLD];
  __shared__ __attribute__((aligned(16))) E Vt[2][P][HDP][VLD];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, grp = lane >> 4;

  const int nqb = (a.S + BM - 1) / BM;
  const int lin = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = lin / nqb;
  int qb = lin % nqb;
  const bool causal = a.flags & KF_FLASH_CAUSAL;
  if (causal) qb = (qb & 1) ? nqb - 1 - (qb >> 1) : (qb >> 1);   // heavy/light interleave
  const int b = bh / a.H, h = bh % a.H;

  const int kvlen = a.kv_len ? a.kv_len[b] : a.S;
  // prefix: keys [0, kvlen) are all valid, so kvlen alone decides validity (keep unread)
  const bool prefix = a.keep == nullptr || (a.kv_len && a.prefix && a.prefix[b] != 0);
  const bool skip_pad = (a.flags & KF_FLASH_SKIP_PAD_ROWS) && a.kv_len;

  const int q_lo = qb * BM;
  const int qw0 = q_lo + wave * 16 * QG;         // first query row of this wavefront
  const int64_t obase = (int64_t)b * a.os0 + (int64_t)h * a.os1;

  auto write_zero_rows = [&](int q0) {
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

  // ---- query fragments (MFMA "B" operand of S^T): lane (r, grp) holds q[qw0+16qg+r][32dc+8grp..+7]
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
          ld8<IT>(a.q, qbase + (int64_t)qi * a.qs2 + d, x);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = 0.0f;
        }
        if constexpr (TR::split) split8<E, V>(x, qf[qg][dc][0], qf[qg][dc][P - 1]);
        else round8<E, V>(x, qf[qg][dc][0]);
      }
  }

  float m_i[QG], l_i[QG];
  f32x4 acc[QG][NT];
#pragma unroll
  for (int qg = 0; qg < QG; ++qg) {
    m_i[qg] = kNegInf;
    l_i[qg] = 0.0f;
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[qg][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // ---- K/V staging: global -> registers -> (split) -> LDS
  const int64_t kbase_g = (int64_t)b * a.ks0 + (int64_t)h * a.ks1;
  const int64_t vbase_g = (int64_t)b * a.vs0 + (int64_t)h * a.vs1;
  float kreg[NCHUNK][8], vreg[NCHUNK][8];
  auto load_tile = [&](int t) {
    const int k0 = t * BN;
#pragma unroll
    for (int i = 0; i < NCHUNK; ++i) {
      const int c = tid + 256 * i;
      {   // K: consecutive threads walk d within a key row
        const int key = k0 + c / (HDP / 8), d8 = (c % (HDP / 8)) * 8;
        if (key < kend_blk && d8 < a.hd) ld8<IT>(a.k, kbase_g + (int64_t)key * a.ks2 + d8, kreg[i]);
        else for (int e = 0; e < 8; ++e) kreg[i][e] = 0.0f;
      }
      {   // V: consecutive threads walk keys, so the transposed LDS writes are contiguous
        const int key = k0 + c % BN, d8 = (c / BN) * 8;
        if (key < kend_blk && d8 < a.hd) ld8<IT>(a.v, vbase_g + (int64_t)key * a.vs2 + d8, vreg[i]);
        else for (int e = 0; e < 8; ++e) vreg[i][e] = 0.0f;
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < NCHUNK; ++i) {
      const int c = tid + 256 * i;
      {
        const int key = c / (HDP / 8), d8 = (c % (HDP / 8)) * 8;
        V hi, lo;
        if constexpr (TR::split) split8<E, V>(kreg[i], hi, lo);
        else round8<E, V>(kreg[i], hi);
        *(U4*)&Ks[buf][0][key][d8] = as_u4(hi);
        if constexpr (TR::split) *(U4*)&Ks[buf][P - 1][key][d8] = as_u4(lo);
      }
      {
        const int key = c % BN, d8 = (c / BN) * 8;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const E hv = (E)vreg[i][e];
          Vt[buf][0][d8 + e][key] = hv;
          if constexpr (TR::split) Vt[buf][P - 1][d8 + e][key] = (E)(vreg[i][e] - (float)hv);
        }
      }
    }
  };

  const int ntiles = (kend_blk + BN - 1) / BN;
  if (ntiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    const int k0 = t * BN;
    if (t + 1 < ntiles) load_tile(t + 1);

    if (wave_active && k0 < kend_w) {
      // ---- S^T = K . Q^T for BN keys and every query group of this wavefront
      f32x4 s[QG][NC][2];
#pragma unroll
      for (int qg = 0; qg < QG; ++qg)
#pragma unroll
        for (int c = 0; c < NC; ++c) s[qg][c][0] = s[qg][c][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const int krow = 32 * c + (r >> 2) * 8 + 4 * tt + (r & 3);
#pragma unroll
          for (int dc = 0; dc < ND; ++dc) {
            V kf[P];
#pragma unroll
            for (int p = 0; p < P; ++p) kf[p] = from_u4<V>(*(const U4*)&Ks[buf][p][krow][dc * 32 + grp * 8]);
#pragma unroll
            for (int qg = 0; qg < QG; ++qg) {
              if constexpr (TR::split) {
                s[qg][c][tt] = mma16(kf[0], qf[qg][dc][1], s[qg][c][tt]);
                s[qg][c][tt] = mma16(kf[1], qf[qg][dc][0], s[qg][c][tt]);
              }
              s[qg][c][tt] = mma16(kf[0], qf[qg][dc][0], s[qg][c][tt]);
            }
          }
        }

      // ---- online softmax per query group; lane holds keys k0 + 32c + 8grp + (4tt + i)
      V pf[QG][NC][P];
#pragma unroll
      for (int qg = 0; qg < QG; ++qg) {
        const int qg0 = qw0 + qg * 16;
        const int qi = qg0 + r;
        const bool full = prefix && k0 + BN <= kvlen && (!causal || k0 + BN - 1 <= qg0);
        float x[NC][8];
        float mloc = kNegInf;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) {
            float val = s[qg][c][jj >> 2][jj & 3] * a.scale_log2;
            if (!full) {
              const int key = k0 + 32 * c + 8 * grp + jj;
              bool ok = key < kvlen && (!causal || key <= qi);
              if (ok && !prefix) ok = ld_elem(a.keep, a.keep_dtype, (int64_t)b * a.ld_keep + key) != 0.0f;
              val = ok ? val : kNegInf;
            }
            x[c][jj] = val;
            mloc = fmaxf(mloc, val);
          }
        mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
        const float m_new = fmaxf(m_i[qg], mloc);
        const float m_safe = m_new == kNegInf ? 0.0f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_i[qg] - m_safe);
        float psum = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          float pv[8];
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) {
            pv[jj] = __builtin_amdgcn_exp2f(x[c][jj] - m_safe);
            psum += pv[jj];
          }
          if constexpr (TR::split) split8<E, V>(pv, pf[qg][c][0], pf[qg][c][P - 1]);
          else round8<E, V>(pv, pf[qg][c][0]);
        }
        l_i[qg] = l_i[qg] * alpha + psum;
        m_i[qg] = m_new;
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[qg][j] *= alpha;
      }

      // ---- O^T += V^T . P^T
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          if (16 * j >= a.hd) continue;
          V vf[P];
#pragma unroll
          for (int p = 0; p < P; ++p) vf[p] = from_u4<V>(*(const U4*)&Vt[buf][p][16 * j + r][32 * c + 8 * grp]);
#pragma unroll
          for (int qg = 0; qg < QG; ++qg) {
            if constexpr (TR::split) {
              acc[qg][j] = mma16(vf[0], pf[qg][c][1], acc[qg][j]);
              acc[qg][j] = mma16(vf[1], pf[qg][c][0], acc[qg][j]);
            }
            acc[qg][j] = mma16(vf[0], pf[qg][c][0], acc[qg][j]);
          }
        }
    }

    if (t + 1 < ntiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- finalize: reduce the row sum over the four lane groups, normalise, store
  if (!wave_active) {
    if (qw0 < a.S) write_zero_rows(qw0);
    return;
  }
#pragma unroll
  for (int qg = 0; qg < QG; ++qg) {
    float l = l_i[qg];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
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

// kv_len[b] = 1 + last valid position (0 if none); prefix[b] = all of [0, kv_len) valid.
__global__ __launch_bounds__(256) void mask_prep_kernel(const void* keep, int dtype, int64_t ld,
                                                        int S, int32_t* kv_len, int32_t* prefix) {
  __shared__ int smax[4], scnt[4];
  const int b = blockIdx.x;
  int last = -1, cnt = 0;
  for (int s = threadIdx.x; s < S; s += blockDim.x) {
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

template <int MODE, int IT, int HDP>
static void launch_flash(const FlashArgs& a, hipStream_t st) {
  const int nqb = (a.S + FlashTile<HDP>::BM - 1) / FlashTile<HDP>::BM;
  const int64_t blocks = (int64_t)nqb * a.B * a.H;
  hipLaunchKernelGGL((flash_fwd_kernel<MODE, IT, HDP>), dim3((unsigned)blocks), dim3(256), 0, st, a);
}

template <int MODE, int IT>
static void launch_hd(const FlashArgs& a, int hdp, hipStream_t st) {
  switch (hdp) {
    case 32: launch_flash<MODE, IT, 32>(a, st); break;
    case 64: launch_flash<MODE, IT, 64>(a, st); break;
    case 128: launch_flash<MODE, IT, 128>(a, st); break;
    default: launch_flash<MODE, IT, 256>(a, st); break;
  }
}

}  // namespace kf

using namespace kf;

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

extern "C" int kf_flash_fwd(const void* q, const int64_t* qs, const void* k, const int64_t* ks,
                            const void* v, const int64_t* vs, int in_dtype,
                            void* o, void* o_lo, const int64_t* os, int o_dtype,
                            const void* keep, int keep_dtype, int64_t ld_keep,
                            const int32_t* kv_len, const int32_t* prefix,
                            int64_t B, int64_t H, int64_t S, int64_t hd,
                            float sm_scale, int mode, int flags, void* stream) {
  if (!q || !k || !v || !o || !qs || !ks || !vs || !os || B < 0 || H <= 0 || S < 0) {
    kf_set_error("kf_flash_fwd: bad arguments");
    return KF_EINVAL;
  }
  if (hd != 8 && hd != 16 && hd != 32 && hd != 64 && hd != 128 && hd != 256) {
    kf_set_error("kf_flash_fwd: unsupported head_dim %lld (8, 16, 32, 64, 128, 256)", (long long)hd);
    return KF_EUNSUPPORTED;
  }
  if (qs[3] != 1 || ks[3] != 1 || vs[3] != 1 || os[3] != 1) {
    kf_set_error("kf_flash_fwd: head_dim stride must be 1");
    return KF_EINVAL;
  }
  if (keep && (keep_dtype < KF_F32 || keep_dtype > KF_U8 || ld_keep < S)) {
    kf_set_error("kf_flash_fwd: bad keep mask");
    return KF_EINVAL;
  }
  const bool o_planes = o_dtype == KF_F16X2 || o_dtype == KF_BF16X2;
  if (in_dtype < KF_F32 || in_dtype > KF_BF16 || o_dtype < KF_F32 || o_dtype == KF_U8 ||
      o_dtype > KF_BF16X2 || (o_planes && !o_lo)) {
    kf_set_error("kf_flash_fwd: bad dtype (or missing output lo plane)");
    return KF_EINVAL;
  }
  // Input storage and MFMA precision pairs: fp32 storage with any mode; 16-bit storage with
  // its own single-pass mode.
  const bool pair_ok = (in_dtype == KF_F32 && mode != KF_MMA_F32) ||
                       (in_dtype == KF_F16 && mode == KF_MMA_F16) ||
                       (in_dtype == KF_BF16 && mode == KF_MMA_BF16);
  if (!pair_ok) {
    kf_set_error("kf_flash_fwd: storage dtype %d with MFMA mode %d is not supported", in_dtype, mode);
    return KF_EUNSUPPORTED;
  }
  // vector loads: 8-element chunks must be aligned to 16 bytes (16-bit) / 32 bytes (fp32) or at
  // least to the 16-byte vector width
  const int64_t vec = in_dtype == KF_F32 ? 4 : 8;
  for (const int64_t* s : {qs, ks, vs})
    for (int i = 0; i < 3; ++i)
      if (s[i] % vec) { kf_set_error("kf_flash_fwd: input strides must be multiples of %lld", (long long)vec); return KF_EUNSUPPORTED; }
  for (int i = 0; i < 3; ++i)
    if (os[i] % 4) { kf_set_error("kf_flash_fwd: output strides must be multiples of 4"); return KF_EUNSUPPORTED; }
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v) & 15 || ((uintptr_t)o & (o_dtype == KF_F32 ? 15 : 7)) ||
      (o_planes && ((uintptr_t)o_lo & 7))) {
    kf_set_error("kf_flash_fwd: pointers must be 16-byte aligned");
    return KF_EUNSUPPORTED;
  }
  if (S > (1 << 30) || B * H > (1LL << 31)) { kf_set_error("kf_flash_fwd: problem too large"); return KF_EUNSUPPORTED; }
  if (B == 0 || S == 0) return KF_OK;
  FlashArgs a{q, qs[0], qs[1], qs[2], k, ks[0], ks[1], ks[2], v, vs[0], vs[1], vs[2],
              o, o_lo, os[0], os[1], os[2], o_dtype, keep, keep_dtype, ld_keep, kv_len, prefix,
              (int)B, (int)H, (int)S, (int)hd, sm_scale * 1.4426950408889634f, flags};
  const int hdp = hd < 32 ? 32 : (int)hd;
  const int64_t nqb = (S + FlashTile<64>::BM - 1) / FlashTile<64>::BM;
  if (nqb * B * H * 2 > 0x7fffffffLL) { kf_set_error("kf_flash_fwd: grid too large"); return KF_EUNSUPPORTED; }
  hipStream_t st = (hipStream_t)stream;
  switch (mode) {
    case KF_MMA_F16:
      if (in_dtype == KF_F16) launch_hd<MODE_F16, KF_F16>(a, hdp, st);
      else launch_hd<MODE_F16, KF_F32>(a, hdp, st);
      break;
    case KF_MMA_BF16:
      if (in_dtype == KF_BF16) launch_hd<MODE_BF16, KF_BF16>(a, hdp, st);
      else launch_hd<MODE_BF16, KF_F32>(a, hdp, st);
      break;
    case KF_MMA_F16X3: launch_hd<MODE_F16X3, KF_F32>(a, hdp, st); break;
    default: launch_hd<MODE_BF16X3, KF_F32>(a, hdp, st); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { kf_set_error("kf_flash_fwd: launch failed: %s", hipGetErrorString(e)); return KF_ELAUNCH; }
  return KF_OK;
}
