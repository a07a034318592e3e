// Kernels of the gfx950 GEMM (shared by the per-mode translation units gemm_*.hip).
//
// MFMA GEMM with bias / erf-GELU / cast epilogue for gfx950:
//   C[M, N] = act(A[M, K] . W[N, K]^T + bias[N])
// covering the fused QKV projection, out_proj, ffn_in(+GELU) and ffn_out of the layer
// (kernelforge/optimized.py:441-446, 483, 572-574).
//
// Two kernels share the epilogues below. gemm_dma_kernel (16-bit operands, what the
// layer's producers write) is persistent and copies tiles global -> LDS by DMA, several
// stages deep; gemm16_kernel (any operand, including fp32 A converted on the fly) stages
// through registers. The rest of this note describes what both do.
//
// Tiling: a 256-thread block (four wavefronts, WGM x WGN) computes a BM x BN tile of C.
// The product is formed as C^T = W . A^T -- W rows are the MFMA "A" operand, A rows the
// "B" operand of v_mfma_f32_16x16x32 -- so each lane ends with four consecutive output
// columns of one row and stores them with one vector write. K advances BK at a time
// through two LDS stages: the global loads of stage k+1 are issued before the MFMAs of
// stage k, and one barrier per stage separates the LDS writes of one buffer from the
// reads of the other.
//
// LDS layout: rows of BK 16-bit values with no padding, 16-byte chunks XOR-swizzled by
// row. gemm16_kernel stores chunk c of row r at c ^ ((r / (128 / BK)) % (BK / 8)), which
// measures ~124 of 256 B/clk/CU for its fragment reads; gemm_dma_kernel uses the
// swizzle of dswz (below), chosen by measurement. A 128 x 128 x 32 split-mode stage is
// 32 KB.
//
// Operand formats: fp32 activations are rounded (single-pass modes) or split into hi/lo
// (split modes) on their way into LDS; activations that a producer already stored as
// X2 planes (LayerNorm output, GELU output, attention output) are copied as they are.
// Weights arrive pre-split from kf_split. Split modes issue hi*lo + lo*hi + hi*hi per
// tile. KF_MMA_F32 runs the fp32 MFMA (16x16x4) on fp32 tiles (separate kernel below).
#pragma once

#include <type_traits>

#include "kf_common.h"

namespace kf {

struct GemmArgs {
  const void* a; const void* a_lo; int64_t lda;
  const void* w_hi; const void* w_lo; int64_t ldw;
  const float* bias;
  void* c; void* c_lo; int c_dtype; int64_t ldc;
  int M, N, K; int act;
  // attention-operand epilogue (kf_gemm_qkv): columns [0, d) -> q (fp32 [M, d]),
  // [d, 2d) -> k (kv_dtype, [M, d]), [2d, 3d) -> v^T (kv_dtype, [B, H, hd, sp])
  float* q_out; void* k_hi; void* k_lo; void* vt_hi; void* vt_lo; int kv_dtype;
  int64_t sp; int S, H, hd;
  // 16-bit outputs (c, or k of the QKV epilogue) may be stored 8 columns per lane:
  // row stride a multiple of 8 elements and 16-byte aligned planes
  int wide16;
  // QKV epilogue: log2(S) and log2(hd) where they are powers of two, else -1 (divide)
  int s_shift, hd_shift;
  // row blocks per group of the persistent kernel's tile walk (set at launch; tile_rc)
  int group;
};

// Store eight consecutive values at element offset `off` of a 16-bit (or X2) output:
// one 16-byte store per plane.
__device__ __forceinline__ void store8_16(void* p, void* p_lo, int dtype, int64_t off,
                                          const float* v) {
  if (dtype == KF_F16) {
    half8 hi;
#pragma unroll
    for (int e = 0; e < 8; ++e) hi[e] = (_Float16)v[e];
    *(half8*)((_Float16*)p + off) = hi;
  } else if (dtype == KF_F16X2) {
    half8 hi, lo;
    split_n<_Float16, 8>(v, hi, lo);
    *(half8*)((_Float16*)p + off) = hi;
    *(half8*)((_Float16*)p_lo + off) = lo;
  } else if (dtype == KF_BF16) {
    bhalf8 hi;
#pragma unroll
    for (int e = 0; e < 8; ++e) hi[e] = (__bf16)v[e];
    *(bhalf8*)((__bf16*)p + off) = hi;
  } else {
    bhalf8 hi, lo;
    split_n<__bf16, 8>(v, hi, lo);
    *(bhalf8*)((__bf16*)p + off) = hi;
    *(bhalf8*)((__bf16*)p_lo + off) = lo;
  }
}

// store8_16 with the type fixed at compile time
template <int DT>
__device__ __forceinline__ void store8_t(void* p, void* p_lo, int64_t off, const float* v) {
  if constexpr (DT == KF_F16) {
    half8 hi;
#pragma unroll
    for (int e = 0; e < 8; ++e) hi[e] = (_Float16)v[e];
    *(half8*)((_Float16*)p + off) = hi;
  } else if constexpr (DT == KF_F16X2) {
    half8 hi, lo;
    split_n<_Float16, 8>(v, hi, lo);
    *(half8*)((_Float16*)p + off) = hi;
    *(half8*)((_Float16*)p_lo + off) = lo;
  } else if constexpr (DT == KF_BF16) {
    bhalf8 hi;
#pragma unroll
    for (int e = 0; e < 8; ++e) hi[e] = (__bf16)v[e];
    *(bhalf8*)((__bf16*)p + off) = hi;
  } else {
    static_assert(DT == KF_BF16X2, "16-bit output types");
    bhalf8 hi, lo;
    split_n<__bf16, 8>(v, hi, lo);
    *(bhalf8*)((__bf16*)p + off) = hi;
    *(bhalf8*)((__bf16*)p_lo + off) = lo;
  }
}

// k / v^T storage type of the QKV epilogue for an MFMA mode (what kf_gemm_qkv sets in
// GemmArgs::kv_dtype): split planes for the split modes and f16x2, else the mode's type.
// KVT < 0: read it from GemmArgs at run time.
template <int MODE> constexpr int qkv_kv_dtype() {
  return (MODE == MODE_F16X3 || MODE == MODE_F16X2) ? KF_F16X2
       : MODE == MODE_BF16X3 ? KF_BF16X2 : MODE == MODE_F16 ? KF_F16 : KF_BF16;
}
// The QKV epilogue's k / v^T type with one 16-bit plane (EPI 5: a split-mode GEMM whose
// attention reads single-pass operands -- the planes' hi part, the values rounded to
// nearest -- so the lo planes are not written).
template <int MODE> constexpr int qkv_kv_single() {
  return (MODE == MODE_BF16X3 || MODE == MODE_BF16) ? KF_BF16 : KF_F16;
}

// BIAS false: the caller has added the bias already (the LDS-DMA kernel, from scalar loads).
template <bool BIAS = true>
__device__ __forceinline__ void epilogue_store(const GemmArgs& g, int m, int n, f32x4 acc) {
  if (m >= g.M || n >= g.N) return;
  float v[4] = {acc[0], acc[1], acc[2], acc[3]};
  if (BIAS && g.bias) {
    const float4 bv = *(const float4*)(g.bias + n);
    v[0] += bv.x; v[1] += bv.y; v[2] += bv.z; v[3] += bv.w;
  }
  if (g.act == KF_ACT_GELU_ERF) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = gelu_erf(v[i]);
  }
  store4_any(g.c, g.c_lo, g.c_dtype, (int64_t)m * g.ldc + n, v);
}

// Plain epilogues with the output type and activation fixed at compile time (EPI 2-4 of
// gemm_dma_kernel, chosen by the host for the combinations the layer uses), so no
// per-fragment dtype or activation branches. Same arithmetic as epilogue_store.
template <int MODE, int EPI> constexpr int epi_ctype() {
  constexpr bool f16 = MODE == MODE_F16 || MODE == MODE_F16X3 || MODE == MODE_F16X2;
  return EPI == 2 ? KF_F32 : EPI == 3 ? (f16 ? KF_F16 : KF_BF16) : (f16 ? KF_F16X2 : KF_BF16X2);
}
template <int CT, bool GELU, bool BIAS = true>
__device__ __forceinline__ void epilogue_store_t(const GemmArgs& g, int m, int n, f32x4 acc) {
  if (m >= g.M || n >= g.N) return;
  float v[4] = {acc[0], acc[1], acc[2], acc[3]};
  if (BIAS && g.bias) {
    const float4 bv = *(const float4*)(g.bias + n);
    v[0] += bv.x; v[1] += bv.y; v[2] += bv.z; v[3] += bv.w;
  }
  if constexpr (GELU) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = gelu_erf(v[i]);
  }
  store4_t<CT>(g.c, g.c_lo, (int64_t)m * g.ldc + n, v);
}

// Epilogue of the fused QKV projection: the four columns n..n+3 of row m (= token b*S+s)
// belong to one of q, k, v (d % 4 == 0) and to one head h; q and k keep the token-major
// [M, d] layout, v is written transposed to [B, H, hd, sp] so that attention stages V^T
// rows (keys contiguous) without a transpose.
template <int KVT = -1, bool BIAS = true>
__device__ __forceinline__ void epilogue_qkv(const GemmArgs& g, int m, int n, f32x4 acc) {
  if (m >= g.M || n >= g.N) return;
  float v[4] = {acc[0], acc[1], acc[2], acc[3]};
  if constexpr (BIAS) {
    const float4 bv = *(const float4*)(g.bias + n);
    v[0] += bv.x; v[1] += bv.y; v[2] += bv.z; v[3] += bv.w;
  }
  const int d = g.K;
  const int which = (n >= d ? 1 : 0) + (n >= 2 * d ? 1 : 0), within = n - which * d;
  if (which == 0) {
    *(float4*)(g.q_out + (int64_t)m * d + within) = make_float4(v[0], v[1], v[2], v[3]);
  } else if (which == 1) {
    if constexpr (KVT < 0) store4_any(g.k_hi, g.k_lo, g.kv_dtype, (int64_t)m * d + within, v);
    else store4_t<KVT>(g.k_hi, g.k_lo, (int64_t)m * d + within, v);
  } else {
    const int b = g.s_shift >= 0 ? m >> g.s_shift : m / g.S, s = m - b * g.S;
    const int h = g.hd_shift >= 0 ? within >> g.hd_shift : within / g.hd, dd = within - h * g.hd;
    const int64_t base = (((int64_t)b * g.H + h) * g.hd + dd) * g.sp + s;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (KVT < 0) st_elem(g.vt_hi, g.kv_dtype, base + i * g.sp, v[i], g.vt_lo);
      else st16_t<KVT>(g.vt_hi, g.vt_lo, base + i * g.sp, v[i]);
    }
  }
}

// Eight-column variants (columns n..n+7 of row m; n % 8 == 0) used when g.wide16.
template <bool BIAS = true>
__device__ __forceinline__ void epilogue_store8(const GemmArgs& g, int m, int n, float* v) {
  if (m >= g.M || n >= g.N) return;
  if (BIAS && g.bias) {
    const float4 b0 = *(const float4*)(g.bias + n), b1 = *(const float4*)(g.bias + n + 4);
    v[0] += b0.x; v[1] += b0.y; v[2] += b0.z; v[3] += b0.w;
    v[4] += b1.x; v[5] += b1.y; v[6] += b1.z; v[7] += b1.w;
  }
  if (g.act == KF_ACT_GELU_ERF) {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = gelu_erf(v[i]);
  }
  store8_16(g.c, g.c_lo, g.c_dtype, (int64_t)m * g.ldc + n, v);
}

template <int CT, bool GELU, bool BIAS = true>
__device__ __forceinline__ void epilogue_store8_t(const GemmArgs& g, int m, int n, float* v) {
  static_assert(CT != KF_F32, "8-column stores are for 16-bit outputs");
  if (m >= g.M || n >= g.N) return;
  if (BIAS && g.bias) {
    const float4 b0 = *(const float4*)(g.bias + n), b1 = *(const float4*)(g.bias + n + 4);
    v[0] += b0.x; v[1] += b0.y; v[2] += b0.z; v[3] += b0.w;
    v[4] += b1.x; v[5] += b1.y; v[6] += b1.z; v[7] += b1.w;
  }
  if constexpr (GELU) {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = gelu_erf(v[i]);
  }
  store8_t<CT>(g.c, g.c_lo, (int64_t)m * g.ldc + n, v);
}

template <int KVT = -1, bool BIAS = true>
__device__ __forceinline__ void epilogue_qkv8(const GemmArgs& g, int m, int n, float* v) {
  if (m >= g.M || n >= g.N) return;
  if constexpr (BIAS) {
    const float4 b0 = *(const float4*)(g.bias + n), b1 = *(const float4*)(g.bias + n + 4);
    v[0] += b0.x; v[1] += b0.y; v[2] += b0.z; v[3] += b0.w;
    v[4] += b1.x; v[5] += b1.y; v[6] += b1.z; v[7] += b1.w;
  }
  const int d = g.K;
  const int which = (n >= d ? 1 : 0) + (n >= 2 * d ? 1 : 0), within = n - which * d;
  if (which == 0) {
    float* q = g.q_out + (int64_t)m * d + within;
    *(float4*)q = make_float4(v[0], v[1], v[2], v[3]);
    *(float4*)(q + 4) = make_float4(v[4], v[5], v[6], v[7]);
  } else if (which == 1) {
    if constexpr (KVT < 0) store8_16(g.k_hi, g.k_lo, g.kv_dtype, (int64_t)m * d + within, v);
    else store8_t<KVT>(g.k_hi, g.k_lo, (int64_t)m * d + within, v);
  } else {
    const int b = g.s_shift >= 0 ? m >> g.s_shift : m / g.S, s = m - b * g.S;
    const int h = g.hd_shift >= 0 ? within >> g.hd_shift : within / g.hd, dd = within - h * g.hd;
    const int64_t base = (((int64_t)b * g.H + h) * g.hd + dd) * g.sp + s;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if constexpr (KVT < 0) st_elem(g.vt_hi, g.kv_dtype, base + i * g.sp, v[i], g.vt_lo);
      else st16_t<KVT>(g.vt_hi, g.vt_lo, base + i * g.sp, v[i]);
    }
  }
}

// Bias of the sixteen columns [c, c + 16) for a wavefront (c wave-uniform), as wave-uniform
// values read through the scalar data cache: those loads count on lgkmcnt, whereas a vector
// load counts on vmcnt behind the LDS copies still in flight, and waiting for it waited for
// every one of them (the epilogue of the LDS-DMA kernel drained its copy pipeline once per
// fragment). Columns at or past n read as 0; they are never stored.
__device__ __forceinline__ void bias16(const float* bias, int c, int n, float (&s)[16]) {
  using CF = const __attribute__((address_space(4))) float;
  CF* p = (CF*)bias;
  if (c + 16 <= n) {
#pragma unroll
    for (int e = 0; e < 16; ++e) s[e] = p[c + e];
  } else {
#pragma unroll
    for (int e = 0; e < 16; ++e) s[e] = c + e < n ? p[c + e] : 0.f;
  }
}
// Lane value of four wave-uniform candidates by the lane's column group.
__device__ __forceinline__ float sel4(int grp, float a, float b, float c, float d) {
  const float lo = (grp & 1) ? b : a, hi = (grp & 1) ? d : c;
  return (grp & 2) ? hi : lo;
}

template <int BM_, int BN_, int BK_, int WGM_> struct GemmCfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WGM = WGM_, WGN = 4 / WGM_;
  static constexpr int TM = BM / WGM, TN = BN / WGN;    // wavefront tile (m, n)
  static constexpr int FM = TM / 16, FN = TN / 16;      // 16x16 MFMA tiles per wavefront
  static constexpr int CPR = BK / 8;                    // 16-byte chunks per LDS row
  static constexpr int RPS = 128 / BK;                  // rows per 256-byte bank sweep
  static constexpr int NA = BM * CPR / 256;             // A chunks staged per thread
  static constexpr int NW = BN * CPR / 256;             // W chunks staged per thread
  static_assert(NA >= 1 && NW >= 1 && FM >= 1 && FN >= 1, "tile too small for 256 threads");
  static_assert(BK % 32 == 0, "BK must be a multiple of the MFMA K (32)");
};

template <class C>
__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * C::BK + ((chunk ^ ((row / C::RPS) % C::CPR)) << 3);
}

// ------------------------------------------------------------------ 16-bit MFMA modes
// AT: KF_F32 (convert on load), the mode's 16-bit type (single-pass modes), or its X2
// planes (split modes).
template <int MODE, int AT, class C, int EPI>
__global__ __launch_bounds__(256) void gemm16_kernel(GemmArgs g) {
  using TR = ModeTraits<MODE>;
  using V = typename TR::vec;
  using E = typename TR::elem;
  constexpr int P = TR::split ? 2 : 1;
  constexpr bool A32 = AT == KF_F32;
  __shared__ __attribute__((aligned(16))) E As[2][P][C::BM * C::BK];
  __shared__ __attribute__((aligned(16))) E Ws[2][P][C::BN * C::BK];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, grp = lane >> 4;
  const int wm = wave % C::WGM, wn = wave / C::WGM;
  const int ntn = (g.N + C::BN - 1) / C::BN;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int tm = tile / ntn, tn = tile % ntn;
  const int m0 = tm * C::BM, n0 = tn * C::BN;

  float areg[A32 ? C::NA : 1][8];
  U4 a16[A32 ? 1 : C::NA][P];
  U4 wreg[C::NW][P];

  auto load_tile = [&](int kt) KF_INLINE {
    const int k0 = kt * C::BK;
#pragma unroll
    for (int i = 0; i < C::NA; ++i) {
      const int q = threadIdx.x + 256 * i;
      const int row = q / C::CPR, ch = q % C::CPR;
      const int64_t gm = (int64_t)m0 + row;
      const int kk = k0 + ch * 8;
      const bool ok = gm < g.M && kk < g.K;
      if constexpr (A32) {
        if (ok) ld8<KF_F32>(g.a, gm * g.lda + kk, areg[i]);
        else for (int e = 0; e < 8; ++e) areg[i][e] = 0.0f;
      } else {
#pragma unroll
        for (int p = 0; p < P; ++p) {
          const E* ap = (const E*)(p == 0 ? g.a : g.a_lo);
          a16[i][p] = ok ? *(const U4*)(ap + gm * g.lda + kk) : U4{0, 0, 0, 0};
        }
      }
    }
#pragma unroll
    for (int i = 0; i < C::NW; ++i) {
      const int q = threadIdx.x + 256 * i;
      const int row = q / C::CPR, ch = q % C::CPR;
      const int64_t gn = (int64_t)n0 + row;
      const int kk = k0 + ch * 8;
      const bool ok = gn < g.N && kk < g.K;
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const E* wp = (const E*)(p == 0 ? g.w_hi : g.w_lo);
        wreg[i][p] = ok ? *(const U4*)(wp + gn * g.ldw + kk) : U4{0, 0, 0, 0};
      }
    }
  };
  auto store_tile = [&](int buf) KF_INLINE {
#pragma unroll
    for (int i = 0; i < C::NA; ++i) {
      const int q = threadIdx.x + 256 * i;
      const int off = lds_off<C>(q / C::CPR, q % C::CPR);
      if constexpr (A32) {
        V hi, lo;
        if constexpr (TR::split) split8<E, V>(areg[i], hi, lo);
        else round8<E, V>(areg[i], hi);
        *(U4*)&As[buf][0][off] = as_u4(hi);
        if constexpr (TR::split) *(U4*)&As[buf][P - 1][off] = as_u4(lo);
      } else {
#pragma unroll
        for (int p = 0; p < P; ++p) *(U4*)&As[buf][p][off] = a16[i][p];
      }
    }
#pragma unroll
    for (int i = 0; i < C::NW; ++i) {
      const int q = threadIdx.x + 256 * i;
      const int off = lds_off<C>(q / C::CPR, q % C::CPR);
#pragma unroll
      for (int p = 0; p < P; ++p) *(U4*)&Ws[buf][p][off] = wreg[i][p];
    }
  };

  f32x4 acc[C::FN][C::FM];
#pragma unroll
  for (int i = 0; i < C::FN; ++i)
#pragma unroll
    for (int j = 0; j < C::FM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = (g.K + C::BK - 1) / C::BK;
  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load_tile(kt + 1);
#pragma unroll
    for (int ks = 0; ks < C::BK / 32; ++ks) {
      V wf[C::FN][P], af[C::FM][P];
#pragma unroll
      for (int i = 0; i < C::FN; ++i) {
        const int off = lds_off<C>(wn * C::TN + 16 * i + r, ks * 4 + grp);
#pragma unroll
        for (int p = 0; p < P; ++p) wf[i][p] = from_u4<V>(*(const U4*)&Ws[buf][p][off]);
      }
#pragma unroll
      for (int j = 0; j < C::FM; ++j) {
        const int off = lds_off<C>(wm * C::TM + 16 * j + r, ks * 4 + grp);
#pragma unroll
        for (int p = 0; p < P; ++p) af[j][p] = from_u4<V>(*(const U4*)&As[buf][p][off]);
      }
#pragma unroll
      for (int i = 0; i < C::FN; ++i)
#pragma unroll
        for (int j = 0; j < C::FM; ++j) {
          if constexpr (TR::split) {
            acc[i][j] = mma16(wf[i][0], af[j][1], acc[i][j]);
            acc[i][j] = mma16(wf[i][1], af[j][0], acc[i][j]);
          }
          acc[i][j] = mma16(wf[i][0], af[j][0], acc[i][j]);
        }
    }
    if (kt + 1 < nk) store_tile(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < C::FN; ++i)
#pragma unroll
    for (int j = 0; j < C::FM; ++j) {
      const int m = m0 + wm * C::TM + 16 * j + r, n = n0 + wn * C::TN + 16 * i + 4 * grp;
      if constexpr (EPI == 1) epilogue_qkv(g, m, n, acc[i][j]);
      else epilogue_store(g, m, n, acc[i][j]);
    }
}

// ------------------------------------------------------------------ LDS-DMA pipeline
// Operands already in 16-bit form (the mode's type or its X2 planes, which every producer
// of the layer writes) skip the register round trip: global_load_lds_dwordx4 copies them
// straight into LDS, STAGES buffers deep, so the copies of later stages are in flight
// while the MFMAs consume the current one, with no VGPRs and no LDS write instructions
// spent on staging.
//
// LDS layout: a stage of BK k holds, per operand plane, BK / 32 sub-tiles of 32 k (rows of
// 64 bytes, four 16-byte chunks, the chunk swizzled by dswz(row)). The copies land
// lane-linearly, so the swizzle is applied to the source address instead: LDS chunk q of a
// sub-tile holds row q / 4, logical chunk (q % 4) ^ dswz(row). A stage's copies are issued
// sub-tile innermost, so a wavefront's consecutive copies read the two 64-byte halves of
// the same 128-byte lines: measured on MI355X (L2-resident source, 128 KB in flight per
// CU), 27.8 B/clk/CU when the halves are fetched a stage apart, as 32-k stages do, and
// 54.2 B/clk/CU when they are fetched back to back. Rows past M or N re-read the last
// valid row (finite data whose products fall in outputs that are never stored); K must
// be a multiple of BK.
//
// The kernel is persistent: a block walks a list of output tiles and the copy pipeline
// runs on across tile boundaries, so the first stages of the next tile load while the
// current one finishes and stores its epilogue. Blocks are numbered onto XCDs
// round-robin; each XCD owns one contiguous range of row-major tiles, so the tiles that
// share an A row panel (and all of W) stay in one L2.
// Output tile of linear index t: tiles are walked in groups of `group` row blocks, column
// by column inside a group (row-major when group is 1). Consecutive indices -- the tiles an
// XCD's blocks hold at one time -- then share `group` A row panels and a few W column
// panels in that XCD's L2 instead of every W panel. A bijection of [0, ntm * ntn).
__device__ __forceinline__ void tile_rc(int t, int ntm, int ntn, int group, int& tm, int& tn) {
  if (group <= 1) {
    tm = t / ntn;
    tn = t % ntn;
  } else {
    const int per = group * ntn;
    const int grp = t / per, idx = t % per;
    const int r0 = grp * group;
    const int rows = min(group, ntm - r0);
    tm = r0 + idx % rows;
    tn = idx / rows;
  }
}

// WPE_ > 0: wavefronts per SIMD the kernel is compiled to fit (registers), capped by what
// the tile's LDS allows in the mode; 0: only what one block needs.
template <int BM_, int BN_, int BK_, int ST_, int WGM_, int WGN_, int WPE_ = 0> struct DmaCfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, STAGES = ST_, WGM = WGM_, WGN = WGN_;
  static constexpr int WPE = WPE_;
  static constexpr int NWAVES = WGM * WGN, NT = 64 * NWAVES;
  static constexpr int TM = BM / WGM, TN = BN / WGN;
  static constexpr int FM = TM / 16, FN = TN / 16;
  static constexpr int NS = BK / 32;                    // 32-k sub-tiles per stage
  // 16-byte copies per thread per plane and stage (chunks: rows x 4 x NS)
  static constexpr int NA = BM * 4 * NS / NT, NW = BN * 4 * NS / NT;
  static_assert(BK == 32 || BK == 64 || BK == 128, "BK must be 32, 64 or 128");
  static_assert(NA >= 1 && NW >= 1 && (BM * 4 * NS) % NT == 0 && (BN * 4 * NS) % NT == 0,
                "a stage must be a whole number of block-wide copies");
  static_assert((BM * 4) % 64 == 0 && (BN * 4) % 64 == 0,
                "a wavefront's copies must stay in one sub-tile");
  static_assert(FM >= 1 && FN >= 1, "bad wavefront tiling");
  static_assert(STAGES >= 2 && STAGES <= 6, "the schedule takes 2 to 6 stages");
  static constexpr int lds_bytes(int pa, int pw) { return STAGES * (pa * BM + pw * BN) * BK * 2; }
};

// Chunk swizzle of a 64-byte LDS row (four 16-byte chunks) for fragment loads, where lane
// (r, g) reads row R + r, logical chunk g. Chosen by measuring the ds_read_b128
// throughput of this kernel's read sequence on MI355X over every bit-select swizzle of the
// row index: ~187 B/clk/CU of the 256 B/clk peak, against 111 unswizzled and 124 for the
// classic (row / rows-per-128B) % chunks swizzle.
__device__ __forceinline__ int dswz(int row) { return (row >> 1) & 3; }

// Copy c (0 <= c < count) of thread t for one operand plane of `rows` rows: its sub-tile and
// its chunk q within the sub-tile. Where a sub-tile has at least one chunk per thread the
// sub-tile index runs fastest (a thread's consecutive copies read both halves of a line);
// otherwise the block's threads cover the sub-tiles side by side.
template <int NT, int NS>
__device__ __forceinline__ void copy_slot(int rows, int c, int t, int& sub, int& q) {
  const int per = rows * 4;                    // chunks per sub-tile
  if (per >= NT) {
    sub = c % NS;
    q = (c / NS) * NT + t;
  } else {
    const int k = c * NT + t;
    sub = k / per;
    q = k % per;
  }
}

// Occupancy the kernel of tile C in MODE is compiled for (wavefronts per SIMD, through
// the register budget): C::WPE where the tile asks for one, capped by the blocks its LDS
// lets a CU hold in this mode; else one block's worth. (The 128 x 128 x 64 tile asks for
// four: an fp16 epilogue one register past 128 had halved its resident blocks.)
template <int MODE, class C> constexpr int dma_waves_per_simd() {
  constexpr int lds = C::lds_bytes(a_planes<MODE>(), w_planes<MODE>());
  constexpr int blocks = lds <= 160 * 1024 ? 160 * 1024 / lds : 1;
  constexpr int by_lds = blocks * C::NWAVES / 4;
  constexpr int one = C::NWAVES / 4 < 1 ? 1 : C::NWAVES / 4;
  constexpr int w = C::WPE > 0 ? (C::WPE < by_lds ? C::WPE : by_lds) : one;
  return w < one ? one : w > 8 ? 8 : w;
}

template <int MODE, class C, int EPI>
__global__ __launch_bounds__(C::NT)
__attribute__((amdgpu_waves_per_eu(dma_waves_per_simd<MODE, C>())))
void gemm_dma_kernel(GemmArgs g) {
  using TR = ModeTraits<MODE>;
  using V = typename TR::vec;
  using E = typename TR::elem;
  constexpr int PA = a_planes<MODE>(), PW = w_planes<MODE>();   // operand planes
  constexpr int NT = C::NT;
  constexpr int SA = C::BM * C::BK, SW = C::BN * C::BK, STG = PA * SA + PW * SW;
  constexpr int NL = PA * C::NA + PW * C::NW;  // copies per thread per stage
  constexpr int KS = C::BK / 32;               // MFMA k-steps per stage
  static_assert(NL * (C::STAGES - 1) < 64, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) E smem[C::STAGES * STG];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: LDS targets in SGPRs
  const int r = lane & 15, grp = lane >> 4;
  const int wm = wave % C::WGM, wn = wave / C::WGM;
  const int ntm = (g.M + C::BM - 1) / C::BM, ntn = (g.N + C::BN - 1) / C::BN;
  const int T = ntm * ntn;
  const int nk = g.K / C::BK;

  // this block's tiles: lo + j, lo + j + GX, ... below hi
  int lo = 0, hi = T, j = blockIdx.x, GX = gridDim.x;
  if (gridDim.x % kXcds == 0) {
    GX = gridDim.x / kXcds;
    j = blockIdx.x / kXcds;
    const int per = (T + kXcds - 1) / kXcds;
    lo = (blockIdx.x % kXcds) * per;
    hi = min(T, lo + per);
  }
  const int my_tiles = hi - lo > j ? (hi - lo - j + GX - 1) / GX : 0;
  if (my_tiles == 0) return;
  const int Q = my_tiles * nk;       // stages of this block
  const int U = Q * KS;              // MFMA k-steps of this block

  const E* src_a[PA];
  const E* src_w[PW];
  src_a[0] = (const E*)g.a;
  src_w[0] = (const E*)g.w_hi;
  if constexpr (PA == 2) src_a[1] = (const E*)g.a_lo;
  if constexpr (PW == 2) src_w[1] = (const E*)g.w_lo;
  // per copy: row within the tile, source k offset (sub-tile and swizzled chunk), and the
  // LDS element offset within its plane (wavefront-uniform base + lane * 8)
  int arow[C::NA], ak[C::NA], adst[C::NA], wrow[C::NW], wk[C::NW], wdst[C::NW];
#pragma unroll
  for (int i = 0; i < C::NA; ++i) {
    int sub, q;
    copy_slot<NT, C::NS>(C::BM, i, tid, sub, q);
    arow[i] = q / 4;
    ak[i] = 32 * sub + (((q % 4) ^ dswz(arow[i])) << 3);
    int subw, qw;
    copy_slot<NT, C::NS>(C::BM, i, wave * 64, subw, qw);
    adst[i] = (subw * C::BM * 4 + qw) * 8;
  }
#pragma unroll
  for (int i = 0; i < C::NW; ++i) {
    int sub, q;
    copy_slot<NT, C::NS>(C::BN, i, tid, sub, q);
    wrow[i] = q / 4;
    wk[i] = 32 * sub + (((q % 4) ^ dswz(wrow[i])) << 3);
    int subw, qw;
    copy_slot<NT, C::NS>(C::BN, i, wave * 64, subw, qw);
    wdst[i] = (subw * C::BN * 4 + qw) * 8;
  }

  // Copy cursor: the stages are issued in order, walking this block's tiles; a tile's
  // row offsets (one division for its origin) are found when the cursor enters it, and
  // the per-stage issue only adds the uniform column offset: no index math per stage.
  int c_tile = 0, c_k0 = 0, c_buf = 0;
  int64_t off_a[C::NA], off_w[C::NW];
  auto aim = [&]() KF_INLINE {
    int tm, tn;
    tile_rc(lo + j + c_tile * GX, ntm, ntn, g.group, tm, tn);
    const int m0 = tm * C::BM, n0 = tn * C::BN;
#pragma unroll
    for (int i = 0; i < C::NA; ++i)
      off_a[i] = (int64_t)min(m0 + arow[i], g.M - 1) * g.lda + ak[i];
#pragma unroll
    for (int i = 0; i < C::NW; ++i)
      off_w[i] = (int64_t)min(n0 + wrow[i], g.N - 1) * g.ldw + wk[i];
  };
  aim();
  auto issue = [&]() KF_INLINE {
    E* dst = smem + c_buf * STG;
#pragma unroll
    for (int p = 0; p < PA; ++p)
#pragma unroll
      for (int i = 0; i < C::NA; ++i) dma16(src_a[p] + c_k0 + off_a[i], dst + p * SA + adst[i]);
#pragma unroll
    for (int p = 0; p < PW; ++p)
#pragma unroll
      for (int i = 0; i < C::NW; ++i) dma16(src_w[p] + c_k0 + off_w[i], dst + PA * SA + p * SW + wdst[i]);
    if (++c_buf == C::STAGES) c_buf = 0;
    c_k0 += C::BK;
    if (c_k0 == g.K) {
      c_k0 = 0;
      if (++c_tile < my_tiles) aim();
    }
  };

  // Fragment offsets (elements within a stage) of this lane, per k-step (= sub-tile).
  int wrow_off[C::FN][KS], arow_off[C::FM][KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
    for (int i = 0; i < C::FN; ++i) {
      const int row = wn * C::TN + 16 * i + r;
      wrow_off[i][ks] = PA * SA + ks * C::BN * 32 + row * 32 + ((grp ^ dswz(row)) << 3);
    }
#pragma unroll
    for (int jj = 0; jj < C::FM; ++jj) {
      const int row = wm * C::TM + 16 * jj + r;
      arow_off[jj][ks] = ks * C::BM * 32 + row * 32 + ((grp ^ dswz(row)) << 3);
    }
  }

  struct Frags { V w[C::FN][PW]; V a[C::FM][PA]; };
  auto read_frags = [&](int buf, int ks, Frags& f) KF_INLINE {
    const E* base = smem + buf * STG;
#pragma unroll
    for (int i = 0; i < C::FN; ++i)
#pragma unroll
      for (int p = 0; p < PW; ++p) f.w[i][p] = from_u4<V>(*(const U4*)&base[wrow_off[i][ks] + p * SW]);
#pragma unroll
    for (int jj = 0; jj < C::FM; ++jj)
#pragma unroll
      for (int p = 0; p < PA; ++p) f.a[jj][p] = from_u4<V>(*(const U4*)&base[arow_off[jj][ks] + p * SA]);
  };

  f32x4 acc[C::FN][C::FM];
  auto zero_acc = [&]() KF_INLINE {
#pragma unroll
    for (int i = 0; i < C::FN; ++i)
#pragma unroll
      for (int jj = 0; jj < C::FM; ++jj) acc[i][jj] = f32x4{0.f, 0.f, 0.f, 0.f};
  };
  zero_acc();

  auto mfmas = [&](const Frags& f) KF_INLINE {
#pragma unroll
    for (int i = 0; i < C::FN; ++i)
#pragma unroll
      for (int jj = 0; jj < C::FM; ++jj) {
        if constexpr (TR::split) {
          acc[i][jj] = mma16(f.w[i][0], f.a[jj][PA - 1], acc[i][jj]);
          acc[i][jj] = mma16(f.w[i][PW - 1], f.a[jj][0], acc[i][jj]);
        } else if constexpr (PW == 2) {          // f16x2: the weights' lo plane only
          acc[i][jj] = mma16(f.w[i][PW - 1], f.a[jj][0], acc[i][jj]);
        }
        acc[i][jj] = mma16(f.w[i][0], f.a[jj][0], acc[i][jj]);
      }
  };

  // The bias enters from scalar loads (bias16) and is added here, in the order the other
  // kernels add it (accumulator + bias, then the activation).
  auto epilogue = [&](int ti) KF_INLINE {
    int tm, tn;
    tile_rc(lo + j + ti * GX, ntm, ntn, g.group, tm, tn);
    const int m0 = tm * C::BM, n0 = tn * C::BN;
    const int cw = n0 + wn * C::TN;          // this wavefront's first column (uniform)
    const bool has_bias = g.bias != nullptr;
    if constexpr (C::FN % 2 == 0 && EPI != 2) {
      // V^T columns are written transposed (2-byte pieces per key): the wide layout buys
      // nothing there, so tiles that reach into the V part keep the 4-column path.
      if (g.wide16 && ((EPI != 1 && EPI != 5) || n0 + C::BN <= 2 * g.K)) {
        // Lanes of column groups 2q and 2q+1 trade quads of adjacent 16-column tiles
        // (v_permlane16_swap), so each lane holds 8 consecutive columns of its row and
        // a row's 16-bit output leaves in 64-byte pieces instead of 32-byte ones.
        const bool odd = grp & 1;
#pragma unroll
        for (int i = 0; i < C::FN; i += 2) {
          // this lane's columns: 16i + {0, 16, 8, 24}[grp] + e of the wavefront's range
          float bl[8];
          if (has_bias) {
            float s0[16], s1[16];
            bias16(g.bias, cw + 16 * i, g.N, s0);
            bias16(g.bias, cw + 16 * (i + 1), g.N, s1);
#pragma unroll
            for (int e = 0; e < 8; ++e) bl[e] = sel4(grp, s0[e], s1[e], s0[8 + e], s1[8 + e]);
          }
#pragma unroll
          for (int jj = 0; jj < C::FM; ++jj) {
            float v[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const auto pr = __builtin_amdgcn_permlane16_swap(
                  __float_as_uint(acc[i][jj][e]), __float_as_uint(acc[i + 1][jj][e]), false, false);
              v[e] = __uint_as_float(pr[0]);
              v[4 + e] = __uint_as_float(pr[1]);
            }
            if (has_bias) {
#pragma unroll
              for (int e = 0; e < 8; ++e) v[e] += bl[e];
            }
            const int m = m0 + wm * C::TM + 16 * jj + r;
            const int n = cw + 16 * (i + (odd ? 1 : 0)) + 4 * (grp - (odd ? 1 : 0));
            if constexpr (EPI == 1) epilogue_qkv8<qkv_kv_dtype<MODE>(), false>(g, m, n, v);
            else if constexpr (EPI == 5) epilogue_qkv8<qkv_kv_single<MODE>(), false>(g, m, n, v);
            else if constexpr (EPI == 3 || EPI == 4) epilogue_store8_t<epi_ctype<MODE, EPI>(), true, false>(g, m, n, v);
            else epilogue_store8<false>(g, m, n, v);
          }
        }
        return;
      }
    }
#pragma unroll
    for (int i = 0; i < C::FN; ++i) {
      float bl[4];               // this lane's columns: 16i + 4 grp + e
      if (has_bias) {
        float s[16];
        bias16(g.bias, cw + 16 * i, g.N, s);
#pragma unroll
        for (int e = 0; e < 4; ++e) bl[e] = sel4(grp, s[e], s[4 + e], s[8 + e], s[12 + e]);
      }
#pragma unroll
      for (int jj = 0; jj < C::FM; ++jj) {
        f32x4 a = acc[i][jj];
        if (has_bias) {
#pragma unroll
          for (int e = 0; e < 4; ++e) a[e] += bl[e];
        }
        const int m = m0 + wm * C::TM + 16 * jj + r, n = cw + 16 * i + 4 * grp;
        if constexpr (EPI == 1) epilogue_qkv<qkv_kv_dtype<MODE>(), false>(g, m, n, a);
        else if constexpr (EPI == 5) epilogue_qkv<qkv_kv_single<MODE>(), false>(g, m, n, a);
        else if constexpr (EPI >= 2) epilogue_store_t<epi_ctype<MODE, EPI>(), EPI >= 3, false>(g, m, n, a);
        else epilogue_store<false>(g, m, n, a);
      }
    }
  };

  // Wait until stage q has landed given that `pending` later stages may still be in
  // flight. Global loads (and the LDS copies) complete in issue order, so any
  // unfinished copy of stage q keeps at least pending * NL + 1 operations outstanding;
  // epilogue stores in between may complete in any order without breaking this.
  auto wait_stage = [&](int pending) KF_INLINE {
    if constexpr (C::STAGES >= 6) {
      if (pending >= 5) { wait_vmcnt<5 * NL>(); return; }
    }
    if constexpr (C::STAGES >= 5) {
      if (pending >= 4) { wait_vmcnt<4 * NL>(); return; }
    }
    if constexpr (C::STAGES >= 4) {
      if (pending >= 3) { wait_vmcnt<3 * NL>(); return; }
    }
    if constexpr (C::STAGES >= 3) {
      if (pending >= 2) { wait_vmcnt<2 * NL>(); return; }
    }
    if (pending >= 1) { wait_vmcnt<NL>(); return; }
    wait_vmcnt<0>();
  };

  // Schedule over k-steps u (stage u / KS). Step u issues the LDS reads of step u + 1
  // among its own MFMAs, so fragment latency hides behind a step of MFMAs. Entering
  // stage q + 1 needs its copies landed in every wavefront (vmcnt, then the barrier),
  // which also retires every read of stage q, whose buffer then takes stage q + STAGES:
  // STAGES - 1 stages of copies stay in flight behind the one being consumed.
#pragma unroll
  for (int q = 0; q < C::STAGES; ++q)
    if (q < Q) issue();
  wait_stage(min(C::STAGES - 1, Q - 1));
  lds_barrier();

  // Read cursor: buffer of the stage the next fragment read comes from (step u reads the
  // fragments of step u + 1). The reads are unconditional so that the MFMAs of a step
  // never wait on a join of paths with different LDS traffic: the last step reads the
  // buffer after its own, which no copy targets any more (every stage has landed by
  // then), and discards it. The step loop is unrolled over a stage, so a step's k-step and
  // the k-step it reads are compile-time constants and fragment offsets index statically.
  int r_buf = 0;
  const int tile_steps = nk * KS;
  int q_cur = 0, t_step = 0, e_tile = 0;   // stage of step u, k-step within its tile
  auto step = [&](auto KR, int u, Frags& cur, Frags& nxt, auto EP) KF_INLINE {
    constexpr int kr = decltype(KR)::value;  // k-step of the fragments this step reads
    constexpr bool kEp = decltype(EP)::value;  // this step may end a tile (its epilogue)
    if constexpr (kr == 0) {                 // step u + 1 starts stage q_cur + 1
      if (u + 1 < U) {
        wait_stage(min(C::STAGES - 2, Q - 2 - q_cur));
        lds_barrier();
        if (q_cur + C::STAGES < Q) issue();
        ++q_cur;
      }
      if (++r_buf == C::STAGES) r_buf = 0;
    }
    mfmas(cur);
    read_frags(r_buf, kr, nxt);
    // Order: one MFMA, then the next step's fragment reads paired one-to-one with MFMAs,
    // then the rest of the MFMAs. The copies are FLAT-encoded LDS writes, so the compiler
    // waits for every LDS read outstanding (lgkmcnt(0)) before a step's first MFMA: with
    // that MFMA ahead of the reads the wait covers only the previous step's reads, issued
    // early in that step, instead of a read issued just before it (bit-identical; per
    // call 1-5 % faster, C4 out_proj 218 -> 208 us).
    constexpr int NR = C::FN * PW + C::FM * PA;
    constexpr int NM = C::FN * C::FM * (TR::split ? 3 : PW == 2 ? 2 : 1);
    constexpr int NI = NR < NM - 1 ? NR : NM - 1;     // reads paired one-to-one with MFMAs
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);          // DS read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);          // MFMA
    }
    if constexpr (NR > NI) __builtin_amdgcn_sched_group_barrier(0x100, NR - NI, 0);
    if constexpr (NM - 1 - NI > 0) __builtin_amdgcn_sched_group_barrier(0x008, NM - 1 - NI, 0);
    if constexpr (kEp) {
      if (++t_step == tile_steps) {          // tile complete
        t_step = 0;
        epilogue(e_tile++);
        zero_acc();
      }
    }
  };
  using K0 = std::integral_constant<int, 0>;
  using K1 = std::integral_constant<int, 1>;
  using K2 = std::integral_constant<int, 2>;
  using K3 = std::integral_constant<int, 3>;
  constexpr std::true_type kEpi{};

  Frags f0, f1;
  read_frags(0, 0, f0);
  // 256 x 256 tiles where the weight has two planes (the split modes and f16x2): 64 x 128
  // per wavefront holds 128 accumulator registers and 80-96 of fragments, so the fragments
  // are single-buffered -- a step's reads of the next k-step land in the registers its own
  // MFMAs have finished with (each read waits for the last MFMA that used its registers);
  // double-buffered, the split-mode kernel spilled ~140 VGPRs. A tile's last step runs its
  // MFMAs, then the epilogue, then the next step's reads, so no fragment is live across the
  // epilogue (with the reads before it the QKV and GELU epilogues spilled 19-61 VGPRs). The
  // loops nest (tiles, then k-steps) so the two step forms run in sequence: one loop
  // branching between them made the allocator keep both forms' registers (~330 spilled).
  constexpr bool kSingle = C::BM == 256 && C::BN == 256 && PW == 2;
  if constexpr (KS == 1 && kSingle) {
    auto step_last = [&](int u) KF_INLINE {
      if (u + 1 < U) {                       // step u + 1 starts stage q_cur + 1
        wait_stage(min(C::STAGES - 2, Q - 2 - q_cur));
        lds_barrier();
        if (q_cur + C::STAGES < Q) issue();
        ++q_cur;
      }
      if (++r_buf == C::STAGES) r_buf = 0;
      mfmas(f0);
      t_step = 0;
      epilogue(e_tile++);
      zero_acc();
      read_frags(r_buf, 0, f0);
    };
    int u = 0;
    for (int ti = 0; ti < my_tiles; ++ti) {
      for (int ks = 0; ks + 1 < tile_steps; ++ks, ++u) step(K0{}, u, f0, f0, std::false_type{});
      step_last(u++);
    }
  } else if constexpr (KS == 1) {
    for (int u = 0; u < U; u += 2) {
      step(K0{}, u, f0, f1, kEpi);
      if (u + 1 < U) step(K0{}, u + 1, f1, f0, kEpi);
    }
  } else if constexpr (KS == 2) {
    for (int u = 0; u < U; u += 2) {
      step(K1{}, u, f0, f1, kEpi);
      step(K0{}, u + 1, f1, f0, kEpi);
    }
  } else {
    static_assert(KS == 4, "1, 2 or 4 k-steps per stage");
    for (int u = 0; u < U; u += 4) {
      step(K1{}, u, f0, f1, kEpi);
      step(K2{}, u + 1, f1, f0, kEpi);
      step(K3{}, u + 2, f0, f1, kEpi);
      step(K0{}, u + 3, f1, f0, kEpi);
    }
  }
}

// ------------------------------------------------------------------ fp32 MFMA mode
// v_mfma_f32_16x16x4f32 takes one fp32 value per lane per operand. Lane (r, grp) supplies
// k = grp * 8 + s on sub-step s (s = 0..7), the same k for both operands, so 8 sub-steps
// cover a 32-wide K tile.
constexpr int GBM = 128, GBN = 128, GBK = 32;

template <int AT>
__global__ __launch_bounds__(256, 2) void gemm32_kernel(GemmArgs g) {
  constexpr int LDK = GBK + 4;
  __shared__ __attribute__((aligned(16))) float As[2][GBM][LDK];
  __shared__ __attribute__((aligned(16))) float Ws[2][GBN][LDK];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, grp = lane >> 4;
  const int wn = wave >> 1, wm = wave & 1;
  const int ntn = (g.N + GBN - 1) / GBN;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int tm = tile / ntn, tn = tile % ntn;
  const int m0 = tm * GBM, n0 = tn * GBN;
  const int lrow = tid >> 1, lkc = (tid & 1) * 16;
  const int64_t am = (int64_t)m0 + lrow, wnrow = (int64_t)n0 + lrow;
  float areg[16], wreg[16];

  auto load_tile = [&](int kt) KF_INLINE {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int kk = kt * GBK + lkc + 8 * c;
      if (am < g.M && kk < g.K) ld8<AT>(g.a, am * g.lda + kk, areg + 8 * c);
      else for (int i = 0; i < 8; ++i) areg[8 * c + i] = 0.0f;
      if (wnrow < g.N && kk < g.K) ld8<KF_F32>(g.w_hi, wnrow * g.ldw + kk, wreg + 8 * c);
      else for (int i = 0; i < 8; ++i) wreg[8 * c + i] = 0.0f;
    }
  };
  auto store_tile = [&](int buf) KF_INLINE {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      *(float4*)&As[buf][lrow][lkc + 4 * q] =
          make_float4(areg[4 * q], areg[4 * q + 1], areg[4 * q + 2], areg[4 * q + 3]);
      *(float4*)&Ws[buf][lrow][lkc + 4 * q] =
          make_float4(wreg[4 * q], wreg[4 * q + 1], wreg[4 * q + 2], wreg[4 * q + 3]);
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = (g.K + GBK - 1) / GBK;
  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load_tile(kt + 1);
    float wf[4][8], af[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 w0 = *(const float4*)&Ws[buf][wn * 64 + 16 * i + r][grp * 8];
      const float4 w1 = *(const float4*)&Ws[buf][wn * 64 + 16 * i + r][grp * 8 + 4];
      const float4 a0 = *(const float4*)&As[buf][wm * 64 + 16 * i + r][grp * 8];
      const float4 a1 = *(const float4*)&As[buf][wm * 64 + 16 * i + r][grp * 8 + 4];
      wf[i][0] = w0.x; wf[i][1] = w0.y; wf[i][2] = w0.z; wf[i][3] = w0.w;
      wf[i][4] = w1.x; wf[i][5] = w1.y; wf[i][6] = w1.z; wf[i][7] = w1.w;
      af[i][0] = a0.x; af[i][1] = a0.y; af[i][2] = a0.z; af[i][3] = a0.w;
      af[i][4] = a1.x; af[i][5] = a1.y; af[i][6] = a1.z; af[i][7] = a1.w;
    }
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(wf[i][s], af[j][s], acc[i][j], 0, 0, 0);
    if (kt + 1 < nk) store_tile(buf ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      epilogue_store(g, m0 + wm * 64 + 16 * j + r, n0 + wn * 64 + 16 * i + 4 * grp, acc[i][j]);
}


// ------------------------------------------------------------------ tile selection
// Register-staged configurations (BM, BN, BK, wavefronts along m) serve fp32 A operands
// (converted on their way into LDS) and K not a multiple of the DMA tile's BK; the
// LDS-DMA configurations (BM, BN, BK, stages, wavefronts along m) serve 16-bit operands.
typedef GemmCfg<128, 128, 32, 2> Cfg128x128k32;
typedef GemmCfg<128, 128, 64, 2> Cfg128x128k64;
typedef GemmCfg<64, 128, 64, 2> Cfg64x128k64;
typedef GemmCfg<128, 64, 64, 2> Cfg128x64k64;
typedef GemmCfg<64, 64, 64, 2> Cfg64x64k64;


// Tile identifiers (kf_gemm_tiled / kf_gemm_tile_info): 0 chooses automatically;
// register-staged tiles first, then the persistent LDS-DMA tiles (BM x BN x BK, stages,
// wavefronts). The automatic choice uses only some of these; the rest stay selectable so
// that tests can pin bit-identity across tilings and sweeps can compare them.
enum {
  TILE_AUTO = 0, TILE_128x128k32 = 1, TILE_128x128k64 = 2, TILE_64x128k64 = 3,
  TILE_128x64k64 = 4, TILE_64x64k64 = 5,
  DMA_FIRST = 6,
  DMA_128x128k32s4w4 = 6, DMA_128x128k32s4w8 = 7, DMA_128x64k32s3w4 = 8,
  DMA_256x128k32s3w8 = 9, DMA_128x256k32s3w8 = 10, DMA_64x64k32s3w4 = 11,
  DMA_128x128k32s3w8 = 12, DMA_128x64k64s3w8 = 13, DMA_128x128k64s2w4 = 14,
  DMA_128x128k64s2w8 = 15, DMA_128x256k64s2w8 = 16, DMA_128x256k64s3w8 = 17,
  DMA_256x128k64s2w8 = 18, DMA_256x256k64s2w8 = 19, DMA_256x256k32s2w8 = 20,
  TILE_LAST = 20
};

// (BM, BN, BK, stages, wavefronts, LDS-DMA) of every tile id, in id order; the launch
// switch in launch_tile instantiates exactly these.
struct TileInfo { int bm, bn, bk, stages, waves, dma; };
constexpr TileInfo kTileInfo[TILE_LAST + 1] = {
    {0, 0, 0, 0, 0, 0},
    {128, 128, 32, 2, 4, 0}, {128, 128, 64, 2, 4, 0}, {64, 128, 64, 2, 4, 0},
    {128, 64, 64, 2, 4, 0}, {64, 64, 64, 2, 4, 0},
    {128, 128, 32, 4, 4, 1}, {128, 128, 32, 4, 8, 1}, {128, 64, 32, 3, 4, 1},
    {256, 128, 32, 3, 8, 1}, {128, 256, 32, 3, 8, 1}, {64, 64, 32, 3, 4, 1},
    {128, 128, 32, 3, 8, 1}, {128, 64, 64, 3, 8, 1}, {128, 128, 64, 2, 4, 1},
    {128, 128, 64, 2, 8, 1}, {128, 256, 64, 2, 8, 1}, {128, 256, 64, 3, 8, 1},
    {256, 128, 64, 2, 8, 1}, {256, 256, 64, 2, 8, 1}, {256, 256, 32, 2, 8, 1},
};

template <int MODE, int AT, class C, int EPI>
static void launch_cfg(const GemmArgs& g, hipStream_t st) {
  const int64_t blocks = ((int64_t)(g.M + C::BM - 1) / C::BM) * ((g.N + C::BN - 1) / C::BN);
  hipLaunchKernelGGL((gemm16_kernel<MODE, AT, C, EPI>), dim3((unsigned)blocks), dim3(256), 0, st, g);
}

template <int MODE, class C, int EPI>
static void launch_dma(const GemmArgs& g, hipStream_t st) {
  constexpr int LDS = C::lds_bytes(a_planes<MODE>(), w_planes<MODE>());
  if constexpr (LDS > 160 * 1024) {      // too big for this mode: default tile
    launch_dma<MODE, DmaCfg<128, 128, 32, 4, 2, 4>, EPI>(g, st);
  } else {
    constexpr int per_cu_lds = 160 * 1024 / LDS;
    constexpr int per_cu_waves = 32 / C::NWAVES;           // 8 wavefronts per SIMD
    constexpr int occ = per_cu_lds < per_cu_waves ? per_cu_lds : per_cu_waves;
    const int64_t tiles = ((int64_t)(g.M + C::BM - 1) / C::BM) * ((g.N + C::BN - 1) / C::BN);
    int64_t grid = (int64_t)cu_count() * occ;
    // Grids that cover every tile at once keep one tile per block (rounding them down to
    // the XCD count would give some blocks a second tile: C1's QKV GEMM, 12 tiles, ran
    // two rounds on 8 blocks); larger ones are a multiple of the XCD count, each XCD
    // walking a contiguous tile range.
    if (grid >= tiles) grid = tiles;
    else if (grid >= kXcds) grid -= grid % kXcds;
    // Grouped tile walk where the grid takes many rounds of tiles: measured on MI355X
    // (outputs bit-identical), C5's QKV GEMM (96 rounds) 5.3 -> 4.8 ms with groups of 8
    // row blocks, C4's ffn_in (~16 rounds) 390 -> 365 us with 4; grids of one or two rounds
    // (C2) ran up to 18 % slower grouped, so they keep the row-major walk.
    GemmArgs ga = g;
    const int64_t rounds = tiles / grid;
    ga.group = rounds >= 32 ? 8 : rounds >= 8 ? 4 : 1;
    hipLaunchKernelGGL((gemm_dma_kernel<MODE, C, EPI>), dim3((unsigned)grid), dim3(C::NT), 0, st, ga);
  }
}

template <int MODE, int AT, int EPI = 0>
static void launch_tile(const GemmArgs& g, int tile, hipStream_t st) {
  static_assert(MODE != MODE_F16X2 || AT == KF_F16, "f16x2 takes one fp16 A plane");
  if constexpr (AT != KF_F32) {
    switch (tile) {
      case DMA_128x128k32s4w4: return launch_dma<MODE, DmaCfg<128, 128, 32, 4, 2, 2>, EPI>(g, st);
      case DMA_128x128k32s4w8: return launch_dma<MODE, DmaCfg<128, 128, 32, 4, 2, 4>, EPI>(g, st);
      case DMA_128x64k32s3w4: return launch_dma<MODE, DmaCfg<128, 64, 32, 3, 2, 2>, EPI>(g, st);
      case DMA_256x128k32s3w8: return launch_dma<MODE, DmaCfg<256, 128, 32, 3, 4, 2>, EPI>(g, st);
      case DMA_128x256k32s3w8: return launch_dma<MODE, DmaCfg<128, 256, 32, 3, 2, 4>, EPI>(g, st);
      case DMA_64x64k32s3w4: return launch_dma<MODE, DmaCfg<64, 64, 32, 3, 2, 2>, EPI>(g, st);
      case DMA_128x128k32s3w8: return launch_dma<MODE, DmaCfg<128, 128, 32, 3, 2, 4>, EPI>(g, st);
      case DMA_128x64k64s3w8: return launch_dma<MODE, DmaCfg<128, 64, 64, 3, 4, 2>, EPI>(g, st);
      case DMA_128x128k64s2w4: return launch_dma<MODE, DmaCfg<128, 128, 64, 2, 2, 2>, EPI>(g, st);
      case DMA_128x128k64s2w8: return launch_dma<MODE, DmaCfg<128, 128, 64, 2, 2, 4, 4>, EPI>(g, st);
      case DMA_128x256k64s2w8: return launch_dma<MODE, DmaCfg<128, 256, 64, 2, 2, 4>, EPI>(g, st);
      case DMA_128x256k64s3w8: return launch_dma<MODE, DmaCfg<128, 256, 64, 3, 2, 4>, EPI>(g, st);
      case DMA_256x128k64s2w8: return launch_dma<MODE, DmaCfg<256, 128, 64, 2, 4, 2>, EPI>(g, st);
      case DMA_256x256k64s2w8: return launch_dma<MODE, DmaCfg<256, 256, 64, 2, 4, 2>, EPI>(g, st);
      case DMA_256x256k32s2w8: return launch_dma<MODE, DmaCfg<256, 256, 32, 2, 4, 2>, EPI>(g, st);
      default: break;
    }
  }
  if constexpr (MODE == MODE_F16X2) {
    return;      // the entry points only pass DMA tiles for f16x2 (checked there)
  } else {
  // register-staged kernels: the generic attention-layout epilogue (k / v^T type read from
  // GemmArgs at run time) or the generic plain one
  constexpr int ER = (EPI == 1 || EPI == 5) ? 1 : 0;
  switch (tile) {
    case TILE_128x128k32: launch_cfg<MODE, AT, Cfg128x128k32, ER>(g, st); break;
    case TILE_128x128k64: launch_cfg<MODE, AT, Cfg128x128k64, ER>(g, st); break;
    case TILE_64x128k64: launch_cfg<MODE, AT, Cfg64x128k64, ER>(g, st); break;
    case TILE_128x64k64: launch_cfg<MODE, AT, Cfg128x64k64, ER>(g, st); break;
    default: launch_cfg<MODE, AT, Cfg64x64k64, ER>(g, st); break;
  }
  }
}

// One MFMA mode, every A format it accepts and every epilogue (EPI 0: generic, 1:
// attention layout, 2: fp32 out, 3: GELU to the mode's 16-bit type, 4: GELU to its
// planes, 5: attention layout with single-plane k / v^T from a split mode; 2-4 only for
// 16-bit A, the LDS-DMA kernels). Instantiated once per mode, each in its own
// translation unit.
template <int MODE, int AT>
void launch_epi(const GemmArgs& g, int tile, int epi, hipStream_t st) {
  switch (epi) {
    case 1: launch_tile<MODE, AT, 1>(g, tile, st); break;
    case 5:
      if constexpr (MODE == MODE_F16X3 || MODE == MODE_BF16X3) launch_tile<MODE, AT, 5>(g, tile, st);
      break;
    case 2: launch_tile<MODE, AT, 2>(g, tile, st); break;
    case 3: launch_tile<MODE, AT, 3>(g, tile, st); break;
    case 4: launch_tile<MODE, AT, 4>(g, tile, st); break;
    default: launch_tile<MODE, AT, 0>(g, tile, st); break;
  }
}
template <int MODE, int A16>
void launch_mode(const GemmArgs& g, int a_dtype, int tile, int epi, hipStream_t st) {
  if constexpr (MODE == MODE_F16X2) {
    launch_epi<MODE, KF_F16>(g, tile, epi, st);
  } else {
    if (a_dtype == KF_F32) {
      if (epi == 1 || epi == 5) launch_tile<MODE, KF_F32, 1>(g, tile, st);   // run-time k type
      else launch_tile<MODE, KF_F32, 0>(g, tile, st);
    } else {
      launch_epi<MODE, A16>(g, tile, epi, st);
    }
  }
}

void gemm_launch_f16(const GemmArgs& g, int a_dtype, int tile, int epi, hipStream_t st);
void gemm_launch_bf16(const GemmArgs& g, int a_dtype, int tile, int epi, hipStream_t st);
void gemm_launch_f16x3(const GemmArgs& g, int a_dtype, int tile, int epi, hipStream_t st);
void gemm_launch_bf16x3(const GemmArgs& g, int a_dtype, int tile, int epi, hipStream_t st);
void gemm_launch_f16x2(const GemmArgs& g, int a_dtype, int tile, int epi, hipStream_t st);
void gemm_launch_f32(const GemmArgs& g, int a_dtype, hipStream_t st);

}  // namespace kf
