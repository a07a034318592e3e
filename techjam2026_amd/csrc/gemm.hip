// MFMA GEMM with bias / erf-GELU / cast epilogue for gfx950:
//   C[M, N] = act(A[M, K] . W[N, K]^T + bias[N])
// covering the fused QKV projection, out_proj, ffn_in(+GELU) and ffn_out of the layer
// (kernelforge/optimized.py:441-446, 483, 572-574).
//
// Tiling: a 256-thread block computes a 128 x 128 tile of C with four wavefronts arranged
// 2 x 2, each owning 64 (n) x 64 (m) = 4 x 4 v_mfma_f32_16x16x32 tiles. The product is
// formed as C^T = W . A^T (W rows are the MFMA "A" operand, A rows the "B" operand), so
// every lane ends with four consecutive output columns of one row and stores them with one
// vector write. K advances 32 at a time through a double-buffered LDS stage: the global
// loads for step k+1 are issued before the MFMAs of step k, and a single barrier per step
// separates the LDS write of one buffer from the reads of the other.
//
// Precision: fp32 activations are rounded (F16/BF16) or split into hi + lo (F16X3/BF16X3)
// while they are written to LDS; weights arrive pre-split from kf_split. Split modes issue
// hi*hi + hi*lo + lo*hi per tile. KF_MMA_F32 runs the fp32 MFMA (16x16x4) on fp32 tiles.
#include "kf_common.h"

namespace kf {

struct GemmArgs {
  const void* a; int64_t lda;
  const void* w_hi; const void* w_lo; int64_t ldw;
  const float* bias;
  void* c; int c_dtype; int64_t ldc;
  int M, N, K; int act;
};

constexpr int GBM = 128, GBN = 128, GBK = 32;

__device__ __forceinline__ void epilogue_store(const GemmArgs& g, int m, int n, f32x4 acc) {
  if (m >= g.M || n >= g.N) return;
  float v[4] = {acc[0], acc[1], acc[2], acc[3]};
  if (g.bias) {
    const float4 bv = *(const float4*)(g.bias + n);
    v[0] += bv.x; v[1] += bv.y; v[2] += bv.z; v[3] += bv.w;
  }
  if (g.act == KF_ACT_GELU_ERF) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = gelu_erf(v[i]);
  }
  const int64_t off = (int64_t)m * g.ldc + n;
  if (g.c_dtype == KF_F32) {
    *(float4*)((float*)g.c + off) = make_float4(v[0], v[1], v[2], v[3]);
  } else if (g.c_dtype == KF_F16) {
    half4 o = {(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
    *(half4*)((_Float16*)g.c + off) = o;
  } else {
    typedef __bf16 b4 __attribute__((ext_vector_type(4)));
    b4 o = {(__bf16)v[0], (__bf16)v[1], (__bf16)v[2], (__bf16)v[3]};
    *(b4*)((__bf16*)g.c + off) = o;
  }
}

// ------------------------------------------------------------------ 16-bit MFMA modes
template <int MODE, int AT>
__global__ __launch_bounds__(256, 2) void gemm16_kernel(GemmArgs g) {
  using TR = ModeTraits<MODE>;
  using V = typename TR::vec;
  using E = typename TR::elem;
  constexpr int P = TR::split ? 2 : 1;
  constexpr int LDK = GBK + 8;   // 80-byte rows: conflict-free 16-byte fragment reads
  __shared__ __attribute__((aligned(16))) E As[2][P][GBM][LDK];
  __shared__ __attribute__((aligned(16))) E Ws[2][P][GBN][LDK];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, grp = lane >> 4;
  const int wn = wave >> 1, wm = wave & 1;
  const int ntn = (g.N + GBN - 1) / GBN;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int tm = tile / ntn, tn = tile % ntn;
  const int m0 = tm * GBM, n0 = tn * GBN;

  // global -> register staging: thread loads row (tid >> 1), 16 k-values at (tid & 1) * 16
  const int lrow = tid >> 1, lkc = (tid & 1) * 16;
  const int64_t am = (int64_t)m0 + lrow, wnrow = (int64_t)n0 + lrow;
  float areg[16];
  U4 wreg[P][2];

  auto load_tile = [&](int kt) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int kk = kt * GBK + lkc + 8 * c;
      const bool ok = am < g.M && kk < g.K;
      if (ok) {
        ld8<AT>(g.a, am * g.lda + kk, areg + 8 * c);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) areg[8 * c + i] = 0.0f;
      }
      const bool okw = wnrow < g.N && kk < g.K;
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const E* wp = (const E*)(p == 0 ? g.w_hi : g.w_lo);
        wreg[p][c] = okw ? *(const U4*)(wp + wnrow * g.ldw + kk) : U4{0, 0, 0, 0};
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      V hi, lo;
      if constexpr (TR::split) split8<E, V>(areg + 8 * c, hi, lo);
      else round8<E, V>(areg + 8 * c, hi);
      *(U4*)&As[buf][0][lrow][lkc + 8 * c] = as_u4(hi);
      if constexpr (TR::split) *(U4*)&As[buf][P - 1][lrow][lkc + 8 * c] = as_u4(lo);
#pragma unroll
      for (int p = 0; p < P; ++p) *(U4*)&Ws[buf][p][lrow][lkc + 8 * c] = wreg[p][c];
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
    V wf[4][P], af[4][P];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int p = 0; p < P; ++p) {
        wf[i][p] = from_u4<V>(*(const U4*)&Ws[buf][p][wn * 64 + 16 * i + r][grp * 8]);
        af[i][p] = from_u4<V>(*(const U4*)&As[buf][p][wm * 64 + 16 * i + r][grp * 8]);
      }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (TR::split) {
          acc[i][j] = mma16(wf[i][0], af[j][1], acc[i][j]);
          acc[i][j] = mma16(wf[i][1], af[j][0], acc[i][j]);
        }
        acc[i][j] = mma16(wf[i][0], af[j][0], acc[i][j]);
      }
    if (kt + 1 < nk) store_tile(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      epilogue_store(g, m0 + wm * 64 + 16 * j + r, n0 + wn * 64 + 16 * i + 4 * grp, acc[i][j]);
}

// ------------------------------------------------------------------ fp32 MFMA mode
// v_mfma_f32_16x16x4f32 takes one fp32 value per lane per operand. Lane (r, grp) supplies
// k = grp * 8 + s on sub-step s (s = 0..7), the same k for both operands, so 8 sub-steps
// cover the 32-wide K tile.
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

  auto load_tile = [&](int kt) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int kk = kt * GBK + lkc + 8 * c;
      if (am < g.M && kk < g.K) ld8<AT>(g.a, am * g.lda + kk, areg + 8 * c);
      else for (int i = 0; i < 8; ++i) areg[8 * c + i] = 0.0f;
      if (wnrow < g.N && kk < g.K) ld8<KF_F32>(g.w_hi, wnrow * g.ldw + kk, wreg + 8 * c);
      else for (int i = 0; i < 8; ++i) wreg[8 * c + i] = 0.0f;
    }
  };
  auto store_tile = [&](int buf) {
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

// ------------------------------------------------------------------ weight preparation
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

template <int MODE, int AT>
static void launch16(const GemmArgs& g, int blocks, hipStream_t st) {
  hipLaunchKernelGGL((gemm16_kernel<MODE, AT>), dim3(blocks), dim3(256), 0, st, g);
}

template <int MODE>
static void launch_mode(const GemmArgs& g, int a_dtype, int blocks, hipStream_t st) {
  switch (a_dtype) {
    case KF_F32: launch16<MODE, KF_F32>(g, blocks, st); break;
    case KF_F16: launch16<MODE, KF_F16>(g, blocks, st); break;
    default: launch16<MODE, KF_BF16>(g, blocks, st); break;
  }
}

static inline bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace kf

using namespace kf;

extern "C" int kf_gemm(const void* a, int a_dtype, int64_t lda,
                       const void* w_hi, const void* w_lo, int64_t ldw,
                       const float* bias,
                       void* c, int c_dtype, int64_t ldc,
                       int64_t M, int64_t N, int64_t K, int mode, int act, void* stream) {
  if (!a || !w_hi || !c || M < 0 || N <= 0 || K <= 0) {
    kf_set_error("kf_gemm: bad arguments (M=%lld N=%lld K=%lld)", (long long)M, (long long)N,
                 (long long)K);
    return KF_EINVAL;
  }
  if (mode < KF_MMA_F32 || mode > KF_MMA_BF16X3 || a_dtype < KF_F32 || a_dtype > KF_BF16 ||
      c_dtype < KF_F32 || c_dtype > KF_BF16 || (act != KF_ACT_NONE && act != KF_ACT_GELU_ERF)) {
    kf_set_error("kf_gemm: bad mode/dtype/act (%d/%d/%d/%d)", mode, a_dtype, c_dtype, act);
    return KF_EINVAL;
  }
  if ((mode == KF_MMA_F16X3 || mode == KF_MMA_BF16X3) && !w_lo) {
    kf_set_error("kf_gemm: split mode needs the lo weight plane");
    return KF_EINVAL;
  }
  if (K % 8 || N % 4 || lda % 8 || ldw % 8 || ldc % 4 || lda < K || ldw < K || ldc < N ||
      !al16(a) || !al16(w_hi) || (w_lo && !al16(w_lo)) || !al16(c) || (bias && !al16(bias))) {
    kf_set_error("kf_gemm: unsupported shape/alignment (M=%lld N=%lld K=%lld lda=%lld "
                 "ldw=%lld ldc=%lld): needs K%%8 == 0, N%%4 == 0 and 16-byte aligned rows",
                 (long long)M, (long long)N, (long long)K, (long long)lda, (long long)ldw,
                 (long long)ldc);
    return KF_EUNSUPPORTED;
  }
  if (M > (1LL << 30) || N > (1LL << 30) || K > (1LL << 30)) {
    kf_set_error("kf_gemm: dimension too large");
    return KF_EUNSUPPORTED;
  }
  if (M == 0) return KF_OK;
  const int64_t tiles = ((M + GBM - 1) / GBM) * ((N + GBN - 1) / GBN);
  if (tiles > 0x7fffffff) { kf_set_error("kf_gemm: grid too large"); return KF_EUNSUPPORTED; }
  GemmArgs g{a, lda, w_hi, w_lo, ldw, bias, c, c_dtype, ldc, (int)M, (int)N, (int)K, act};
  hipStream_t st = (hipStream_t)stream;
  const int blocks = (int)tiles;
  switch (mode) {
    case KF_MMA_F16: launch_mode<MODE_F16>(g, a_dtype, blocks, st); break;
    case KF_MMA_BF16: launch_mode<MODE_BF16>(g, a_dtype, blocks, st); break;
    case KF_MMA_F16X3: launch_mode<MODE_F16X3>(g, a_dtype, blocks, st); break;
    case KF_MMA_BF16X3: launch_mode<MODE_BF16X3>(g, a_dtype, blocks, st); break;
    default:
      switch (a_dtype) {
        case KF_F32: hipLaunchKernelGGL((gemm32_kernel<KF_F32>), dim3(blocks), dim3(256), 0, st, g); break;
        case KF_F16: hipLaunchKernelGGL((gemm32_kernel<KF_F16>), dim3(blocks), dim3(256), 0, st, g); break;
        default: hipLaunchKernelGGL((gemm32_kernel<KF_BF16>), dim3(blocks), dim3(256), 0, st, g); break;
      }
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    kf_set_error("kf_gemm: launch failed: %s", hipGetErrorString(e));
    return KF_ELAUNCH;
  }
  return KF_OK;
}

extern "C" int kf_split(const float* src, int64_t n, int mode, void* hi, void* lo, void* stream) {
  if (!src || !hi || n < 0) { kf_set_error("kf_split: bad arguments"); return KF_EINVAL; }
  const bool split = mode == KF_MMA_F16X3 || mode == KF_MMA_BF16X3;
  if (split && !lo) { kf_set_error("kf_split: split mode needs lo"); return KF_EINVAL; }
  if (n == 0) return KF_OK;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipStream_t st = (hipStream_t)stream;
  switch (mode) {
    case KF_MMA_F16: case KF_MMA_F16X3:
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
