// Shared definitions for the gfx950 kernels of libkf950.
//
// Everything here is CDNA4-specific: 64-lane wavefronts, v_mfma_f32_16x16x32_{f16,bf16}
// (eight 16-bit operands per lane), 160 KB of LDS per CU and 8 XCDs that each own an L2.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kf950.h"

// Kernel-local lambdas capture register arrays (accumulators, fragments) by reference;
// a lambda left out of line forces those arrays into scratch memory, so every one is
// inlined. (Measured: the QKV epilogue made the inliner give up on 4-tile-wide
// GEMM configurations, which then ran ~30x slower from scratch.)
#define KF_INLINE __attribute__((always_inline))

namespace kf {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bhalf8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef __bf16 bhalf4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kXcds = 8;

// ---------------------------------------------------------------- numerics
// MFMA input precision. The split modes carry each fp32 operand as hi + lo in a 16-bit
// format and accumulate hi*hi + hi*lo + lo*hi in fp32: f16x3 keeps 22 significand bits
// (fp32 needs 24), bf16x3 keeps 16 bits but cannot overflow.
enum Mode : int {
  MODE_F16 = KF_MMA_F16,
  MODE_BF16 = KF_MMA_BF16,
  MODE_F16X3 = KF_MMA_F16X3,
  MODE_BF16X3 = KF_MMA_BF16X3,
  MODE_F16X2 = KF_MMA_F16X2,
  MODE_F32 = KF_MMA_F32,
};

template <int M> struct ModeTraits;
template <> struct ModeTraits<MODE_F16> { typedef half8 vec; typedef _Float16 elem; static constexpr bool split = false; };
template <> struct ModeTraits<MODE_BF16> { typedef bhalf8 vec; typedef __bf16 elem; static constexpr bool split = false; };
template <> struct ModeTraits<MODE_F16X3> { typedef half8 vec; typedef _Float16 elem; static constexpr bool split = true; };
template <> struct ModeTraits<MODE_BF16X3> { typedef bhalf8 vec; typedef __bf16 elem; static constexpr bool split = true; };
// A single fp16 plane, W split (GEMM only): "split" (3-MFMA, both operands in planes) is false
template <> struct ModeTraits<MODE_F16X2> { typedef half8 vec; typedef _Float16 elem; static constexpr bool split = false; };
// planes of the A and W operands of a GEMM in MFMA mode M
template <int M> constexpr int a_planes() { return ModeTraits<M>::split ? 2 : 1; }
template <int M> constexpr int w_planes() { return (ModeTraits<M>::split || M == MODE_F16X2) ? 2 : 1; }

__device__ __forceinline__ f32x4 mma16(const half8& a, const half8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma16(const bhalf8& a, const bhalf8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// 16-byte value as raw dwords, for LDS stores of eight 16-bit elements.
struct alignas(16) U4 { uint32_t x, y, z, w; };

template <typename V> __device__ __forceinline__ U4 as_u4(const V& v) {
  static_assert(sizeof(V) == 16, "16-byte vector expected");
  return __builtin_bit_cast(U4, v);
}
template <typename V> __device__ __forceinline__ V from_u4(const U4& u) {
  return __builtin_bit_cast(V, u);
}


template <typename E, typename V>
__device__ __forceinline__ void round8(const float* x, V& hi) {
#pragma unroll
  for (int i = 0; i < 8; ++i) hi[i] = (E)x[i];
}

// The fp32 value a hi / lo plane split starts from, made opaque to the optimizer. Under
// floating-point contraction the compiler may fold the producer's last product into each
// 16-bit conversion separately -- the hi plane rounded from the fp32 product, the
// residual taken against a hi re-rounded from the exact product -- and where a value lies
// on an fp16 tie those two hi differ by an ulp, so hi + lo missed the value by that ulp
// (measured: 56 of 768000 GELU outputs, errors of 2^-9 at 2.0). Splitting one
// materialised fp32 value gives hi = round(v) and lo = round(v - hi) in every kernel.
__device__ __forceinline__ float plane_src(float x) {
  asm volatile("" : "+v"(x));
  return x;
}
// hi / lo planes of N values (16-bit type T, vectors V), and of one value
template <typename T, int N, typename V>
__device__ __forceinline__ void split_n(const float* v, V& hi, V& lo) {
#pragma unroll
  for (int e = 0; e < N; ++e) {
    const float x = plane_src(v[e]);
    const T h = (T)x;
    hi[e] = h;
    lo[e] = (T)(x - (float)h);
  }
}
template <typename T>
__device__ __forceinline__ void split_1(float v, T& hi, T& lo) {
  const float x = plane_src(v);
  hi = (T)x;
  lo = (T)(x - (float)hi);
}

// Split eight fp32 values into hi (nearest 16-bit value) and lo (nearest 16-bit value of
// the exact remainder x - hi), from one opaque fp32 value each (plane_src).
template <typename E, typename V>
__device__ __forceinline__ void split8(const float* x, V& hi, V& lo) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float v = plane_src(x[i]);
    const E h = (E)v;
    hi[i] = h;
    lo[i] = (E)(v - (float)h);
  }
}

__device__ __forceinline__ half4 cvt4h(const float* v) {
  return half4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
}
__device__ __forceinline__ bhalf4 cvt4b(const float* v) {
  return bhalf4{(__bf16)v[0], (__bf16)v[1], (__bf16)v[2], (__bf16)v[3]};
}

// Store four fp32 values at element offset `off` as dtype (X2: hi plane at p, lo at p_lo).
__device__ __forceinline__ void store4_any(void* p, void* p_lo, int dtype, int64_t off,
                                           const float* v) {
  switch (dtype) {
    case KF_F32: *(float4*)((float*)p + off) = make_float4(v[0], v[1], v[2], v[3]); break;
    case KF_F16: *(half4*)((_Float16*)p + off) = cvt4h(v); break;
    case KF_BF16: *(bhalf4*)((__bf16*)p + off) = cvt4b(v); break;
    case KF_F16X2: {
      half4 hi, lo;
      split_n<_Float16, 4>(v, hi, lo);
      *(half4*)((_Float16*)p + off) = hi;
      *(half4*)((_Float16*)p_lo + off) = lo;
      break;
    }
    default: {
      bhalf4 hi, lo;
      split_n<__bf16, 4>(v, hi, lo);
      *(bhalf4*)((__bf16*)p + off) = hi;
      *(bhalf4*)((__bf16*)p_lo + off) = lo;
      break;
    }
  }
}

// store4_any with the output type fixed at compile time (no per-element dtype branches).
template <int DT>
__device__ __forceinline__ void store4_t(void* p, void* p_lo, int64_t off, const float* v) {
  if constexpr (DT == KF_F32) {
    *(float4*)((float*)p + off) = make_float4(v[0], v[1], v[2], v[3]);
  } else if constexpr (DT == KF_F16) {
    *(half4*)((_Float16*)p + off) = cvt4h(v);
  } else if constexpr (DT == KF_BF16) {
    *(bhalf4*)((__bf16*)p + off) = cvt4b(v);
  } else if constexpr (DT == KF_F16X2) {
    half4 hi, lo;
    split_n<_Float16, 4>(v, hi, lo);
    *(half4*)((_Float16*)p + off) = hi;
    *(half4*)((_Float16*)p_lo + off) = lo;
  } else {
    static_assert(DT == KF_BF16X2, "output types");
    bhalf4 hi, lo;
    split_n<__bf16, 4>(v, hi, lo);
    *(bhalf4*)((__bf16*)p + off) = hi;
    *(bhalf4*)((__bf16*)p_lo + off) = lo;
  }
}

// one element of a 16-bit (or X2) output, type fixed at compile time: p[i] (and p_lo[i])
template <int DT>
__device__ __forceinline__ void st16_t(void* p, void* p_lo, int64_t i, float v) {
  if constexpr (DT == KF_F16) {
    ((_Float16*)p)[i] = (_Float16)v;
  } else if constexpr (DT == KF_BF16) {
    ((__bf16*)p)[i] = (__bf16)v;
  } else if constexpr (DT == KF_F16X2) {
    _Float16 h, l;
    split_1<_Float16>(v, h, l);
    ((_Float16*)p)[i] = h;
    ((_Float16*)p_lo)[i] = l;
  } else {
    static_assert(DT == KF_BF16X2, "16-bit output types");
    __bf16 h, l;
    split_1<__bf16>(v, h, l);
    ((__bf16*)p)[i] = h;
    ((__bf16*)p_lo)[i] = l;
  }
}

// ------------------------------------------------------------- element I/O
__device__ __forceinline__ float ld_elem(const void* p, int dtype, int64_t i) {
  switch (dtype) {
    case KF_F32: return ((const float*)p)[i];
    case KF_F16: return (float)((const _Float16*)p)[i];
    case KF_BF16: return (float)((const __bf16*)p)[i];
    default: return (float)((const uint8_t*)p)[i];
  }
}
__device__ __forceinline__ void st_elem(void* p, int dtype, int64_t i, float v,
                                        void* p_lo = nullptr) {
  switch (dtype) {
    case KF_F32: ((float*)p)[i] = v; break;
    case KF_F16: ((_Float16*)p)[i] = (_Float16)v; break;
    case KF_BF16: ((__bf16*)p)[i] = (__bf16)v; break;
    case KF_F16X2: {
      _Float16 h, l;
      split_1<_Float16>(v, h, l);
      ((_Float16*)p)[i] = h;
      ((_Float16*)p_lo)[i] = l;
      break;
    }
    default: {
      __bf16 h, l;
      split_1<__bf16>(v, h, l);
      ((__bf16*)p)[i] = h;
      ((__bf16*)p_lo)[i] = l;
      break;
    }
  }
}

// Load 8 consecutive elements starting at p[i] as fp32 (16- or 32-byte aligned vector loads).
template <int DT> __device__ __forceinline__ void ld8(const void* p, int64_t i, float* out);
template <> __device__ __forceinline__ void ld8<KF_F32>(const void* p, int64_t i, float* out) {
  const float4* q = (const float4*)((const float*)p + i);
  float4 a = q[0], b = q[1];
  out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
  out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
}
template <> __device__ __forceinline__ void ld8<KF_F16>(const void* p, int64_t i, float* out) {
  half8 v = *(const half8*)((const _Float16*)p + i);
#pragma unroll
  for (int k = 0; k < 8; ++k) out[k] = (float)v[k];
}
template <> __device__ __forceinline__ void ld8<KF_BF16>(const void* p, int64_t i, float* out) {
  bhalf8 v = *(const bhalf8*)((const __bf16*)p + i);
#pragma unroll
  for (int k = 0; k < 8; ++k) out[k] = (float)v[k];
}

// ------------------------------------------------------------ LDS DMA
// global_load_lds_dwordx4: every lane copies 16 bytes from its own global address; the
// wavefront's 64 chunks land contiguously (lane order) from a wave-uniform LDS address.
typedef __attribute__((address_space(3))) void* lds_addr_t;
typedef __attribute__((address_space(1))) void* gbl_addr_t;

__device__ __forceinline__ void dma16(const void* src, void* lds_dst) {
  __builtin_amdgcn_global_load_lds((gbl_addr_t)const_cast<void*>(src), (lds_addr_t)lds_dst, 16, 0, 0);
}

// The same copy through a buffer resource (MUBUF buffer_load_dwordx4 ... lds): counted on
// vmcnt only. The FLAT-encoded global_load_lds also counts as a possible LDS access in the
// compiler's wait tracking, which then waits for every outstanding LDS read (lgkmcnt(0))
// wherever one result is needed; with buffer copies in flight its LDS-read waits stay exact.
// The resource spans the whole address range (no bounds clamp); voff is the lane's byte
// offset, soff a wave-uniform byte offset.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, -1, 0x00020000);
}
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t r, int voff, int soff, void* lds_dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_addr_t)lds_dst, 16, voff, soff, 0, 0);
}

// Wait until at most N vector-memory operations of this wavefront are outstanding
// (vmcnt only; LDS and export counters left unconstrained).
template <int N> __device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (((N >> 4) & 3) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier that does not drain outstanding global->LDS copies (the fence of
// __syncthreads waits for vmcnt(0), which would serialise a multi-stage copy pipeline).
// This wavefront's own LDS reads are complete before it arrives; visibility of copied
// data is established by wait_vmcnt in every wavefront before the barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// ------------------------------------------------------------ wave helpers
template <int WIDTH>
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = WIDTH / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, WIDTH);
  return v;
}

// Blocks are dealt to the 8 XCDs round-robin by linear block id. Renumber so that each XCD
// receives a contiguous range of logical tiles: tiles that share operands (the same
// attention head, the same GEMM row panel) then share one L2.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  if (nblocks % kXcds != 0) return bid;
  const int per = nblocks / kXcds;
  return (bid % kXcds) * per + bid / kXcds;
}

// Compute units of the current device (host side, cached; abi.hip).
int cu_count();

__device__ __forceinline__ float gelu_erf(float x) {
  return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f));
}

}  // namespace kf

// Error reporting shared by the entry points (defined in abi.hip).
// per-thread error message behind kf_last_error (library-internal: not exported)
extern "C" __attribute__((visibility("hidden"))) void kf_set_error(const char* fmt, ...);
