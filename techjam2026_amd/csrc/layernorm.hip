// Fused residual add + row mask + LayerNorm for gfx950.
//
// Semantics of kernelforge/ops/layernorm.py:40-86 (one row of the residual stream at a
// time, fp32 arithmetic): s = (x + y) * keep; mean; centred biased variance;
// h = (s - mean) / sqrt(var + eps) * w + b; optionally h *= keep.
//
// Layout: rows are independent and HBM-bound (16 B per element with every flag on), so
// the fast path keeps a whole row in registers of LPR lanes (LPR = 64 for d >= 256, fewer
// lanes and several rows per wavefront for narrow rows such as d = 64), reads and writes
// it with 128-bit accesses exactly once, and reduces with cross-lane shuffles. A block of
// four wavefronts strides over row groups.
#include "kf_common.h"

namespace kf {

struct LnArgs {
  const float* x; int64_t ldx;
  const float* y; int64_t ldy;
  const void* keep; int keep_dtype;
  const float* w; const float* b;
  float* s; int64_t lds;
  void* h; void* h_lo; int h_dtype; int64_t ldh;
  int64_t M; int d; float eps; int flags;
};

// Streaming (non-temporal) 16-byte accesses for data read or written exactly once.
__device__ __forceinline__ float4 ld_stream4(const float* p) {
  const f32x4 v = __builtin_nontemporal_load((const f32x4*)p);
  return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void st_stream4(float* p, const float* v) {
  __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]}, (f32x4*)p);
}

__device__ __forceinline__ float keep_value(const void* keep, int dtype, int64_t row) {
  return ld_elem(keep, dtype, row) != 0.0f ? 1.0f : 0.0f;
}

// LPR lanes per row, NV float4 per lane (4 * LPR * NV >= d > 4 * LPR * (NV - 1)).
// The grid is sized to keep every CU busy and each row group strides over rows, loading
// the next row's x and y while it reduces and stores the current one; w and b are loaded
// once per thread.
// NT: stream x, y and s past the caches (non-temporal accesses).
template <int LPR, int NV, int HT, bool NT>
__global__ __launch_bounds__(256) void ln_rows_kernel(LnArgs a) {
  constexpr int kRowsPerWave = kWave / LPR;
  constexpr int kRowsPerBlock = kRowsPerWave * 4;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int li = lane % LPR;
  const int sub = lane / LPR;
  const bool has_y = a.flags & KF_LN_HAS_Y;
  const bool has_mask = a.flags & KF_LN_HAS_MASK;
  const bool mask_out = a.flags & KF_LN_MASK_OUT;
  const bool write_s = a.flags & KF_LN_WRITE_S;
  const float inv_d = 1.0f / (float)a.d;

  float4 wv[NV], bv[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (li + LPR * j) * 4;
    if (c < a.d) {
      wv[j] = *(const float4*)(a.w + c);
      bv[j] = *(const float4*)(a.b + c);
    } else {
      wv[j] = bv[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }

  auto load = [&](int64_t row, float4* xv, float4* yv) KF_INLINE {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      // Lanes past d load column 0 (always in bounds) and select zero: a conditional
      // load here was compiled as a select between the global address and a zero in
      // scratch memory, read with a flat load.
      const int c = (li + LPR * j) * 4;
      const bool ok = c < a.d;
      const int cc = ok ? c : 0;
      const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
      float4 xt, yt = z;
      if constexpr (NT) {
        xt = ld_stream4(a.x + row * a.ldx + cc);
        if (has_y) yt = ld_stream4(a.y + row * a.ldy + cc);
      } else {
        xt = *(const float4*)(a.x + row * a.ldx + cc);
        if (has_y) yt = *(const float4*)(a.y + row * a.ldy + cc);
      }
      xv[j] = ok ? xt : z;
      yv[j] = ok ? yt : z;
    }
  };

  const int64_t stride = (int64_t)gridDim.x * kRowsPerBlock;
  int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + wave * kRowsPerWave + sub;
  float4 xc[NV], yc[NV];
  if (row < a.M) load(row, xc, yc);
  for (; row < a.M; row += stride) {
    const int64_t nrow = row + stride;
    float4 xn[NV], yn[NV];
    if (nrow < a.M) load(nrow, xn, yn);
    float kv = 1.0f;
    if (has_mask) kv = keep_value(a.keep, a.keep_dtype, row);
    float v[NV][4];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      v[j][0] = (xc[j].x + yc[j].x) * kv;
      v[j][1] = (xc[j].y + yc[j].y) * kv;
      v[j][2] = (xc[j].z + yc[j].z) * kv;
      v[j][3] = (xc[j].w + yc[j].w) * kv;
    }
    if (write_s) {
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int c = (li + LPR * j) * 4;
        if (c < a.d)
          if constexpr (NT) st_stream4(a.s + row * a.lds + c, v[j]);
          else *(float4*)(a.s + row * a.lds + c) = make_float4(v[j][0], v[j][1], v[j][2], v[j][3]);
      }
    }
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) sum += (v[j][0] + v[j][1]) + (v[j][2] + v[j][3]);
    const float mean = wave_sum<LPR>(sum) * inv_d;
    float sq = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int c = (li + LPR * j) * 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[j][e] = (c < a.d) ? v[j][e] - mean : 0.0f;
        sq += v[j][e] * v[j][e];
      }
    }
    const float var = wave_sum<LPR>(sq) * inv_d;
    const float rstd = 1.0f / sqrtf(var + a.eps);
    const float hscale = (mask_out && has_mask) ? kv : 1.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int c = (li + LPR * j) * 4;
      if (c < a.d) {
        float o[4];
        o[0] = (v[j][0] * rstd * wv[j].x + bv[j].x) * hscale;
        o[1] = (v[j][1] * rstd * wv[j].y + bv[j].y) * hscale;
        o[2] = (v[j][2] * rstd * wv[j].z + bv[j].z) * hscale;
        o[3] = (v[j][3] * rstd * wv[j].w + bv[j].w) * hscale;
        store4_any(a.h, a.h_lo, HT, row * a.ldh + c, o);
      }
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      xc[j] = xn[j];
      yc[j] = yn[j];
    }
  }
}

// Generic path: any d, any element types. One block per row, three passes over global
// memory (sum, centred sum of squares, output).
struct LnGenericArgs {
  const void* x; int x_dtype; int64_t ldx;
  const void* y; int y_dtype; int64_t ldy;
  const void* keep; int keep_dtype;
  const void* w; const void* b; int wb_dtype;
  void* s; int s_dtype; int64_t lds;
  void* h; void* h_lo; int h_dtype; int64_t ldh;
  int64_t M; int64_t d; float eps; int flags;
};

__device__ float block_sum(float v, float* red) {
  v = wave_sum<kWave>(v);
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.0f;
  for (int i = 0; i < (int)(blockDim.x / kWave); ++i) t += red[i];
  return t;
}

__global__ __launch_bounds__(256) void ln_generic_kernel(LnGenericArgs a) {
  __shared__ float red[4];
  const bool has_y = a.flags & KF_LN_HAS_Y;
  const bool has_mask = a.flags & KF_LN_HAS_MASK;
  for (int64_t row = blockIdx.x; row < a.M; row += gridDim.x) {
    const float kv = has_mask ? keep_value(a.keep, a.keep_dtype, row) : 1.0f;
    auto sval = [&](int64_t c) KF_INLINE {
      float t = ld_elem(a.x, a.x_dtype, row * a.ldx + c);
      if (has_y) t += ld_elem(a.y, a.y_dtype, row * a.ldy + c);
      return t * kv;
    };
    float sum = 0.0f;
    for (int64_t c = threadIdx.x; c < a.d; c += blockDim.x) sum += sval(c);
    const float mean = block_sum(sum, red) / (float)a.d;
    float sq = 0.0f;
    for (int64_t c = threadIdx.x; c < a.d; c += blockDim.x) {
      const float t = sval(c) - mean;
      sq += t * t;
    }
    const float var = block_sum(sq, red) / (float)a.d;
    const float rstd = 1.0f / sqrtf(var + a.eps);
    const float hscale = ((a.flags & KF_LN_MASK_OUT) && has_mask) ? kv : 1.0f;
    for (int64_t c = threadIdx.x; c < a.d; c += blockDim.x) {
      const float t = sval(c);
      if (a.flags & KF_LN_WRITE_S) st_elem(a.s, a.s_dtype, row * a.lds + c, t);
      const float o = ((t - mean) * rstd * ld_elem(a.w, a.wb_dtype, c) +
                       ld_elem(a.b, a.wb_dtype, c)) * hscale;
      st_elem(a.h, a.h_dtype, row * a.ldh + c, o, a.h_lo);
    }
  }
}

template <int LPR, int NV>
static hipError_t launch_rows(const LnArgs& a, hipStream_t st) {
  constexpr int kRowsPerBlock = (kWave / LPR) * 4;
  const int64_t xbytes = a.M * a.d * 4;
  int64_t blocks = (a.M + kRowsPerBlock - 1) / kRowsPerBlock;
  // Blocks per CU (rows beyond: grid stride): operands of 64 MB and more stream best from
  // two blocks per CU, measured on MI355X (d 1024, x, y, s fp32): 262144 rows 5.10 -> 5.25
  // TB/s with f16x2 h and 5.16 -> 5.35 with fp16 h against eight blocks per CU, 131072
  // rows 5.23 -> 5.36 / 6.35 -> 6.53, 32768 rows unchanged. Smaller operands: four blocks
  // per CU for rows of 64 lanes (8192 x 512: 10.8 -> 10.2 us, each wave takes two rows and
  // prefetches the second), eight for the narrow rows (65536 x 64: 10.9 us at eight, 11.3
  // at four).
  const int64_t resident = (int64_t)cu_count() * (xbytes >= (64LL << 20) ? 2 : LPR == 64 ? 4 : 8);
  if (blocks > resident) blocks = resident;
  if (blocks < 1) blocks = 1;
  // Streaming accesses measured on MI355X (x, y, s fp32, h f16x2): 32768 x 1024 rows
  // 5.28 -> 6.43 TB/s, 262144 x 1024 5.13 -> 4.97, 8192 x 512 slower; so they are used
  // for operands between 64 MB and 512 MB only.
  const bool nt = xbytes >= (64LL << 20) && xbytes <= (512LL << 20);
#define KF_LN_LAUNCH(HT)                                                                           \
  if (nt) hipLaunchKernelGGL((ln_rows_kernel<LPR, NV, HT, true>), dim3(blocks), dim3(256), 0, st, a); \
  else hipLaunchKernelGGL((ln_rows_kernel<LPR, NV, HT, false>), dim3(blocks), dim3(256), 0, st, a)
  switch (a.h_dtype) {
    case KF_F32: KF_LN_LAUNCH(KF_F32); break;
    case KF_F16: KF_LN_LAUNCH(KF_F16); break;
    case KF_BF16: KF_LN_LAUNCH(KF_BF16); break;
    case KF_F16X2: KF_LN_LAUNCH(KF_F16X2); break;
    default: KF_LN_LAUNCH(KF_BF16X2); break;
  }
#undef KF_LN_LAUNCH
  return hipGetLastError();
}

static hipError_t dispatch_rows(const LnArgs& a, hipStream_t st) {
  const int nv4 = (a.d + 3) / 4;   // float4 per row
  if (nv4 <= 16) return launch_rows<16, 1>(a, st);
  if (nv4 <= 32) return launch_rows<32, 1>(a, st);
  switch ((nv4 + 63) / 64) {
    case 1: return launch_rows<64, 1>(a, st);
    case 2: return launch_rows<64, 2>(a, st);
    case 3: return launch_rows<64, 3>(a, st);
    case 4: return launch_rows<64, 4>(a, st);
    case 5: case 6: return launch_rows<64, 6>(a, st);
    case 7: case 8: return launch_rows<64, 8>(a, st);
    case 9: case 10: case 11: case 12: return launch_rows<64, 12>(a, st);
    default: return launch_rows<64, 16>(a, st);
  }
}

static inline bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace kf

using namespace kf;

extern "C" int kf_add_mask_ln(const void* x, int x_dtype, int64_t ldx,
                              const void* y, int y_dtype, int64_t ldy,
                              const void* keep, int keep_dtype,
                              const void* w, const void* b, int wb_dtype,
                              void* s_out, int s_dtype, int64_t lds,
                              void* h_out, void* h_lo, int h_dtype, int64_t ldh,
                              int64_t M, int64_t d, float eps, int flags, void* stream) {
  const bool has_y = flags & KF_LN_HAS_Y, has_mask = flags & KF_LN_HAS_MASK;
  const bool write_s = flags & KF_LN_WRITE_S;
  if (M < 0 || d <= 0 || !x || !w || !b || !h_out || (has_y && !y) || (has_mask && !keep) ||
      (write_s && !s_out)) {
    kf_set_error("kf_add_mask_ln: bad arguments (M=%lld d=%lld flags=%d)", (long long)M,
                 (long long)d, flags);
    return KF_EINVAL;
  }
  if (ldx < d || (has_y && ldy < d) || (write_s && lds < d) || ldh < d) {
    kf_set_error("kf_add_mask_ln: row stride smaller than d");
    return KF_EINVAL;
  }
  for (int t : {x_dtype, y_dtype, s_dtype, wb_dtype})
    if (t < KF_F32 || t > KF_BF16) { kf_set_error("kf_add_mask_ln: bad dtype %d", t); return KF_EINVAL; }
  const bool h_planes = h_dtype == KF_F16X2 || h_dtype == KF_BF16X2;
  if (h_dtype < KF_F32 || h_dtype == KF_U8 || h_dtype > KF_BF16X2 || (h_planes && !h_lo)) {
    kf_set_error("kf_add_mask_ln: bad h dtype %d (or missing lo plane)", h_dtype);
    return KF_EINVAL;
  }
  if (keep_dtype < KF_F32 || keep_dtype > KF_U8) { kf_set_error("kf_add_mask_ln: bad keep dtype"); return KF_EINVAL; }
  if (M == 0) return KF_OK;
  hipStream_t st = (hipStream_t)stream;

  const bool fast = d <= 4096 && d % 4 == 0 && x_dtype == KF_F32 && wb_dtype == KF_F32 &&
                    (!has_y || y_dtype == KF_F32) && (!write_s || s_dtype == KF_F32) &&
                    ldx % 4 == 0 && (!has_y || ldy % 4 == 0) && (!write_s || lds % 4 == 0) &&
                    ldh % 4 == 0 && al16(x) && (!has_y || al16(y)) && (!write_s || al16(s_out)) &&
                    al16(h_out) && (!h_planes || al16(h_lo)) && al16(w) && al16(b);
  hipError_t e;
  if (fast) {
    LnArgs a{(const float*)x, ldx, (const float*)y, ldy, keep, keep_dtype, (const float*)w,
             (const float*)b, (float*)s_out, lds, h_out, h_lo, h_dtype, ldh, M, (int)d, eps, flags};
    e = dispatch_rows(a, st);
  } else {
    LnGenericArgs a{x, x_dtype, ldx, y, y_dtype, ldy, keep, keep_dtype, w, b, wb_dtype,
                    s_out, s_dtype, lds, h_out, h_lo, h_dtype, ldh, M, d, eps, flags};
    int64_t blocks = M < 65536 ? M : 65536;
    hipLaunchKernelGGL(ln_generic_kernel, dim3(blocks), dim3(256), 0, st, a);
    e = hipGetLastError();
  }
  if (e != hipSuccess) {
    kf_set_error("kf_add_mask_ln: launch failed: %s", hipGetErrorString(e));
    return KF_ELAUNCH;
  }
  return KF_OK;
}
