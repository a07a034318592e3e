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

__device__ __forceinline__ float keep_value(const void* keep, int dtype, int64_t row) {
  return ld_elem(keep, dtype, row) != 0.0f ? 1.0f : 0.0f;
}

// LPR lanes per row, NV float4 per lane (4 * LPR * NV >= d > 4 * LPR * (NV - 1)).
template <int LPR, int NV, int HT>
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

  for (int64_t base = (int64_t)blockIdx.x * kRowsPerBlock; base < a.M;
       base += (int64_t)gridDim.x * kRowsPerBlock) {
    const int64_t row = base + wave * kRowsPerWave + sub;
    if (row >= a.M) continue;   // whole row-group of lanes leaves together
    float v[NV][4];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int c = (li + LPR * j) * 4;
      if (c < a.d) {
        float4 xv = *(const float4*)(a.x + row * a.ldx + c);
        v[j][0] = xv.x; v[j][1] = xv.y; v[j][2] = xv.z; v[j][3] = xv.w;
        if (has_y) {
          float4 yv = *(const float4*)(a.y + row * a.ldy + c);
          v[j][0] += yv.x; v[j][1] += yv.y; v[j][2] += yv.z; v[j][3] += yv.w;
        }
      } else {
        v[j][0] = v[j][1] = v[j][2] = v[j][3] = 0.0f;
      }
    }
    float kv = 1.0f;
    if (has_mask) {
      kv = keep_value(a.keep, a.keep_dtype, row);
#pragma unroll
      for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[j][e] *= kv;
    }
    if (write_s) {
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int c = (li + LPR * j) * 4;
        if (c < a.d)
          *(float4*)(a.s + row * a.lds + c) = make_float4(v[j][0], v[j][1], v[j][2], v[j][3]);
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
        float4 wv = *(const float4*)(a.w + c);
        float4 bv = *(const float4*)(a.b + c);
        float o[4];
        o[0] = (v[j][0] * rstd * wv.x + bv.x) * hscale;
        o[1] = (v[j][1] * rstd * wv.y + bv.y) * hscale;
        o[2] = (v[j][2] * rstd * wv.z + bv.z) * hscale;
        o[3] = (v[j][3] * rstd * wv.w + bv.w) * hscale;
        store4_any(a.h, a.h_lo, HT, row * a.ldh + c, o);
      }
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
    auto sval = [&](int64_t c) {
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
  int64_t blocks = (a.M + kRowsPerBlock - 1) / kRowsPerBlock;
  if (blocks > 65536) blocks = 65536;   // grid-stride beyond this
  if (blocks < 1) blocks = 1;
  switch (a.h_dtype) {
    case KF_F32: hipLaunchKernelGGL((ln_rows_kernel<LPR, NV, KF_F32>), dim3(blocks), dim3(256), 0, st, a); break;
    case KF_F16: hipLaunchKernelGGL((ln_rows_kernel<LPR, NV, KF_F16>), dim3(blocks), dim3(256), 0, st, a); break;
    case KF_BF16: hipLaunchKernelGGL((ln_rows_kernel<LPR, NV, KF_BF16>), dim3(blocks), dim3(256), 0, st, a); break;
    case KF_F16X2: hipLaunchKernelGGL((ln_rows_kernel<LPR, NV, KF_F16X2>), dim3(blocks), dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL((ln_rows_kernel<LPR, NV, KF_BF16X2>), dim3(blocks), dim3(256), 0, st, a); break;
  }
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
