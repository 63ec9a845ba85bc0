// Gated RMS norm of the GDN core output (HF RMSNormGated,
// transformers modeling_qwen3_5_moe.py:169-185, applied at :535-538):
//   y = weight * x * rsqrt(mean(x^2) + eps) * silu(z)    per (token, head) row
// One pass over HBM (x, z in, y out) instead of the module's chain of
// elementwise torch ops.  Arithmetic in fp32, one rounding to y's dtype
// (the module rounds x * rsqrt(.) to the input dtype before the weight; the
// difference is within one output ulp).
#include "gdn_common.h"

namespace gdn {
namespace {

constexpr int ND = 128;          // row length (v head dim)
constexpr int ROWS_PER_WG = 16;  // 16 lanes x 8 values per row, 4 rows per wave

struct NormArgs {
  const void *x, *z, *w;
  void *y;
  int x_dt, z_dt, w_dt, y_dt;
  int64_t xs, zs, ys;  // token strides (elements)
  int64_t rows;        // tokens * H (informational)
  int H;
  float eps;
};

typedef __attribute__((ext_vector_type(4))) unsigned u32x4;

// 8 consecutive values of dtype dt starting at element i (16-byte aligned for
// 2-byte types, 32-byte for fp32).
__device__ __forceinline__ void load8(const void *p, int64_t i, int dt, float (&v)[8]) {
  if (dt == GDN_DTYPE_F32) {
    const u32x4 a = *reinterpret_cast<const u32x4 *>(static_cast<const float *>(p) + i);
    const u32x4 b = *reinterpret_cast<const u32x4 *>(static_cast<const float *>(p) + i + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = __uint_as_float(a[e]);
      v[4 + e] = __uint_as_float(b[e]);
    }
  } else {
    const u32x4 a = *reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(p) + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (dt == GDN_DTYPE_BF16) {
        v[2 * e] = bf16_bits_to_f32(a[e] & 0xffffu);
        v[2 * e + 1] = bf16_bits_to_f32(a[e] >> 16);
      } else {
        v[2 * e] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(a[e] & 0xffffu)));
        v[2 * e + 1] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(a[e] >> 16)));
      }
    }
  }
}

__device__ __forceinline__ void store8(void *p, int64_t i, int dt, const float (&v)[8]) {
  if (dt == GDN_DTYPE_F32) {
    u32x4 a, b;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a[e] = __float_as_uint(v[e]);
      b[e] = __float_as_uint(v[4 + e]);
    }
    *reinterpret_cast<u32x4 *>(static_cast<float *>(p) + i) = a;
    *reinterpret_cast<u32x4 *>(static_cast<float *>(p) + i + 4) = b;
  } else {
    u32x4 a;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      uint32_t lo, hi;
      if (dt == GDN_DTYPE_BF16) {
        lo = f32_to_bf16_bits(v[2 * e]);
        hi = f32_to_bf16_bits(v[2 * e + 1]);
      } else {
        lo = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v[2 * e]));
        hi = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v[2 * e + 1]));
      }
      a[e] = lo | (hi << 16);
    }
    *reinterpret_cast<u32x4 *>(static_cast<uint16_t *>(p) + i) = a;
  }
}

// Grid: x = token, y = group of 16 heads.  A workgroup normalises 16 rows
// of one token; 16 lanes per row, 8 values per lane.
__global__ __launch_bounds__(256) void rmsnorm_gated_kernel(NormArgs a) {
  const int64_t t = blockIdx.x;
  const int hh = static_cast<int>(blockIdx.y) * ROWS_PER_WG + static_cast<int>(threadIdx.x >> 4);
  const int c0 = (threadIdx.x & 15) * 8;  // this lane's 8 columns
  const bool valid = hh < a.H;            // (all lanes take part in the row reduction)
  float x[8], z[8], w[8];
  load8(a.w, c0, a.w_dt, w);
  if (valid) {
    load8(a.x, t * a.xs + static_cast<int64_t>(hh) * ND + c0, a.x_dt, x);
    load8(a.z, t * a.zs + static_cast<int64_t>(hh) * ND + c0, a.z_dt, z);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = z[e] = 0.f;
  }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
  ss = row16_sum(ss);
  const float r = rsqrtf(ss * (1.f / ND) + a.eps);
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = w[e] * (x[e] * r) * (z[e] / (1.f + __expf(-z[e])));
  if (valid) store8(a.y, t * a.ys + static_cast<int64_t>(hh) * ND + c0, a.y_dt, y);
}

// 8 two-byte values (bf16 or fp16) as one 16-byte load, converted apart
// from the load so that a kernel can issue all of its loads first.
__device__ __forceinline__ u32x4 raw8(const void *p, int64_t i) {
  return *reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(p) + i);
}

__device__ __forceinline__ void cvt8(const u32x4 a, int dt, float (&v)[8]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (dt == GDN_DTYPE_BF16) {
      v[2 * e] = bf16_bits_to_f32(a[e] & 0xffffu);
      v[2 * e + 1] = bf16_bits_to_f32(a[e] >> 16);
    } else {
      v[2 * e] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(a[e] & 0xffffu)));
      v[2 * e + 1] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(a[e] >> 16)));
    }
  }
}

// x, z and y in 2-byte types (the layer's case; the weight in fp32 when
// W32): the same rows and arithmetic as rmsnorm_gated_kernel, with the x, z
// and weight loads issued back to back before any conversion, so that a
// workgroup waits for one memory latency instead of three in turn.  Lanes
// of a row past H load the last row and store nothing.
template <bool W32>
__global__ __launch_bounds__(256) void rmsnorm_gated_h_kernel(NormArgs a) {
  const int64_t t = blockIdx.x;
  const int hr = static_cast<int>(blockIdx.y) * ROWS_PER_WG + static_cast<int>(threadIdx.x >> 4);
  const bool valid = hr < a.H;
  const int hh = valid ? hr : a.H - 1;
  const int c0 = (threadIdx.x & 15) * 8;
  const u32x4 xr = raw8(a.x, t * a.xs + static_cast<int64_t>(hh) * ND + c0);
  const u32x4 zr = raw8(a.z, t * a.zs + static_cast<int64_t>(hh) * ND + c0);
  float x[8], z[8], w[8];
  if constexpr (W32) {
    const u32x4 w0 = *reinterpret_cast<const u32x4 *>(static_cast<const float *>(a.w) + c0);
    const u32x4 w1 = *reinterpret_cast<const u32x4 *>(static_cast<const float *>(a.w) + c0 + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      w[e] = __uint_as_float(w0[e]);
      w[4 + e] = __uint_as_float(w1[e]);
    }
  } else {
    cvt8(raw8(a.w, c0), a.w_dt, w);
  }
  cvt8(xr, a.x_dt, x);
  cvt8(zr, a.z_dt, z);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
  ss = row16_sum(ss);
  const float r = rsqrtf(ss * (1.f / ND) + a.eps);
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = w[e] * (x[e] * r) * (z[e] / (1.f + __expf(-z[e])));
  if (valid) store8(a.y, t * a.ys + static_cast<int64_t>(hh) * ND + c0, a.y_dt, y);
}

bool aligned_rows(const void *p, int dt, int64_t stride) {
  const int64_t unit = 8;  // rows start on 8-element boundaries: 16 bytes (2-byte types) or 32 (fp32)
  const size_t align = dt == GDN_DTYPE_F32 ? 32 : 16;
  return reinterpret_cast<uintptr_t>(p) % align == 0 && stride % unit == 0;
}

}  // namespace
}  // namespace gdn

extern "C" int gdn_rmsnorm_gated_fwd(const void *x, int x_dtype, int64_t x_stride_t,
                                     const void *z, int z_dtype, int64_t z_stride_t,
                                     const void *weight, int w_dtype,
                                     void *y, int y_dtype, int64_t y_stride_t,
                                     int64_t n_tokens, int32_t H, int32_t D, float eps, void *stream) {
  using namespace gdn;
  if (D != ND) return fail(GDN_ERR_UNSUPPORTED, "gdn_rmsnorm_gated_fwd: D=%d; only D=128 is built", D);
  if (n_tokens < 0 || H <= 0) return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_rmsnorm_gated_fwd: bad sizes");
  if (!valid_dtype(x_dtype) || !valid_dtype(z_dtype) || !valid_dtype(w_dtype) || !valid_dtype(y_dtype))
    return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_rmsnorm_gated_fwd: bad dtype");
  if (!(eps >= 0.f)) return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_rmsnorm_gated_fwd: eps must be >= 0");
  if (n_tokens == 0) return ok();
  if (!x || !z || !weight || !y) return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_rmsnorm_gated_fwd: null pointer");
  const int64_t row_len = static_cast<int64_t>(H) * D;
  if (x_stride_t < row_len || z_stride_t < row_len || y_stride_t < row_len)
    return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_rmsnorm_gated_fwd: token stride smaller than H*D");
  if (!aligned_rows(x, x_dtype, x_stride_t) || !aligned_rows(z, z_dtype, z_stride_t) ||
      !aligned_rows(y, y_dtype, y_stride_t))
    return fail(GDN_ERR_INVALID_ARGUMENT,
                "gdn_rmsnorm_gated_fwd: x/z/y must be 16-byte (32 for fp32) aligned with strides multiple of 8");
  if (n_tokens > 0x7fffffff || H > 65535 * ROWS_PER_WG)
    return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_rmsnorm_gated_fwd: grid too large");
  if (reinterpret_cast<uintptr_t>(weight) % (w_dtype == GDN_DTYPE_F32 ? 32 : 16))
    return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_rmsnorm_gated_fwd: weight must be 16-byte (32 for fp32) aligned");
  NormArgs a{x, z, weight, y, x_dtype, z_dtype, w_dtype, y_dtype, x_stride_t, z_stride_t, y_stride_t,
             n_tokens * H, H, eps};
  const dim3 grid(static_cast<unsigned>(n_tokens), static_cast<unsigned>((H + ROWS_PER_WG - 1) / ROWS_PER_WG));
  const auto st = static_cast<hipStream_t>(stream);
  const bool half_io = x_dtype != GDN_DTYPE_F32 && z_dtype != GDN_DTYPE_F32 && y_dtype != GDN_DTYPE_F32;
  if (half_io && w_dtype == GDN_DTYPE_F32)
    hipLaunchKernelGGL(rmsnorm_gated_h_kernel<true>, grid, dim3(256), 0, st, a);
  else if (half_io)
    hipLaunchKernelGGL(rmsnorm_gated_h_kernel<false>, grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(rmsnorm_gated_kernel, grid, dim3(256), 0, st, a);
  return check_launch("gdn_rmsnorm_gated_fwd");
}
