// Causal depthwise conv1d (+ optional SiLU) feeding the GDN q/k/v split.
//
// Prefill: each thread owns 8 consecutive channels and walks a tile of
// tokens of the packed token-major stream, keeping the previous 3 inputs of
// its channels in registers; a sequence start (from cu_seqlens) reloads the
// window from the cached history (or zeros).  A second small kernel writes
// the final windows.  A token row of x is read by
// one coalesced 16-byte load per thread, so the kernel is one read of x and
// one write of y (HBM roofline), plus the small state rows.
// Update: one thread per (sequence, channel) shifts the cached window by
// the T new tokens in place.
//
// Storage bf16, fp16 or fp32 (x, weight, bias, windows and y share it);
// arithmetic in fp32, one rounding on the store.
// Semantics: transformers modeling_qwen3_5_moe.py:200-240 (causal_conv1d_fn
// and causal_conv1d_update) and cache_utils.py:1032-1068 (cached window).
#include "gdn_common.h"

namespace gdn {
namespace {

constexpr int CPT = 8;         // channels per thread
constexpr int CONV_NT = 256;   // threads per workgroup
// Tokens per workgroup tile: 32 when a 64-token grid would leave CUs
// without a workgroup (short inputs), else the longest of 64, 56 and 48
// whose busiest CU streams the fewest tokens, ceil(workgroups / CUs) x tile:
// a long tile halves the re-read 3-token halo against 32 and keeps more loads
// in flight per thread, and a grid that is not a whole number of rounds over
// the CUs leaves some CUs one workgroup more than the rest (configuration 3,
// 13,794 tokens: 864 workgroups of 64 tokens, 3.4 per CU; 988 of 56)
constexpr int TILE_SHORT = 32, TILE_LONG = 64;
constexpr int CONV_CUS = 256;

template <typename T> struct Vec8;
template <> struct Vec8<uint16_t> {
  struct Raw { uint4 u; };
  static constexpr int PF = 4;  // tokens loaded ahead per batch
  static __device__ __forceinline__ Raw load_raw(const uint16_t *p) { return Raw{*reinterpret_cast<const uint4 *>(p)}; }
  static __device__ __forceinline__ void cvt(const Raw &r, float *o) {
    const uint32_t w[4] = {r.u.x, r.u.y, r.u.z, r.u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = bf16_bits_to_f32(w[i] & 0xffffu);
      o[2 * i + 1] = bf16_bits_to_f32(w[i] >> 16);
    }
  }
  static __device__ __forceinline__ void load(const uint16_t *p, float *o) { cvt(load_raw(p), o); }
  static __device__ __forceinline__ void store(uint16_t *p, const float *x) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = static_cast<uint32_t>(f32_to_bf16_bits(x[2 * i])) |
             (static_cast<uint32_t>(f32_to_bf16_bits(x[2 * i + 1])) << 16);
    *reinterpret_cast<uint4 *>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  }
};
template <> struct Vec8<float> {
  struct Raw { float4 a, b; };
  static constexpr int PF = 4;
  static __device__ __forceinline__ Raw load_raw(const float *p) {
    return Raw{reinterpret_cast<const float4 *>(p)[0], reinterpret_cast<const float4 *>(p)[1]};
  }
  static __device__ __forceinline__ void cvt(const Raw &r, float *o) {
    o[0] = r.a.x; o[1] = r.a.y; o[2] = r.a.z; o[3] = r.a.w; o[4] = r.b.x; o[5] = r.b.y; o[6] = r.b.z; o[7] = r.b.w;
  }
  static __device__ __forceinline__ void load(const float *p, float *o) { cvt(load_raw(p), o); }
  static __device__ __forceinline__ void store(float *p, const float *x) {
    reinterpret_cast<float4 *>(p)[0] = make_float4(x[0], x[1], x[2], x[3]);
    reinterpret_cast<float4 *>(p)[1] = make_float4(x[4], x[5], x[6], x[7]);
  }
};

template <> struct Vec8<_Float16> {
  struct Raw { uint4 u; };
  static constexpr int PF = 4;
  static __device__ __forceinline__ Raw load_raw(const _Float16 *p) { return Raw{*reinterpret_cast<const uint4 *>(p)}; }
  static __device__ __forceinline__ void cvt(const Raw &r, float *o) {
    const uint32_t w[4] = {r.u.x, r.u.y, r.u.z, r.u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w[i] & 0xffffu)));
      o[2 * i + 1] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w[i] >> 16)));
    }
  }
  static __device__ __forceinline__ void load(const _Float16 *p, float *o) { cvt(load_raw(p), o); }
  static __device__ __forceinline__ void store(_Float16 *p, const float *x) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)  // round to nearest even, as torch's fp16 cast
      w[i] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(x[2 * i]))) |
             (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(x[2 * i + 1]))) << 16);
    *reinterpret_cast<uint4 *>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  }
};

template <typename T> __device__ __forceinline__ float ld1(const T *p);
template <> __device__ __forceinline__ float ld1<uint16_t>(const uint16_t *p) { return bf16_bits_to_f32(*p); }
template <> __device__ __forceinline__ float ld1<float>(const float *p) { return *p; }
template <> __device__ __forceinline__ float ld1<_Float16>(const _Float16 *p) { return static_cast<float>(*p); }
template <typename T> __device__ __forceinline__ void st1(T *p, float x);
template <> __device__ __forceinline__ void st1<uint16_t>(uint16_t *p, float x) { *p = f32_to_bf16_bits(x); }
template <> __device__ __forceinline__ void st1<float>(float *p, float x) { *p = x; }
template <> __device__ __forceinline__ void st1<_Float16>(_Float16 *p, float x) { *p = static_cast<_Float16>(x); }

__device__ __forceinline__ float silu(float x) { return x / (1.f + expf(-x)); }
// SiLU with the hardware exp2 and reciprocal (a few ulp; the prefill kernel's
// per-token arithmetic is otherwise dominated by the IEEE exp and division)
__device__ __forceinline__ float silu_fast(float x) { return x * __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

struct ConvArgs {
  const void *x;
  int64_t xs;
  const void *w, *bias;
  void *y;
  int64_t ys;
  const void *st_in;
  const int64_t *in_idx;
  int64_t in_rows;
  void *st_out;
  const int64_t *out_idx;
  int64_t out_rows;
  const int32_t *cu;
  int n_seqs, T, C, width, silu;
  int64_t total;
};

constexpr int WIN = 3;  // previous inputs kept in registers (width <= 4)

// History row (SL inputs, oldest first) -> value `d` tokens before the
// sequence start (d >= 1), or 0 when there is no history.
template <typename T, int SL>
__device__ __forceinline__ float history_at(const ConvArgs &a, int64_t row, int c, int d) {
  if (row < 0 || d > SL) return 0.f;
  return ld1<T>(static_cast<const T *>(a.st_in) + (row * a.C + c) * SL + (SL - d));
}

// (n is the same across the calling lanes; a repeated slot id selects no row)
__device__ __forceinline__ int64_t in_row_of(const ConvArgs &a, int n) {
  return a.st_in ? pool_row_first(a.in_idx, n, a.in_rows) : -1;
}

template <typename T, int SL, bool SILU, int TILE_T>
__global__ __launch_bounds__(CONV_NT) void conv_fwd_kernel(ConvArgs a) {
  const int c0 = (blockIdx.x * CONV_NT + threadIdx.x) * CPT;
  if (c0 >= a.C) return;
  const int64_t tbeg = static_cast<int64_t>(blockIdx.y) * TILE_T;
  if (tbeg >= a.total) return;
  const int64_t tend = min(tbeg + TILE_T, a.total);

  // sequence containing tbeg: last n with start(n) <= tbeg < end(n)
  int n;
  int64_t s_beg, s_end;
  if (a.cu) {
    int lo = 0, hi = a.n_seqs;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (a.cu[mid] <= tbeg) lo = mid; else hi = mid;
    }
    n = lo;
  } else {
    n = static_cast<int>(tbeg / a.T);
  }
  {
    int len;
    seq_range(a.cu, n, a.T, a.total, &s_beg, &len);
    s_end = s_beg + len;
  }
  if (tbeg < s_beg || tbeg >= s_end) return;  // tokens outside every sequence

  // taps aligned to the newest input: wt[k] multiplies x_{t - 3 + k}; a
  // narrower kernel's missing oldest taps are zero (same sums, same order)
  float wt[4][CPT];
  {
    const T *wp = static_cast<const T *>(a.w);
    const int lead = 4 - a.width;
#pragma unroll
    for (int i = 0; i < CPT; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k) wt[k][i] = k >= lead ? ld1<T>(wp + (int64_t)(c0 + i) * a.width + (k - lead)) : 0.f;
  }
  float bias[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) bias[i] = a.bias ? ld1<T>(static_cast<const T *>(a.bias) + c0 + i) : 0.f;

  // win[j] = input at t - WIN + j (oldest first) for the current token t
  float win[WIN][CPT];
  {
    const int64_t hrow = in_row_of(a, n);
#pragma unroll
    for (int j = 0; j < WIN; ++j) {
      const int64_t tt = tbeg - WIN + j;
      if (tt >= s_beg) {
        Vec8<T>::load(static_cast<const T *>(a.x) + tt * a.xs + c0, win[j]);
      } else {
#pragma unroll
        for (int i = 0; i < CPT; ++i) win[j][i] = history_at<T, SL>(a, hrow, c0 + i, static_cast<int>(s_beg - tt));
      }
    }
  }

  // Tokens in batches of PF: a batch's inputs are requested one batch ahead
  // (two batches in registers), so each thread keeps up to 2 PF loads in
  // flight instead of waiting on one load per token.
  constexpr int PF = Vec8<T>::PF;
  using Raw = typename Vec8<T>::Raw;
  const T *xc = static_cast<const T *>(a.x) + c0;
  T *yc = static_cast<T *>(a.y) + c0;
  // One token: output from the window and the raw input, then slide the window.
  auto token = [&](const Raw &raw, int64_t t) {
    float xv[CPT];
    Vec8<T>::cvt(raw, xv);
    float out[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      float acc = bias[i];
#pragma unroll
      for (int k = 0; k < 4; ++k) acc += wt[k][i] * (k == 3 ? xv[i] : win[k][i]);
      out[i] = SILU ? silu_fast(acc) : acc;
    }
    Vec8<T>::store(yc + t * a.ys, out);
#pragma unroll
    for (int j = 0; j < WIN - 1; ++j)
#pragma unroll
      for (int i = 0; i < CPT; ++i) win[j][i] = win[j + 1][i];
#pragma unroll
    for (int i = 0; i < CPT; ++i) win[WIN - 1][i] = xv[i];
  };

  if (tend - tbeg == TILE_T && tend <= s_end) {
    // The whole tile lies in one sequence (the common case): fully unrolled,
    // no per-token bounds or sequence checks.
    constexpr int NB = TILE_T / PF;
    Raw r[2][PF];
#pragma unroll
    for (int u = 0; u < PF; ++u) r[0][u] = Vec8<T>::load_raw(xc + (tbeg + u) * a.xs);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (b + 1 < NB) {
#pragma unroll
        for (int u = 0; u < PF; ++u) r[(b + 1) & 1][u] = Vec8<T>::load_raw(xc + (tbeg + (b + 1) * PF + u) * a.xs);
      }
#pragma unroll
      for (int u = 0; u < PF; ++u) token(r[b & 1][u], tbeg + b * PF + u);
    }
    return;
  }

  // General tile: a sequence boundary or the end of the input falls inside it.
  // The tile is walked one sequence segment at a time.  Inside a segment the
  // loads run one batch ahead as in the full tile (addresses clamped to the
  // segment's last token, so a batch past its end re-reads a cached row) and
  // only the token step is guarded; between segments the window is reloaded
  // from the next sequence's history.
  int64_t sb = tbeg;  // first token of the current segment
  for (;;) {
    const int64_t se = min(tend, s_end);  // sb < se
    auto fetch = [&](Raw (&r)[PF], int64_t tb) {
#pragma unroll
      for (int u = 0; u < PF; ++u) r[u] = Vec8<T>::load_raw(xc + min(tb + u, se - 1) * a.xs);
    };
    Raw r0[PF], r1[PF];
    fetch(r0, sb);
    for (int64_t tb = sb; tb < se; tb += 2 * PF) {
      fetch(r1, tb + PF);
#pragma unroll
      for (int u = 0; u < PF; ++u)
        if (tb + u < se) token(r0[u], tb + u);
      fetch(r0, tb + 2 * PF);
#pragma unroll
      for (int u = 0; u < PF; ++u)
        if (tb + PF + u < se) token(r1[u], tb + PF + u);
    }
    if (se >= tend) return;
    // the next sequence starts at se, inside this tile
    ++n;
    if (a.cu) {
      while (n < a.n_seqs && a.cu[n + 1] <= se) ++n;  // skip empty sequences
      if (n >= a.n_seqs) return;
    }
    {
      int len;
      seq_range(a.cu, n, a.T, a.total, &s_beg, &len);
      s_end = s_beg + len;
    }
    if (se < s_beg || se >= s_end) return;  // tokens outside every sequence
    const int64_t hrow = in_row_of(a, n);
#pragma unroll
    for (int j = 0; j < WIN; ++j)
#pragma unroll
      for (int i = 0; i < CPT; ++i) win[j][i] = history_at<T, SL>(a, hrow, c0 + i, WIN - j);
    sb = se;
  }
}

// Final windows: the last SL inputs of cat(history, x) per sequence.  Run
// after the conv kernel (stream order) so that a pool updated in place is
// never overwritten while a tile still reads its history; each thread reads
// all SL values of its (sequence, channel) before writing any.
template <typename T, int SL>
__global__ __launch_bounds__(CONV_NT) void conv_final_state_kernel(ConvArgs a) {
  const int c = blockIdx.x * CONV_NT + threadIdx.x;
  const int n = blockIdx.y;
  if (c >= a.C) return;
  const int64_t row = pool_row_first(a.out_idx, n, a.out_rows);
  if (row < 0) return;
  int64_t s_beg;
  int len;
  seq_range(a.cu, n, a.T, a.total, &s_beg, &len);
  const int64_t s_end = s_beg + len;
  const int64_t hrow = in_row_of(a, n);
  float vals[SL];
#pragma unroll
  for (int j = 0; j < SL; ++j) {
    const int64_t pos = s_end - SL + j;
    vals[j] = pos >= s_beg ? ld1<T>(static_cast<const T *>(a.x) + pos * a.xs + c)
                           : history_at<T, SL>(a, hrow, c, static_cast<int>(s_beg - pos));
  }
  T *st = static_cast<T *>(a.st_out) + (row * a.C + c) * SL;
#pragma unroll
  for (int j = 0; j < SL; ++j) st1<T>(st + j, vals[j]);
}

struct UpdArgs {
  const void *x;
  int64_t xs;
  void *st;
  const int64_t *idx;
  int64_t rows;
  const void *w, *bias;
  void *y;
  int64_t ys;
  int n_seqs, T, C, width, silu;
};

template <typename T, int SL>
__global__ __launch_bounds__(CONV_NT) void conv_update_kernel(UpdArgs a) {
  const int c = blockIdx.x * CONV_NT + threadIdx.x;
  const int n = blockIdx.y;
  if (c >= a.C) return;
  const int64_t row = pool_row_first(a.idx, n, a.rows);
  T *st = row >= 0 ? static_cast<T *>(a.st) + (row * a.C + c) * SL : nullptr;
  float full[SL + 1];  // cached window (oldest first) followed by the new input
#pragma unroll
  for (int j = 0; j < SL; ++j) full[j] = st ? ld1<T>(st + j) : 0.f;
  float wt[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) wt[j] = j < a.width ? ld1<T>(static_cast<const T *>(a.w) + (int64_t)c * a.width + j) : 0.f;
  const float b = a.bias ? ld1<T>(static_cast<const T *>(a.bias) + c) : 0.f;
  for (int t = 0; t < a.T; ++t) {
    const int64_t tok = static_cast<int64_t>(n) * a.T + t;
    full[SL] = ld1<T>(static_cast<const T *>(a.x) + tok * a.xs + c);
    float acc = b;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (j < a.width) acc += wt[j] * full[SL + 1 - a.width + j];
    st1<T>(static_cast<T *>(a.y) + tok * a.ys + c, a.silu ? silu(acc) : acc);
#pragma unroll
    for (int j = 0; j < SL; ++j) full[j] = full[j + 1];
  }
  if (st) {
#pragma unroll
    for (int j = 0; j < SL; ++j) st1<T>(st + j, full[j]);
  }
}

template <typename T, int SL, int TILE_T>
void launch_tiles(const ConvArgs &a, unsigned gx, hipStream_t s) {
  const unsigned gy = static_cast<unsigned>((a.total + TILE_T - 1) / TILE_T);
  if (a.silu)
    hipLaunchKernelGGL((conv_fwd_kernel<T, SL, true, TILE_T>), dim3(gx, gy), dim3(CONV_NT), 0, s, a);
  else
    hipLaunchKernelGGL((conv_fwd_kernel<T, SL, false, TILE_T>), dim3(gx, gy), dim3(CONV_NT), 0, s, a);
}

template <typename T, int SL>
int launch_fwd(const ConvArgs &a, hipStream_t s) {
  const unsigned gx = (a.C / CPT + CONV_NT - 1) / CONV_NT;
  if (a.total > 0) {
    auto busiest = [&](int64_t tile) {  // tokens streamed by the CU with the most workgroups
      const int64_t n = gx * ((a.total + tile - 1) / tile);
      return (n + CONV_CUS - 1) / CONV_CUS * tile;
    };
    if (gx * ((a.total + TILE_LONG - 1) / TILE_LONG) < CONV_CUS) {
      launch_tiles<T, SL, TILE_SHORT>(a, gx, s);
    } else {
      int tile = TILE_LONG;
      for (const int t : {56, 48})
        if (busiest(t) < busiest(tile)) tile = t;
      if (tile == 56)
        launch_tiles<T, SL, 56>(a, gx, s);
      else if (tile == 48)
        launch_tiles<T, SL, 48>(a, gx, s);
      else
        launch_tiles<T, SL, TILE_LONG>(a, gx, s);
    }
  }
  if (a.st_out)
    hipLaunchKernelGGL((conv_final_state_kernel<T, SL>), dim3((a.C + CONV_NT - 1) / CONV_NT, a.n_seqs),
                       dim3(CONV_NT), 0, s, a);
  return check_launch("causal_conv1d_fwd");
}

template <typename T, int SL>
int launch_upd(const UpdArgs &a, hipStream_t s) {
  hipLaunchKernelGGL((conv_update_kernel<T, SL>), dim3((a.C + CONV_NT - 1) / CONV_NT, a.n_seqs),
                     dim3(CONV_NT), 0, s, a);
  return check_launch("causal_conv1d_update");
}

}  // namespace
}  // namespace gdn

extern "C" int causal_conv1d_fwd(const void *x, int64_t x_stride_t, const void *w, const void *bias,
                                 void *y, int64_t y_stride_t,
                                 const void *state_in, const int64_t *state_in_idx, int64_t state_in_rows,
                                 void *state_out, const int64_t *state_out_idx, int64_t state_out_rows,
                                 const int32_t *cu_seqlens, int32_t n_seqs, int32_t T,
                                 int32_t C, int32_t width, int32_t state_len,
                                 int silu, int dtype, void *stream) {
  using namespace gdn;
  if (!valid_dtype(dtype))
    return fail(GDN_ERR_UNSUPPORTED, "causal_conv1d_fwd: dtype must be bf16, fp16 or fp32");
  if (width < 1 || width > 4 || (state_len != 3 && state_len != 4))
    return fail(GDN_ERR_UNSUPPORTED, "causal_conv1d_fwd: width=%d state_len=%d (need width<=4, state_len in {3,4})",
                width, state_len);
  if (C <= 0 || C % CPT || n_seqs < 0 || T < 0 || n_seqs > 65535)
    return fail(GDN_ERR_INVALID_ARGUMENT, "causal_conv1d_fwd: bad sizes C=%d n_seqs=%d T=%d", C, n_seqs, T);
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) % 16)
    return fail(GDN_ERR_INVALID_ARGUMENT, "causal_conv1d_fwd: x and y must be 16-byte aligned");
  if (!x || !w || !y) return fail(GDN_ERR_INVALID_ARGUMENT, "causal_conv1d_fwd: null x/w/y");
  if (x_stride_t < C || y_stride_t < C || (x_stride_t % CPT) || (y_stride_t % CPT))
    return fail(GDN_ERR_INVALID_ARGUMENT, "causal_conv1d_fwd: token strides must be >= C and multiples of 8");
  if (!rows_cover(state_in, state_in_idx, state_in_rows, n_seqs) ||
      !rows_cover(state_out, state_out_idx, state_out_rows, n_seqs))
    return fail(GDN_ERR_INVALID_ARGUMENT, "causal_conv1d_fwd: state rows (%lld in, %lld out) do not cover %d sequences",
                static_cast<long long>(state_in_rows), static_cast<long long>(state_out_rows), n_seqs);
  if (n_seqs == 0) return ok();
  ConvArgs a{x, x_stride_t, w, bias, y, y_stride_t, state_in, state_in_idx, state_in_rows, state_out, state_out_idx,
             state_out_rows, cu_seqlens, n_seqs, T, C, width, silu};
  a.total = cu_seqlens ? static_cast<int64_t>(T) : static_cast<int64_t>(n_seqs) * T;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == GDN_DTYPE_BF16)
    return state_len == 4 ? launch_fwd<uint16_t, 4>(a, s) : launch_fwd<uint16_t, 3>(a, s);
  if (dtype == GDN_DTYPE_F16)
    return state_len == 4 ? launch_fwd<_Float16, 4>(a, s) : launch_fwd<_Float16, 3>(a, s);
  return state_len == 4 ? launch_fwd<float, 4>(a, s) : launch_fwd<float, 3>(a, s);
}

extern "C" int causal_conv1d_update(const void *x, int64_t x_stride_t, void *conv_state,
                                    const int64_t *state_idx, int64_t state_rows, const void *w, const void *bias,
                                    void *y, int64_t y_stride_t, int32_t n_seqs, int32_t T,
                                    int32_t C, int32_t width, int32_t state_len,
                                    int silu, int dtype, void *stream) {
  using namespace gdn;
  if (!valid_dtype(dtype))
    return fail(GDN_ERR_UNSUPPORTED, "causal_conv1d_update: dtype must be bf16, fp16 or fp32");
  if (width < 1 || width > 4 || (state_len != 3 && state_len != 4) || width > state_len + 1)
    return fail(GDN_ERR_UNSUPPORTED, "causal_conv1d_update: width=%d state_len=%d (need width<=min(4,state_len+1))",
                width, state_len);
  if (C <= 0 || n_seqs < 0 || T < 0 || x_stride_t < C || y_stride_t < C)
    return fail(GDN_ERR_INVALID_ARGUMENT, "causal_conv1d_update: bad sizes");
  if (!x || !w || !y || !conv_state) return fail(GDN_ERR_INVALID_ARGUMENT, "causal_conv1d_update: null pointer");
  if (!rows_cover(conv_state, state_idx, state_rows, n_seqs))
    return fail(GDN_ERR_INVALID_ARGUMENT, "causal_conv1d_update: %lld state rows do not cover %d sequences",
                static_cast<long long>(state_rows), n_seqs);
  if (n_seqs == 0) return ok();
  if (n_seqs > 65535) return fail(GDN_ERR_INVALID_ARGUMENT, "causal_conv1d_update: n_seqs > 65535");
  UpdArgs a{x, x_stride_t, conv_state, state_idx, state_rows, w, bias, y, y_stride_t, n_seqs, T, C, width, silu};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == GDN_DTYPE_BF16)
    return state_len == 4 ? launch_upd<uint16_t, 4>(a, s) : launch_upd<uint16_t, 3>(a, s);
  if (dtype == GDN_DTYPE_F16)
    return state_len == 4 ? launch_upd<_Float16, 4>(a, s) : launch_upd<_Float16, 3>(a, s);
  return state_len == 4 ? launch_upd<float, 4>(a, s) : launch_upd<float, 3>(a, s);
}
