// Shared device helpers and host-side error plumbing for libgdn_mi355x.
// gfx950 (CDNA4) only: wave64, bf16 MFMA, 160 KiB LDS per CU.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "gdn_capi.h"

namespace gdn {

// ---------------------------------------------------------------- host side

// Records a formatted message for gdn_last_error_string() and returns `code`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the thread's message; returns GDN_OK.
int ok();
// Maps a launch error (hipGetLastError after a launch) to a status.
int check_launch(const char *what);

inline bool valid_dtype(int dt) { return dt == GDN_DTYPE_F32 || dt == GDN_DTYPE_BF16 || dt == GDN_DTYPE_F16; }
inline size_t dtype_size(int dt) { return dt == GDN_DTYPE_F32 ? 4 : 2; }

// A state tensor of `rows` rows (a slot pool, or one row per sequence)
// addressed per sequence through `idx` (NULL: row n).  Host check: without
// indices, the rows must cover the sequences; with them, out-of-range ids are
// handled on the device (pool_row).
inline bool rows_cover(const void *state, const int64_t *idx, int64_t rows, int32_t n_seqs) {
  return !state || (rows >= 0 && (idx || rows >= n_seqs));
}

// ---------------------------------------------------------------- device side

constexpr int BUF_DWORD3 = 0x00020000;  // raw (untyped) buffer resource word 3 on CDNA
constexpr int BUF_NT = 2;               // buffer load/store cache policy: non-temporal

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits (inputs here are finite).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float load_elem(const void *p, int64_t i, int dt) {
  if (dt == GDN_DTYPE_F32) return static_cast<const float *>(p)[i];
  if (dt == GDN_DTYPE_BF16) return bf16_bits_to_f32(static_cast<const uint16_t *>(p)[i]);
  return static_cast<float>(static_cast<const _Float16 *>(p)[i]);
}

// load_elem in two halves: the raw bits (f32, or a 2-byte type zero-extended)
// and their conversion, so that a load can be issued long before its value is
// needed without the conversion pulling the wait forward.
__device__ __forceinline__ uint32_t load_bits(const void *p, int64_t i, int dt) {
  if (dt == GDN_DTYPE_F32) return static_cast<const uint32_t *>(p)[i];
  return static_cast<const uint16_t *>(p)[i];
}
__device__ __forceinline__ float bits_to_f32(uint32_t b, int dt) {
  if (dt == GDN_DTYPE_F32) return __uint_as_float(b);
  if (dt == GDN_DTYPE_BF16) return bf16_bits_to_f32(static_cast<uint16_t>(b));
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b)));
}

__device__ __forceinline__ void store_elem(void *p, int64_t i, int dt, float x) {
  if (dt == GDN_DTYPE_F32) {
    static_cast<float *>(p)[i] = x;
  } else if (dt == GDN_DTYPE_BF16) {
    static_cast<uint16_t *>(p)[i] = f32_to_bf16_bits(x);
  } else {
    static_cast<_Float16 *>(p)[i] = static_cast<_Float16>(x);
  }
}

// Gate inputs of one (token, v-head).  Precomputed: g (fp32 log-decay) and
// beta (dtype `dt`), both [tokens, Hv] with token stride `stride`.  Raw (the
// HF Qwen3.5 GDN layer's projections, engine reference: the layer forward
// computes them before the kernel, transformers modeling_qwen3_5_moe.py:495-497):
//   beta = sigmoid(b),  g = -exp(A_log[h]) * softplus(a + dt_bias[h]),
// softplus(x) = x for x > 20 (torch's threshold), log1p(e^x) otherwise; a and b
// in dtype `dt`, A_log and dt_bias fp32 [Hv].  Raw mode when A_log is set.
struct GateArgs {
  const void *g_or_a;
  const void *beta_or_b;
  int dt;
  int64_t stride;
  const float *A_log;
  const float *dt_bias;
};
__device__ __forceinline__ void load_gates(const GateArgs &ga, int64_t tok, int h, float *g, float *beta) {
  const int64_t i = tok * ga.stride + h;
  if (ga.A_log) {
    const float x = load_elem(ga.g_or_a, i, ga.dt) + ga.dt_bias[h];
    const float sp = x > 20.f ? x : log1pf(expf(x));
    *g = -expf(ga.A_log[h]) * sp;
    *beta = 1.f / (1.f + expf(-load_elem(ga.beta_or_b, i, ga.dt)));
  } else {
    *g = static_cast<const float *>(ga.g_or_a)[i];
    *beta = load_elem(ga.beta_or_b, i, ga.dt);
  }
}

// load_bits for a wave-uniform address, always as a vector memory instruction
// (a buffer load).  A plain uniform load becomes a scalar load for one dtype
// and a vector load for another, and the dtype branches then serialise their
// waits.
__device__ __forceinline__ uint32_t load_bits_vmem(const void *p, int64_t i, int dt) {
  const int es = dt == GDN_DTYPE_F32 ? 4 : 2;
  const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(static_cast<const char *>(p) + i * es), 0, 4,
                                                    BUF_DWORD3);
  return dt == GDN_DTYPE_F32 ? static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(rs, 0, 0, 0))
                             : static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b16(rs, 0, 0, 0));
}

// load_gates in two halves (raw loads, then the gate math), for the same reason
// as load_bits; tok and h are wave-uniform.
struct GateRaw {
  uint32_t ga, gb;        // a (or g) and b (or beta), raw bits
  float a_log, dt_bias;   // raw mode only
};
__device__ __forceinline__ GateRaw load_gates_raw(const GateArgs &ga, int64_t tok, int h) {
  const int64_t i = tok * ga.stride + h;
  GateRaw r;
  if (ga.A_log) {
    r.ga = load_bits_vmem(ga.g_or_a, i, ga.dt);
    r.a_log = ga.A_log[h];
    r.dt_bias = ga.dt_bias[h];
  } else {
    r.ga = load_bits_vmem(ga.g_or_a, i, GDN_DTYPE_F32);
    r.a_log = r.dt_bias = 0.f;
  }
  r.gb = load_bits_vmem(ga.beta_or_b, i, ga.dt);
  return r;
}
__device__ __forceinline__ void gates_from_raw(const GateArgs &ga, const GateRaw &r, float *g, float *beta) {
  if (ga.A_log) {
    const float x = bits_to_f32(r.ga, ga.dt) + r.dt_bias;
    const float sp = x > 20.f ? x : log1pf(expf(x));
    *g = -expf(r.a_log) * sp;
    *beta = 1.f / (1.f + expf(-bits_to_f32(r.gb, ga.dt)));
  } else {
    *g = __uint_as_float(r.ga);
    *beta = bits_to_f32(r.gb, ga.dt);
  }
}

// Sum over the 16 lanes of a DPP row (every lane receives the sum).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_mov<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp_mov<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp_mov<0x141>(x);  // row_half_mirror
  x += dpp_mov<0x140>(x);  // row_mirror
  return x;
}

// Inclusive prefix sum over the 64 lanes of a wave on DPP (no LDS round
// trip): shifts by 1, 2, 4, 8 within each row of 16 lanes (a lane whose
// source lies before its row's start adds 0), then row 0's total into row 1
// and row 2's into row 3 (row_bcast:15, rows 1 and 3 enabled), then the
// total of lanes 0..31 into rows 2 and 3 (row_bcast:31).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_from(float v) {
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf, false));
}
__device__ __forceinline__ float wave_incl_scan(float x) {
  x += dpp_from<0x111, 0xf>(x);  // row_shr:1
  x += dpp_from<0x112, 0xf>(x);  // row_shr:2
  x += dpp_from<0x114, 0xf>(x);  // row_shr:4
  x += dpp_from<0x118, 0xf>(x);  // row_shr:8
  x += dpp_from<0x142, 0xa>(x);  // row_bcast:15
  x += dpp_from<0x143, 0xc>(x);  // row_bcast:31
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
  return x;
}

// Row of sequence n in a state tensor of `rows` rows addressed through `idx`
// (NULL: row n).  An id outside [0, rows) means no row, like a negative slot
// id: zero state in, nothing written.
__device__ __forceinline__ int64_t pool_row(const int64_t *idx, int64_t n, int64_t rows) {
  const int64_t r = idx ? idx[n] : n;
  return (r >= 0 && r < rows) ? r : -1;
}

// Slot ids repeated within one call.  The reference's CUDA-graph runner pads
// a batch bucket by repeating row 0 (engine/runtime/cuda_graphs.py:478-482);
// its cache gathers, computes and scatters with index_copy_, so the copies
// are harmless there.  Here pools are read and written in place, so only the
// first row that names a slot uses it: a row whose id equals the id of an
// earlier row of the same index array selects no row (zero state in, nothing
// written), like a negative id.
//
// repeats_earlier: n must be the same in every active lane (a workgroup- or
// wave-level sequence index); the active lanes split the earlier ids among
// themselves and vote.
__device__ __forceinline__ bool repeats_earlier(const int64_t *idx, int64_t n) {
  if (!idx || n <= 0) return false;
  const uint64_t act = __builtin_amdgcn_read_exec();
  const int cnt = __popcll(act);
  const int pos = static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(act >> 32),
                                                            __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(act), 0u)));
  const int64_t id = idx[n];
  for (int64_t base = 0; base < n; base += cnt) {
    const int64_t m = base + pos;
    if (__ballot(m < n && idx[m] == id)) return true;
  }
  return false;
}

// repeats_earlier in two halves for one full wave (all 64 lanes active, n
// uniform): the earlier ids, one per lane, can be requested ahead of a long
// stream of vector loads and tested after it.  Vector loads complete in order,
// so the test then waits for these ids only, not for the stream.  `id` is
// idx[n]; ids beyond the first 64 rows are read in the test itself.
__device__ __forceinline__ int64_t earlier_id_of_lane(const int64_t *idx, int64_t n, int lane) {
  return (idx && lane < n) ? idx[lane] : 0;
}
__device__ __forceinline__ bool repeats_earlier_wave(const int64_t *idx, int64_t n, int64_t id, int64_t lane_id,
                                                     int lane) {
  if (!idx || n <= 0) return false;
  if (__ballot(lane < n && lane_id == id)) return true;
  for (int64_t base = 64; base < n; base += 64) {
    const int64_t m = base + lane;
    if (__ballot(m < n && idx[m] == id)) return true;
  }
  return false;
}

// The same test when n differs between lanes (one thread per sequence).
__device__ __forceinline__ bool repeats_earlier_thread(const int64_t *idx, int64_t n) {
  if (!idx || n <= 0) return false;
  const int64_t id = idx[n];
  bool hit = false;
  for (int64_t m = 0; m < n; ++m) hit |= idx[m] == id;
  return hit;
}

// pool_row with repeated ids mapped to "no row" (n uniform as for repeats_earlier).
__device__ __forceinline__ int64_t pool_row_first(const int64_t *idx, int64_t n, int64_t rows) {
  const int64_t r = pool_row(idx, n, rows);
  return (r >= 0 && repeats_earlier(idx, n)) ? -1 : r;
}

// Sequence n's token range [*t0, *t0 + *len), clamped to the [0, total)
// tokens the caller passed, so that a malformed device-side cu_seqlens can
// never move an access outside the tensors.
__device__ __forceinline__ void seq_range(const int32_t *cu_seqlens, int n, int T, int64_t total,
                                          int64_t *t0, int *len) {
  int64_t a, b;
  if (cu_seqlens) {
    a = cu_seqlens[n];
    b = cu_seqlens[n + 1];
  } else {
    a = static_cast<int64_t>(n) * T;
    b = a + T;
  }
  a = a < 0 ? 0 : (a > total ? total : a);
  b = b < a ? a : (b > total ? total : b);
  *t0 = a;
  *len = static_cast<int>(b - a);
}

}  // namespace gdn
