// Chunk-64 gated delta rule prefill on bf16 MFMA (gfx950).
//
// The reference algorithm (engine/kernels/delta_rule.py:286-349) per chunk
// of 64 tokens and v-head, with gamma = chunk-local cumsum(g):
//   L = strict_lower(diag(beta) K~K~^T * Gamma),  T = (I + L)^-1
//   U = T (beta V),  W = T (beta e^gamma K~)
//   V' = U - W S ;  O = (e^gamma Q~) S + lower(Q~K~^T * Gamma) V'
//   S <- e^{gamma_63} S + (e^{gamma_63 - gamma} K~)^T V'
// runs as three launches:
//   chunk_table_kernel  chunk -> sequence table (cu_seqlens aware)
//   chunk_prep_kernel   one workgroup per (chunk, v-head), all in parallel:
//                       K K^T and Q K^T on MFMA from the raw bf16 rows (exact
//                       products; l2norm and gate factors scale the fp32
//                       results), T by blocked substitution in fp32 (LDS),
//                       W = T' K and U = T'' V on MFMA with T', T'' split into
//                       bf16 hi + lo parts.  Every operand the scan needs is
//                       written pre-swizzled: one 1 KiB block per (MFMA, wave),
//                       lane l's 16 bytes at offset 16 l.
//   chunk_scan_kernel   one wave per (sequence, v-head, 16 state columns),
//                       serial over the chunks; the state slice lives in MFMA
//                       accumulators for the whole sequence.  The next chunk's
//                       operand blocks stream into a second LDS buffer with
//                       buffer_load ... lds while the current chunk computes.
// Precision (checked against an fp64 restatement at T=4096): the state is fed
// to MFMA as bf16, U stays fp32 (it initialises the V' accumulator), the state
// increment K^T V'' uses V'' split into bf16 hi + lo.
//
// MFMA: v_mfma_f32_16x16x32_bf16.  Lane l holds A[l%16][8(l/16)+j] and
// B[8(l/16)+j][l%16] (j<8), and D[4(l/16)+i][l%16] (i<4).  When an
// accumulator tile pair (rows 0-15, 16-31 of a 32-long reduction) is reused
// as the B operand of the next product, lane group g = l/16 holds reduction
// indices {4g..4g+3, 16+4g..16+4g+3} ("pi" order); the scan's A-operand
// blocks are stored in the same order, so no accumulator goes through LDS.
#include <algorithm>
#include <type_traits>

#include "gdn_common.h"

namespace gdn {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) unsigned u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned u32x2;

constexpr int CK = 64;     // chunk length
constexpr int DK = 128;    // k head dim
constexpr int DV = 128;    // v head dim
constexpr int SCAL = 256;  // per (chunk, v-head) scalars: sq[64], sk[64], eL (1 KiB block)

// Operand blocks (64 lanes x 16 bytes) per chunk, in two contiguous regions
// so that one chunk's scan operands are two straight copies:
//   per (chunk, v-head): -W [p 0..3][s 0..3], A [p 0..3][s 0..1] (6 used), scalars
//   per (chunk, k-head): Q [p 0..3][s 0..3], K^T [i 0..7][s 0..1]
constexpr int NB_W = 16;
constexpr int NB_A = 8;
constexpr int NB_SC = SCAL / 64;  // scalars as blocks (1)
constexpr int NB_Q = 16;
constexpr int NB_KT = 16;
constexpr int VH_W = 0, VH_A = VH_W + NB_W, VH_SC = VH_A + NB_A, NB_VH = VH_SC + NB_SC;
constexpr int KH_Q = 0, KH_KT = KH_Q + NB_Q, NB_KH = KH_KT + NB_KT;

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 u) { return __builtin_bit_cast(bf16x8, u); }
__device__ __forceinline__ int64_t uniform64(int64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(x));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(x) >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}
__device__ __forceinline__ uint16_t bf16_rne(float x) {  // hardware round-to-nearest-even
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
}
__device__ __forceinline__ bf16x8 ld8(const uint16_t *p) {
  return as_bf16x8(*reinterpret_cast<const u32x4 *>(p));
}
__device__ __forceinline__ bf16x8 zero8() {
  u32x4 u = {0u, 0u, 0u, 0u};
  return as_bf16x8(u);
}
__device__ __forceinline__ bf16x8 pack_hi(f32x4 a, f32x4 b) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r[i] = static_cast<__bf16>(a[i]);
    r[4 + i] = static_cast<__bf16>(b[i]);
  }
  return r;
}
__device__ __forceinline__ void pack_hilo(f32x4 a, f32x4 b, bf16x8 &hi, bf16x8 &lo) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const __bf16 ha = static_cast<__bf16>(a[i]);
    const __bf16 hb = static_cast<__bf16>(b[i]);
    hi[i] = ha;
    hi[4 + i] = hb;
    lo[i] = static_cast<__bf16>(a[i] - static_cast<float>(ha));
    lo[4 + i] = static_cast<__bf16>(b[i] - static_cast<float>(hb));
  }
}

struct ChunkArgs {
  const uint16_t *q, *k, *v;  // bf16
  int64_t qs, ks, vs;         // token strides (elements)
  const float *g;
  const void *beta;
  int beta_dt;
  const float *h0;
  const int64_t *h0_idx;
  float *hT;
  const int64_t *hT_idx;
  void *o;
  int o_dt;
  const int32_t *cu;
  int n_seqs, T, Hk, Hv;
  int64_t total;
  float scale;
  int l2norm;
  int max_chunks;
  int seg_begin, seg_end;  // global chunk range of this launch (workspace holds SEG chunks)
  // workspace
  int32_t *chunk_start;  // [n_seqs + 1]
  u32x4 *vh;             // [SEG][Hv][NB_VH][64]   -W, A, scalars
  u32x4 *kh;             // [SEG][Hk][NB_KH][64]   Q, K^T
  float *Ut;             // [SEG][Hv][8 x 4 blocks][64][4]  U, fp32
  float *carry;          // [n_seqs][Hv][128][128] state between segments
};

__device__ __forceinline__ void seq_bounds(const ChunkArgs &a, int n, int64_t *s0, int *len) {
  seq_range(a.cu, n, a.T, a.total, s0, len);
}

// ------------------------------------------------------------------ chunk table
__global__ __launch_bounds__(256) void chunk_table_kernel(ChunkArgs a) {
  __shared__ int32_t part[256];
  int32_t carry = 0;
  if (threadIdx.x == 0) a.chunk_start[0] = 0;
  for (int base = 0; base < a.n_seqs; base += 256) {
    const int n = base + threadIdx.x;
    int64_t s0;
    int len = 0;
    if (n < a.n_seqs) seq_bounds(a, n, &s0, &len);
    part[threadIdx.x] = (len + CK - 1) / CK;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {  // inclusive scan
      const int32_t x = threadIdx.x >= off ? part[threadIdx.x - off] : 0;
      __syncthreads();
      part[threadIdx.x] += x;
      __syncthreads();
    }
    if (n < a.n_seqs) a.chunk_start[n + 1] = carry + part[threadIdx.x];
    carry += part[255];
    __syncthreads();
  }
}

// ------------------------------------------------------------------ phase A
constexpr int LT_LD = CK + 4;    // fp32 row stride of L / T (16-byte aligned rows)
constexpr int WS_LD = DK + 8;    // bf16 row stride of the -W staging tile (same bytes as L / T)
static_assert(CK * LT_LD * 4 == CK * WS_LD * 2, "W staging reuses the L/T buffer");

// Transposed [128][64] bf16 tiles (K^T, V^T): 16-byte segment seg of row r is
// stored at segment seg ^ f(r), f(r) = ((r >> 1) ^ (r >> 3)) & 7.  With this
// swizzle the MFMA operand reads (16 consecutive rows, one segment) touch
// distinct banks, and the transposing 2-byte writes (rows 8 apart, one
// column) collide at most 2-way.
__device__ __forceinline__ int tsw(int row, int col) {
  return row * CK + ((((col >> 3) ^ (row >> 1) ^ (row >> 3)) & 7) << 3) + (col & 7);
}

// Row-major [64][128] bf16 K tile: 16-byte segment seg of row r at seg ^ (r & 15).
__device__ __forceinline__ int nsw(int row, int col) {
  return row * DK + ((((col >> 3) ^ row) & 15) << 3) + (col & 7);
}
constexpr int AS_LD = CK + 8;  // bf16 row stride of the A staging tile

__global__ __launch_bounds__(256) void chunk_prep_kernel(ChunkArgs a) {
  __shared__ __align__(16) uint16_t kn_s[CK * DK];   // K rows (MFMA operands of K K^T, Q K^T)
  __shared__ __align__(16) uint16_t kt_s[DK * CK];   // K^T (B operand of W, scan operand blocks)
  __shared__ __align__(16) uint16_t vt_s[DV * CK];   // V^T (B operand of U)
  __shared__ __align__(16) float lt[CK * LT_LD];      // L, then T in place, then -W staging
  __shared__ __align__(16) uint16_t as_s[CK * AS_LD]; // A staging
  __shared__ __align__(16) float xs[3][16][17];
  __shared__ float gam_s[CK], beta_s[CK], nk_s[CK], nq_s[CK], colw_s[CK];

  const int h = blockIdx.x;
  const int j = a.seg_begin + static_cast<int>(blockIdx.y);  // global chunk index
  if (j >= a.seg_end || j >= a.chunk_start[a.n_seqs]) return;
  int lo = 0, hi = a.n_seqs;  // sequence owning chunk j: last n with chunk_start[n] <= j
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (a.chunk_start[mid] <= j) lo = mid; else hi = mid;
  }
  const int n = lo;
  int64_t s0;
  int slen;
  seq_bounds(a, n, &s0, &slen);
  const int c = j - a.chunk_start[n];
  const int64_t t0 = s0 + static_cast<int64_t>(c) * CK;
  const int len = min(CK, slen - c * CK);
  if (len <= 0) return;
  const int ratio = a.Hv / a.Hk;
  const int hk = h / ratio;
  const bool khead_writer = (h % ratio) == 0;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g4 = lane >> 4;
  const int r16 = lane & 15;
  const int jl = static_cast<int>(blockIdx.y);  // chunk index within the segment's workspace
  const size_t ch = static_cast<size_t>(jl) * a.Hv + h;
  const size_t chk = static_cast<size_t>(jl) * a.Hk + hk;
  const int p = wave;  // row block of K K^T / Q K^T / W / U owned by this wave

  // ---- issue every global load up front
  const int seg = tid & 15;
  u32x4 ku[4], qu[4], vu[4];
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int row = (tid >> 4) + 16 * it;
    const int64_t tok = t0 + row;
    const u32x4 z = {0u, 0u, 0u, 0u};
    ku[it] = row < len ? *reinterpret_cast<const u32x4 *>(a.k + tok * a.ks + (int64_t)hk * DK + seg * 8) : z;
    qu[it] = row < len ? *reinterpret_cast<const u32x4 *>(a.q + tok * a.qs + (int64_t)hk * DK + seg * 8) : z;
    vu[it] = row < len ? *reinterpret_cast<const u32x4 *>(a.v + tok * a.vs + (int64_t)h * DV + seg * 8) : z;
  }
  bf16x8 aq[4];  // Q rows of block p (A operands of Q K^T)
  {
    const int row = 16 * p + r16;
    const uint16_t *qrow = a.q + (t0 + row) * a.qs + (int64_t)hk * DK + 8 * g4;
#pragma unroll
    for (int s = 0; s < 4; ++s) aq[s] = row < len ? ld8(qrow + 32 * s) : zero8();
  }
  float gv = 0.f, bv = 0.f;
  if (wave == 0 && lane < len) {
    gv = a.g[(t0 + lane) * a.Hv + h];
    bv = load_elem(a.beta, (t0 + lane) * a.Hv + h, a.beta_dt);
  }

  // ---- A.1: K (rows and transposed), V^T into LDS; row norms; chunk-local cumsum of g
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int row = (tid >> 4) + 16 * it;
    *reinterpret_cast<u32x4 *>(kn_s + nsw(row, seg * 8)) = ku[it];
    float sk = 0.f, sq = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t kw = ku[it][e], qw = qu[it][e], vw = vu[it][e];
      const float k0 = bf16_bits_to_f32(kw & 0xffffu), k1 = bf16_bits_to_f32(kw >> 16);
      const float q0 = bf16_bits_to_f32(qw & 0xffffu), q1 = bf16_bits_to_f32(qw >> 16);
      sk += k0 * k0 + k1 * k1;
      sq += q0 * q0 + q1 * q1;
      const int d0 = seg * 8 + 2 * e;
      kt_s[tsw(d0, row)] = static_cast<uint16_t>(kw & 0xffffu);
      kt_s[tsw(d0 + 1, row)] = static_cast<uint16_t>(kw >> 16);
      vt_s[tsw(d0, row)] = static_cast<uint16_t>(vw & 0xffffu);
      vt_s[tsw(d0 + 1, row)] = static_cast<uint16_t>(vw >> 16);
    }
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) {
      sk += __shfl_xor(sk, m, 64);
      sq += __shfl_xor(sq, m, 64);
    }
    if (seg == 0) {
      nk_s[row] = a.l2norm ? rsqrtf(sk + 1e-6f) : 1.f;
      nq_s[row] = (a.l2norm ? rsqrtf(sq + 1e-6f) : 1.f) * a.scale;
    }
  }
  if (wave == 0) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float x = __shfl_up(gv, off, 64);
      if (lane >= off) gv += x;
    }
    gam_s[lane] = gv;
    beta_s[lane] = bv;
  }
  // Q operand blocks for the scan (pi order), straight from the loaded rows
  if (khead_writer) {
    u32x4 *qop = a.kh + chk * (NB_KH * 64) + KH_Q * 64;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int row = (tid >> 4) + 16 * it;
      const int s = seg >> 2, m = seg & 3;       // columns 32 s + 8 m .. +8
      const int blk = (row >> 4) * 4 + s;
      const int half = m >> 1;                   // slots 0-3 or 4-7
      const int gA = 2 * (m & 1);                // lane group of columns +0..3; +4..7 -> gA + 1
      u32x2 *base = reinterpret_cast<u32x2 *>(qop + blk * 64);
      base[2 * ((row & 15) + 16 * gA) + half] = u32x2{qu[it][0], qu[it][1]};
      base[2 * ((row & 15) + 16 * (gA + 1)) + half] = u32x2{qu[it][2], qu[it][3]};
    }
  }
  __syncthreads();

  // ---- A.2: K K^T -> L (fp32, LDS), Q K^T -> A (bf16, LDS staging)
  if (wave == 0) colw_s[lane] = beta_s[lane] * expf(gam_s[lane]) * nk_s[lane];  // W's column scale
  {
    bf16x8 ak[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) ak[s] = ld8(kn_s + nsw(16 * p + r16, 32 * s + 8 * g4));
    float gi[4], ni[4], qi[4], bi[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int ii = 16 * p + 4 * g4 + e;
      gi[e] = gam_s[ii];
      ni[e] = nk_s[ii];
      qi[e] = nq_s[ii];
      bi[e] = beta_s[ii];
    }
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      f32x4 kk = {0.f, 0.f, 0.f, 0.f}, qk = kk;
      if (cb <= p) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const bf16x8 bk = ld8(kn_s + nsw(16 * cb + r16, 32 * s + 8 * g4));
          kk = mfma(ak[s], bk, kk);
          qk = mfma(aq[s], bk, qk);
        }
      }
      const int jj = 16 * cb + r16;
      const float gj = gam_s[jj], nj = nk_s[jj];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int ii = 16 * p + 4 * g4 + e;
        float lval = 0.f, aval = 0.f;
        if (cb <= p && ii >= jj) {
          const float dec = expf(gi[e] - gj);
          aval = qi[e] * nj * qk[e] * dec;
          if (ii > jj) lval = bi[e] * ni[e] * nj * kk[e] * dec;
        }
        lt[ii * LT_LD + jj] = lval;
        as_s[ii * AS_LD + jj] = bf16_rne(aval);
      }
    }
  }
  __syncthreads();
  {  // A operand blocks (pi order) -> global: blocks 0, 2, 4, 5, 6, 7 of [p][s]
    u32x4 *aop = a.vh + ch * (NB_VH * 64) + VH_A * 64;
    for (int e = tid; e < 6 * 64; e += 256) {
      const int id = e >> 6, l = e & 63;
      const int blk = id == 0 ? 0 : (id == 1 ? 2 : id + 2);  // ids 0..5 -> blocks 0, 2, 4, 5, 6, 7
      const int bp = blk >> 1, bs = blk & 1;
      const uint16_t *src = as_s + (16 * bp + (l & 15)) * AS_LD + 32 * bs + 4 * (l >> 4);
      const u32x2 x0 = *reinterpret_cast<const u32x2 *>(src);
      const u32x2 x1 = *reinterpret_cast<const u32x2 *>(src + 16);
      aop[blk * 64 + l] = u32x4{x0.x, x0.y, x1.x, x1.y};
    }
  }

  // ---- A.3: T = (I + L)^-1 in place (16x16 diagonal blocks by substitution)
  {
    float x[16];
    const int b = tid >> 4, cc = tid & 15;
    if (tid < 64) {
#pragma unroll
      for (int i = 0; i < 16; ++i) x[i] = (i == cc) ? 1.f : 0.f;
      const float *lb = lt + (16 * b) * LT_LD + 16 * b;
#pragma unroll
      for (int i = 1; i < 16; ++i) {
        if (i > cc) {
          float sacc = 0.f;
#pragma unroll
          for (int jx = 0; jx < i; ++jx) sacc += lb[i * LT_LD + jx] * x[jx];
          x[i] = -sacc;
        }
      }
    }
    __syncthreads();
    if (tid < 64) {
      float *tb = lt + (16 * b) * LT_LD + 16 * b;
#pragma unroll
      for (int i = 0; i < 16; ++i) tb[i * LT_LD + cc] = x[i];
    }
    __syncthreads();
  }
  for (int ab = 1; ab < 4; ++ab) {
    for (int e = tid; e < ab * 256; e += 256) {  // X_b = sum_{kb=b}^{ab-1} L[ab][kb] T[kb][b]
      const int b = e >> 8, r = (e >> 4) & 15, cc = e & 15;
      float sacc = 0.f;
      for (int kb = b; kb < ab; ++kb) {
        const float *lrow = lt + (16 * ab + r) * LT_LD + 16 * kb;
        const float *tcol = lt + (16 * kb) * LT_LD + 16 * b + cc;
#pragma unroll
        for (int qx = 0; qx < 16; ++qx) sacc += lrow[qx] * tcol[qx * LT_LD];
      }
      xs[b][r][cc] = sacc;
    }
    __syncthreads();
    for (int e = tid; e < ab * 256; e += 256) {  // T[ab][b] = -T[ab][ab] X_b
      const int b = e >> 8, r = (e >> 4) & 15, cc = e & 15;
      const float *trow = lt + (16 * ab + r) * LT_LD + 16 * ab;
      float sacc = 0.f;
#pragma unroll
      for (int qx = 0; qx < 16; ++qx) sacc += trow[qx] * xs[b][qx][cc];
      lt[(16 * ab + r) * LT_LD + 16 * b + cc] = -sacc;
    }
    __syncthreads();
  }

  // ---- A.4: W = T diag(beta e^gamma nk) K,  U = T diag(beta) V  (T split hi + lo)
  f32x4 wacc[8];
  {
    const int nsteps = p >= 2 ? 2 : 1;  // T is lower triangular
    bf16x8 wa_hi[2], wa_lo[2], ua_hi[2], ua_lo[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const float *trow = lt + (16 * p + r16) * LT_LD + 32 * s + 8 * g4;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int col = 32 * s + 8 * g4 + e;
        const float t = s < nsteps ? trow[e] : 0.f;
        const float tb = t * beta_s[col];
        const float tw = t * colw_s[col];
        const __bf16 hw = static_cast<__bf16>(tw), hu = static_cast<__bf16>(tb);
        wa_hi[s][e] = hw;
        wa_lo[s][e] = static_cast<__bf16>(tw - static_cast<float>(hw));
        ua_hi[s][e] = hu;
        ua_lo[s][e] = static_cast<__bf16>(tb - static_cast<float>(hu));
      }
    }
    // U in scan operand order: 1 KiB block (column tile nb, row tile p),
    // lane (g, c) holding rows 16p + 4g + 0..3 of column 16 nb + c
    float *Uout = a.Ut + ch * (DV * CK);
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      f32x4 w = {0.f, 0.f, 0.f, 0.f}, u = w;
      const int row = 16 * nb + r16;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        if (s < nsteps) {
          const bf16x8 bk2 = ld8(kt_s + tsw(row, 32 * s + 8 * g4));
          const bf16x8 bv2 = ld8(vt_s + tsw(row, 32 * s + 8 * g4));
          w = mfma(wa_hi[s], bk2, w);
          w = mfma(wa_lo[s], bk2, w);
          u = mfma(ua_hi[s], bv2, u);
          u = mfma(ua_lo[s], bv2, u);
        }
      }
      wacc[nb] = w;
      *reinterpret_cast<f32x4 *>(Uout + ((4 * nb + p) * 64 + lane) * 4) = u;
    }
  }
  __syncthreads();  // T no longer read: reuse lt as the -W staging tile [64][WS_LD] bf16
  {
    uint16_t *ws = reinterpret_cast<uint16_t *>(lt);
#pragma unroll
    for (int nb = 0; nb < 8; ++nb)
#pragma unroll
      for (int e = 0; e < 4; ++e) ws[(16 * p + 4 * g4 + e) * WS_LD + 16 * nb + r16] = f32_to_bf16_bits(-wacc[nb][e]);
  }
  __syncthreads();

  // ---- A.5: operand blocks (-W, K^T) and per-position scalars
  {
    const uint16_t *ws = reinterpret_cast<const uint16_t *>(lt);
    u32x4 *wop = a.vh + ch * (NB_VH * 64) + VH_W * 64;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int e = tid + 256 * it;          // block e/64, lane e%64
      const int blk = e >> 6, l = e & 63;
      const int bp = blk >> 2, bs = blk & 3;
      const uint16_t *src = ws + (16 * bp + (l & 15)) * WS_LD + 32 * bs + 4 * (l >> 4);
      const u32x2 x0 = *reinterpret_cast<const u32x2 *>(src);
      const u32x2 x1 = *reinterpret_cast<const u32x2 *>(src + 16);
      wop[e] = u32x4{x0.x, x0.y, x1.x, x1.y};
    }
    if (khead_writer) {
      u32x4 *kop = a.kh + chk * (NB_KH * 64) + KH_KT * 64;
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int e = tid + 256 * it;
        const int blk = e >> 6, l = e & 63;
        const int bi = blk >> 1, bs = blk & 1;
        const int row = 16 * bi + (l & 15);
        const int col = 32 * bs + 4 * (l >> 4);
        const u32x2 x0 = *reinterpret_cast<const u32x2 *>(kt_s + tsw(row, col));
        const u32x2 x1 = *reinterpret_cast<const u32x2 *>(kt_s + tsw(row, col + 16));
        kop[e] = u32x4{x0.x, x0.y, x1.x, x1.y};
      }
    }
    if (tid < CK) {
      float *sc = reinterpret_cast<float *>(a.vh + ch * (NB_VH * 64) + VH_SC * 64);
      const float gl = gam_s[CK - 1];
      sc[tid] = expf(gam_s[tid]) * nq_s[tid];
      sc[CK + tid] = expf(gl - gam_s[tid]) * nk_s[tid];
      if (tid == 0) sc[2 * CK] = expf(gl);
    }
  }
}

// ------------------------------------------------------------------ phase B
// LDS stage: one chunk's scan operands for a workgroup of NW waves: the
// v-head region, the k-head region, then U for the workgroup's 16*NW
// columns, 4 blocks per wave.
constexpr int ST_W = VH_W * 64;
constexpr int ST_A = VH_A * 64;
constexpr int ST_SC = VH_SC * 64;
constexpr int ST_Q = (NB_VH + KH_Q) * 64;
constexpr int ST_KT = (NB_VH + KH_KT) * 64;
constexpr int ST_U = (NB_VH + NB_KH) * 64;
template <int NW> struct Stage {
  static constexpr int blocks = NB_VH + NB_KH + 4 * NW;
  static constexpr int u4 = blocks * 64;  // size in 16-byte units
};

constexpr int BUF_DWORD3 = 0x00020000;  // raw (untyped) buffer resource word 3 on CDNA

// Copies nb 1 KiB blocks of a region into LDS with buffer_load ... lds: a
// uniform base (no per-lane 64-bit address math), 64 lanes x 16 bytes per
// instruction.  Wave w issues blocks w, w + NW, ...; a wave with no block
// left in the last round copies the region's last block again (same bytes to
// the same LDS address), which keeps the copy free of branches.
template <int NW>
__device__ __forceinline__ void copy_region(u32x4 *dst, const void *src, int nb, int wave, int lane) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(src), 0, nb * 1024, BUF_DWORD3);
#pragma unroll
  for (int i = 0; i < (nb + NW - 1) / NW; ++i) {
    const int t = min(i * NW + wave, nb - 1);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst + t * 64, 16, lane * 16, t * 1024, 0, 0);
  }
}

template <int NW>
__device__ __forceinline__ void stage_load(u32x4 *st, const ChunkArgs &a, size_t ch, size_t chk, int ct, int wave,
                                           int lane) {
  copy_region<NW>(st, a.vh + ch * (NB_VH * 64), NB_VH, wave, lane);
  copy_region<NW>(st + NB_VH * 64, a.kh + chk * (NB_KH * 64), NB_KH, wave, lane);
  copy_region<NW>(st + ST_U, a.Ut + ch * (DV * CK) + ct * (NW * 4 * 256), 4 * NW, wave, lane);
}

// Output of one chunk: lane (g, c) holds rows 16p + 4g + e of its column.  The
// buffer resource starts at the chunk's first token and ends after its last
// valid row, so stores past the sequence end are dropped by the hardware
// range check; voff[4p + e] is the byte offset of row 16p + 4g + e.
template <bool BF16_OUT>
__device__ __forceinline__ void store_chunk(const f32x4 (&o)[4], __amdgpu_buffer_rsrc_t r, const int (&voff)[16]) {
#pragma unroll
  for (int p = 0; p < 4; ++p)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (BF16_OUT)
        __builtin_amdgcn_raw_buffer_store_b16(bf16_rne(o[p][e]), r, voff[4 * p + e], 0, 0);
      else
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, o[p][e]), r, voff[4 * p + e], 0, 0);
    }
}

// sched_group_barrier masks
constexpr int SG_VALU = 0x2, SG_MFMA = 0x8, SG_VMEM_WR = 0x40, SG_DS_RD = 0x100;
#define GDN_SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)
#define GDN_GROUP(mask, n) __builtin_amdgcn_sched_group_barrier(mask, n, 0)

// One chunk of the scan for this wave's 16 state columns, in three
// scheduling regions.  The scan runs one wave per SIMD, so the vector ALU
// work is interleaved with the MFMAs by hand (sched_group_barrier patterns):
//   R1  V' = U - W S            16 MFMAs | S *= e^{gamma_63}, previous chunk's
//                                          output stores; reads Q, scales
//   R2  acc = Q S               16 MFMAs | V' to bf16, V'' = sk V' split hi + lo;
//                                          reads A, K^T
//   R3  S += K^T V'' (hi, lo)   32 MFMAs | O = sq acc, then O += A V' (6 MFMAs),
//                                          next chunk's bf16 state operands
// sb holds the state as bf16 B operands (k-steps over the 128 state rows);
// on return it holds the updated state, o holds this chunk's output.
template <bool BF16_OUT>
__device__ __forceinline__ void scan_chunk(const u32x4 *st, int ubase, f32x4 (&S)[8], bf16x8 (&sb)[4], f32x4 (&o)[4],
                                           __amdgpu_buffer_rsrc_t prev_out, const int (&voff)[16], int lane) {
  const int g4 = lane >> 4;
  const float *sc = reinterpret_cast<const float *>(st + ST_SC);

  // ---- R1
  u32x4 wb[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) wb[i] = st[ST_W + i * 64 + lane];
  f32x4 vp[4];  // V' rows 16p + 4g + e
#pragma unroll
  for (int p = 0; p < 4; ++p) vp[p] = __builtin_bit_cast(f32x4, st[ubase + p * 64 + lane]);
  const float eL = sc[2 * CK];
  u32x4 qb[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) qb[i] = st[ST_Q + i * 64 + lane];
  f32x4 sk[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) sk[p] = *reinterpret_cast<const f32x4 *>(sc + CK + 16 * p + 4 * g4);
  store_chunk<BF16_OUT>(o, prev_out, voff);
#pragma unroll
  for (int s2 = 0; s2 < 4; ++s2)
#pragma unroll
    for (int p = 0; p < 4; ++p) vp[p] = mfma(as_bf16x8(wb[4 * p + s2]), sb[s2], vp[p]);
#pragma unroll
  for (int i = 0; i < 8; ++i) S[i] = S[i] * eL;
  GDN_GROUP(SG_DS_RD, 21);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    GDN_GROUP(SG_MFMA, 1);
    GDN_GROUP(SG_DS_RD, 1);
    GDN_GROUP(SG_VALU, 3);
    GDN_GROUP(SG_VMEM_WR, 1);
  }
  GDN_SCHED_FENCE();

  // ---- R2
  u32x4 ab[6], kb[16];  // A blocks 0, 2, 4, 5, 6, 7 (the others are zero); K^T tiles
  ab[0] = st[ST_A + 0 * 64 + lane];
  ab[1] = st[ST_A + 2 * 64 + lane];
  ab[2] = st[ST_A + 4 * 64 + lane];
  ab[3] = st[ST_A + 5 * 64 + lane];
  ab[4] = st[ST_A + 6 * 64 + lane];
  ab[5] = st[ST_A + 7 * 64 + lane];
#pragma unroll
  for (int i = 0; i < 16; ++i) kb[i] = st[ST_KT + i * 64 + lane];
  f32x4 sq[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) sq[p] = *reinterpret_cast<const f32x4 *>(sc + 16 * p + 4 * g4);
  f32x4 acc[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) acc[p] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s2 = 0; s2 < 4; ++s2)
#pragma unroll
    for (int p = 0; p < 4; ++p) acc[p] = mfma(as_bf16x8(qb[4 * p + s2]), sb[s2], acc[p]);
  bf16x8 vb[2], vh[2], vl[2];
  vb[0] = pack_hi(vp[0], vp[1]);
  vb[1] = pack_hi(vp[2], vp[3]);
#pragma unroll
  for (int p2 = 0; p2 < 2; ++p2)  // V'' = diag(e^{gamma_63 - gamma} nk) V', hi + lo
    pack_hilo(vp[2 * p2] * sk[2 * p2], vp[2 * p2 + 1] * sk[2 * p2 + 1], vh[p2], vl[p2]);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    GDN_GROUP(SG_MFMA, 1);
    GDN_GROUP(SG_DS_RD, 2);
    GDN_GROUP(SG_VALU, 4);
  }
  GDN_SCHED_FENCE();

  // ---- R3
#pragma unroll
  for (int half = 0; half < 2; ++half)
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
#pragma unroll
      for (int t = 0; t < 4; ++t) S[4 * half + t] = mfma(as_bf16x8(kb[2 * (4 * half + t) + s2]), vh[s2], S[4 * half + t]);
#pragma unroll
      for (int t = 0; t < 4; ++t) S[4 * half + t] = mfma(as_bf16x8(kb[2 * (4 * half + t) + s2]), vl[s2], S[4 * half + t]);
    }
#pragma unroll
  for (int p = 0; p < 4; ++p) o[p] = acc[p] * sq[p];
  o[0] = mfma(as_bf16x8(ab[0]), vb[0], o[0]);
  o[1] = mfma(as_bf16x8(ab[1]), vb[0], o[1]);
  o[2] = mfma(as_bf16x8(ab[2]), vb[0], o[2]);
  o[3] = mfma(as_bf16x8(ab[4]), vb[0], o[3]);
  o[2] = mfma(as_bf16x8(ab[3]), vb[1], o[2]);
  o[3] = mfma(as_bf16x8(ab[5]), vb[1], o[3]);
#pragma unroll
  for (int s2 = 0; s2 < 4; ++s2) sb[s2] = pack_hi(S[2 * s2], S[2 * s2 + 1]);
#pragma unroll
  for (int i = 0; i < 38; ++i) {
    GDN_GROUP(SG_MFMA, 1);
    GDN_GROUP(SG_VALU, 1);
  }
  GDN_SCHED_FENCE();
}

// Workgroup = NW waves = 16*NW state columns of one (sequence, v-head).  The
// two LDS stages leave room for one workgroup per CU, so each SIMD runs one
// wave and may use the whole register file.
template <int NW, bool BF16_OUT>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(1, 1))) void chunk_scan_kernel(ChunkArgs a) {
  __shared__ u32x4 stage0[Stage<NW>::u4];
  __shared__ u32x4 stage1[Stage<NW>::u4];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g4 = lane >> 4;
  const int r16 = lane & 15;
  const int nh = a.n_seqs * a.Hv;
  const int ct = blockIdx.x / nh;    // the column tiles of one head share bid % 8,
  const int rest = blockIdx.x % nh;  // i.e. one XCD and its L2
  const int n = rest / a.Hv;
  const int h = rest % a.Hv;
  const int hk = h / (a.Hv / a.Hk);
  const int col = 16 * NW * ct + 16 * wave + r16;
  const int ubase = ST_U + wave * 4 * 64;  // this wave's U blocks in a stage

  // Values read from memory are workgroup-uniform; readfirstlane tells the
  // compiler so (buffer resources built from them must live in SGPRs).
  int64_t s0;
  int slen;
  seq_bounds(a, n, &s0, &slen);
  s0 = uniform64(s0);
  slen = __builtin_amdgcn_readfirstlane(slen);
  // Chunks [cs, ce) of sequence n; this launch covers global chunks
  // [seg_begin, seg_end).  chunk_start is built from clamped lengths, so it
  // never exceeds the workspace bound; the min() keeps that true here too.
  const int cs = __builtin_amdgcn_readfirstlane(a.chunk_start[n]);
  const int ce = __builtin_amdgcn_readfirstlane(max(cs, min(a.chunk_start[n + 1], a.max_chunks)));
  const int lo = max(cs, a.seg_begin), hi = min(ce, a.seg_end);
  const int64_t in_row = a.h0 ? uniform64(a.h0_idx ? a.h0_idx[n] : n) : -1;
  const int64_t out_row = a.hT ? uniform64(a.hT_idx ? a.hT_idx[n] : n) : -1;
  const int64_t kv = static_cast<int64_t>(DK) * DV;
  if (cs == ce) {  // empty sequence: the final state is the initial one (handled once)
    if (a.seg_begin == 0 && out_row >= 0) {
      float *dst = a.hT + (out_row * a.Hv + h) * kv + col;
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 16 * i + 4 * g4 + e;
          dst[r * DV] = in_row >= 0 ? a.h0[(in_row * a.Hv + h) * kv + r * DV + col] : 0.f;
        }
    }
    return;
  }
  if (lo >= hi) return;  // no chunk of this sequence in this segment
  const int nch = hi - lo;
  const int c0 = lo - a.seg_begin;                             // first chunk, workspace-local
  const int64_t seq_off = static_cast<int64_t>(lo - cs) * CK;  // its first token within the sequence
  float *carry = a.carry + (static_cast<int64_t>(n) * a.Hv + h) * kv + col;

  f32x4 S[8];
  const float *src = lo == cs ? (in_row >= 0 ? a.h0 + (in_row * a.Hv + h) * kv + col : nullptr) : carry;
  if (src) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) S[i][e] = src[(16 * i + 4 * g4 + e) * DV];
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) S[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  bf16x8 sb[4];
#pragma unroll
  for (int s2 = 0; s2 < 4; ++s2) sb[s2] = pack_hi(S[2 * s2], S[2 * s2 + 1]);

  // Output addressing: byte offsets of rows 16p + 4g + e within a chunk.
  typedef typename std::conditional<BF16_OUT, uint16_t, float>::type OT;
  const int64_t ostep = static_cast<int64_t>(a.Hv) * DV;  // elements per token
  int voff[16];
#pragma unroll
  for (int p = 0; p < 4; ++p)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      voff[4 * p + e] = static_cast<int>(((16 * p + 4 * g4 + e) * ostep + h * DV + col) * sizeof(OT));
  auto out_rsrc = [&](int c) {  // chunk c of this launch: rows [0, min(64, rest of sequence))
    const int64_t toff = seq_off + static_cast<int64_t>(c) * CK;
    const int rows = static_cast<int>(min<int64_t>(CK, slen - toff));
    OT *base = static_cast<OT *>(a.o) + (s0 + toff) * ostep;
    return __builtin_amdgcn_make_buffer_rsrc(base, 0, static_cast<int>(rows * ostep * sizeof(OT)), BUF_DWORD3);
  };
  // Before the first chunk there is no output to store: a zero-sized range.
  __amdgpu_buffer_rsrc_t prev = __builtin_amdgcn_make_buffer_rsrc(a.o, 0, 0, BUF_DWORD3);
  f32x4 o[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) o[p] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto load_stage = [&](u32x4 *st, int cidx) {
    const size_t j = static_cast<size_t>(c0 + cidx);
    stage_load<NW>(st, a, j * a.Hv + h, j * a.Hk + hk, ct, wave, lane);
  };
  // A chunk's output is stored during the next chunk (vmcnt counts stores
  // too, so the wait at the end of each chunk then finds them long done).
  load_stage(stage0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int c = 0; c < nch; c += 2) {
    if (c + 1 < nch) load_stage(stage1, c + 1);
    scan_chunk<BF16_OUT>(stage0, ubase, S, sb, o, prev, voff, lane);
    prev = out_rsrc(c);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (c + 1 >= nch) break;
    if (c + 2 < nch) load_stage(stage0, c + 2);
    scan_chunk<BF16_OUT>(stage1, ubase, S, sb, o, prev, voff, lane);
    prev = out_rsrc(c + 1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  store_chunk<BF16_OUT>(o, prev, voff);

  float *dst = hi == ce ? (out_row >= 0 ? a.hT + (out_row * a.Hv + h) * kv + col : nullptr) : carry;
  if (dst) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) dst[(16 * i + 4 * g4 + e) * DV] = S[i][e];
  }
}

// Scan workgroup shape (measured on MI355X at T=4096, 32 v-heads): 4 waves =
// 64 state columns per workgroup.  With 8 waves per workgroup every wave
// re-reads the whole operand stage from LDS and the LDS bandwidth becomes the
// limit; with 2 the stage is streamed four times.
constexpr int SCAN_WAVES = 4;

// Chunks per prep + scan segment: the operand workspace of one segment
// (about 2.3 MiB per chunk at 32 v-heads) stays resident in the 256 MB
// Infinity Cache between the producer and the consumer launch.
constexpr int SEG_CHUNKS = 16;

struct WsLayout {
  size_t chunk_start, vh, kh, Ut, carry, total;
};

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

WsLayout ws_layout(int n_seqs, int64_t seg_chunks, int Hv, int Hk, bool need_carry) {
  WsLayout l;
  size_t off = 0;
  l.chunk_start = off;
  off = align256(off + sizeof(int32_t) * (n_seqs + 1));
  l.vh = off;
  off = align256(off + 16ull * seg_chunks * Hv * NB_VH * 64);
  l.kh = off;
  off = align256(off + 16ull * seg_chunks * Hk * NB_KH * 64);
  l.Ut = off;
  off = align256(off + sizeof(float) * seg_chunks * Hv * DV * CK);
  l.carry = off;
  if (need_carry) off = align256(off + sizeof(float) * static_cast<size_t>(n_seqs) * Hv * DK * DV);
  l.total = off;
  return l;
}

int64_t max_chunks_of(int n_seqs, int64_t total_tokens, bool varlen, int T) {
  if (!varlen) return static_cast<int64_t>(n_seqs) * ((T + CK - 1) / CK);
  return (total_tokens + CK - 1) / CK + n_seqs;
}

}  // namespace
}  // namespace gdn

extern "C" size_t gdn_chunk_workspace_bytes(int32_t n_seqs, int64_t total_tokens, int32_t Hv, int32_t K,
                                            int32_t V) {
  using namespace gdn;
  if (n_seqs <= 0 || total_tokens < 0 || Hv <= 0 || K != DK || V != DV) return 0;
  // Upper bound valid with or without cu_seqlens; k-head blocks counted at Hk = Hv.
  const int64_t nc = (total_tokens + CK - 1) / CK + n_seqs;
  return ws_layout(n_seqs, std::min<int64_t>(nc, SEG_CHUNKS), Hv, Hv, nc > SEG_CHUNKS).total;
}

extern "C" int gdn_chunk_fwd(const void *q, const void *k, const void *v, int qkv_dtype,
                             int64_t q_stride_t, int64_t k_stride_t, int64_t v_stride_t,
                             const float *g, const void *beta, int beta_dtype,
                             const float *h0, const int64_t *h0_idx,
                             float *hT, const int64_t *hT_idx,
                             void *o, int o_dtype,
                             const int32_t *cu_seqlens, int32_t n_seqs, int32_t T,
                             int32_t Hk, int32_t Hv, int32_t K, int32_t V,
                             float scale, int l2norm_qk,
                             void *workspace, size_t workspace_bytes, void *stream) {
  using namespace gdn;
  if (K != DK || V != DV) return fail(GDN_ERR_UNSUPPORTED, "gdn_chunk_fwd: K=%d V=%d; only K=V=128 is built", K, V);
  if (qkv_dtype != GDN_DTYPE_BF16)
    return fail(GDN_ERR_UNSUPPORTED, "gdn_chunk_fwd: q/k/v must be bf16 (MFMA operands)");
  if (n_seqs < 0 || T < 0 || Hk <= 0 || Hv <= 0 || Hv % Hk)
    return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_chunk_fwd: bad sizes n_seqs=%d T=%d Hk=%d Hv=%d", n_seqs, T, Hk, Hv);
  if (!valid_dtype(beta_dtype)) return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_chunk_fwd: bad beta dtype");
  if (o_dtype != GDN_DTYPE_BF16 && o_dtype != GDN_DTYPE_F32)
    return fail(GDN_ERR_UNSUPPORTED, "gdn_chunk_fwd: output must be bf16 or fp32");
  if (n_seqs == 0) return ok();
  if (!q || !k || !v || !g || !beta || !o) return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_chunk_fwd: null q/k/v/g/beta/o");
  if (q_stride_t < Hk * K || k_stride_t < Hk * K || v_stride_t < Hv * V || (q_stride_t | k_stride_t | v_stride_t) % 8)
    return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_chunk_fwd: token strides must cover a row and be multiples of 8");
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) % 16)
    return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_chunk_fwd: q/k/v must be 16-byte aligned");
  const int64_t total = cu_seqlens ? static_cast<int64_t>(T) : static_cast<int64_t>(n_seqs) * T;
  const int64_t nc = max_chunks_of(n_seqs, total, cu_seqlens != nullptr, T);
  const int64_t seg = std::min<int64_t>(nc, SEG_CHUNKS);
  const WsLayout l = ws_layout(n_seqs, seg, Hv, Hk, nc > SEG_CHUNKS);
  if (!workspace || workspace_bytes < l.total)
    return fail(GDN_ERR_WORKSPACE, "gdn_chunk_fwd: workspace %zu bytes < %zu needed", workspace_bytes, l.total);
  if (reinterpret_cast<uintptr_t>(workspace) % 256)
    return fail(GDN_ERR_WORKSPACE, "gdn_chunk_fwd: workspace must be 256-byte aligned");
  if (nc > 65535) return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_chunk_fwd: %lld chunks exceed one launch", (long long)nc);
  const int64_t scan_blocks = static_cast<int64_t>(n_seqs) * Hv * (DV / (16 * SCAN_WAVES));
  if (scan_blocks > 0x7fffffff) return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_chunk_fwd: grid too large");
  char *ws = static_cast<char *>(workspace);
  ChunkArgs a{static_cast<const uint16_t *>(q), static_cast<const uint16_t *>(k), static_cast<const uint16_t *>(v),
              q_stride_t, k_stride_t, v_stride_t, g, beta, beta_dtype, h0, h0_idx, hT, hT_idx, o, o_dtype,
              cu_seqlens, n_seqs, T, Hk, Hv, total, scale, l2norm_qk, static_cast<int>(nc), 0, 0,
              reinterpret_cast<int32_t *>(ws + l.chunk_start), reinterpret_cast<u32x4 *>(ws + l.vh),
              reinterpret_cast<u32x4 *>(ws + l.kh), reinterpret_cast<float *>(ws + l.Ut),
              reinterpret_cast<float *>(ws + l.carry)};
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(chunk_table_kernel, dim3(1), dim3(256), 0, s, a);
  // One prep + scan pair per segment of SEG_CHUNKS global chunks (at least one
  // pair, so that empty sequences still pass their initial state through).
  for (int64_t sb = 0; sb == 0 || sb < nc; sb += seg) {
    a.seg_begin = static_cast<int>(sb);
    a.seg_end = static_cast<int>(std::min<int64_t>(sb + seg, nc));
    if (seg > 0) hipLaunchKernelGGL(chunk_prep_kernel, dim3(Hv, static_cast<unsigned>(seg)), dim3(256), 0, s, a);
    if (o_dtype == GDN_DTYPE_BF16)
      hipLaunchKernelGGL((chunk_scan_kernel<SCAN_WAVES, true>), dim3(static_cast<unsigned>(scan_blocks)),
                         dim3(64 * SCAN_WAVES), 0, s, a);
    else
      hipLaunchKernelGGL((chunk_scan_kernel<SCAN_WAVES, false>), dim3(static_cast<unsigned>(scan_blocks)),
                         dim3(64 * SCAN_WAVES), 0, s, a);
  }
  return check_launch("gdn_chunk_fwd");
}
