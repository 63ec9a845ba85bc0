// Chunk-64 gated delta rule prefill on bf16 MFMA (gfx950).
//
// The reference algorithm (engine/kernels/delta_rule.py:286-349) per chunk
// of 64 tokens and v-head, with gamma = chunk-local cumsum(g):
//   L = strict_lower(diag(beta) K~K~^T * Gamma),  T = (I + L)^-1
//   U = T (beta V),  W = T (beta e^gamma K~)
//   V' = U - W S ;  O = (e^gamma Q~) S + lower(Q~K~^T * Gamma) V'
//   S <- e^{gamma_63} S + (e^{gamma_63 - gamma} K~)^T V'
// is split into three launches:
//   chunk_table_kernel  chunk -> (sequence, first token) table (cu_seqlens aware)
//   chunk_prep_kernel   one workgroup per (chunk, v-head), all in parallel:
//                       K K^T and Q K^T on MFMA from the raw bf16 rows (exact
//                       products; the l2norm and gate factors are applied to
//                       the fp32 results), T by blocked forward substitution
//                       in fp32 (LDS), then W = T' K and U = T'' V on MFMA with
//                       T', T'' split into bf16 hi + lo parts.
//   chunk_scan_kernel   one wave per (sequence, v-head, 16 state columns), serial
//                       over the chunks: the state slice lives in MFMA
//                       accumulators for the whole sequence.
// Precision (checked against an fp64 restatement at T=4096): the state is fed
// to MFMA as bf16, U stays fp32 (it initialises the V' accumulator) and the
// state increment K^T V'' uses V'' split into bf16 hi + lo.
//
// MFMA: v_mfma_f32_16x16x32_bf16.  Lane l holds A[l%16][8(l/16)+j] and
// B[8(l/16)+j][l%16] (j<8) and D[4(l/16)+i][l%16] (i<4).  When an
// accumulator tile pair (rows 0-15, 16-31 of a 32-long reduction) is reused
// as the B operand of the next product, lane group g = l/16 holds reduction
// indices {4g..4g+3, 16+4g..16+4g+3}; the matching A operand reads the same
// index set ("pi" order) with two 8-byte loads.  No LDS round trip.
#include "gdn_common.h"

namespace gdn {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) unsigned u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned u32x2;

constexpr int CK = 64;    // chunk length
constexpr int DK = 128;   // k head dim
constexpr int DV = 128;   // v head dim
constexpr int SCAL = 132; // per (chunk, head) scalars: sq[64], sk[64], eL, pad

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 u) { return __builtin_bit_cast(bf16x8, u); }

// 8 consecutive bf16 at p (16-byte aligned)
__device__ __forceinline__ bf16x8 ld8(const uint16_t *p) {
  return as_bf16x8(*reinterpret_cast<const u32x4 *>(p));
}
// pi-order operand: p[0..3] and p[16..19] (each 8-byte aligned)
__device__ __forceinline__ bf16x8 ld_pi(const uint16_t *p) {
  const u32x2 a = *reinterpret_cast<const u32x2 *>(p);
  const u32x2 b = *reinterpret_cast<const u32x2 *>(p + 16);
  u32x4 u = {a.x, a.y, b.x, b.y};
  return as_bf16x8(u);
}
__device__ __forceinline__ bf16x8 zero8() {
  u32x4 u = {0u, 0u, 0u, 0u};
  return as_bf16x8(u);
}

// two accumulator tiles -> one pi-order B operand (bf16 hi part)
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
  // workspace
  int32_t *chunk_start;  // [n_seqs + 1]
  uint16_t *W;           // [NC][Hv][64][128]   -W, bf16
  float *Ut;             // [NC][Hv][128][64]   U transposed, fp32
  uint16_t *A;           // [NC][Hv][64][64]    lower(Q~K~^T Gamma), bf16
  uint16_t *Kt;          // [NC][Hk][128][64]   raw K transposed, bf16
  float *scal;           // [NC][Hv][SCAL]
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
    const int32_t nc = (len + CK - 1) / CK;
    part[threadIdx.x] = nc;
    __syncthreads();
    // inclusive scan (Hillis-Steele) over 256 entries
    for (int off = 1; off < 256; off <<= 1) {
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
constexpr int KT_LD = CK + 8;   // LDS row stride (bf16) of the transposed K / V tiles
constexpr int TF_LD = CK + 4;   // LDS row stride (fp32) of L / T

__global__ __launch_bounds__(256) void chunk_prep_kernel(ChunkArgs a) {
  __shared__ __align__(16) uint16_t kt_s[DK * KT_LD];
  __shared__ __align__(16) uint16_t vt_s[DV * KT_LD];
  __shared__ __align__(16) float lf[CK * TF_LD];   // L (strict lower)
  __shared__ __align__(16) float tf[CK * TF_LD];   // T = (I + L)^-1
  __shared__ __align__(16) float xs[3][16][17];    // block products
  __shared__ float gam_s[CK], beta_s[CK], nk_s[CK], nq_s[CK];

  const int h = blockIdx.x;
  const int j = blockIdx.y;
  const int total_chunks = a.chunk_start[a.n_seqs];
  if (j >= total_chunks) return;
  // sequence owning chunk j: last n with chunk_start[n] <= j
  int lo = 0, hi = a.n_seqs;
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
  const int hk = h / (a.Hv / a.Hk);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g4 = lane >> 4;   // lane group
  const int r16 = lane & 15;

  // ---- A.1: K^T and V^T tiles into LDS, row norms, gates
  for (int i = tid; i < CK * TF_LD; i += 256) tf[i] = 0.f;
  {
    const int seg = tid & 15;         // 8-element column segment
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int row = (tid >> 4) + 16 * it;
      const bool live = row < len;
      const int64_t tok = t0 + row;
      u32x4 ku = {0u, 0u, 0u, 0u}, qu = ku, vu = ku;
      if (live) {
        ku = *reinterpret_cast<const u32x4 *>(a.k + tok * a.ks + (int64_t)hk * DK + seg * 8);
        qu = *reinterpret_cast<const u32x4 *>(a.q + tok * a.qs + (int64_t)hk * DK + seg * 8);
        vu = *reinterpret_cast<const u32x4 *>(a.v + tok * a.vs + (int64_t)h * DV + seg * 8);
      }
      float sk = 0.f, sq = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t kw = ku[e], qw = qu[e], vw = vu[e];
        const float k0 = bf16_bits_to_f32(kw & 0xffffu), k1 = bf16_bits_to_f32(kw >> 16);
        const float q0 = bf16_bits_to_f32(qw & 0xffffu), q1 = bf16_bits_to_f32(qw >> 16);
        sk += k0 * k0 + k1 * k1;
        sq += q0 * q0 + q1 * q1;
        kt_s[(seg * 8 + 2 * e) * KT_LD + row] = static_cast<uint16_t>(kw & 0xffffu);
        kt_s[(seg * 8 + 2 * e + 1) * KT_LD + row] = static_cast<uint16_t>(kw >> 16);
        vt_s[(seg * 8 + 2 * e) * KT_LD + row] = static_cast<uint16_t>(vw & 0xffffu);
        vt_s[(seg * 8 + 2 * e + 1) * KT_LD + row] = static_cast<uint16_t>(vw >> 16);
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
      const bool live = lane < len;
      float gv = live ? a.g[(t0 + lane) * a.Hv + h] : 0.f;
      const float bv = live ? load_elem(a.beta, (t0 + lane) * a.Hv + h, a.beta_dt) : 0.f;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float x = __shfl_up(gv, off, 64);
        if (lane >= off) gv += x;
      }
      gam_s[lane] = gv;
      beta_s[lane] = bv;
    }
  }
  __syncthreads();

  // ---- A.2: K K^T and Q K^T (wave w owns row block p = w)
  const size_t ch = static_cast<size_t>(j) * a.Hv + h;
  {
    const int p = wave;
    const int row = 16 * p + r16;
    const bool live_r = row < len;
    const uint16_t *krow = a.k + (t0 + row) * a.ks + (int64_t)hk * DK;
    const uint16_t *qrow = a.q + (t0 + row) * a.qs + (int64_t)hk * DK;
    uint16_t *Aout = a.A + ch * (CK * CK);
    for (int cb = 0; cb < 4; ++cb) {
      f32x4 kk = {0.f, 0.f, 0.f, 0.f}, qk = kk;
      if (cb <= p) {
        const int col = 16 * cb + r16;
        const bool live_c = col < len;
        const uint16_t *kcol = a.k + (t0 + col) * a.ks + (int64_t)hk * DK;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int off = 32 * s + 8 * g4;
          const bf16x8 ak = live_r ? ld8(krow + off) : zero8();
          const bf16x8 aq = live_r ? ld8(qrow + off) : zero8();
          const bf16x8 bk = live_c ? ld8(kcol + off) : zero8();
          kk = mfma(ak, bk, kk);
          qk = mfma(aq, bk, qk);
        }
      }
      const int jj = 16 * cb + r16;  // column (key position) of this lane
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int ii = 16 * p + 4 * g4 + e;  // row (query position)
        float lval = 0.f, aval = 0.f;
        if (cb <= p && ii >= jj) {
          const float dec = expf(gam_s[ii] - gam_s[jj]);
          aval = nq_s[ii] * nk_s[jj] * qk[e] * dec;
          if (ii > jj) lval = beta_s[ii] * nk_s[ii] * nk_s[jj] * kk[e] * dec;
        }
        lf[ii * TF_LD + jj] = lval;
        Aout[ii * CK + jj] = f32_to_bf16_bits(aval);
      }
    }
  }
  __syncthreads();

  // ---- A.3: T = (I + L)^-1, blocked (16x16 diagonal blocks by substitution)
  if (tid < 64) {
    const int b = tid >> 4, cc = tid & 15;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = (i == cc) ? 1.f : 0.f;
    const float *lb = lf + (16 * b) * TF_LD + 16 * b;
#pragma unroll
    for (int i = 1; i < 16; ++i) {
      if (i > cc) {
        float s = 0.f;
#pragma unroll
        for (int jx = 0; jx < i; ++jx) s += lb[i * TF_LD + jx] * x[jx];
        x[i] = -s;
      }
    }
    float *tb = tf + (16 * b) * TF_LD + 16 * b;
#pragma unroll
    for (int i = 0; i < 16; ++i) tb[i * TF_LD + cc] = x[i];
  }
  __syncthreads();
  for (int ab = 1; ab < 4; ++ab) {
    // X_b = sum_{kb=b}^{ab-1} L[ab][kb] T[kb][b]   for b < ab
    for (int e = tid; e < ab * 256; e += 256) {
      const int b = e >> 8, r = (e >> 4) & 15, cc = e & 15;
      float s = 0.f;
      for (int kb = b; kb < ab; ++kb) {
        const float *lrow = lf + (16 * ab + r) * TF_LD + 16 * kb;
        const float *tcol = tf + (16 * kb) * TF_LD + 16 * b + cc;
#pragma unroll
        for (int qx = 0; qx < 16; ++qx) s += lrow[qx] * tcol[qx * TF_LD];
      }
      xs[b][r][cc] = s;
    }
    __syncthreads();
    // T[ab][b] = -T[ab][ab] X_b
    for (int e = tid; e < ab * 256; e += 256) {
      const int b = e >> 8, r = (e >> 4) & 15, cc = e & 15;
      const float *trow = tf + (16 * ab + r) * TF_LD + 16 * ab;
      float s = 0.f;
#pragma unroll
      for (int qx = 0; qx < 16; ++qx) s += trow[qx] * xs[b][qx][cc];
      tf[(16 * ab + r) * TF_LD + 16 * b + cc] = -s;
    }
    __syncthreads();
  }

  // ---- A.4: W = T diag(beta e^gamma nk) K,  U = T diag(beta) V  (hi + lo T)
  {
    const int p = wave;
    const int nsteps = p >= 2 ? 2 : 1;  // T is lower triangular
    bf16x8 wa_hi[2], wa_lo[2], ua_hi[2], ua_lo[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      if (s < nsteps) {
        const float *trow = tf + (16 * p + r16) * TF_LD + 32 * s + 8 * g4;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int col = 32 * s + 8 * g4 + e;
          const float t = trow[e];
          const float tb = t * beta_s[col];
          const float tw = tb * expf(gam_s[col]) * nk_s[col];
          const __bf16 hw = static_cast<__bf16>(tw), hu = static_cast<__bf16>(tb);
          wa_hi[s][e] = hw;
          wa_lo[s][e] = static_cast<__bf16>(tw - static_cast<float>(hw));
          ua_hi[s][e] = hu;
          ua_lo[s][e] = static_cast<__bf16>(tb - static_cast<float>(hu));
        }
      }
    }
    uint16_t *Wout = a.W + ch * (CK * DK);
    float *Uout = a.Ut + ch * (DV * CK);
#pragma unroll 2
    for (int nb = 0; nb < 8; ++nb) {
      f32x4 w = {0.f, 0.f, 0.f, 0.f}, u = w;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        if (s < nsteps) {
          const bf16x8 bk = ld8(kt_s + (16 * nb + r16) * KT_LD + 32 * s + 8 * g4);
          const bf16x8 bv = ld8(vt_s + (16 * nb + r16) * KT_LD + 32 * s + 8 * g4);
          w = mfma(wa_hi[s], bk, w);
          w = mfma(wa_lo[s], bk, w);
          u = mfma(ua_hi[s], bv, u);
          u = mfma(ua_lo[s], bv, u);
        }
      }
      // D layout: column 16nb + r16, rows 16p + 4g4 + e
#pragma unroll
      for (int e = 0; e < 4; ++e) Wout[(16 * p + 4 * g4 + e) * DK + 16 * nb + r16] = f32_to_bf16_bits(-w[e]);
      *reinterpret_cast<f32x4 *>(Uout + (16 * nb + r16) * CK + 16 * p + 4 * g4) = u;
    }
  }

  // ---- A.5: per-position scalars and the transposed raw K tile
  if (tid < CK) {
    float *sc = a.scal + ch * SCAL;
    const float gl = gam_s[CK - 1];
    sc[tid] = expf(gam_s[tid]) * nq_s[tid];
    sc[CK + tid] = expf(gl - gam_s[tid]) * nk_s[tid];
    if (tid == 0) sc[2 * CK] = expf(gl);
  }
  if (h % (a.Hv / a.Hk) == 0) {
    uint16_t *kt_out = a.Kt + (static_cast<size_t>(j) * a.Hk + hk) * (DK * CK);
    for (int e = tid; e < DK * CK / 8; e += 256) {
      const int row = e >> 3, seg = e & 7;
      *reinterpret_cast<u32x4 *>(kt_out + row * CK + seg * 8) =
          *reinterpret_cast<const u32x4 *>(kt_s + row * KT_LD + seg * 8);
    }
  }
}

// ------------------------------------------------------------------ phase B
// Workgroup = 4 waves = 64 state columns of one (sequence, v-head); wave w owns
// columns 16*(4*half + w) .. +16 and all 128 state rows (8 accumulator tiles).
__global__ __launch_bounds__(256) void chunk_scan_kernel(ChunkArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g4 = lane >> 4;
  const int r16 = lane & 15;
  const int nh = a.n_seqs * a.Hv;
  const int half = blockIdx.x / nh;  // heads of a sequence are adjacent: all
  const int rest = blockIdx.x % nh;  // tiles of a head land on one XCD
  const int n = rest / a.Hv;
  const int h = rest % a.Hv;
  const int hk = h / (a.Hv / a.Hk);
  const int vt = 4 * half + wave;
  const int col = 16 * vt + r16;     // this lane's state column

  int64_t s0;
  int slen;
  seq_bounds(a, n, &s0, &slen);
  const int c0 = a.chunk_start[n];
  // chunk_start is built from the clamped lengths, so it never exceeds the
  // workspace bound; the min() keeps that true by construction here too.
  const int nch = max(0, min(a.chunk_start[n + 1], a.max_chunks) - c0);

  f32x4 S[8];
  const int64_t in_row = a.h0 ? (a.h0_idx ? a.h0_idx[n] : n) : -1;
  if (in_row >= 0) {
    const float *src = a.h0 + (in_row * a.Hv + h) * (int64_t)(DK * DV) + col;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) S[i][e] = src[(16 * i + 4 * g4 + e) * DV];
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) S[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  for (int c = 0; c < nch; ++c) {
    const int j = c0 + c;
    const size_t ch = static_cast<size_t>(j) * a.Hv + h;
    const int64_t t0 = s0 + static_cast<int64_t>(c) * CK;
    const int len = min(CK, slen - c * CK);
    const uint16_t *Wc = a.W + ch * (CK * DK);
    const float *Uc = a.Ut + ch * (DV * CK) + col * CK;
    const uint16_t *Ac = a.A + ch * (CK * CK);
    const uint16_t *Ktc = a.Kt + (static_cast<size_t>(j) * a.Hk + hk) * (DK * CK);
    const float *sc = a.scal + ch * SCAL;

    // state as bf16 B operands (k-steps over the 128 state rows)
    bf16x8 sb[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) sb[s] = pack_hi(S[2 * s], S[2 * s + 1]);

    // V' = U - W S     (rows: chunk positions 16p + 4g4 + e)
    f32x4 vp[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      vp[p] = *reinterpret_cast<const f32x4 *>(Uc + 16 * p + 4 * g4);
      const uint16_t *wrow = Wc + (16 * p + r16) * DK + 4 * g4;
#pragma unroll
      for (int s = 0; s < 4; ++s) vp[p] = mfma(ld_pi(wrow + 32 * s), sb[s], vp[p]);
    }

    // O = diag(e^gamma nq) (Q S) + A V'
    bf16x8 vb[2];
    vb[0] = pack_hi(vp[0], vp[1]);
    vb[1] = pack_hi(vp[2], vp[3]);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int row = 16 * p + r16;
      const bool live = row < len;
      const uint16_t *qrow = a.q + (t0 + row) * a.qs + (int64_t)hk * DK + 4 * g4;
      f32x4 oq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) oq = mfma(live ? ld_pi(qrow + 32 * s) : zero8(), sb[s], oq);
      const f32x4 sq = *reinterpret_cast<const f32x4 *>(sc + 16 * p + 4 * g4);
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = oq[e] * sq[e];
      const uint16_t *arow = Ac + row * CK + 4 * g4;
      o = mfma(ld_pi(arow), vb[0], o);
      if (p >= 2) o = mfma(ld_pi(arow + 32), vb[1], o);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int orow = 16 * p + 4 * g4 + e;
        if (orow < len) store_elem(a.o, ((t0 + orow) * a.Hv + h) * (int64_t)DV + col, a.o_dt, o[e]);
      }
    }

    // S <- e^{gamma_63} S + K^T diag(e^{gamma_63 - gamma} nk) V'   (V'' hi + lo)
    bf16x8 vh[2], vl[2];
#pragma unroll
    for (int p2 = 0; p2 < 2; ++p2) {
      const f32x4 ska = *reinterpret_cast<const f32x4 *>(sc + CK + 32 * p2 + 4 * g4);
      const f32x4 skb = *reinterpret_cast<const f32x4 *>(sc + CK + 32 * p2 + 16 + 4 * g4);
      f32x4 xa, xb;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xa[e] = vp[2 * p2][e] * ska[e];
        xb[e] = vp[2 * p2 + 1][e] * skb[e];
      }
      pack_hilo(xa, xb, vh[p2], vl[p2]);
    }
    const float eL = sc[2 * CK];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) S[i][e] *= eL;
      const uint16_t *krow = Ktc + (16 * i + r16) * CK + 4 * g4;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const bf16x8 ak = ld_pi(krow + 32 * s);
        S[i] = mfma(ak, vh[s], S[i]);
        S[i] = mfma(ak, vl[s], S[i]);
      }
    }
  }

  const int64_t out_row = a.hT ? (a.hT_idx ? a.hT_idx[n] : n) : -1;
  if (out_row >= 0) {
    float *dst = a.hT + (out_row * a.Hv + h) * (int64_t)(DK * DV) + col;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) dst[(16 * i + 4 * g4 + e) * DV] = S[i][e];
  }
}

struct WsLayout {
  size_t chunk_start, W, Ut, A, Kt, scal, total;
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

WsLayout ws_layout(int n_seqs, int64_t max_chunks, int Hv, int Hk) {
  WsLayout l;
  size_t off = 0;
  l.chunk_start = off;
  off = align256(off + sizeof(int32_t) * (n_seqs + 1));
  l.W = off;
  off = align256(off + sizeof(uint16_t) * max_chunks * Hv * CK * DK);
  l.Ut = off;
  off = align256(off + sizeof(float) * max_chunks * Hv * DV * CK);
  l.A = off;
  off = align256(off + sizeof(uint16_t) * max_chunks * Hv * CK * CK);
  l.Kt = off;
  off = align256(off + sizeof(uint16_t) * max_chunks * Hk * DK * CK);
  l.scal = off;
  off = align256(off + sizeof(float) * max_chunks * Hv * SCAL);
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
  // Upper bound valid with or without cu_seqlens; K tiles counted at Hk = Hv.
  const int64_t nc = (total_tokens + CK - 1) / CK + n_seqs;
  return ws_layout(n_seqs, nc, Hv, Hv).total;
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
  if (!valid_dtype(beta_dtype) || !valid_dtype(o_dtype)) return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_chunk_fwd: bad dtype");
  if (n_seqs == 0) return ok();
  if (!q || !k || !v || !g || !beta || !o) return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_chunk_fwd: null q/k/v/g/beta/o");
  if (q_stride_t < Hk * K || k_stride_t < Hk * K || v_stride_t < Hv * V || (q_stride_t | k_stride_t | v_stride_t) % 8)
    return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_chunk_fwd: token strides must cover a row and be multiples of 8");
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) % 16)
    return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_chunk_fwd: q/k/v must be 16-byte aligned");
  const int64_t total = cu_seqlens ? static_cast<int64_t>(T) : static_cast<int64_t>(n_seqs) * T;
  const int64_t nc = max_chunks_of(n_seqs, total, cu_seqlens != nullptr, T);
  const WsLayout l = ws_layout(n_seqs, nc, Hv, Hk);
  if (!workspace || workspace_bytes < l.total)
    return fail(GDN_ERR_WORKSPACE, "gdn_chunk_fwd: workspace %zu bytes < %zu needed", workspace_bytes, l.total);
  if (nc > 65535) return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_chunk_fwd: %lld chunks exceed one launch", (long long)nc);
  if (static_cast<int64_t>(n_seqs) * Hv * 2 > 0x7fffffff) return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_chunk_fwd: grid");
  char *ws = static_cast<char *>(workspace);
  ChunkArgs a{static_cast<const uint16_t *>(q), static_cast<const uint16_t *>(k), static_cast<const uint16_t *>(v),
              q_stride_t, k_stride_t, v_stride_t, g, beta, beta_dtype, h0, h0_idx, hT, hT_idx, o, o_dtype,
              cu_seqlens, n_seqs, T, Hk, Hv, total, scale, l2norm_qk, static_cast<int>(nc),
              reinterpret_cast<int32_t *>(ws + l.chunk_start), reinterpret_cast<uint16_t *>(ws + l.W),
              reinterpret_cast<float *>(ws + l.Ut), reinterpret_cast<uint16_t *>(ws + l.A),
              reinterpret_cast<uint16_t *>(ws + l.Kt), reinterpret_cast<float *>(ws + l.scal)};
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(chunk_table_kernel, dim3(1), dim3(256), 0, s, a);
  if (nc > 0) hipLaunchKernelGGL(chunk_prep_kernel, dim3(Hv, static_cast<unsigned>(nc)), dim3(256), 0, s, a);
  hipLaunchKernelGGL(chunk_scan_kernel, dim3(static_cast<unsigned>(n_seqs * Hv * 2)), dim3(256), 0, s, a);
  return check_launch("gdn_chunk_fwd");
}
