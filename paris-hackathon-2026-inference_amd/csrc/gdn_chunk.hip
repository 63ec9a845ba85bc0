// Chunk-64 gated delta rule prefill on bf16 MFMA (gfx950).
//
// The reference algorithm (engine/kernels/delta_rule.py:286-349) per chunk
// of 64 tokens and v-head, with gamma = chunk-local cumsum(g):
//   L = strict_lower(diag(beta) K~K~^T * Gamma),  T = (I + L)^-1
//   U = T (beta V),  W = T (beta e^gamma K~)
//   V' = U - W S ;  O = (e^gamma Q~) S + lower(Q~K~^T * Gamma) V'
//   S <- e^{gamma_63} S + (e^{gamma_63 - gamma} K~)^T V'
// runs on one of two paths.  Batches of 160 or more (sequence, v-head) pairs,
// and batches whose longest sequence has one chunk (or two, from 96 pairs),
// take chunk_local_kernel: one 8-wave workgroup per pair walks its
// sequence's chunks, 4 waves preparing chunk k while 4 run chunk k - 1's
// state chain, every operand kept in LDS (no workspace); with cu_seqlens the
// workgroups take the sequences longest first.  Otherwise up to three
// launches:
//   chunk_table_kernel  chunk -> sequence table (only with cu_seqlens)
//   chunk_prep_kernel   one workgroup per (chunk, v-head), all in parallel:
//                       K K^T and K Q^T on MFMA from the raw bf16 rows (exact
//                       products; l2norm and gate factors scale the fp32
//                       results), computed transposed so that L and A come out
//                       in the layout their consumers read; T = (I + L)^-1 by
//                       substitution on the 16x16 diagonal blocks and fp32 MFMA
//                       below them; W = T' K and U = T'' V on MFMA with T', T''
//                       split into bf16 hi + lo parts and K, V read transposed
//                       (ds_read_b64_tr_b16).  -W, U, the A blocks and the
//                       scalars are written pre-swizzled for the scan: one
//                       1 KiB block per (MFMA, wave), lane l's 16 bytes at
//                       offset 16 l (the scan reads q and k rows from the
//                       inputs themselves).
//   chunk_scan_kernel   one workgroup per (sequence, v-head, 16 state
//                       columns), serial over the chunks: four compute waves,
//                       each owning 16 chunk positions and 32 state rows (its
//                       state slice lives in MFMA accumulators for the whole
//                       sequence), exchange V'' and the state through LDS;
//                       two loader waves stream the operand blocks of the
//                       chunk after next into a double-buffered LDS stage
//                       with buffer_load ... lds.
// Inputs longer than one segment (64 chunks) run prep / scan per segment,
// one segment after the other on the caller's stream; several sequences
// (varlen or a batch) are scanned by one workgroup per (v-head, 16 state
// columns) walking all of them (chunk_scan_persist_kernel).
// Precision (checked against an fp64 restatement at T=4096): the state is fed
// to MFMA as bf16, U stays fp32 (it initialises the V' accumulator), the state
// increment K^T V'' uses V'' split into bf16 hi + lo.
//
// MFMA: v_mfma_f32_16x16x32_bf16.  Lane l holds A[l%16][8(l/16)+j] and
// B[8(l/16)+j][l%16] (j<8), and D[4(l/16)+i][l%16] (i<4).  When an
// accumulator tile pair (rows 0-15, 16-31 of a 32-long reduction) is reused
// as the B operand of the next product, lane group g = l/16 holds reduction
// indices {4g..4g+3, 16+4g..16+4g+3} ("pi" order); the scan's A-operand
// blocks are stored in the same order, so an accumulator becomes an operand
// by conversion to bf16 alone (in the scan, between waves, through LDS
// without any reordering).
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

// Operand blocks (64 lanes x 16 bytes) per (chunk, v-head), one contiguous
// region so that a chunk's prep operands are one straight copy:
// -W [p 0..3][s 0..3], A [p 0..3][s 0..1] (6 used), scalars.  (The scan reads
// q and k rows from the inputs themselves.)
constexpr int NB_W = 16;
constexpr int NB_A = 8;
constexpr int NB_SC = SCAL / 64;  // scalars as blocks (1)
constexpr int VH_W = 0, VH_A = VH_W + NB_W, VH_SC = VH_A + NB_A, NB_VH = VH_SC + NB_SC;

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 u) { return __builtin_bit_cast(bf16x8, u); }
__device__ __forceinline__ int64_t uniform64(int64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(x));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(x) >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
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
  GateArgs gate;
  const float *h0;
  const int64_t *h0_idx;
  int64_t h0_rows;
  float *hT;
  const int64_t *hT_idx;
  int64_t hT_rows;
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
  int32_t *chunk_start;  // [n_seqs + 2]: chunk starts, then the empty-sequence count
  u32x4 *vh;             // [SEG][Hv][NB_VH][64]   -W, A, scalars
  float *Ut;             // [SEG][Hv][8 x 4 blocks][64][4]  U, fp32
  float *carry;          // [n_seqs][Hv][128][128] state between segments
  int64_t *seqrec;       // [n_seqs][SEQREC]: per-sequence record for the persistent scan
  // [SEG][Hv / 2]: the chunk's q and k rows of v-head 2i + 1 equal those of 2i
  // (q and k given per v-head, Hk == Hv: the caller repeated them); null
  // unless the prep checks and the scan uses it
  int32_t *dup;
};

// Per-sequence record written by chunk_table_kernel for the persistent scan:
// token start, state rows in / out (-1: none), end chunk, length, and the
// next non-empty sequence (n_seqs: none).
constexpr int SEQREC = 6;
enum { SR_S0 = 0, SR_IN, SR_OUT, SR_CE, SR_LEN, SR_NXT };

__device__ __forceinline__ void seq_bounds(const ChunkArgs &a, int n, int64_t *s0, int *len) {
  seq_range(a.cu, n, a.T, a.total, s0, len);
}
// First global chunk of sequence n (n = n_seqs: the chunk count).  Without
// cu_seqlens every sequence has ceil(T / 64) chunks and no table is built.
__device__ __forceinline__ int chunk_start_at(const ChunkArgs &a, int n) {
  return a.cu ? a.chunk_start[n] : n * ((a.T + CK - 1) / CK);
}

// Workgroup order that keeps the workgroups reading one k-head's q and k
// (its R = Hv / Hk v-heads, GQA; and for the scan their column tiles) on one
// XCD, so that they share its L2: the dispatcher hands workgroup `bid` to XCD
// bid % 8, so bid = x + 8 t with t = per * gq + m serves group g = 8 gq + x,
// member m < per.  Needs the group count to be a multiple of 8 (else the
// caller keeps its plain order).
__device__ __forceinline__ void xcd_group_order(int bid, int per, int *g, int *m) {
  const int x = bid & 7, t = bid >> 3;
  *g = 8 * (t / per) + x;
  *m = t % per;
}

// ------------------------------------------------------------------ chunk table
// chunk_start[0 .. n_seqs]: first global chunk of each sequence (and the
// total); chunk_start[n_seqs + 1]: the number of empty sequences.
__global__ __launch_bounds__(256) void chunk_table_kernel(ChunkArgs a) {
  __shared__ int32_t part[256];
  __shared__ int32_t empties;
  int32_t carry = 0;
  if (threadIdx.x == 0) {
    a.chunk_start[0] = 0;
    empties = 0;
  }
  __syncthreads();
  for (int base = 0; base < a.n_seqs; base += 256) {
    const int n = base + threadIdx.x;
    int64_t s0;
    int len = 0;
    if (n < a.n_seqs) {
      seq_bounds(a, n, &s0, &len);
      if (len == 0) atomicAdd(&empties, 1);
    }
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
  if (threadIdx.x == 0) a.chunk_start[a.n_seqs + 1] = empties;
  __syncthreads();  // chunk_start complete (workgroup-visible)
  for (int n = threadIdx.x; n < a.n_seqs; n += 256) {
    int64_t s0;
    int len;
    seq_bounds(a, n, &s0, &len);
    int k = n + 1;
    while (k < a.n_seqs && a.chunk_start[k] == a.chunk_start[k + 1]) ++k;  // skip empty sequences
    int64_t *r = a.seqrec + static_cast<int64_t>(n) * SEQREC;
    r[SR_S0] = s0;
    const int64_t rin = a.h0 ? pool_row(a.h0_idx, n, a.h0_rows) : -1;
    const int64_t rout = a.hT ? pool_row(a.hT_idx, n, a.hT_rows) : -1;
    r[SR_IN] = rin >= 0 && repeats_earlier_thread(a.h0_idx, n) ? -1 : rin;  // repeated slot ids: no row
    r[SR_OUT] = rout >= 0 && repeats_earlier_thread(a.hT_idx, n) ? -1 : rout;
    r[SR_CE] = a.chunk_start[n + 1];
    r[SR_LEN] = len;
    r[SR_NXT] = k;
  }
}

// ------------------------------------------------------------------ phase A
// One workgroup of 4 waves per (chunk, v-head); wave p owns chunk rows
// 16p..16p+15.  Fragment layouts used below (lane = 16 g + r, r < 16):
//   pi fragment of X (bf16 MFMA operand, k-step s):  lane holds row r of the
//     tile, columns 32s + 4g + 0..3 and 32s + 16 + 4g + 0..3;
//   row layout (16x16 fp32 block):  lane holds X[r][4g + e], e < 4;
//   D layout (16x16 fp32 block):    lane holds X[4g + e][r] (an MFMA result).

// Row-major [64][128] bf16 tile (K or V): 16-byte segment seg of row r is
// stored at segment seg ^ (r & 15).  Row writes, pi-fragment reads and the
// transposing reads below are all free of bank conflicts with it.
__device__ __forceinline__ int nsw(int row, int col) {
  return row * DK + ((((col >> 3) ^ row) & 15) << 3) + (col & 7);
}

typedef __attribute__((ext_vector_type(4))) short s16x4;
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives 16-bit
// element (i % 4) of the 8 bytes addressed by source lanes 4k + i / 4 of the
// group, k = 0..3.  With source lane L pointing at X[j0 + L/4][n0 + 4 (L%4)],
// lane i therefore holds X[j0 + k][n0 + i]: four consecutive rows of column
// n0 + i, which is the MFMA operand layout of X^T.
__device__ __forceinline__ s16x4 ld_tr(const uint16_t *tile, int j0, int n0, int lane) {
  const int L = lane & 15;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_s16x4 *)(const_cast<uint16_t *>(tile) + nsw(j0 + (L >> 2), n0 + 4 * (L & 3))));
}
// Pi fragment of X^T for k-step s over the rows of X and columns n0..n0+15.
__device__ __forceinline__ bf16x8 frag_tr(const uint16_t *tile, int s, int n0, int lane) {
  const int g4 = lane >> 4;
  const s16x4 lo = ld_tr(tile, 32 * s + 4 * g4, n0, lane);
  const s16x4 hi = ld_tr(tile, 32 * s + 16 + 4 * g4, n0, lane);
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}
// Pi fragment of rows row0..row0+15 of X, k-step s.
__device__ __forceinline__ bf16x8 frag_pi(const uint16_t *tile, int row0, int s, int lane) {
  const int r = row0 + (lane & 15), g4 = lane >> 4;
  const u32x2 a = *reinterpret_cast<const u32x2 *>(tile + nsw(r, 32 * s + 4 * g4));
  const u32x2 b = *reinterpret_cast<const u32x2 *>(tile + nsw(r, 32 * s + 16 + 4 * g4));
  return as_bf16x8(u32x4{a.x, a.y, b.x, b.y});
}

// 16x16x16 fp32 product on MFMA (v_mfma_f32_16x16x4_f32: lane (r, g) gives
// A[r][g] and B[g][r]).  With X in row layout and Y in D layout, call kc
// reduces over the indices 4g + kc, so mm16(X, Y) is X Y in D layout, and
// mm16(Y, X) (arguments swapped) is the same product in row layout.
__device__ __forceinline__ f32x4 mm16(f32x4 a, f32x4 b, f32x4 acc) {
#pragma unroll
  for (int kc = 0; kc < 4; ++kc) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[kc], b[kc], acc, 0, 0, 0);
  return acc;
}

__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

// T[p][p] = (I + L[p][p])^-1 in D layout: each lane solves for column r16 by
// forward substitution, x[i] = [i == r16] - sum_{j < i} L[i][j] x[j], with
// L[p][p]'s entries (row layout: row i, columns 4q .. 4q + 3 in lane
// i + 16 q) broadcast from the lanes that hold them by v_readlane, so the
// 16 dependent rows wait on no memory.
__device__ __forceinline__ f32x4 diag_inverse(const f32x4 lf[4], int p, int lane) {
  const int r16 = lane & 15, g4 = lane >> 4, pu = __builtin_amdgcn_readfirstlane(p);
  // (the entries are read as ints of the whole vector's bit cast: a bit cast
  // of one vector element was lowered as a read of element 0, and the builtin
  // takes ints, so a float argument would be converted by value)
  const u32x4 lpp = __builtin_bit_cast(u32x4, pu == 0 ? lf[0] : pu == 1 ? lf[1] : pu == 2 ? lf[2] : lf[3]);
  float x[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    float acc = i == r16 ? 1.f : 0.f;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (4 * q4 + e < i) {
          const float lij = __builtin_bit_cast(float, __builtin_amdgcn_readlane(static_cast<int>(lpp[e]), i + 16 * q4));
          acc = __builtin_fmaf(-lij, x[4 * q4 + e], acc);
        }
    x[i] = acc;
  }
  f32x4 d;
#pragma unroll
  for (int e = 0; e < 4; ++e) {  // x[4 g4 + e]
    // (the candidates are pinned in registers first: LLVM turns a select
    // between elements of x into an indexed load, which puts x in scratch)
    float c0 = x[e], c1 = x[4 + e], c2 = x[8 + e], c3 = x[12 + e];
    asm volatile("" : "+v"(c0), "+v"(c1), "+v"(c2), "+v"(c3));
    d[e] = g4 == 0 ? c0 : g4 == 1 ? c1 : g4 == 2 ? c2 : c3;
  }
  return d;
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void chunk_prep_kernel(ChunkArgs a) {
  __shared__ __align__(16) uint16_t kn[CK * DK];  // K rows (swizzled)
  // V rows (swizzled) share 16 KiB with the solve's exchange buffers: V is
  // first read by the W/U products, after the solve's last exchange, and
  // waits in registers until then.  (4 workgroups fit a CU's LDS instead of 3.)
  __shared__ __align__(16) f32x4 shared16k[1024];
  uint16_t *vn = reinterpret_cast<uint16_t *>(shared16k);
  f32x4 *lbuf = shared16k;                // [4 * 64] diagonal blocks of L, row layout by lane
  f32x4 *dxch = shared16k + 4 * 64;       // [4 * 64] diagonal blocks of T, D layout by lane
  f32x4 *txch = shared16k + 8 * 64;       // [3 * 64] T[1][0], T[2][1], T[2][0], D layout by lane
  float(*dtr)[16 * 20] = reinterpret_cast<float(*)[16 * 20]>(shared16k + 11 * 64);  // D -> row layout
  static_assert(CK * DV * 2 == sizeof(f32x4) * 1024 && (11 * 64) * 16 + 4 * 16 * 20 * 4 == 16384, "layout");
  __shared__ __align__(16) float gam_s[CK], beta_s[CK], nk_s[CK], nq_s[CK], colw_s[CK];

  const int ratio = a.Hv / a.Hk;
  // the v-heads that read the same q / k rows (those of one k-head; a checked
  // pair with repeated q / k) on one XCD: grp heads per group, hg groups
  const int grp = a.dup ? 2 : ratio, hg = a.Hv / grp;
  int h = blockIdx.x, jl = blockIdx.y;  // v-head; chunk index within the segment's workspace
  if ((hg * static_cast<int>(gridDim.y)) % 8 == 0) {
    int g, m;
    xcd_group_order(blockIdx.x + gridDim.x * blockIdx.y, grp, &g, &m);
    h = (g % hg) * grp + m;
    jl = g / hg;
  }
  const int j = a.seg_begin + jl;  // global chunk index
  if (j >= a.seg_end || j >= chunk_start_at(a, a.n_seqs)) return;
  int lo = 0, hi = a.n_seqs;  // sequence owning chunk j: last n with chunk_start[n] <= j
  if (!a.cu) {
    lo = j / ((a.T + CK - 1) / CK);
  } else {
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (a.chunk_start[mid] <= j) lo = mid; else hi = mid;
    }
  }
  const int n = lo;
  int64_t s0;
  int slen;
  seq_bounds(a, n, &s0, &slen);
  const int c = j - chunk_start_at(a, n);
  const int64_t t0 = s0 + static_cast<int64_t>(c) * CK;
  const int len = min(CK, slen - c * CK);
  if (len <= 0) {
    if (a.dup && (h & 1) && threadIdx.x == 0) a.dup[jl * (a.Hv / 2) + h / 2] = 1;  // (no rows: nothing differs)
    return;
  }
  const int hk = h / ratio;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int p = tid >> 6;  // this wave's row block
  const int g4 = lane >> 4;
  const int r16 = lane & 15;
  const size_t ch = static_cast<size_t>(jl) * a.Hv + h;
  const int irow = 16 * p + r16;  // this lane's chunk row in row-layout / pi fragments

  // ---- global loads: K, V rows (16 bytes per thread), this wave's Q rows as
  // pi fragments, and the gates
  const int seg = tid & 15;
  u32x4 ku[4], vu[4];
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int row = (tid >> 4) + 16 * it;
    const int64_t tok = t0 + row;
    const u32x4 z = {0u, 0u, 0u, 0u};
    ku[it] = row < len ? *reinterpret_cast<const u32x4 *>(a.k + tok * a.ks + (int64_t)hk * DK + seg * 8) : z;
    vu[it] = row < len ? *reinterpret_cast<const u32x4 *>(a.v + tok * a.vs + (int64_t)h * DV + seg * 8) : z;
  }
  bf16x8 qf[4];
  {
    const uint16_t *qrow = a.q + (t0 + irow) * a.qs + (int64_t)hk * DK + 4 * g4;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x2 x0 = {0u, 0u}, x1 = {0u, 0u};
      if (irow < len) {
        x0 = *reinterpret_cast<const u32x2 *>(qrow + 32 * s);
        x1 = *reinterpret_cast<const u32x2 *>(qrow + 32 * s + 16);
      }
      qf[s] = as_bf16x8(u32x4{x0.x, x0.y, x1.x, x1.y});
    }
  }
  // an odd v-head with per-v-head q / k (dup): its rows against the even
  // partner's, the same loads from head hk - 1 (on this XCD's L2), requested
  // with its own rows and the gates and compared once all of them are in
  const bool chk = a.dup && (h & 1);
  u32x4 kpart[4], qpart[4];
  if (chk) {  // rows clamped to the chunk's last one (len >= 1), those past it not compared
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int row = min((tid >> 4) + 16 * it, len - 1);
      kpart[it] = *reinterpret_cast<const u32x4 *>(a.k + (t0 + row) * a.ks + (int64_t)(hk - 1) * DK + seg * 8);
    }
    const uint16_t *qrow = a.q + (t0 + min(irow, len - 1)) * a.qs + (int64_t)(hk - 1) * DK + 4 * g4;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const u32x2 x0 = *reinterpret_cast<const u32x2 *>(qrow + 32 * s);
      const u32x2 x1 = *reinterpret_cast<const u32x2 *>(qrow + 32 * s + 16);
      qpart[s] = u32x4{x0.x, x0.y, x1.x, x1.y};
    }
  }
  GateRaw graw{0u, 0u, 0.f, 0.f};
  if (p == 0 && lane < len) {
    const int64_t gi = (t0 + lane) * a.gate.stride + h;
    graw.ga = load_bits(a.gate.g_or_a, gi, a.gate.A_log ? a.gate.dt : GDN_DTYPE_F32);
    graw.gb = load_bits(a.gate.beta_or_b, gi, a.gate.dt);
  }
  if (a.gate.A_log) {
    graw.a_log = a.gate.A_log[h];
    graw.dt_bias = a.gate.dt_bias[h];
  }
  bool same = true;
  if (chk) {
    uint32_t diff = 0u;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      uint32_t d = 0u;
#pragma unroll
      for (int e = 0; e < 4; ++e) d |= kpart[it][e] ^ ku[it][e];
      diff |= (tid >> 4) + 16 * it < len ? d : 0u;
    }
    uint32_t dq = 0u;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const u32x4 own = __builtin_bit_cast(u32x4, qf[s]);
#pragma unroll
      for (int e = 0; e < 4; ++e) dq |= qpart[s][e] ^ own[e];
    }
    diff |= irow < len ? dq : 0u;
    same = diff == 0u;
  }
  float gv = 0.f, bv = 0.f;
  if (p == 0 && lane < len) gates_from_raw(a.gate, graw, &gv, &bv);

  // ---- A.1: K, V rows into LDS; K row norms; chunk-local cumsum of g; Q row norms
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int row = (tid >> 4) + 16 * it;
    *reinterpret_cast<u32x4 *>(kn + nsw(row, seg * 8)) = ku[it];
    float sk = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t kw = ku[it][e];
      const float k0 = bf16_bits_to_f32(kw & 0xffffu), k1 = bf16_bits_to_f32(kw >> 16);
      sk += k0 * k0 + k1 * k1;
    }
    sk = row16_sum(sk);
    if (seg == 0) nk_s[row] = a.l2norm ? rsqrtf(sk + 1e-6f) : 1.f;
  }
  {
    float sq = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = static_cast<float>(qf[s][e]);
        sq += x * x;
      }
    sq += __shfl_xor(sq, 16, 64);
    sq += __shfl_xor(sq, 32, 64);
    if (g4 == 0) nq_s[irow] = (a.l2norm ? rsqrtf(sq + 1e-6f) : 1.f) * a.scale;
  }
  if (p == 0) {
    gv = wave_incl_scan(gv);  // chunk-local cumsum of g
    gam_s[lane] = gv;
    beta_s[lane] = bv;
  }
  if (a.dup) {
    const int all_same = __syncthreads_and(same);
    if ((h & 1) && tid == 0) a.dup[jl * (a.Hv / 2) + h / 2] = all_same;
  } else {
    __syncthreads();
  }

  // Per-position scalars: the scan's output / state-increment scales, and W's column scale.
  if (p == 0) {
    float *sc = reinterpret_cast<float *>(a.vh + ch * (NB_VH * 64) + VH_SC * 64);
    const float gl = gam_s[CK - 1], gm = gam_s[lane];
    sc[lane] = fast_exp(gm) * nq_s[lane];
    sc[CK + lane] = fast_exp(gl - gm) * nk_s[lane];
    if (lane == 0) sc[2 * CK] = fast_exp(gl);
    colw_s[lane] = beta_s[lane] * fast_exp(gm) * nk_s[lane];
  }

  // ---- A.2: tiles (cb, p), cb <= p, of K K^T and K Q^T.  The MFMA result
  // lane holds (K_cb K_p^T)[4g + e][r] = k_j . k_i with i = 16p + r (this
  // lane's row) and j = 16cb + 4g + e: L and A come out in row layout.
  const float gi = gam_s[irow], bi = beta_s[irow], nki = nk_s[irow], nqi = nq_s[irow];
  // (register arrays are only indexed by unrolled loop counters; the wave's
  // own block is selected with uniform branches)
  bf16x8 kown[4];  // pi fragments of this wave's K rows
#pragma unroll
  for (int s = 0; s < 4; ++s) kown[s] = frag_pi(kn, 16 * p, s, lane);
  f32x4 lf[4], af[4];  // L and A blocks (p, cb), row layout
#pragma unroll
  for (int cb = 0; cb < 4; ++cb) {
    lf[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
    af[cb] = lf[cb];
    if (cb <= p) {
      f32x4 kk = {0.f, 0.f, 0.f, 0.f}, qk = kk;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 kcb = frag_pi(kn, 16 * cb, s, lane);
        kk = mfma(kcb, kown[s], kk);
        qk = mfma(kcb, qf[s], qk);
      }
      const f32x4 gj = *reinterpret_cast<const f32x4 *>(gam_s + 16 * cb + 4 * g4);
      const f32x4 nj = *reinterpret_cast<const f32x4 *>(nk_s + 16 * cb + 4 * g4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int jj = 16 * cb + 4 * g4 + e;
        const float dec = jj <= irow ? fast_exp(gi - gj[e]) : 0.f;
        af[cb][e] = nqi * nj[e] * qk[e] * dec;
        lf[cb][e] = jj < irow ? bi * nki * nj[e] * kk[e] * dec : 0.f;
      }
    }
  }
  {  // the scan's A operand blocks (p, s) = A tiles 2s, 2s + 1 (zero past the diagonal)
    u32x4 *aop = a.vh + ch * (NB_VH * 64) + VH_A * 64;
    aop[(2 * p) * 64 + lane] = __builtin_bit_cast(u32x4, pack_hi(af[0], af[1]));
    if (p >= 2) aop[(2 * p + 1) * 64 + lane] = __builtin_bit_cast(u32x4, pack_hi(af[2], af[3]));
  }

  // ---- A.3: T = (I + L)^-1.  Diagonal blocks by substitution (each lane one
  // column, rows of L broadcast from LDS), then the blocks below the diagonal
  // on fp32 MFMA: T[p][b] = -T[p][p] sum_{b <= kb < p} L[p][kb] T[kb][b].
  f32x4 dl, drow;  // T[p][p] in D layout and row layout
  {
    f32x4 *lb = lbuf + p * 64;
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
      if (cb == p) lb[lane] = lf[cb];
    __builtin_amdgcn_wave_barrier();
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float acc = i == r16 ? 1.f : 0.f;
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
        if (4 * q4 < i) {
          const f32x4 lrow = lb[i + 16 * q4];  // L[i][4 q4 .. 4 q4 + 3]
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (4 * q4 + e < i) acc -= lrow[e] * x[4 * q4 + e];
        }
      x[i] = acc;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
      dl[e] = g4 == 0 ? x[e] : g4 == 1 ? x[4 + e] : g4 == 2 ? x[8 + e] : x[12 + e];
    dxch[p * 64 + lane] = dl;
    float *tr = dtr[p];
#pragma unroll
    for (int e = 0; e < 4; ++e) tr[(4 * g4 + e) * 20 + r16] = dl[e];
    __builtin_amdgcn_wave_barrier();
    drow = *reinterpret_cast<const f32x4 *>(tr + r16 * 20 + 4 * g4);
  }
  __syncthreads();
  f32x4 trow[4];  // T[p][b], row layout
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int b = 0; b < 4; ++b) trow[b] = b == p ? drow : z4;
  // step 1: T[p][p-1] = -T[p][p] L[p][p-1] T[p-1][p-1]
#pragma unroll
  for (int b = 0; b < 3; ++b)
    if (b == p - 1) {
      const f32x4 x = mm16(lf[b], dxch[b * 64 + lane], z4);
      trow[b] = -mm16(x, drow, z4);
      if (b <= 1) txch[b * 64 + lane] = -mm16(drow, x, z4);  // T[1][0], T[2][1]
    }
  __syncthreads();
  // step 2: T[p][p-2] = -T[p][p] (L[p][p-2] T[p-2][p-2] + L[p][p-1] T[p-1][p-2])
#pragma unroll
  for (int b = 0; b < 2; ++b)
    if (b == p - 2) {
      f32x4 x = mm16(lf[b], dxch[b * 64 + lane], z4);
      x = mm16(lf[b + 1], txch[b * 64 + lane], x);  // T[b+1][b]: T[1][0] or T[2][1]
      trow[b] = -mm16(x, drow, z4);
      if (b == 0) txch[2 * 64 + lane] = -mm16(drow, x, z4);  // T[2][0]
    }
  __syncthreads();
  if (p == 3) {  // step 3: T[3][0]
    f32x4 x = mm16(lf[0], dxch[lane], z4);
    x = mm16(lf[1], txch[lane], x);           // T[1][0]
    x = mm16(lf[2], txch[2 * 64 + lane], x);  // T[2][0]
    trow[0] = -mm16(x, drow, z4);
  }
  __syncthreads();  // the exchange buffers are free: V rows take their place
#pragma unroll
  for (int it = 0; it < 4; ++it)
    *reinterpret_cast<u32x4 *>(vn + nsw((tid >> 4) + 16 * it, seg * 8)) = vu[it];
  __syncthreads();

  // ---- A.4: W^T = K^T (T diag(colw))^T and U = T diag(beta) V on bf16 MFMA,
  // with the T factors split into bf16 hi + lo.  Reduction over chunk
  // positions in pi order: k-step s covers T blocks 2s and 2s + 1.
  f32x4 wt[8], ut[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) {
    wt[nb] = z4;
    ut[nb] = z4;
  }
  const int nsteps = p >= 2 ? 2 : 1;  // T is lower triangular
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    if (s < nsteps) {
      const f32x4 cw0 = *reinterpret_cast<const f32x4 *>(colw_s + 32 * s + 4 * g4);
      const f32x4 cw1 = *reinterpret_cast<const f32x4 *>(colw_s + 32 * s + 16 + 4 * g4);
      const f32x4 be0 = *reinterpret_cast<const f32x4 *>(beta_s + 32 * s + 4 * g4);
      const f32x4 be1 = *reinterpret_cast<const f32x4 *>(beta_s + 32 * s + 16 + 4 * g4);
      bf16x8 whi, wlo, uhi, ulo;
      pack_hilo(trow[2 * s] * cw0, trow[2 * s + 1] * cw1, whi, wlo);
      pack_hilo(trow[2 * s] * be0, trow[2 * s + 1] * be1, uhi, ulo);
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) {
        const bf16x8 kt = frag_tr(kn, s, 16 * nb, lane);
        const bf16x8 vf = frag_tr(vn, s, 16 * nb, lane);
        wt[nb] = mfma(kt, whi, wt[nb]);
        wt[nb] = mfma(kt, wlo, wt[nb]);
        ut[nb] = mfma(uhi, vf, ut[nb]);
        ut[nb] = mfma(ulo, vf, ut[nb]);
      }
    }
  }

  // ---- A.5: outputs.  -W blocks (p, s) = W^T tiles 2s, 2s + 1; U blocks in
  // the scan's lane order (column tile nb, row tile p).
  u32x4 *wop = a.vh + ch * (NB_VH * 64) + VH_W * 64;
#pragma unroll
  for (int s = 0; s < 4; ++s) wop[(4 * p + s) * 64 + lane] = __builtin_bit_cast(u32x4, pack_hi(-wt[2 * s], -wt[2 * s + 1]));
  float *Uout = a.Ut + ch * (DV * CK);
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) *reinterpret_cast<f32x4 *>(Uout + ((4 * nb + p) * 64 + lane) * 4) = ut[nb];
}

// ------------------------------------------------------------------ phase B

// sched_group_barrier masks
constexpr int SG_MFMA = 0x8, SG_DS_RD = 0x100;
#define GDN_SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)
#define GDN_GROUP(mask, n) __builtin_amdgcn_sched_group_barrier(mask, n, 0)

// ------------------------------------------------------------ row-split scan
// Workgroup = 6 waves for one (sequence, v-head, 16 state columns):
//
// * compute waves q = 0..3.  Wave q owns chunk positions 16q..16q+15 (its
//   rows of V' and O) and state rows 32q..32q+31 (state tiles 2q, 2q+1:
//   k-step q of every product with S).  No operand one compute wave reads is
//   read by another, and LDS carries the two exchanges of each chunk:
//     xv  after V' = U - W S:   V' (bf16) and V'' = diag(sk) V' (bf16 hi + lo)
//     xs  after S += K^T V'':   the updated state rows (bf16)
//   each followed by a barrier.  A compute wave runs 17-18 MFMAs per chunk.
// * loader waves 4, 5 stream each chunk's operands (61 KiB: the v-head
//   region, the k-head region and this column tile's U blocks) from global
//   memory into a double-buffered LDS stage with buffer_load ... lds, two
//   chunks ahead, so that the CU's vector-memory path (about 55 B/clk with
//   two waves issuing) runs the whole time instead of in bursts between the
//   barriers; the compute waves read their operands from the stage one chunk
//   ahead (LDS reads, about 39 B/clk per wave).
//
// Stage buffer c % 2 holds chunk c.  Loaders: during chunk c they copy
// chunk c + 2 into buffer c % 2 (half before barrier 1, half before barrier
// 2) and, before barrier 1, wait for chunk c + 1's copies.  Compute waves:
// between barriers 1 and 2 of chunk c they read chunk c + 1's operands from
// buffer (c + 1) % 2.  So a buffer is rewritten only after the barrier that
// follows its last read, and read only after the barrier that follows the
// wait for its copies.  The barriers fence LDS only (the loaders wait for
// their copies with an explicit vmcnt).
// stage blocks per chunk: the v-head region, K and Q rows (raw, 4 rows per
// block, swizzled as nsw), U
constexpr int RS_VH = 0, RS_K = NB_VH, RS_Q = RS_K + 16, RS_U = RS_Q + 16, RS_BLOCKS = RS_U + 4;  // 61 blocks
// Loader 0 copies the v-head region but for the two A blocks the compute
// waves never read ((p, s) = (0, 1), (1, 1): zero, and left unwritten by the
// prep), then the U blocks; loader 1 the K and Q rows.
constexpr int RS_VH_COPIES = NB_VH - 2;
constexpr int RS_LOADER0 = RS_VH_COPIES + 4;
constexpr int RS_LOADER1 = 32;
constexpr int SCAN_WAVES = 6;
constexpr int SCAN_COLS = 16;  // state columns per workgroup
constexpr int SCAN_PERSIST_BLOCKS = 256;  // one scan workgroup per CU (MI355X: 256 CUs)

struct RowOps {     // one chunk's operands of one compute wave
  u32x4 w[4];       // -W rows 16q.., k-steps 0..3
  u32x4 qm[4];      // Q rows 16q.., k-steps 0..3
  u32x4 kt[4];      // K^T tiles 2q + t, k-steps s: [2t + s]
  u32x4 am[2];      // A rows 16q.., k-steps 0, 1 (the second only for q >= 2)
  f32x4 u, sk;      // U rows 16q + 4g + e of this lane's column; their V'' scales
  float sq, eL;     // output scale of position 16q + (lane % 16); e^{gamma_63}
};
// Token ranges of global chunks visited in increasing order (a scan
// loader's walk): one search for the first chunk's sequence, then the next
// sequence is entered when a chunk crosses the current one's end, with that
// sequence's table entries read one crossing earlier.  Uniform; the chunk
// table and cu_seqlens are read as scalar loads.
struct ChunkWalk {
  int n, cs, next_cs, slen;
  int64_t s0;
  int p_cs, p_slen;  // the next sequence's end chunk and length, read one crossing ahead
  int64_t p_s0;
  __device__ void prefetch(const ChunkArgs &a) {
    const int m = min(n + 1, a.n_seqs - 1);
    p_cs = chunk_start_at(a, m + 1);
    seq_bounds(a, m, &p_s0, &p_slen);
  }
  __device__ void start(const ChunkArgs &a, int j) {
    int lo = 0, hi = a.n_seqs;  // last n with chunk_start[n] <= j
    if (!a.cu) {
      lo = j / ((a.T + CK - 1) / CK);
    } else {
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (a.chunk_start[mid] <= j) lo = mid; else hi = mid;
      }
    }
    n = lo;
    cs = chunk_start_at(a, lo);
    next_cs = chunk_start_at(a, lo + 1);
    seq_bounds(a, lo, &s0, &slen);
    prefetch(a);
  }
  // chunk j's first token and length (j at or after the previous call's)
  __device__ void at(const ChunkArgs &a, int j, int64_t *t0, int *len) {
    while (j >= next_cs && n + 1 < a.n_seqs) {  // (empty sequences have no chunks: cs == next_cs)
      ++n;
      cs = next_cs;
      next_cs = p_cs;
      s0 = p_s0;
      slen = p_slen;
      prefetch(a);
    }
    const int c = j - cs;
    *t0 = s0 + static_cast<int64_t>(c) * CK;
    *len = min(CK, slen - c * CK);
  }
};
struct RowSrc {     // one chunk's sources: its workspace regions (v-head operands, U) and raw k, q rows
  __amdgpu_buffer_rsrc_t vh, ut, k, q;
};
// ch: the (chunk, v-head) index within the workspace; the chunk's tokens
// [t0, t0 + len).  Rows past the chunk's end read as zero (their offsets are
// range checked).
__device__ __forceinline__ RowSrc row_src(const ChunkArgs &a, size_t ch, int64_t t0, int len, int hk) {
  const int64_t kb = (len - 1) * a.ks * 2 + DK * 2, qb = (len - 1) * a.qs * 2 + DK * 2;
  return RowSrc{__builtin_amdgcn_make_buffer_rsrc(a.vh + ch * (NB_VH * 64), 0, NB_VH * 1024, BUF_DWORD3),
                __builtin_amdgcn_make_buffer_rsrc(a.Ut + ch * (DV * CK), 0, DV * CK * 4, BUF_DWORD3),
                __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(a.k) + t0 * a.ks + (int64_t)hk * DK, 0,
                                                  static_cast<int>(kb < 0 ? 0 : kb), BUF_DWORD3),
                __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(a.q) + t0 * a.qs + (int64_t)hk * DK, 0,
                                                  static_cast<int>(qb < 0 ? 0 : qb), BUF_DWORD3)};
}

// Loader ld's copies [i0, i1) of one chunk into stage st (1 KiB each, lane l's
// 16 bytes at 16 l; a raw row block i holds rows 4i .. 4i + 3, LDS segment ps
// of a row holding its logical segment ps ^ (row & 15), the nsw layout).
template <int LD>
__device__ __forceinline__ void stage_copy(u32x4 *st, const RowSrc &r, const ChunkArgs &a, int ct, int i0, int i1,
                                           int lane) {
  const int rl = lane >> 4, ps = lane & 15;
  for (int i = i0; i < i1; ++i) {
    if constexpr (LD == 0) {
      if (i < RS_VH_COPIES) {
        const int blk = i + (i > VH_A) + (i > VH_A + 1);  // (skips blocks VH_A + 1, VH_A + 3)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r.vh, st + (RS_VH + blk) * 64, 16, lane * 16, blk * 1024, 0, 0);
      } else {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r.ut, st + (RS_U + i - RS_VH_COPIES) * 64, 16, lane * 16,
                                                 (4 * ct + i - RS_VH_COPIES) * 1024, 0, 0);
      }
    } else {
      const int b = i & 15, row = 4 * b + rl;
      const int seg = 16 * (ps ^ (row & 15));  // (the whole offset is in the range-checked vector offset)
      if (i < 16)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r.k, st + (RS_K + b) * 64, 16, row * static_cast<int>(a.ks * 2) + seg,
                                                 0, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r.q, st + (RS_Q + b) * 64, 16, row * static_cast<int>(a.qs * 2) + seg,
                                                 0, 0, 0);
    }
  }
}

// A compute wave's operands of one chunk from its stage buffer, in groups
// read at different points of the previous chunk.
template <int G>
__device__ __forceinline__ void read_rows(RowOps &op, const u32x4 *st, int q, int lane) {
  const float *sc = reinterpret_cast<const float *>(st + (RS_VH + VH_SC) * 64);
  if constexpr (G == 0) {  // V' = U - W S and its scales
#pragma unroll
    for (int s = 0; s < 4; ++s) op.w[s] = st[(RS_VH + VH_W + 4 * q + s) * 64 + lane];
    op.u = __builtin_bit_cast(f32x4, st[(RS_U + q) * 64 + lane]);
    op.sk = *reinterpret_cast<const f32x4 *>(sc + CK + 16 * q + 4 * (lane >> 4));
    op.eL = sc[2 * CK];
  } else if constexpr (G == 1) {  // Q S: pi fragments of q rows 16q..
    const uint16_t *qn = reinterpret_cast<const uint16_t *>(st + RS_Q * 64);
#pragma unroll
    for (int s = 0; s < 4; ++s) op.qm[s] = __builtin_bit_cast(u32x4, frag_pi(qn, 16 * q, s, lane));
  } else if constexpr (G == 2) {  // S += K^T V'': K^T tiles 2q + t, read transposed from the k rows
    const uint16_t *kn = reinterpret_cast<const uint16_t *>(st + RS_K * 64);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int s = 0; s < 2; ++s) op.kt[2 * t + s] = __builtin_bit_cast(u32x4, frag_tr(kn, s, 32 * q + 16 * t, lane));
  } else {  // the output
    op.am[0] = st[(RS_VH + VH_A + 2 * q) * 64 + lane];
    op.am[1] = st[(RS_VH + VH_A + 2 * q + 1) * 64 + lane];  // (unused for q < 2)
    op.sq = sc[16 * q + (lane & 15)];
  }
}

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
__device__ __forceinline__ u32x2 pack4(f32x4 x) {
  bf16x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = static_cast<__bf16>(x[i]);
  return __builtin_bit_cast(u32x2, r);
}

// One chunk of compute wave q (TWO_A: q >= 2, whose output rows see V' rows
// of both k-steps).  sb: the whole state as bf16 B operands by k-step; S:
// this wave's state rows (fp32).  On return sb and S hold the updated state
// and store_out(o) has been called with the chunk's output rows.  nst: the
// stage buffer of the next chunk, whose operands are read into nx here.
//
// The chain that carries the state from chunk to chunk -- V' = U - W S, V''
// to LDS, barrier, S += K^T V'', S to LDS, barrier, S back from LDS -- runs
// first in each of three regions; the products off that chain (Q S and the
// output) and the operand reads fill its waits:
//   R1  V' (4 MFMAs), V'' to LDS
//   R2  (after barrier 1, V'' reads in flight) Q S (4 MFMAs), then
//       S += K^T V'' (8 MFMAs) | next chunk's operands from the stage
//   R3  (after barrier 2, state reads in flight) O (1-2 MFMAs), its store
// xv[kind][k-step][lane] holds, per lane, 4 bf16 of wave 2 k-step and then 4
// of wave 2 k-step + 1: a B operand in pi order.
//
// O is computed transposed, O^T = (S^T Q^T) diag(sq) + V'^T A^T: the
// registers of an A operand are those of the transposed B operand, so sb,
// the V' exchange and the Q and A blocks serve unchanged, and lane (g, r)
// ends with O[16q + r][4g .. 4g + 3], one 8-byte store.
template <bool TWO_A, class StoreOut, class AtState>
__device__ __forceinline__ void scan_rows_chunk(const RowOps &op, RowOps &nx, const u32x4 *nst, bf16x8 (&sb)[4],
                                                f32x4 (&S)[2], u32x2 (*xv)[2][64][2], u32x4 (*xs)[64], int q,
                                                int lane, const StoreOut &store_out, const AtState &at_state) {
  // ---- R1
  f32x4 vp = op.u;
#pragma unroll
  for (int s = 0; s < 4; ++s) vp = mfma(as_bf16x8(op.w[s]), sb[s], vp);
#pragma unroll
  for (int t = 0; t < 2; ++t) S[t] = S[t] * op.eL;
  {
    const f32x4 v2 = vp * op.sk;
    f32x4 hf;
    bf16x4 h, l;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      h[i] = static_cast<__bf16>(v2[i]);
      hf[i] = static_cast<float>(h[i]);
      l[i] = static_cast<__bf16>(v2[i] - hf[i]);
    }
    xv[0][q >> 1][lane][q & 1] = pack4(vp);
    xv[1][q >> 1][lane][q & 1] = __builtin_bit_cast(u32x2, h);
    xv[2][q >> 1][lane][q & 1] = __builtin_bit_cast(u32x2, l);
  }
  lds_barrier();

  // ---- R2
  bf16x8 vh[2], vl[2], vb[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    vh[s] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(&xv[1][s][lane][0]));
    vl[s] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(&xv[2][s][lane][0]));
  }
  vb[0] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(&xv[0][0][lane][0]));
  if constexpr (TWO_A) vb[1] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(&xv[0][1][lane][0]));
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = mfma(sb[s], as_bf16x8(op.qm[s]), acc);
  read_rows<0>(nx, nst, q, lane);
  GDN_SCHED_FENCE();
#pragma unroll
  for (int s = 0; s < 2; ++s) {
#pragma unroll
    for (int t = 0; t < 2; ++t) S[t] = mfma(as_bf16x8(op.kt[2 * t + s]), vh[s], S[t]);
#pragma unroll
    for (int t = 0; t < 2; ++t) S[t] = mfma(as_bf16x8(op.kt[2 * t + s]), vl[s], S[t]);
  }
  read_rows<1>(nx, nst, q, lane);
  read_rows<2>(nx, nst, q, lane);
  read_rows<3>(nx, nst, q, lane);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    GDN_GROUP(SG_MFMA, 1);
    GDN_GROUP(SG_DS_RD, 2);
  }
  GDN_SCHED_FENCE();
  at_state(S);  // (persistent scan: a sequence that ends here hands over to the next one's initial state)
  xs[q][lane] = __builtin_bit_cast(u32x4, pack_hi(S[0], S[1]));
  lds_barrier();

  // ---- R3
#pragma unroll
  for (int s = 0; s < 4; ++s) sb[s] = __builtin_bit_cast(bf16x8, xs[s][lane]);
  f32x4 o = acc * op.sq;
  o = mfma(vb[0], as_bf16x8(op.am[0]), o);
  if constexpr (TWO_A) o = mfma(vb[1], as_bf16x8(op.am[1]), o);
  store_out(o);
  GDN_SCHED_FENCE();
}

// s_waitcnt operand that waits for vmcnt <= n only (lgkmcnt and expcnt at their maxima)
constexpr int vmcnt_only(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }

// A loader wave's part of the scan (LD = 0, 1): the copies and the barriers,
// matching the compute waves' barrier for barrier.  A loader touches LDS only
// through its copies, whose completion it waits for explicitly, so its
// barriers carry no fence (a release fence would wait for every copy in
// flight, including those for the chunk after next).
template <int LD>
__device__ __forceinline__ void scan_rows_loader(u32x4 (*stage)[RS_BLOCKS * 64], int nch, int ct, int lane,
                                                 const ChunkArgs &a, int c0, int h, int hk) {
  constexpr int N = LD == 0 ? RS_LOADER0 : RS_LOADER1;  // copies per chunk
  constexpr int H = N / 2;                               // of which before barrier 1
  ChunkWalk walk;
  walk.start(a, a.seg_begin + c0);
  auto src_of = [&](int c) {  // (called with increasing c)
    const size_t j = static_cast<size_t>(c0 + c);
    int64_t t0;
    int len;
    walk.at(a, a.seg_begin + c0 + c, &t0, &len);
    return row_src(a, j * a.Hv + h, t0, len, hk);
  };
  stage_copy<LD>(stage[0], src_of(0), a, ct, 0, N, lane);
  if (nch > 1) {
    stage_copy<LD>(stage[1], src_of(1), a, ct, 0, N, lane);
    __builtin_amdgcn_s_waitcnt(vmcnt_only(N));  // chunk 0 landed
  } else {
    __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
  }
  __builtin_amdgcn_s_barrier();  // state exchange; chunk 0 staged
  __builtin_amdgcn_s_barrier();  // compute waves have read chunk 0
  for (int c = 0; c < nch; ++c) {
    if (c + 2 < nch) {
      const RowSrc r = src_of(c + 2);
      stage_copy<LD>(stage[c & 1], r, a, ct, 0, H, lane);
      __builtin_amdgcn_s_waitcnt(vmcnt_only(H));  // chunk c + 1 landed
      __builtin_amdgcn_s_barrier();
      stage_copy<LD>(stage[c & 1], r, a, ct, H, N, lane);
    } else {
      __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
      __builtin_amdgcn_s_barrier();
    }
    __builtin_amdgcn_s_barrier();
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
}

template <bool BF16_OUT>
__global__ __launch_bounds__(64 * SCAN_WAVES) void chunk_scan_kernel(ChunkArgs a) {
  __shared__ u32x4 stage[2][RS_BLOCKS * 64];  // 122 KiB
  __shared__ u32x4 xs[4][64];                 // state rows by k-step (bf16), lane order
  __shared__ u32x2 xv[3][2][64][2];           // V', V'' hi, V'' lo by k-step, lane, half
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = wave & 3;
  const int g4 = lane >> 4;
  const int nh = a.n_seqs * a.Hv;
  const int ratio = a.Hv / a.Hk;
  const int grp = a.dup ? 2 : ratio, hg = a.Hv / grp;  // v-heads reading the same q / k rows
  int ct = blockIdx.x / nh;    // plain order: the column tiles of one head share bid % 8,
  int rest = blockIdx.x % nh;  // i.e. one XCD and its L2
  if ((a.n_seqs * hg) % 8 == 0) {  // also the v-heads of one k-head (of a checked pair)
    int g, m;
    xcd_group_order(blockIdx.x, grp * (DV / SCAN_COLS), &g, &m);
    ct = m % (DV / SCAN_COLS);
    rest = (g / hg) * a.Hv + (g % hg) * grp + m / (DV / SCAN_COLS);
  }
  const int n = rest / a.Hv;
  const int h = rest % a.Hv;
  int hk = h / ratio;
  const int col = 16 * ct + (lane & 15);

  int64_t s0;
  int slen;
  seq_bounds(a, n, &s0, &slen);
  s0 = uniform64(s0);
  slen = __builtin_amdgcn_readfirstlane(slen);
  const int cs = __builtin_amdgcn_readfirstlane(chunk_start_at(a, n));
  const int ce = __builtin_amdgcn_readfirstlane(max(cs, min(chunk_start_at(a, n + 1), a.max_chunks)));
  const int lo = max(cs, a.seg_begin), hi = min(ce, a.seg_end);
  const int64_t in_row = a.h0 ? uniform64(pool_row_first(a.h0_idx, n, a.h0_rows)) : -1;
  const int64_t out_row = a.hT ? uniform64(pool_row_first(a.hT_idx, n, a.hT_rows)) : -1;
  const int64_t kv = static_cast<int64_t>(DK) * DV;
  const int row0 = 32 * q;  // first state row of a compute wave
  if (cs == ce) {  // empty sequence: the final state is the initial one (handled once)
    if (wave < 4 && a.seg_begin == 0 && out_row >= 0) {
      float *dst = a.hT + (out_row * a.Hv + h) * kv + col;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = row0 + 16 * t + 4 * g4 + e;
          dst[r * DV] = in_row >= 0 ? a.h0[(in_row * a.Hv + h) * kv + r * DV + col] : 0.f;
        }
    }
    return;
  }
  if (lo >= hi) return;  // no chunk of this sequence in this segment
  const int nch = hi - lo;
  const int c0 = lo - a.seg_begin;                             // first chunk, workspace-local
  const int64_t seq_off = static_cast<int64_t>(lo - cs) * CK;  // its first token within the sequence
  if (a.dup && (h & 1)) {  // every chunk of the range repeats the even partner's q / k rows: read that copy
    bool all = true;
    for (int i0 = 0; i0 < nch; i0 += 64) {
      const int i = i0 + lane;
      all = all && __all(i >= nch || a.dup[(c0 + i) * (a.Hv / 2) + h / 2] != 0);
    }
    if (all) hk = h - 1;
  }
  if (wave >= 4) {
    if (wave == 4)
      scan_rows_loader<0>(stage, nch, ct, lane, a, c0, h, hk);
    else
      scan_rows_loader<1>(stage, nch, ct, lane, a, c0, h, hk);
    return;
  }
  float *carry = a.carry + (static_cast<int64_t>(n) * a.Hv + h) * kv + col;

  f32x4 S[2];  // state rows row0 + 16t + 4g + e of this lane's column
  const float *src = lo == cs ? (in_row >= 0 ? a.h0 + (in_row * a.Hv + h) * kv + col : nullptr) : carry;
  if (src) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) S[t][e] = src[(row0 + 16 * t + 4 * g4 + e) * DV];
  } else {
#pragma unroll
    for (int t = 0; t < 2; ++t) S[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // Output addressing: byte offset of this lane's row 16q + r, columns
  // 16 ct + 4g .. +3, within a chunk (rows past the sequence end fall outside
  // the buffer range and are dropped).
  typedef typename std::conditional<BF16_OUT, uint16_t, float>::type OT;
  const int64_t ostep = static_cast<int64_t>(a.Hv) * DV;  // elements per token
  const int voff = static_cast<int>(((16 * q + (lane & 15)) * ostep + h * DV + 16 * ct + 4 * g4) * sizeof(OT));
  auto store_out = [&](const f32x4 &o, int c) {  // chunk c of this launch: rows [0, min(64, rest of sequence))
    const int64_t toff = seq_off + static_cast<int64_t>(c) * CK;
    const int rows = static_cast<int>(min<int64_t>(CK, slen - toff));
    OT *base = static_cast<OT *>(a.o) + (s0 + toff) * ostep;
    const auto r = __builtin_amdgcn_make_buffer_rsrc(base, 0, static_cast<int>(rows * ostep * sizeof(OT)), BUF_DWORD3);
    if constexpr (BF16_OUT)
      __builtin_amdgcn_raw_buffer_store_b64(pack4(o), r, voff, 0, 0);
    else
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), r, voff, 0, 0);
  };
  bf16x8 sb[4];  // the whole state as bf16 B operands, by k-step
  auto chunk = [&](const RowOps &op, RowOps &nx, int c) {
    // (after the last chunk the "next" reads take the idle buffer's stale contents, unused)
    const u32x4 *nst = stage[(c + 1) & 1];
    auto out = [&](const f32x4 &o) { store_out(o, c); };
    auto keep = [](f32x4 (&)[2]) {};
    if (q >= 2)
      scan_rows_chunk<true>(op, nx, nst, sb, S, xv, xs, q, lane, out, keep);
    else
      scan_rows_chunk<false>(op, nx, nst, sb, S, xv, xs, q, lane, out, keep);
  };

  RowOps op0, op1;
  xs[q][lane] = __builtin_bit_cast(u32x4, pack_hi(S[0], S[1]));
  lds_barrier();  // state exchange; chunk 0 staged
#pragma unroll
  for (int s = 0; s < 4; ++s) sb[s] = __builtin_bit_cast(bf16x8, xs[s][lane]);
  read_rows<0>(op0, stage[0], q, lane);
  read_rows<1>(op0, stage[0], q, lane);
  read_rows<2>(op0, stage[0], q, lane);
  read_rows<3>(op0, stage[0], q, lane);
  lds_barrier();  // chunk 0 read: its buffer may be refilled
  // xv and xs are each written after the barrier that follows their last
  // read, so one buffer of each suffices.
  for (int c = 0; c < nch; c += 2) {
    chunk(op0, op1, c);
    if (c + 1 >= nch) break;
    chunk(op1, op0, c + 1);
  }

  float *dst = hi == ce ? (out_row >= 0 ? a.hT + (out_row * a.Hv + h) * kv + col : nullptr) : carry;
  if (dst) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) dst[(row0 + 16 * t + 4 * g4 + e) * DV] = S[t][e];
  }
}

// Persistent scan for several sequences (varlen or a dense batch): one
// workgroup per (v-head, 16 state columns) walks every chunk of the segment
// in order, sequence after sequence, instead of one workgroup per
// (sequence, v-head, columns) paying its start and end for a few chunks each.
// The loader waves stream the segment's chunks as for one sequence; the
// compute waves track the sequence of each chunk, and where one ends (after
// its last state update, before the state exchange) they store its final
// state and continue from the next one's initial state, loaded into
// registers a sequence ahead.  Used when (v-heads x column tiles) alone fill
// the CUs.
template <bool BF16_OUT>
__global__ __launch_bounds__(64 * SCAN_WAVES) void chunk_scan_persist_kernel(ChunkArgs a) {
  __shared__ u32x4 stage[2][RS_BLOCKS * 64];  // 122 KiB
  __shared__ u32x4 xs[4][64];
  __shared__ u32x2 xv[3][2][64][2];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = wave & 3;
  const int g4 = lane >> 4;
  const int ratio = a.Hv / a.Hk;
  int ct = blockIdx.x / a.Hv;
  int h = blockIdx.x % a.Hv;
  if (a.Hk % 8 == 0) {  // the column tiles and v-heads of one k-head on one XCD
    int g, m;
    xcd_group_order(blockIdx.x, ratio * (DV / SCAN_COLS), &g, &m);
    ct = m % (DV / SCAN_COLS);
    h = g * ratio + m / (DV / SCAN_COLS);
  }
  const int hk = h / ratio;
  const int col = 16 * ct + (lane & 15);
  const int64_t kv = static_cast<int64_t>(DK) * DV;
  const int row0 = 32 * q;
  auto state_at = [&](float *base, int64_t row) { return base + (row * a.Hv + h) * kv + col; };
  auto load_state = [&](const float *src, f32x4 (&S)[2]) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) S[t][e] = src ? src[(row0 + 16 * t + 4 * g4 + e) * DV] : 0.f;
  };
  auto store_state = [&](float *dst, const f32x4 (&S)[2]) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) dst[(row0 + 16 * t + 4 * g4 + e) * DV] = S[t][e];
  };
  auto init_src = [&](int64_t row) -> const float * {
    return row >= 0 ? state_at(const_cast<float *>(a.h0), row) : nullptr;
  };
  // sequence records (chunk_table_kernel, read-only here): uniform, so read
  // through the constant address space as scalar loads into SGPRs
  typedef const __attribute__((address_space(4))) int64_t crec_t;
  crec_t *recp = (crec_t *)(a.seqrec);
  struct Rec {
    int64_t s0, in, out;
    int ce, len, nxt;
  };
  const bool arith = !a.cu && !a.h0_idx && !a.hT_idx;  // a dense batch without slot ids: no table
  auto rec_get = [&](int m) -> Rec {
    if (arith) {
      const int cpb = (a.T + CK - 1) / CK;
      return Rec{static_cast<int64_t>(m) * a.T, a.h0 ? pool_row(nullptr, m, a.h0_rows) : -1,
                 a.hT ? pool_row(nullptr, m, a.hT_rows) : -1, (m + 1) * cpb, a.T, m + 1};
    }
    crec_t *r = recp + static_cast<int64_t>(m) * SEQREC;
    return Rec{r[SR_S0], r[SR_IN], r[SR_OUT], static_cast<int>(r[SR_CE]), static_cast<int>(r[SR_LEN]),
               static_cast<int>(r[SR_NXT])};
  };

  const int lo = a.seg_begin, hi = min(a.seg_end, chunk_start_at(a, a.n_seqs));
  const bool any_empty = a.cu ? a.chunk_start[a.n_seqs + 1] > 0 : a.T == 0;  // (counted by the table kernel)
  if (wave < 4 && a.seg_begin == 0 && any_empty) {  // empty sequences pass their initial state through
    for (int m = 0; m < a.n_seqs; ++m) {
      if (chunk_start_at(a, m) != chunk_start_at(a, m + 1)) continue;
      const Rec r = rec_get(m);
      if (r.out < 0) continue;
      f32x4 Sx[2];
      load_state(init_src(r.in), Sx);
      store_state(state_at(a.hT, r.out), Sx);
    }
  }
  if (lo >= hi) return;
  const int nch = hi - lo;
  if (wave >= 4) {
    if (wave == 4)
      scan_rows_loader<0>(stage, nch, ct, lane, a, 0, h, hk);
    else
      scan_rows_loader<1>(stage, nch, ct, lane, a, 0, h, hk);
    return;
  }

  // the sequence of chunk lo: the last one starting at or before it (non-empty)
  int n;
  {
    int l = 0, r = a.n_seqs;
    while (r - l > 1) {
      const int mid = (l + r) >> 1;
      if (chunk_start_at(a, mid) <= lo) l = mid; else r = mid;
    }
    n = __builtin_amdgcn_readfirstlane(l);
  }
  // Current sequence n, the next one nn (its record and initial state Sn in
  // registers) and the one after, nnn (its record requested): at a sequence
  // end what the next sequence needs is already loaded.
  float *carry = a.carry;
  f32x4 S[2], Sn[2];
  const Rec rc = rec_get(n);
  int cs = __builtin_amdgcn_readfirstlane(chunk_start_at(a, n));
  int ce = rc.ce, slen = rc.len;
  int64_t s0 = rc.s0, orow = rc.out;
  load_state(lo == cs ? init_src(rc.in) : state_at(carry, n), S);
  int nn = ce < hi ? rc.nxt : a.n_seqs;
  int nnn = a.n_seqs;
  Rec rn{0, -1, -1, 0, 0, 0}, r3{0, -1, -1, 0, 0, 0};
  auto take_next = [&]() {  // rn = nn's record: its initial state, and nnn's record
    load_state(init_src(rn.in), Sn);
    nnn = rn.ce < hi ? rn.nxt : a.n_seqs;
    if (nnn < a.n_seqs) r3 = rec_get(nnn);
  };
  if (nn < a.n_seqs) {
    rn = rec_get(nn);
    take_next();
  }

  typedef typename std::conditional<BF16_OUT, uint16_t, float>::type OT;
  const int64_t ostep = static_cast<int64_t>(a.Hv) * DV;
  const int voff = static_cast<int>(((16 * q + (lane & 15)) * ostep + h * DV + 16 * ct + 4 * g4) * sizeof(OT));
  bf16x8 sb[4];
  auto chunk = [&](const RowOps &op, RowOps &nx, int c) {
    const u32x4 *nst = stage[(c + 1) & 1];
    const int j = lo + c;  // global chunk, in sequence n
    const int64_t toff = static_cast<int64_t>(j - cs) * CK;
    const int rows = static_cast<int>(min<int64_t>(CK, slen - toff));
    OT *base = static_cast<OT *>(a.o) + (s0 + toff) * ostep;
    auto out = [base, rows, ostep, voff](const f32x4 &o) {
      const auto r = __builtin_amdgcn_make_buffer_rsrc(base, 0, static_cast<int>(rows * ostep * sizeof(OT)), BUF_DWORD3);
      if constexpr (BF16_OUT)
        __builtin_amdgcn_raw_buffer_store_b64(pack4(o), r, voff, 0, 0);
      else
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), r, voff, 0, 0);
    };
    auto at_state = [&](f32x4 (&St)[2]) {
      if (j + 1 == ce && j + 1 < hi) {  // sequence n ends here, sequence nn starts with the next chunk
        if (orow >= 0) store_state(state_at(a.hT, orow), St);
        St[0] = Sn[0];
        St[1] = Sn[1];
        n = nn;
        cs = ce;
        ce = rn.ce;
        s0 = rn.s0;
        slen = rn.len;
        orow = rn.out;
        nn = nnn;
        if (nn < a.n_seqs) {
          rn = r3;
          take_next();
        }
      }
    };
    if (q >= 2)
      scan_rows_chunk<true>(op, nx, nst, sb, S, xv, xs, q, lane, out, at_state);
    else
      scan_rows_chunk<false>(op, nx, nst, sb, S, xv, xs, q, lane, out, at_state);
  };

  RowOps op0, op1;
  xs[q][lane] = __builtin_bit_cast(u32x4, pack_hi(S[0], S[1]));
  lds_barrier();  // state exchange; chunk 0 staged
#pragma unroll
  for (int s = 0; s < 4; ++s) sb[s] = __builtin_bit_cast(bf16x8, xs[s][lane]);
  read_rows<0>(op0, stage[0], q, lane);
  read_rows<1>(op0, stage[0], q, lane);
  read_rows<2>(op0, stage[0], q, lane);
  read_rows<3>(op0, stage[0], q, lane);
  lds_barrier();  // chunk 0 read: its buffer may be refilled
  for (int c = 0; c < nch; c += 2) {
    chunk(op0, op1, c);
    if (c + 1 >= nch) break;
    chunk(op1, op0, c + 1);
  }
  // the last sequence: finished here, or continued by the next segment
  if (ce <= hi) {
    if (orow >= 0) store_state(state_at(a.hT, orow), S);
  } else {
    store_state(state_at(carry, n), S);
  }
}

// ------------------------------------------------------------------ local prefill
// Batches of (sequence, v-head) pairs that fill the CUs run one workgroup per
// pair over the pair's whole chunk loop, with no workspace: the chunk's
// operands are formed in LDS by loc_prep (the phase-A steps of
// chunk_prep_kernel: K K^T and K Q^T, the solve, W and U) and consumed there
// by the state's chain, the state held in registers for the whole sequence:
//   V' = U - W S                            (-W blocks, U tiles from LDS)
//   O^T = (S^T Q^T) diag(sq) + V'^T A^T     (q fragments, A blocks from LDS)
//   S <- e^{gamma_63} S + K^T V''           (V'' = diag(sk) V' as bf16 hi + lo)
// The state is the B operand of V' and the A operand of O^T straight from the
// accumulators (pi order), V'' the B operand of the state update, so no
// product needs another wave's registers.  The chunk operands live in LDS in
// the layouts their consumers read with one ds_read_b128 per fragment: -W
// and A blocks as in the workspace layout, q rows as pi fragments (written
// from the prep waves' own fragments), K^T fragments (written by the wave of
// the prep that reads all of them), U tiles by (column tile, position tile).
// Same algorithm and precision as prep + scan.
constexpr int LOC_NB_A = 6;  // A blocks (p, s), s <= (p >= 2): those of the lower triangle
__host__ __device__ constexpr int a_blk(int p, int s) { return p < 2 ? p : 2 * p - 2 + s; }
enum { SC_SQ = 0, SC_SK = CK, SC_EL = 2 * CK };  // the scalar block: sq[64], sk[64], eL

struct LocIn {  // one chunk's inputs in prep thread tid's registers (tid < 256)
  u32x4 ku[4], vu[4];
  bf16x8 qf[4];
};

struct LocLds {
  uint16_t *kn;     // [64 * 128] K rows (nsw swizzle)
  f32x4 *s16k;      // [1024]: V rows (nsw) / the solve's exchange buffers
  u32x4 *ktf;       // [16][64] K^T fragments (row tile nb, position k-step s) at 2 nb + s
  u32x4 *qp;        // [16][64] q pi fragments (position tile i, k-step s) at 4 i + s
  u32x4 *wb;        // [16][64] -W blocks (p, s) at 4 p + s
  f32x4 *ub;        // [32][64] U tiles (column tile nb, position tile p) at 4 nb + p
  u32x4 *ab;        // [LOC_NB_A][64] A blocks (p, s) at a_blk(p, s)
  float *sc;        // [256] sq[64], sk[64], eL
  float *gam_s, *beta_s, *nk_s, *nq_s, *colw_s;  // [64] each
  f32x4 *tx;        // [4][4][64] T's rows by position tile (row layout), for the W and U products
};

// One chunk's rows into `in`: part 0 K and Q, part 1 V, part 2 all three.
__device__ __forceinline__ void loc_load(const ChunkArgs &a, LocIn &in, int64_t t0, int len, int h, int hk, int tid,
                                         int part = 2) {
  const int lane = tid & 63, p = tid >> 6, g4 = lane >> 4, irow = 16 * p + (lane & 15), seg = tid & 15;
  // buffer ranges end at the chunk's last row: rows past it read as zero
  auto rows_rsrc = [&](const uint16_t *base, int64_t stride, int head) {
    const int64_t bytes = (len - 1) * stride * 2 + DK * 2;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(base) + t0 * stride + (int64_t)head * DK, 0,
                                             static_cast<int>(bytes < 0 ? 0 : bytes), BUF_DWORD3);
  };
  const auto rk = rows_rsrc(a.k, a.ks, hk), rv = rows_rsrc(a.v, a.vs, h), rq = rows_rsrc(a.q, a.qs, hk);
  const int ks2 = static_cast<int>(a.ks * 2), vs2 = static_cast<int>(a.vs * 2), qs2 = static_cast<int>(a.qs * 2);
  if (part != 1) {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int row = (tid >> 4) + 16 * it;
      in.ku[it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, row * ks2 + seg * 16, 0, 0));
    }
  }
  if (part != 0) {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int row = (tid >> 4) + 16 * it;
      in.vu[it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, row * vs2 + seg * 16, 0, 0));
    }
  }
  if (part == 1) return;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int off = irow * qs2 + (32 * s + 4 * g4) * 2;
    const u32x2 x0 = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rq, off, 0, 0));
    const u32x2 x1 = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rq, off + 32, 0, 0));
    in.qf[s] = as_bf16x8(u32x4{x0.x, x0.y, x1.x, x1.y});
  }
}

// One chunk's gates, raw, into chain wave 4's registers (lane = position;
// positions past the chunk's end read nothing), and from them the gates
// and their chunk-local cumsum into LDS (gam_s, beta_s).  The chain wave
// forms them for chunk k before barrier 1 of step k, in the time it waits
// there, instead of the preparing wave 0 ahead of its own work.
__device__ __forceinline__ GateRaw loc_gates_load(const ChunkArgs &a, int64_t t0, int len, int h, int lane) {
  GateRaw g{0u, 0u, 0.f, 0.f};
  if (lane < len) {
    const int64_t gi = (t0 + lane) * a.gate.stride + h;
    g.ga = load_bits(a.gate.g_or_a, gi, a.gate.A_log ? a.gate.dt : GDN_DTYPE_F32);
    g.gb = load_bits(a.gate.beta_or_b, gi, a.gate.dt);
  }
  if (a.gate.A_log) {
    g.a_log = a.gate.A_log[h];
    g.dt_bias = a.gate.dt_bias[h];
  }
  return g;
}
__device__ __forceinline__ void loc_gates(const ChunkArgs &a, const GateRaw &g, int len, int lane, float *gam_s,
                                          float *beta_s) {
  float gv = 0.f, bv = 0.f;
  if (lane < len) gates_from_raw(a.gate, g, &gv, &bv);
  gam_s[lane] = wave_incl_scan(gv);  // chunk-local cumsum of g
  beta_s[lane] = bv;
}

// Phase A of one chunk on waves 0-3 (thread tid < 256), from the registers of
// loc_load into the LDS operands of the chain.
// after_kq() runs once the chunk's K and Q rows in `in` are consumed (after
// barrier 1) and after_v() once its V rows are (in LDS, before barrier 6):
// the caller requests the next chunk's rows into `in` there, so that no
// load is issued in the interval after barrier 6 (measured: B = 16 x
// T = 1038 and configuration 3's prefill ~1% faster than with all the
// loads after barrier 6).
template <class AfterKQ, class AfterV>
__device__ __forceinline__ void loc_prep(const ChunkArgs &a, const LocIn &in, const LocLds &L, int len, int tid,
                                         const AfterKQ &after_kq, const AfterV &after_v) {
  const int lane = tid & 63, p = tid >> 6, g4 = lane >> 4, r16 = lane & 15, seg = tid & 15;
  const int irow = 16 * p + r16;
  uint16_t *kn = L.kn;
  uint16_t *vn = reinterpret_cast<uint16_t *>(L.s16k);
  // L.s16k[0 .. 4 * 64): unused by the solve
  f32x4 *dxch = L.s16k + 4 * 64;    // [4 * 64] diagonal blocks of T, D layout by lane
  f32x4 *txch = L.s16k + 8 * 64;    // [3 * 64] T[1][0], T[2][1], T[2][0], D layout by lane
  float(*dtr)[16 * 20] = reinterpret_cast<float(*)[16 * 20]>(L.s16k + 11 * 64);  // D -> row layout

  // ---- K rows into LDS; K and Q row norms; the q fragments for the chain (the
  // gates and their cumsum: chain wave 4, loc_gates, before the same barrier 1)
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int row = (tid >> 4) + 16 * it;
    *reinterpret_cast<u32x4 *>(kn + nsw(row, seg * 8)) = in.ku[it];
    float sk = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t kw = in.ku[it][e];
      const float k0 = bf16_bits_to_f32(kw & 0xffffu), k1 = bf16_bits_to_f32(kw >> 16);
      sk += k0 * k0 + k1 * k1;
    }
    sk = row16_sum(sk);
    if (seg == 0) L.nk_s[row] = a.l2norm ? rsqrtf(sk + 1e-6f) : 1.f;
  }
  {
    float sq = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      L.qp[(4 * p + s) * 64 + lane] = __builtin_bit_cast(u32x4, in.qf[s]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = static_cast<float>(in.qf[s][e]);
        sq += x * x;
      }
    }
    sq += __shfl_xor(sq, 16, 64);
    sq += __shfl_xor(sq, 32, 64);
    if (g4 == 0) L.nq_s[irow] = (a.l2norm ? rsqrtf(sq + 1e-6f) : 1.f) * a.scale;
  }
  lds_barrier();  // (1)
  after_kq();

  if (p == 0) {  // per-position scalars of the chain, W's column scale
    const float gl = L.gam_s[CK - 1], gm = L.gam_s[lane], nkl = L.nk_s[lane];
    L.sc[SC_SQ + lane] = fast_exp(gm) * L.nq_s[lane];
    L.sc[SC_SK + lane] = fast_exp(gl - gm) * nkl;
    if (lane == 0) L.sc[SC_EL] = fast_exp(gl);
    L.colw_s[lane] = L.beta_s[lane] * fast_exp(gm) * nkl;
  }

  // ---- tiles (cb, pa), cb <= pa = 3 - p, of K Q^T (A), then tiles (cb, p),
  // cb <= p, of K K^T (L, in row layout, for this wave's solve): 5 tile
  // products per wave instead of 2, 4, 6, 8 (q fragments of other rows from LDS)
  const f32x4 z4a = {0.f, 0.f, 0.f, 0.f};
  {
    const int pa = 3 - p, irow_a = 16 * pa + r16;
    const float gia = L.gam_s[irow_a], nqa = L.nq_s[irow_a];
    bf16x8 qa[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) qa[s] = as_bf16x8(L.qp[(4 * pa + s) * 64 + lane]);
    f32x4 af[4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      af[cb] = z4a;
      if (cb <= pa) {
        f32x4 qk = z4a;
#pragma unroll
        for (int s = 0; s < 4; ++s) qk = mfma(frag_pi(kn, 16 * cb, s, lane), qa[s], qk);
        const f32x4 gj = *reinterpret_cast<const f32x4 *>(L.gam_s + 16 * cb + 4 * g4);
        const f32x4 nj = *reinterpret_cast<const f32x4 *>(L.nk_s + 16 * cb + 4 * g4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int jj = 16 * cb + 4 * g4 + e;
          af[cb][e] = jj <= irow_a ? nqa * nj[e] * qk[e] * fast_exp(gia - gj[e]) : 0.f;
        }
      }
    }
    L.ab[a_blk(pa, 0) * 64 + lane] = __builtin_bit_cast(u32x4, pack_hi(af[0], af[1]));
    if (pa >= 2) L.ab[a_blk(pa, 1) * 64 + lane] = __builtin_bit_cast(u32x4, pack_hi(af[2], af[3]));
  }
  const float gi = L.gam_s[irow], bi = L.beta_s[irow], nki = L.nk_s[irow];
  bf16x8 kown[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) kown[s] = frag_pi(kn, 16 * p, s, lane);
  f32x4 lf[4];
#pragma unroll
  for (int cb = 0; cb < 4; ++cb) {
    lf[cb] = z4a;
    if (cb <= p) {
      f32x4 kk = z4a;
#pragma unroll
      for (int s = 0; s < 4; ++s) kk = mfma(frag_pi(kn, 16 * cb, s, lane), kown[s], kk);
      const f32x4 gj = *reinterpret_cast<const f32x4 *>(L.gam_s + 16 * cb + 4 * g4);
      const f32x4 nj = *reinterpret_cast<const f32x4 *>(L.nk_s + 16 * cb + 4 * g4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int jj = 16 * cb + 4 * g4 + e;
        lf[cb][e] = jj < irow ? bi * nki * nj[e] * kk[e] * fast_exp(gi - gj[e]) : 0.f;
      }
    }
  }

  // ---- T = (I + L)^-1: diagonal blocks by diag_inverse (no LDS round trip on the
  // preparation's longest interval), the blocks below them as in chunk_prep_kernel
  f32x4 dl, drow;
  {
    dl = diag_inverse(lf, p, lane);
    dxch[p * 64 + lane] = dl;
    float *tr = dtr[p];
#pragma unroll
    for (int e = 0; e < 4; ++e) tr[(4 * g4 + e) * 20 + r16] = dl[e];
    __builtin_amdgcn_wave_barrier();
    drow = *reinterpret_cast<const f32x4 *>(tr + r16 * 20 + 4 * g4);
  }
  lds_barrier();  // (2)
  f32x4 trow[4];
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int b = 0; b < 4; ++b) trow[b] = b == p ? drow : z4;
#pragma unroll
  for (int b = 0; b < 3; ++b)
    if (b == p - 1) {
      const f32x4 x = mm16(lf[b], dxch[b * 64 + lane], z4);
      trow[b] = -mm16(x, drow, z4);
      if (b <= 1) txch[b * 64 + lane] = -mm16(drow, x, z4);
    }
  lds_barrier();  // (3)
#pragma unroll
  for (int b = 0; b < 2; ++b)
    if (b == p - 2) {
      f32x4 x = mm16(lf[b], dxch[b * 64 + lane], z4);
      x = mm16(lf[b + 1], txch[b * 64 + lane], x);
      trow[b] = -mm16(x, drow, z4);
      if (b == 0) txch[2 * 64 + lane] = -mm16(drow, x, z4);
    }
  lds_barrier();  // (4)
  if (p == 3) {
    f32x4 x = mm16(lf[0], dxch[lane], z4);
    x = mm16(lf[1], txch[lane], x);
    x = mm16(lf[2], txch[2 * 64 + lane], x);
    trow[0] = -mm16(x, drow, z4);
  }
#pragma unroll
  for (int b = 0; b < 4; ++b) L.tx[(4 * p + b) * 64 + lane] = trow[b];  // for the W and U products
  lds_barrier();  // (5) the exchange buffers are free: V rows take their place
#pragma unroll
  for (int it = 0; it < 4; ++it)
    *reinterpret_cast<u32x4 *>(vn + nsw((tid >> 4) + 16 * it, seg * 8)) = in.vu[it];
  after_v();
  lds_barrier();  // (6)

  // ---- -W = -(T diag(colw) K), as W^T tiles K^T (T diag(colw))^T, for the
  // column tiles 2p and 2p + 1 over every position tile (T's rows from L.tx):
  // 24 products on every wave; the K^T fragments it reads are also left for
  // the chain.  U = T diag(beta) V is formed by the chain waves in the same
  // interval (loc_u).
  bf16x8 kt[2][2];
#pragma unroll
  for (int jn = 0; jn < 2; ++jn)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      kt[jn][s] = frag_tr(kn, s, 16 * (2 * p + jn), lane);
      L.ktf[(2 * (2 * p + jn) + s) * 64 + lane] = __builtin_bit_cast(u32x4, kt[jn][s]);
    }
#pragma unroll
  for (int pt = 0; pt < 4; ++pt) {
    f32x4 w0 = z4, w1 = z4;
#pragma unroll
    for (int s = 0; s < (pt >= 2 ? 2 : 1); ++s) {  // T's rows 0..31 end at column 31
      const f32x4 cw0 = *reinterpret_cast<const f32x4 *>(L.colw_s + 32 * s + 4 * g4);
      const f32x4 cw1 = *reinterpret_cast<const f32x4 *>(L.colw_s + 32 * s + 16 + 4 * g4);
      bf16x8 whi, wlo;
      pack_hilo(L.tx[(4 * pt + 2 * s) * 64 + lane] * cw0, L.tx[(4 * pt + 2 * s + 1) * 64 + lane] * cw1, whi, wlo);
      w0 = mfma(kt[0][s], whi, w0);
      w0 = mfma(kt[0][s], wlo, w0);
      w1 = mfma(kt[1][s], whi, w1);
      w1 = mfma(kt[1][s], wlo, w1);
    }
    L.wb[(4 * pt + p) * 64 + lane] = __builtin_bit_cast(u32x4, pack_hi(-w0, -w1));
  }
  lds_barrier();  // (7) the chunk's operands are in LDS
}

// U = T diag(beta) V for the column tiles 2q and 2q + 1 over every position
// tile, by chain wave 4 + q between barriers 6 and 7 of the chunk's
// preparation: T's rows from L.tx, V's rows from LDS (written before barrier 6).
__device__ __forceinline__ void loc_u(const LocLds &L, int q, int lane) {
  const int g4 = lane >> 4;
  const uint16_t *vn = reinterpret_cast<const uint16_t *>(L.s16k);
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  bf16x8 vf[2][2];
#pragma unroll
  for (int jn = 0; jn < 2; ++jn)
#pragma unroll
    for (int s = 0; s < 2; ++s) vf[jn][s] = frag_tr(vn, s, 16 * (2 * q + jn), lane);
#pragma unroll
  for (int pt = 0; pt < 4; ++pt) {
    f32x4 u0 = z4, u1 = z4;
#pragma unroll
    for (int s = 0; s < (pt >= 2 ? 2 : 1); ++s) {
      const f32x4 be0 = *reinterpret_cast<const f32x4 *>(L.beta_s + 32 * s + 4 * g4);
      const f32x4 be1 = *reinterpret_cast<const f32x4 *>(L.beta_s + 32 * s + 16 + 4 * g4);
      bf16x8 uhi, ulo;
      pack_hilo(L.tx[(4 * pt + 2 * s) * 64 + lane] * be0, L.tx[(4 * pt + 2 * s + 1) * 64 + lane] * be1, uhi, ulo);
      u0 = mfma(uhi, vf[0][s], u0);
      u0 = mfma(ulo, vf[0][s], u0);
      u1 = mfma(uhi, vf[1][s], u1);
      u1 = mfma(ulo, vf[1][s], u1);
    }
    L.ub[(4 * (2 * q) + pt) * 64 + lane] = u0;
    L.ub[(4 * (2 * q + 1) + pt) * 64 + lane] = u1;
  }
}


// The per-pair prefill, the chunk's preparation and the state's chain
// overlapped: one workgroup of 8 waves per (sequence, v-head).  Waves 0-3
// prepare chunk k (loc_prep, 7 barriers) while waves 4-7 run chunk k - 1's
// chain, fitted between the same barriers: V' = U - W S before barrier 1,
// the output and the state update between barriers 1 and 2 (the solve's
// interval, the longest); between barriers 6 and 7 they form chunk k's U
// for their column tiles, and wave 4 forms chunk k + 1's gates before the
// next barrier 1.  The operands the preparation writes before barrier 2
// (q fragments, A blocks, scalars) are double-buffered; -W, U and K^T are
// written after barrier 6, when the chain has read them.  The next chunk's
// K and Q rows are requested after barrier 1 and its V rows before barrier
// 6, each once the current ones are in LDS.
// 159 KiB of LDS: one workgroup per CU.
constexpr int LOC_WAVES = 8;
constexpr int LOC_LPT_MAX = 64 * LOC_WAVES;  // sequences ranked in the prologue, one per thread

// Longest sequences first.  The per-pair workgroups run one per CU, each for
// its sequence's whole length, and start in workgroup order as CUs free up;
// in sequence order a long sequence whose pairs come late starts after a
// short one has finished (configuration 3: 39 chunk steps on the busiest CU
// against 32, its longest sequence).  The workgroup for slot n takes the
// sequence whose length ranks n-th, decreasing, ties by index: each thread
// ranks one sequence against all the lengths (from cu_seqlens, in LDS the
// preparation does not use before barrier 1).  Returns n unchanged for more
// than LOC_LPT_MAX sequences.
__device__ __forceinline__ int loc_longest_first(const ChunkArgs &a, int n, int tid, int *lds) {
  if (a.n_seqs > LOC_LPT_MAX) return n;
  int *lens = lds, *sel = lds + LOC_LPT_MAX;
  if (tid < a.n_seqs) {
    int64_t s0;
    int len;
    seq_bounds(a, tid, &s0, &len);
    lens[tid] = len;
  }
  __syncthreads();
  if (tid < a.n_seqs) {
    const int lm = lens[tid];
    int r = 0;
    for (int j = 0; j < a.n_seqs; ++j) {
      const int lj = lens[j];
      r += (lj > lm) || (lj == lm && j < tid);
    }
    if (r == n) *sel = tid;
  }
  __syncthreads();
  return *sel;
}

template <bool BF16_OUT>
__global__ __launch_bounds__(64 * LOC_WAVES) void chunk_local_kernel(ChunkArgs a) {
  __shared__ __align__(16) uint16_t kn[CK * DK];
  __shared__ __align__(16) f32x4 s16k[1024];
  __shared__ u32x4 ktf[16 * 64], wb[16 * 64], qp2[2][16 * 64], ab2[2][LOC_NB_A * 64];
  __shared__ f32x4 ub[32 * 64];
  __shared__ __align__(16) float sc2[2][SCAL], gam_s[CK], beta_s[CK], nk_s[CK], nq_s[CK], colw_s[CK];
  __shared__ f32x4 tx[16 * 64];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, r16 = lane & 15;
  const int ratio = a.Hv / a.Hk;
  int n = blockIdx.x / a.Hv, h = blockIdx.x % a.Hv;
  if ((a.n_seqs * (a.Hv / ratio)) % 8 == 0) {
    int g, m;
    xcd_group_order(blockIdx.x, ratio, &g, &m);
    n = g / (a.Hv / ratio);
    h = (g % (a.Hv / ratio)) * ratio + m;
  }
  if (a.cu && a.n_seqs > 1) n = __builtin_amdgcn_readfirstlane(loc_longest_first(a, n, tid, reinterpret_cast<int *>(s16k)));
  const int hk = h / ratio;
  int64_t s0;
  int slen;
  seq_bounds(a, n, &s0, &slen);
  s0 = uniform64(s0);
  slen = __builtin_amdgcn_readfirstlane(slen);
  const int nch = (slen + CK - 1) / CK;
  auto chunk_len = [&](int k) { return min(CK, slen - k * CK); };

  if (wave < 4) {  // ---------------- preparation of chunk k at step k
    LocIn in;
    if (nch > 0) loc_load(a, in, s0, chunk_len(0), h, hk, tid);
    for (int k = 0; k < nch; ++k) {
      // the thread index made opaque per chunk: the LDS addresses derived from
      // it are recomputed in the loop instead of hoisted out of it and spilled
      int tk = tid;
      asm volatile("" : "+v"(tk));
      const LocLds L{kn, s16k, ktf, qp2[k & 1], wb, ub, ab2[k & 1], sc2[k & 1], gam_s, beta_s, nk_s, nq_s, colw_s, tx};
      loc_prep(a, in, L, chunk_len(k), tk, [&] {
        if (k + 1 < nch) loc_load(a, in, s0 + static_cast<int64_t>(k + 1) * CK, chunk_len(k + 1), h, hk, tk, 0);
      }, [&] {
        if (k + 1 < nch) loc_load(a, in, s0 + static_cast<int64_t>(k + 1) * CK, chunk_len(k + 1), h, hk, tk, 1);
      });
    }
    if (nch > 0)  // step nch: the chain's last chunk
#pragma unroll 1
      for (int b = 0; b < 7; ++b) lds_barrier();
    return;
  }

  // ---------------- the chain of chunk k - 1 at step k (waves 4-7)
  const int cw = wave - 4;
  const int64_t kv = static_cast<int64_t>(DK) * DV;
  const int64_t in_row = a.h0 ? uniform64(pool_row_first(a.h0_idx, n, a.h0_rows)) : -1;
  const int64_t out_row = a.hT ? uniform64(pool_row_first(a.hT_idx, n, a.hT_rows)) : -1;
  float *dst[2];
  f32x4 S[2][8];  // tile j: state rows 16 t + 4 g + e of column 32 cw + 16 j + r
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = 32 * cw + 16 * j + r16;
    const float *src = in_row >= 0 ? a.h0 + (in_row * a.Hv + h) * kv + col : nullptr;
    dst[j] = out_row >= 0 ? a.hT + (out_row * a.Hv + h) * kv + col : nullptr;
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) S[j][t][e] = src ? src[(16 * t + 4 * g4 + e) * DV] : 0.f;
  }
  typedef typename std::conditional<BF16_OUT, uint16_t, float>::type OT;
  const int64_t ostep = static_cast<int64_t>(a.Hv) * DV;
  // the chain waves' share of the preparation of chunk k: U, between barriers 6 and 7
  const LocLds Lu{kn, s16k, ktf, nullptr, wb, ub, nullptr, nullptr, gam_s, beta_s, nk_s, nq_s, colw_s, tx};
  auto prep_share = [&](int k) {
    int ln = lane;
    asm volatile("" : "+v"(ln));  // per call: keeps LLVM from hoisting loc_u's LDS addresses into the loop
    if (k < nch) loc_u(Lu, cw, ln);
  };
  // chunk k's gates by wave 4 (cw 0) before barrier 1 of step k; the raw
  // values of chunk k + 1 requested after that barrier
  GateRaw gnext{0u, 0u, 0.f, 0.f};
  // step 0: the preparation of chunk 0 alone
  if (nch > 0) {
    if (cw == 0) loc_gates(a, loc_gates_load(a, s0, chunk_len(0), h, lane), chunk_len(0), lane, gam_s, beta_s);
    lds_barrier();  // (1)
    if (cw == 0 && nch > 1) gnext = loc_gates_load(a, s0 + CK, chunk_len(1), h, lane);
#pragma unroll 1
    for (int b = 1; b < 6; ++b) lds_barrier();  // (2) .. (6)
    prep_share(0);
    lds_barrier();  // (7)
  }
  for (int k = 1; k <= nch; ++k) {
    const int c = k - 1;
    const u32x4 *qp = qp2[c & 1], *ab = ab2[c & 1];
    const float *sc = sc2[c & 1];
    const int64_t t0 = s0 + static_cast<int64_t>(c) * CK;
    const int len = chunk_len(c);
    // interval 0: V' = U - W S
    bf16x8 sb[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int s = 0; s < 4; ++s) sb[j][s] = pack_hi(S[j][2 * s], S[j][2 * s + 1]);
    f32x4 vp[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int t = 0; t < 4; ++t) vp[j][t] = ub[(4 * (2 * cw + j) + t) * 64 + lane];
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const bf16x8 w = as_bf16x8(wb[(4 * t + s) * 64 + lane]);
#pragma unroll
        for (int j = 0; j < 2; ++j) vp[j][t] = mfma(w, sb[j][s], vp[j][t]);
      }
    if (cw == 0 && k < nch) loc_gates(a, gnext, chunk_len(k), lane, gam_s, beta_s);
    lds_barrier();  // (1)
    if (cw == 0 && k + 1 < nch) gnext = loc_gates_load(a, s0 + static_cast<int64_t>(k + 1) * CK, chunk_len(k + 1), h, lane);
    // interval 1: O^T = (S^T Q^T) diag(sq) + V'^T A^T, then S <- e^{gamma_63} S + K^T V''
    bf16x8 vb[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int s = 0; s < 2; ++s) vb[j][s] = pack_hi(vp[j][2 * s], vp[j][2 * s + 1]);
    OT *obase = static_cast<OT *>(a.o) + t0 * ostep;
    const auto ro = __builtin_amdgcn_make_buffer_rsrc(obase, 0, static_cast<int>(len * ostep * sizeof(OT)), BUF_DWORD3);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 qv = as_bf16x8(qp[(4 * i + s) * 64 + lane]);
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[j] = mfma(sb[j][s], qv, acc[j]);
      }
      const float sqi = sc[SC_SQ + 16 * i + r16];
      const bf16x8 a0 = as_bf16x8(ab[a_blk(i, 0) * 64 + lane]);
      const bf16x8 a1 = i >= 2 ? as_bf16x8(ab[a_blk(i, 1) * 64 + lane]) : a0;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        f32x4 o = acc[j] * sqi;
        o = mfma(vb[j][0], a0, o);
        if (i >= 2) o = mfma(vb[j][1], a1, o);
        const int voff = static_cast<int>(((16 * i + r16) * ostep + h * DV + 32 * cw + 16 * j + 4 * g4) * sizeof(OT));
        if constexpr (BF16_OUT)
          __builtin_amdgcn_raw_buffer_store_b64(pack4(o), ro, voff, 0, 0);
        else
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), ro, voff, 0, 0);
      }
    }
    bf16x8 vh[2][2], vl[2][2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const f32x4 sk0 = *reinterpret_cast<const f32x4 *>(sc + SC_SK + 32 * s + 4 * g4);
      const f32x4 sk1 = *reinterpret_cast<const f32x4 *>(sc + SC_SK + 32 * s + 16 + 4 * g4);
#pragma unroll
      for (int j = 0; j < 2; ++j) pack_hilo(vp[j][2 * s] * sk0, vp[j][2 * s + 1] * sk1, vh[j][s], vl[j][s]);
    }
    const float eL = sc[SC_EL];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int t = 0; t < 8; ++t) S[j][t] = S[j][t] * eL;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const bf16x8 kt = as_bf16x8(ktf[(2 * t + s) * 64 + lane]);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          S[j][t] = mfma(kt, vh[j][s], S[j][t]);
          S[j][t] = mfma(kt, vl[j][s], S[j][t]);
        }
      }
#pragma unroll 1
    for (int b = 1; b < 6; ++b) lds_barrier();  // (2) .. (6)
    prep_share(k);
    lds_barrier();  // (7)
  }
#pragma unroll
  for (int j = 0; j < 2; ++j)
    if (dst[j]) {
#pragma unroll
      for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[j][(16 * t + 4 * g4 + e) * DV] = S[j][t][e];
    }
}


// Chunks per prep + scan segment: one prep launch produces a segment's
// operands (about 2.3 MiB per chunk at 32 v-heads: 146 MiB for 64 chunks,
// which stay in the 256 MB Infinity Cache until the scan reads them) and one
// scan launch consumes them; longer inputs run segment after segment on the
// caller's stream.  Measured (T = 16384 / 65536 / configuration 3): serial
// 64-chunk segments 478 us / 1.78 ms / 431 us; 96, 128 and 512 chunks, whose
// operands spill to HBM, 532-560 us / 2.0-2.2 ms / 490-518 us; the next
// segment's prep on a second stream beside the scan 700 us / 3.1 ms (the two
// kernels cannot share a CU -- the scan holds 138 KiB of LDS -- so the prep
// takes CUs from the scan's chain).
constexpr int SEG_CHUNKS = 64;
// (sequence, v-head) pairs from which the local kernel runs.  Its time is the
// longest sequence's chunk count times a chunk step, whatever the batch (up
// to one workgroup per CU); prep + scan grows with the total chunks.
// Measured (q/k at 16 heads, Hv = 32): B = 4 x T = 1038 132 (prep + scan)
// against 139 us, B = 6 x T = 1038 193 against 142, B = 4 x T = 4096 459
// against 495, B = 2 x T = 4096 242 against 477: the local kernel from 5
// sequences of 32 v-heads.
constexpr int LOC_MIN_PAIRS = 160;
// Short batches take the local kernel below that as well: one chunk per
// sequence at any batch, two from LOC_SHORT2_PAIRS pairs, where prep + scan's
// fixed latency outweighs a chunk step.  The chunk count is exact for a dense
// batch (no cu_seqlens); with cu_seqlens its bound, the total tokens' chunks
// (one sequence can hold them all), is used.  Measured from graphs (10 calls per
// replay, Hv = 32), local against prep + scan: T = 64 at B = 1 / 2 / 3 / 4
// 14.1 / 14.5 / 15.3 / 15.9 against 15.3 / 17.1 / 19.5 / 22.0 us; T = 128
// 20.5 / 21.0 / 21.5 / 21.9 against 16.5 / 19.4 / 23.7 / 26.7; T = 256
// 33.4-35.5 against 18.6-37.5.  (The workspace size does not depend on
// this: a local call ignores the workspace it is given.)
constexpr int LOC_SHORT2_PAIRS = 96;

// Workspace: the chunk table, the state carried between segments (when
// there are several) and the scan operands of one segment.
struct WsLayout {
  size_t chunk_start, seqrec, carry, total;
  size_t vh, Ut, dup;
};

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

WsLayout ws_layout(int n_seqs, int64_t seg_chunks, int Hv, bool multi) {
  WsLayout l;
  size_t off = 0;
  l.chunk_start = off;
  off = align256(off + sizeof(int32_t) * (n_seqs + 2));
  l.seqrec = off;
  off = align256(off + sizeof(int64_t) * SEQREC * static_cast<size_t>(n_seqs));
  l.carry = off;
  if (multi) off = align256(off + sizeof(float) * static_cast<size_t>(n_seqs) * Hv * DK * DV);
  l.vh = off;
  off = align256(off + 16ull * seg_chunks * Hv * NB_VH * 64);
  l.Ut = off;
  off = align256(off + sizeof(float) * seg_chunks * Hv * DV * CK);
  l.dup = off;
  off = align256(off + sizeof(int32_t) * seg_chunks * ((Hv + 1) / 2));
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
  if (static_cast<int64_t>(n_seqs) * Hv >= LOC_MIN_PAIRS) return 0;  // the local kernel keeps all in LDS
  // Upper bound valid with or without cu_seqlens.
  const int64_t nc = (total_tokens + CK - 1) / CK + n_seqs;
  return ws_layout(n_seqs, std::min<int64_t>(nc, SEG_CHUNKS), Hv, nc > SEG_CHUNKS).total;
}

namespace gdn {
namespace {

int chunk_fwd(const void *q, const void *k, const void *v, int qkv_dtype,
              int64_t q_stride_t, int64_t k_stride_t, int64_t v_stride_t, const GateArgs &gate,
              const float *h0, const int64_t *h0_idx, int64_t h0_rows, float *hT, const int64_t *hT_idx,
              int64_t hT_rows, void *o, int o_dtype, const int32_t *cu_seqlens, int32_t n_seqs, int32_t T,
              int32_t Hk, int32_t Hv, int32_t K, int32_t V, float scale, int l2norm_qk,
              void *workspace, size_t workspace_bytes, void *stream, const char *name) {
  if (K != DK || V != DV) return fail(GDN_ERR_UNSUPPORTED, "%s: K=%d V=%d; only K=V=128 is built", name, K, V);
  if (qkv_dtype != GDN_DTYPE_BF16)
    return fail(GDN_ERR_UNSUPPORTED, "%s: q/k/v must be bf16 (MFMA operands)", name);
  if (n_seqs < 0 || T < 0 || Hk <= 0 || Hv <= 0 || Hv % Hk)
    return fail(GDN_ERR_INVALID_ARGUMENT, "%s: bad sizes n_seqs=%d T=%d Hk=%d Hv=%d", name, n_seqs, T, Hk, Hv);
  if (!valid_dtype(gate.dt)) return fail(GDN_ERR_INVALID_ARGUMENT, "%s: bad gate dtype", name);
  if (o_dtype != GDN_DTYPE_BF16 && o_dtype != GDN_DTYPE_F32)
    return fail(GDN_ERR_UNSUPPORTED, "%s: output must be bf16 or fp32", name);
  if (n_seqs == 0) return ok();
  if (!q || !k || !v || !gate.g_or_a || !gate.beta_or_b || !o)
    return fail(GDN_ERR_INVALID_ARGUMENT, "%s: null q/k/v/gate/o", name);
  if (gate.A_log && !gate.dt_bias) return fail(GDN_ERR_INVALID_ARGUMENT, "%s: null dt_bias", name);
  if (gate.stride < Hv) return fail(GDN_ERR_INVALID_ARGUMENT, "%s: gate token stride smaller than Hv", name);
  if (!rows_cover(h0, h0_idx, h0_rows, n_seqs) || !rows_cover(hT, hT_idx, hT_rows, n_seqs))
    return fail(GDN_ERR_INVALID_ARGUMENT, "%s: state rows (%lld in, %lld out) do not cover %d sequences", name,
                static_cast<long long>(h0_rows), static_cast<long long>(hT_rows), n_seqs);
  if (q_stride_t < Hk * K || k_stride_t < Hk * K || v_stride_t < Hv * V || (q_stride_t | k_stride_t | v_stride_t) % 8)
    return fail(GDN_ERR_INVALID_ARGUMENT, "%s: token strides must cover a row and be multiples of 8", name);
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) % 16)
    return fail(GDN_ERR_INVALID_ARGUMENT, "%s: q/k/v must be 16-byte aligned", name);
  const int64_t total = cu_seqlens ? static_cast<int64_t>(T) : static_cast<int64_t>(n_seqs) * T;
  const int64_t nc = max_chunks_of(n_seqs, total, cu_seqlens != nullptr, T);
  // several sequences: the persistent scan once its (v-head, column tile)
  // workgroups fill the CUs without spreading the sequences over the grid
  // (sequence, v-head) pairs that fill the CUs: the local kernel, one workgroup per pair
  const int64_t pairs = static_cast<int64_t>(n_seqs) * Hv;
  const int64_t longest = cu_seqlens ? (total + CK - 1) / CK : (T + CK - 1) / CK;  // chunks, or their bound
  const bool local = pairs >= LOC_MIN_PAIRS || longest == 1 || (longest == 2 && pairs >= LOC_SHORT2_PAIRS);
  const bool persist = n_seqs > 1 && static_cast<int64_t>(Hv) * (DV / SCAN_COLS) >= SCAN_PERSIST_BLOCKS;
  const int64_t seg = std::min<int64_t>(nc, SEG_CHUNKS);
  const WsLayout l = ws_layout(n_seqs, seg, Hv, nc > SEG_CHUNKS);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (local) {  // one workgroup per (sequence, v-head); no workspace
    if (pairs > 0x7fffffff) return fail(GDN_ERR_INVALID_ARGUMENT, "%s: grid too large", name);
    ChunkArgs a{static_cast<const uint16_t *>(q), static_cast<const uint16_t *>(k), static_cast<const uint16_t *>(v),
                q_stride_t, k_stride_t, v_stride_t, gate, h0, h0_idx, h0_rows, hT, hT_idx, hT_rows, o, o_dtype,
                cu_seqlens, n_seqs, T, Hk, Hv, total, scale, l2norm_qk, static_cast<int>(std::min<int64_t>(nc, 0x7fffffff)),
                0, 0, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(n_seqs) * Hv));
    if (o_dtype == GDN_DTYPE_BF16)
      hipLaunchKernelGGL((chunk_local_kernel<true>), grid, dim3(64 * LOC_WAVES), 0, s, a);
    else
      hipLaunchKernelGGL((chunk_local_kernel<false>), grid, dim3(64 * LOC_WAVES), 0, s, a);
    return check_launch(name);
  }
  if (!workspace || workspace_bytes < l.total)
    return fail(GDN_ERR_WORKSPACE, "%s: workspace %zu bytes < %zu needed", name, workspace_bytes, l.total);
  if (reinterpret_cast<uintptr_t>(workspace) % 256)
    return fail(GDN_ERR_WORKSPACE, "%s: workspace must be 256-byte aligned", name);
  if (nc > 65535) return fail(GDN_ERR_INVALID_ARGUMENT, "%s: %lld chunks exceed one launch", name, (long long)nc);
  const int64_t scan_blocks = static_cast<int64_t>(persist ? 1 : n_seqs) * Hv * (DV / SCAN_COLS);
  if (scan_blocks > 0x7fffffff) return fail(GDN_ERR_INVALID_ARGUMENT, "%s: grid too large", name);
  char *ws = static_cast<char *>(workspace);
  ChunkArgs a{static_cast<const uint16_t *>(q), static_cast<const uint16_t *>(k), static_cast<const uint16_t *>(v),
              q_stride_t, k_stride_t, v_stride_t, gate, h0, h0_idx, h0_rows, hT, hT_idx, hT_rows, o, o_dtype,
              cu_seqlens, n_seqs, T, Hk, Hv, total, scale, l2norm_qk, static_cast<int>(nc), 0, 0,
              reinterpret_cast<int32_t *>(ws + l.chunk_start), reinterpret_cast<u32x4 *>(ws + l.vh),
              reinterpret_cast<float *>(ws + l.Ut),
              reinterpret_cast<float *>(ws + l.carry), reinterpret_cast<int64_t *>(ws + l.seqrec), nullptr};
  // q and k given per v-head (Hk == Hv): the prep checks each chunk's pairs
  // of v-heads for repeated rows and the scan reads one copy of a repeated pair
  if (!persist && Hk == Hv && Hv % 2 == 0) a.dup = reinterpret_cast<int32_t *>(ws + l.dup);
  auto set_segment = [&](int64_t segment) {
    a.seg_begin = static_cast<int>(segment * seg);
    a.seg_end = static_cast<int>(std::min<int64_t>((segment + 1) * seg, nc));
  };
  auto launch_prep = [&](hipStream_t st) {
    hipLaunchKernelGGL(chunk_prep_kernel, dim3(Hv, static_cast<unsigned>(seg)), dim3(256), 0, st, a);
  };
  auto launch_scan = [&](hipStream_t st) {
    if (persist) {
      if (o_dtype == GDN_DTYPE_BF16)
        hipLaunchKernelGGL((chunk_scan_persist_kernel<true>), dim3(static_cast<unsigned>(scan_blocks)),
                           dim3(64 * SCAN_WAVES), 0, st, a);
      else
        hipLaunchKernelGGL((chunk_scan_persist_kernel<false>), dim3(static_cast<unsigned>(scan_blocks)),
                           dim3(64 * SCAN_WAVES), 0, st, a);
      return;
    }
    if (o_dtype == GDN_DTYPE_BF16)
      hipLaunchKernelGGL((chunk_scan_kernel<true>), dim3(static_cast<unsigned>(scan_blocks)),
                         dim3(64 * SCAN_WAVES), 0, st, a);
    else
      hipLaunchKernelGGL((chunk_scan_kernel<false>), dim3(static_cast<unsigned>(scan_blocks)),
                         dim3(64 * SCAN_WAVES), 0, st, a);
  };
  // the chunk table: chunk starts for varlen, per-sequence records for the persistent scan
  // (which computes them itself for a dense batch without slot ids)
  if (cu_seqlens || (persist && (h0_idx || hT_idx)))
    hipLaunchKernelGGL(chunk_table_kernel, dim3(1), dim3(256), 0, s, a);
  const int64_t nseg = seg > 0 ? (nc + seg - 1) / seg : 0;
  if (nseg == 0) {  // only empty sequences: they still pass their state through
    set_segment(0);
    launch_scan(s);
  }
  for (int64_t kseg = 0; kseg < nseg; ++kseg) {  // segment k's scan reads the state carried from k - 1
    set_segment(kseg);
    launch_prep(s);
    launch_scan(s);
  }
  return check_launch(name);
}

}  // namespace
}  // namespace gdn

extern "C" int gdn_chunk_fwd(const void *q, const void *k, const void *v, int qkv_dtype,
                             int64_t q_stride_t, int64_t k_stride_t, int64_t v_stride_t,
                             const float *g, const void *beta, int beta_dtype,
                             const float *h0, const int64_t *h0_idx, int64_t h0_rows,
                             float *hT, const int64_t *hT_idx, int64_t hT_rows,
                             void *o, int o_dtype,
                             const int32_t *cu_seqlens, int32_t n_seqs, int32_t T,
                             int32_t Hk, int32_t Hv, int32_t K, int32_t V,
                             float scale, int l2norm_qk,
                             void *workspace, size_t workspace_bytes, void *stream) {
  const gdn::GateArgs gate{g, beta, beta_dtype, Hv, nullptr, nullptr};
  return gdn::chunk_fwd(q, k, v, qkv_dtype, q_stride_t, k_stride_t, v_stride_t, gate, h0, h0_idx, h0_rows, hT, hT_idx, hT_rows, o,
                        o_dtype, cu_seqlens, n_seqs, T, Hk, Hv, K, V, scale, l2norm_qk, workspace, workspace_bytes,
                        stream, "gdn_chunk_fwd");
}

extern "C" int gdn_chunk_fwd_gated(const void *q, const void *k, const void *v, int qkv_dtype,
                                   int64_t q_stride_t, int64_t k_stride_t, int64_t v_stride_t,
                                   const void *a, const void *b, int ab_dtype, int64_t ab_stride_t,
                                   const float *A_log, const float *dt_bias,
                                   const float *h0, const int64_t *h0_idx, int64_t h0_rows,
                                   float *hT, const int64_t *hT_idx, int64_t hT_rows,
                                   void *o, int o_dtype,
                                   const int32_t *cu_seqlens, int32_t n_seqs, int32_t T,
                                   int32_t Hk, int32_t Hv, int32_t K, int32_t V,
                                   float scale, int l2norm_qk,
                                   void *workspace, size_t workspace_bytes, void *stream) {
  if (!A_log) return gdn::fail(GDN_ERR_INVALID_ARGUMENT, "gdn_chunk_fwd_gated: null A_log");
  const gdn::GateArgs gate{a, b, ab_dtype, ab_stride_t, A_log, dt_bias};
  return gdn::chunk_fwd(q, k, v, qkv_dtype, q_stride_t, k_stride_t, v_stride_t, gate, h0, h0_idx, h0_rows, hT, hT_idx, hT_rows, o,
                        o_dtype, cu_seqlens, n_seqs, T, Hk, Hv, K, V, scale, l2norm_qk, workspace, workspace_bytes,
                        stream, "gdn_chunk_fwd_gated");
}
