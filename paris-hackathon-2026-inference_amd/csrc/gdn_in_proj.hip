// Decode-time input projections of the GDN layer with the causal-conv
// update in the epilogue.
//
// HF's decode step (transformers modeling_qwen3_5_moe.py:443-461) runs four
// skinny GEMMs over the same hidden rows -- in_proj_qkv [2*Hk*K + Hv*V, D],
// in_proj_z [Hv*V, D], in_proj_b / in_proj_a [Hv, D] -- and then
// causal_conv1d_update over the qkv output.  At decode the batch M is small
// (<= 64 rows per workgroup here), so the four GEMMs together are one stream
// of D x (2*Hk*K + 2*Hv*V + 2*Hv) bf16 weights (50.6 MB for the 2048-wide
// Qwen3.5-MoE layer) past a few KiB of activations: bound by HBM, not by the
// matrix cores.  This kernel reads each weight row once, keeps the product
// in registers and applies the conv update (window shift, depthwise taps,
// bias, SiLU) to the qkv columns before anything is written, so the qkv
// projection never round-trips through memory.
//
// Work split (in_proj_xs_kernel): the hidden rows stay in registers, the
// weights stream past them.  Every CU gets a workgroup; its 16 waves split
// K, each holding its K / 16 columns of all 64 rows as MFMA B operands, and
// walk the workgroup's tiles of 16 output columns (3-4 per workgroup for
// the Qwen3.5-MoE layer), each wave multiplying its K / 16 of a tile's
// weight rows as they arrive.  The waves' partial products meet in LDS,
// and waves 0-3 add them in wave order and run the epilogue for one row
// tile each.  Lane (c, g) of a row tile's accumulator holds
// out[16 t + c][col + 4 g .. + 3]: four consecutive channels of one row,
// also the unit of the conv pool ([rows, C, 4] bf16: 32 bytes).
//
// out_proj at decode ([Hv*V -> D], modeling_qwen3_5_moe.py:540: 16.8 MB of
// weights for 64 rows) has only 2048 output columns, so there K is split
// over workgroups (512 of K each, 256 workgroups): each stages its rows'
// 512 columns in LDS by DMA, multiplies them with 64 columns of weights in
// 16 waves (4 column groups x 4 parts of K) and writes its fp32 partial
// block to a workspace; a second small kernel adds the partials in split
// order and writes bf16.  (Letting
// the last workgroup of a column block add them needs agent-scope fences,
// whose L2 writeback and invalidate per workgroup measured 111 us.)
#include <algorithm>
#include <mutex>

#include "gdn_common.h"

namespace gdn {
namespace {

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

constexpr int IP_WAVES = 16;         // waves per workgroup
// GEMV kernels (one or two rows): waves per workgroup.  Smaller workgroups
// spread the weight stream over more CUs.  Measured from HIP graphs over 6
// (in_proj) or 16 (out_proj) weight sets: out_proj at M = 1 5.8 us with 16
// waves per workgroup (64 workgroups), 4.7 / 4.55 / 4.7 us with 8 / 4 / 2;
// in_proj at M = 1 / 2 11.7 / 12.7 us with 16, 11.4 / 12.2 with 8, 12.1 /
// 12.3 with 4; the layer step at B = 1 28.2 us before, 23.9-24.0 us with
// 8 and 4.
constexpr int IN_GEMV_WAVES = 8;
constexpr int IN_GEMV_COLS = 4 * IN_GEMV_WAVES;  // in_proj columns per workgroup
constexpr int OUT_GEMV_WAVES = 4;
constexpr int IP_ROWS = 64;          // hidden rows per workgroup (4 row tiles)
constexpr int IP_OOB = 0x40000000;   // buffer offset past every conv pool: loads read 0, nothing stored
constexpr int IP_GEMV_ROWS = 2;      // up to this many rows: in_proj_gemv_kernel (more spill at K = 2048)
constexpr int IP_COLS = 64;          // n_qkv and n_z come in multiples of this

// Workgroup shape: CG column groups of 16 x KQ parts of K (CG KQ = 16
// waves); a wave holds KS k-steps (of 32) of weights; the hidden rows reach
// LDS in NPH phases, each SP = KS / NPH k-steps of every part: per part 64
// rows of CH = 4 SP chunks of 8 elements (128 KiB at most in all).
template <int CG_, int KQ_, int KS_, int NPH_>
struct ProjShape {
  static constexpr int CG = CG_, KQ = KQ_, KS = KS_, NPH = NPH_;
  static constexpr int COLS = 16 * CG;
  static constexpr int SP = KS / NPH, CH = 4 * SP, RPI = 64 / CH;
  static constexpr int KPART = 32 * KS;
  static constexpr int DMA_PER_WAVE = KQ * CH / IP_WAVES;
  static constexpr int LDS_BLOCKS = KQ * 64 * CH;  // 16-byte entries
  static_assert(CG * KQ == IP_WAVES && KS % NPH == 0 && 64 % CH == 0 && (KQ * CH) % IP_WAVES == 0, "shape");
  static_assert(LDS_BLOCKS * 16 <= 128 * 1024 && KQ * CG * 4 * 64 <= LDS_BLOCKS, "LDS");
};
// out_proj workgroups: 64 columns x 512 of K, or, when K is a multiple of
// 1024, 32 columns x 1024 of K -- half the splits, so half the fp32
// partial sums written and read back (2 MiB each way instead of 4 for the
// Qwen3.5-MoE layer at 64 rows), for twice the staged rows per workgroup
using OutProjShape = ProjShape<4, 4, 4, 1>;
using OutProjShapeWide = ProjShape<2, 8, 4, 1>;
constexpr int OP_KSPAN = OutProjShape::KQ * OutProjShape::KPART;            // 512
constexpr int OP_KSPAN_WIDE = OutProjShapeWide::KQ * OutProjShapeWide::KPART;  // 1024
inline int op_kspan(int K) { return K % OP_KSPAN_WIDE == 0 ? OP_KSPAN_WIDE : OP_KSPAN; }
constexpr int OP_MAX_SPLIT = 16;                  // workgroups per column block (K <= 8192)
constexpr int OP_RED_NT = 256;                    // threads per workgroup of the partials' sum

struct InProjArgs {
  const uint16_t *x;  // [M, K] bf16, row stride xs elements
  int64_t xs;
  const uint16_t *w[4];  // qkv, z, b, a: [n[i], K] bf16, rows contiguous
  int n[4];
  int blocks_qkv, blocks_z;  // column blocks of qkv and z; then one block for b, a (<= 32 columns each)
  int M, K;
  const uint16_t *cw, *cb;  // conv taps [n[0], 4] bf16, bias [n[0]] bf16 or null
  uint16_t *pool;           // conv windows [rows, n[0], 4] bf16, updated in place
  const int64_t *idx;
  int64_t rows;
  uint16_t *y[4];  // conv(qkv) [M, n[0]], z [M, n[1]], b [M, n[2]], a [M, n[3]]
  int silu;
};

__device__ __forceinline__ f32x4_t mfma16(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                 c, 0, 0, 0);
}

__device__ __forceinline__ float silu_f(float v) { return v / (1.f + expf(-v)); }

__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16_bits(lo)) | (static_cast<uint32_t>(f32_to_bf16_bits(hi)) << 16);
}

// This wave's weights, KS k-steps of its part: lane (r, g) of k-step s
// holds W[col + r][k0 + 32 s + 8 g .. + 8].  Rows past the matrix read as zero.
template <int KS>
__device__ __forceinline__ void load_w(u32x4_t (&wr)[KS], __amdgpu_buffer_rsrc_t rw, int k0, int K, int lane) {
  const int voff = ((lane & 15) * K + 8 * (lane >> 4)) * 2;
#pragma unroll
  for (int s = 0; s < KS; ++s) wr[s] = __builtin_amdgcn_raw_buffer_load_b128(rw, voff, (k0 + 32 * s) * 2, 0);
}

// Phase h of every part's hidden rows into LDS by DMA: part q's k-steps
// h SP .. h SP + SP - 1, i.e. CH chunks of 8 elements per row.  LDS holds a
// part row-major, 64 rows of CH chunks, chunk p of row r at position
// p ^ (r % CH) (so that the 16 rows an MFMA operand read touches fall in
// 16 different bank groups).  One DMA instruction fills 64 consecutive
// positions, i.e. 64 / CH whole rows, each lane fetching the chunk its
// position holds: contiguous global reads, 1 KiB per instruction.  Wave w
// copies instructions w, w + 16, ...  Rows past M read as zero.
template <class S>
__device__ __forceinline__ void dma_x(u32x4_t *xl, const uint16_t *xbase, int xbytes, int64_t xs, int h, int wave,
                                      int lane) {
  const auto rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(xbase), 0, xbytes, BUF_DWORD3);
#pragma unroll
  for (int i = 0; i < S::DMA_PER_WAVE; ++i) {
    const int j = wave + IP_WAVES * i;  // part j / CH, rows RPI (j % CH) ..
    const int q = j / S::CH;
    const int r = S::RPI * (j % S::CH) + lane / S::CH, pos = lane % S::CH;
    const int voff = static_cast<int>((r * xs + 8 * (pos ^ (r % S::CH))) * 2);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, xl + j * 64, 16, voff, (q * S::KPART + h * 32 * S::SP) * 2, 0, 0);
  }
}

// Phase PH of this wave's part against its staged rows (all four row tiles):
// B operand of row tile t, k-step s at lane (c, g) = row 16 t + c, chunk 4 s + g.
template <class S, int PH>
__device__ __forceinline__ void phase_mfma(f32x4_t (&acc)[4], const u32x4_t (&wr)[S::KS], const u32x4_t *xq,
                                           int lane) {
  const int c = lane & 15, g = lane >> 4;
#pragma unroll
  for (int s = 0; s < S::SP; ++s)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int r = 16 * t + c;
      acc[t] = mfma16(wr[PH * S::SP + s], xq[r * S::CH + ((4 * s + g) ^ (r % S::CH))], acc[t]);
    }
}

// s_waitcnt operand: vmcnt <= n, lgkmcnt and expcnt unconstrained
constexpr int ip_vmcnt(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }

// A workgroup barrier that orders LDS only: __syncthreads' fence would also
// wait for every outstanding global load and store (the next tile's weights,
// the epilogue's stores), which no other wave reads.  Waits for LDS DMA are
// explicit (ip_vmcnt) where they are needed.
__device__ __forceinline__ void ip_lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// After phase 0's copies and the weights were issued (and POST more loads
// after them): the phases, then the parts' partial sums added in LDS in part
// order.  Returns, for waves of part kq < 4, row tile kq of their column
// group (rows 16 kq + c, columns 4 g .. 4 g + 3 of the group at lane (c, g)).
// copy(h) issues phase h's copies (the kernel's dma_x on its LDS buffer).
template <class S, int POST, class Copy>
__device__ __forceinline__ f32x4_t proj_phases(u32x4_t *xl, const u32x4_t (&wr)[S::KS], const Copy &copy, int wave,
                                               int lane) {
  const int cg = wave % S::CG, kq = wave / S::CG;
  f32x4_t acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const u32x4_t *xq = xl + kq * (64 * S::CH);
  __builtin_amdgcn_s_waitcnt(ip_vmcnt(S::KS + POST));  // this wave's copies landed (the weights may still fly)
  __syncthreads();
  phase_mfma<S, 0>(acc, wr, xq, lane);
#pragma unroll
  for (int h = 1; h < S::NPH; ++h) {
    __syncthreads();  // the previous phase is consumed: the next into the same buffer
    copy(h);
    __builtin_amdgcn_s_waitcnt(ip_vmcnt(0));
    __syncthreads();
    if (h == 1) phase_mfma<S, 1>(acc, wr, xq, lane);
    if constexpr (S::NPH > 2) {
      if (h == 2) phase_mfma<S, 2>(acc, wr, xq, lane);
      if (h == 3) phase_mfma<S, 3>(acc, wr, xq, lane);
    }
  }
  // part partials through LDS (the rows' buffer, once every wave is done with it)
  __syncthreads();
  f32x4_t *red = reinterpret_cast<f32x4_t *>(xl);  // [part][column group][row tile][lane]
#pragma unroll
  for (int t = 0; t < 4; ++t) red[((kq * S::CG + cg) * 4 + t) * 64 + lane] = acc[t];
  __syncthreads();
  f32x4_t o = {0.f, 0.f, 0.f, 0.f};
  if (kq < 4) {
    o = red[(cg * 4 + kq) * 64 + lane];
#pragma unroll
    for (int q = 1; q < S::KQ; ++q) o += red[((q * S::CG + cg) * 4 + kq) * 64 + lane];
  }
  return o;
}

// Conv update of one row's 4 consecutive qkv channels n .. n + 3 (the conv
// update kernel's arithmetic: fp32, bias first, taps oldest first): o the
// projection (fp32 sums, rounded to bf16 as the nn.Linear output), w01 / w23
// the taps of channels n, n + 1 / n + 2, n + 3, bias4 their bf16 biases,
// win0 / win1 their windows (oldest first).  Writes y_qkv and, unless woff
// is IP_OOB, the advanced windows at byte offset woff of the pool.
__device__ __forceinline__ void conv_epilogue(const InProjArgs &a, const f32x4_t &o, const u32x4_t &w01,
                                              const u32x4_t &w23, uint64_t bias4, const u32x4_t &win0,
                                              const u32x4_t &win1, int woff, int me, int n) {
  float y[4];
  uint32_t nw[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const u32x4_t &tv = e < 2 ? w01 : w23;
    const uint32_t tlo = tv[2 * (e & 1)], thi = tv[2 * (e & 1) + 1];
    const u32x4_t &v = e < 2 ? win0 : win1;
    const uint32_t lo = v[2 * (e & 1)], hi = v[2 * (e & 1) + 1];
    const uint16_t xb = f32_to_bf16_bits(o[e]);
    float acc_c = bf16_bits_to_f32(static_cast<uint16_t>(bias4 >> (16 * e)));
    acc_c += bf16_bits_to_f32(tlo & 0xffffu) * bf16_bits_to_f32(lo >> 16);
    acc_c += bf16_bits_to_f32(tlo >> 16) * bf16_bits_to_f32(hi & 0xffffu);
    acc_c += bf16_bits_to_f32(thi & 0xffffu) * bf16_bits_to_f32(hi >> 16);
    acc_c += bf16_bits_to_f32(thi >> 16) * bf16_bits_to_f32(xb);
    y[e] = a.silu ? silu_f(acc_c) : acc_c;
    nw[2 * e] = (lo >> 16) | (hi << 16);                            // s1 | s2
    nw[2 * e + 1] = (hi >> 16) | (static_cast<uint32_t>(xb) << 16);  // s3 | x
  }
  if (woff != IP_OOB) {
    u32x4_t *st = reinterpret_cast<u32x4_t *>(reinterpret_cast<char *>(a.pool) + woff);
    st[0] = u32x4_t{nw[0], nw[1], nw[2], nw[3]};
    st[1] = u32x4_t{nw[4], nw[5], nw[6], nw[7]};
  }
  uint2 *yp = reinterpret_cast<uint2 *>(a.y[0] + static_cast<int64_t>(me) * a.n[0] + n);
  *yp = make_uint2(pack2(y[0], y[1]), pack2(y[2], y[3]));
}

// ---------------------------------------------------------------------------
// Input projections, rows held in registers ("x-stationary").
//
// The qkv and z matrices are cut into tiles of 16 output columns (768 tiles
// for the Qwen3.5-MoE layer); workgroup b of G takes tiles b, b + G, ...
// (G = max(256, tiles / 4), so every CU works and a workgroup has at most
// XS_MAX_TILES).  The b and a projections (64 columns there) are not tiled:
// as 4 more tiles they gave 4 workgroups a fourth tile that set the
// kernel's end.  Workgroup b instead computes columns b, b + G, ... of
// [b | a] as one-column products (an MFMA A operand whose other 15 rows
// are zero) from the hidden rows already in its registers and the column's
// weight row fetched into LDS at the start, in the time waves 4-15 wait for
// the first tile's epilogue; wave 4 adds the waves' partial sums in wave
// order -- the tile path's arithmetic, so the values are the same.  Its 16 waves split K: wave w holds
// K / 16 columns of all 64 hidden rows as MFMA B operands in registers
// (64 VGPRs at K = 2048), loaded once, and streams the matching K / 16 of
// each tile's 16 weight rows, the next tile's requested as soon as the
// current one is multiplied.  The 16 waves' partial
// products of a tile meet in LDS; wave t < 4 adds them in wave order for row
// tile t and runs the epilogue (the conv update for qkv columns, a bf16
// store otherwise) from conv windows, taps and bias that LDS DMA fetched
// at the start.  Per CU: the hidden rows once (256 KiB at K = 2048, L2
// hits after the first) and 3-4 tiles of weights (64 KiB each).
constexpr int XS_WAVES = 16;
constexpr int XS_MAX_TILES = 4;
constexpr int XS_MIN_WGS = 256;  // MI355X CUs
constexpr int XS_BA_MAX = 2;     // b / a columns per workgroup (G >= 32 for the 64 of Qwen3.5-MoE)
constexpr int XS_K_MAX = 2048;   // the largest K built

struct XsTile {
  int mat, col, live;  // matrix (0 qkv, 1 z, 2 b, 3 a), first column, columns in the matrix (<= 16)
};

__device__ __forceinline__ XsTile xs_tile(const InProjArgs &a, const int (&tiles)[4], int j) {
  XsTile t;
  int m = 0;
  while (m < 3 && j >= tiles[m]) {
    j -= tiles[m];
    ++m;
  }
  // (uniform values: readfirstlane keeps the buffer descriptors in SGPRs)
  t.mat = __builtin_amdgcn_readfirstlane(m);
  t.col = __builtin_amdgcn_readfirstlane(16 * j);
  const int n = t.mat == 0 ? a.n[0] : t.mat == 1 ? a.n[1] : t.mat == 2 ? a.n[2] : a.n[3];
  t.live = __builtin_amdgcn_readfirstlane(max(0, min(16, n - t.col)));
  return t;
}

// The b / a columns: this wave's K slice of each column's dot products with
// the 64 rows (lane (c, 0) of row tile t ends with row 16 t + c in element 0),
// into bared; then wave 4 adds the waves' partials per row, in wave order.
template <int NW, int KSW>
__device__ __forceinline__ void xs_ba_partials(const u32x4_t (*baw)[XS_K_MAX / 8], float (*bared)[NW][64],
                                               const u32x4_t (&xr)[4][KSW], int nbc, int kw, int wave, int lane) {
  const int c = lane & 15, g = lane >> 4;
  for (int ci = 0; ci < nbc; ++ci) {
    f32x4_t acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KSW; ++s) {
      const u32x4_t wf = c == 0 ? baw[ci][kw / 8 + 4 * s + g] : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[t] = mfma16(wf, xr[t][s], acc[t]);
    }
    if (g == 0) {
#pragma unroll
      for (int t = 0; t < 4; ++t) bared[ci][wave][16 * t + c] = acc[t][0];
    }
  }
}

template <int NW>
__device__ __forceinline__ void xs_ba_finish(const InProjArgs &a, const float (*bared)[NW][64], int nbc, int G, int m0,
                                             int lane) {  // wave 4, lane = row
  for (int ci = 0; ci < nbc; ++ci) {
    float o = bared[ci][0][lane];
    for (int q = 1; q < NW; ++q) o += bared[ci][q][lane];
    const int jj = static_cast<int>(blockIdx.x) + G * ci;
    const bool is_b = jj < a.n[2];
    const int nmat = is_b ? a.n[2] : a.n[3];
    if (m0 + lane < a.M)
      (is_b ? a.y[2] : a.y[3])[static_cast<int64_t>(m0 + lane) * nmat + (is_b ? jj : jj - a.n[2])] = f32_to_bf16_bits(o);
  }
}

// NW waves, KSW k-steps (of 32) per wave: K = NW * 32 * KSW.
template <int NW, int KSW>
__global__ __launch_bounds__(64 * NW) void in_proj_xs_kernel(InProjArgs a) {
  constexpr int K = NW * 32 * KSW;
  static_assert(NW >= 5, "waves 0-3 run the epilogue, wave 4 fetches the taps");
  __shared__ f32x4_t red[NW][4][64];                       // partial products of one tile
  __shared__ u32x4_t win[XS_MAX_TILES][4][2][64];          // conv windows by tile, row tile, half, lane: 32 KiB
  __shared__ u32x4_t tap[XS_MAX_TILES][64];                // lanes 0-7 taps (2 channels each), 8-9 bias
  // (a fixed bound: with the bound K / 8 on this LDS-DMA target, hipcc emitted
  // no host launch stub for the kernel and the library failed to load)
  static_assert(K <= XS_K_MAX, "K");
  __shared__ u32x4_t baw[XS_BA_MAX][XS_K_MAX / 8];         // weight rows of this workgroup's b / a columns
  __shared__ float bared[XS_BA_MAX][NW][64];               // their partial sums by wave and row
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, g = lane >> 4;
  const int m0 = blockIdx.y * IP_ROWS;
  const int mb = min(IP_ROWS, a.M - m0);
  const int tiles[4] = {(a.n[0] + 15) / 16, (a.n[1] + 15) / 16, 0, 0};  // b and a: columns, below
  const int ntiles = tiles[0] + tiles[1];
  const int G = gridDim.x;
  const int nt = __builtin_amdgcn_readfirstlane((ntiles - static_cast<int>(blockIdx.x) + G - 1) / G);  // <= XS_MAX_TILES
  // this workgroup's columns of [b | a]: blockIdx.x + G ci, ci < nbc (<= XS_BA_MAX: checked on the host)
  const int nba = a.n[2] + a.n[3];
  const int nbc = __builtin_amdgcn_readfirstlane(min(XS_BA_MAX, (nba - static_cast<int>(blockIdx.x) + G - 1) / G));
  // this wave's columns of K: part (wave + blockIdx.x) % NW, so that the CUs
  // (all reading the same rows of x from L2) do not all request the same
  // addresses at the same moment
  const int kw = ((wave + static_cast<int>(blockIdx.x)) % NW) * 32 * KSW;

  // slot id of the row this lane finishes (waves 0-3: row tile = wave)
  const int me = m0 + 16 * wave + c;
  const auto ri = __builtin_amdgcn_make_buffer_rsrc(const_cast<int64_t *>(a.idx), 0, a.idx ? a.M * 8 : 0, BUF_DWORD3);
  uint64_t id_raw = 0;
  if (wave < 4) id_raw = __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(ri, min(me, a.M - 1) * 8, 0, 0));
  __builtin_amdgcn_sched_barrier(0);

  // the hidden rows: B operand of row tile t, k-step s at lane (c, g) = row 16 t + c, k = kw + 32 s + 8 g.
  // Every CU reads the same rows from L2, where a load of 16 rows x 64 bytes
  // (the fragment layout) streams at about half the rate of a contiguous
  // 1 KiB: so they are read contiguously -- instruction q of row tile t holds
  // rows 16 t + RPI q .., lane l row-in-tile RPI q + l / CPR, 16-byte chunk
  // l % CPR of the wave's 64 KSW bytes of the row -- and put in the fragment
  // layout through a wave-private LDS scratch (the tile partials' region,
  // unused until the first tile is multiplied), chunk ch of row r at slot
  // r CPR + (ch ^ r % CPR) so that neither side conflicts on banks.
  constexpr int CPR = 4 * KSW, RPI = 64 / CPR;  // 16-byte chunks per row slice, rows per instruction (KSW of them per tile)
  const auto rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(a.x) + static_cast<int64_t>(m0) * a.xs, 0,
                                                    static_cast<int>(((mb - 1) * a.xs + K) * 2), BUF_DWORD3);
  u32x4_t xr[4][KSW];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int q = 0; q < KSW; ++q)
      xr[t][q] = __builtin_amdgcn_raw_buffer_load_b128(
          rx, static_cast<int>(((16 * t + RPI * q + lane / CPR) * a.xs + kw + 8 * (lane % CPR)) * 2), 0, 0);
  // a tile's weights: lane (r, g) of k-step s holds W[col + r][kw + 32 s + 8 g .. + 8] (rows past the matrix: 0)
  auto load_tile = [&](u32x4_t (&w)[KSW], int i) {
    const XsTile t = xs_tile(a, tiles, static_cast<int>(blockIdx.x) + G * i);
    const uint16_t *wm = t.mat == 0 ? a.w[0] : t.mat == 1 ? a.w[1] : t.mat == 2 ? a.w[2] : a.w[3];
    const auto rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(wm) + static_cast<int64_t>(t.col) * K, 0,
                                                      t.live * K * 2, BUF_DWORD3);
    const int voff = (c * K + kw + 8 * g) * 2;
#pragma unroll
    for (int s = 0; s < KSW; ++s) w[s] = __builtin_amdgcn_raw_buffer_load_b128(rw, voff, 64 * s, 0);
  };
  u32x4_t w[KSW];
  load_tile(w, 0);
  __builtin_amdgcn_sched_barrier(0);

  // conv windows (waves 0-3, their row tile) and taps / bias (wave 4) of the qkv tiles into LDS
  const int64_t id = a.idx ? static_cast<int64_t>(id_raw) : me;  // pool_row's rule
  int wbase = -1;  // byte offset of this lane's row in the pool, -1: no window (waves 0-3)
  if (wave < 4) {
    // a row whose slot id repeats an earlier row's selects no window
    // (the ids read 64 at a time, one per lane, then broadcast lane by lane:
    // one id per iteration from memory was a dependent load per earlier row)
    bool rep = false;
    if (a.idx) {
      const int mlast = min(m0 + 16 * wave + 15, a.M - 1);  // the wave's last row
      for (int base = 0; base < mlast; base += 64) {
        const int64_t v = __builtin_bit_cast(int64_t, __builtin_amdgcn_raw_buffer_load_b64(
                              ri, min(base + lane, a.M - 1) * 8, 0, 0));
        const int jn = min(64, mlast - base);
        for (int j = 0; j < jn; ++j) {
          const int64_t vj = static_cast<int64_t>(
              (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v >> 32), j))) << 32) |
              static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), j)));
          rep |= base + j < me && vj == id;
        }
      }
    }
    const bool has = me < a.M && !rep && id >= 0 && id < a.rows;
    wbase = has ? static_cast<int>(id * a.n[0] * 8) : -1;  // (< IP_OOB: checked on the host)
    const auto rp = __builtin_amdgcn_make_buffer_rsrc(a.pool, 0, static_cast<int>(a.rows * a.n[0] * 8), BUF_DWORD3);
    for (int i = 0; i < nt; ++i) {
      const XsTile t = xs_tile(a, tiles, static_cast<int>(blockIdx.x) + G * i);
      if (t.mat != 0) continue;
      const int woff = wbase >= 0 ? wbase + (t.col + 4 * g) * 8 : IP_OOB;
#pragma unroll
      for (int h = 0; h < 2; ++h) __builtin_amdgcn_raw_ptr_buffer_load_lds(rp, &win[i][wave][h][0], 16, woff, 16 * h, 0, 0);
    }
  } else if (wave == 4) {
    const auto rc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(a.cw), 0, a.n[0] * 8, BUF_DWORD3);
    const auto rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(a.cb), 0, a.cb ? a.n[0] * 2 : 0, BUF_DWORD3);
    for (int i = 0; i < nt; ++i) {
      const XsTile t = xs_tile(a, tiles, static_cast<int>(blockIdx.x) + G * i);
      if (t.mat != 0) continue;
      if (lane < 8)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rc, &tap[i][0], 16, (t.col + 2 * lane) * 8, 0, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, &tap[i][0], 16, lane < 10 ? (t.col + 8 * (lane - 8)) * 2 : IP_OOB, 0,
                                                 0, 0);
    }
    for (int ci = 0; ci < nbc; ++ci) {  // the b / a weight rows, 1 KiB per instruction
      const int jj = static_cast<int>(blockIdx.x) + G * ci;
      const uint16_t *wrow = jj < a.n[2] ? a.w[2] + static_cast<int64_t>(jj) * K : a.w[3] + static_cast<int64_t>(jj - a.n[2]) * K;
      const auto rr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(wrow), 0, K * 2, BUF_DWORD3);
#pragma unroll
      for (int p = 0; p < K / 512; ++p)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, &baw[ci][64 * p], 16, (512 * p + 8 * lane) * 2, 0, 0, 0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  {  // the rows into the fragment layout, one row tile at a time, in place
    u32x4_t *scr = reinterpret_cast<u32x4_t *>(&red[wave][0][0]);  // 16 CPR slots of this wave
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int q = 0; q < KSW; ++q) {
        const int r = RPI * q + lane / CPR, ch = lane % CPR;
        scr[r * CPR + (ch ^ (r % CPR))] = xr[t][q];
      }
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int s2 = 0; s2 < KSW; ++s2) xr[t][s2] = scr[c * CPR + ((4 * s2 + g) ^ (c % CPR))];
      __builtin_amdgcn_wave_barrier();
    }
  }
  auto ba_partials = [&]() { xs_ba_partials<NW, KSW>(baw, bared, xr, nbc, kw, wave, lane); };
  auto ba_finish = [&]() { xs_ba_finish<NW>(a, bared, nbc, G, m0, lane); };

  for (int i = 0; i < nt; ++i) {
    f32x4_t acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KSW; ++s)
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[t] = mfma16(w[s], xr[t][s], acc[t]);
    // the next tile's weights into the same registers, in flight during the
    // epilogue (a second buffer does not fit beside the rows of x)
    const bool more = i + 1 < nt;
    if (more) load_tile(w, i + 1);
#pragma unroll
    for (int t = 0; t < 4; ++t) red[wave][t][lane] = acc[t];
    if (i == 0) {  // the DMAs landed (only the weights just requested may still fly)
      if (more)
        __builtin_amdgcn_s_waitcnt(ip_vmcnt(KSW));
      else
        __builtin_amdgcn_s_waitcnt(ip_vmcnt(0));
    }
    ip_lds_barrier();
    if (i == 0 && wave >= 4) ba_partials();  // (waves 0-3 after their epilogue)
    if (i == 1 && wave == 4) ba_finish();
    if (wave < 4) {
      // row tile `wave`: lane (c, g) holds row me, columns col + 4 g .. + 3; the
      // partials in wave order, four read at a time (the registers hold x)
      f32x4_t o = red[0][wave][lane];
#pragma unroll 1
      for (int q0 = 1; q0 < NW; q0 += 4) {
        const f32x4_t p0 = red[q0][wave][lane];
        const f32x4_t p1 = q0 + 1 < NW ? red[q0 + 1][wave][lane] : f32x4_t{0.f, 0.f, 0.f, 0.f};
        const f32x4_t p2 = q0 + 2 < NW ? red[q0 + 2][wave][lane] : f32x4_t{0.f, 0.f, 0.f, 0.f};
        const f32x4_t p3 = q0 + 3 < NW ? red[q0 + 3][wave][lane] : f32x4_t{0.f, 0.f, 0.f, 0.f};
        o += p0;
        if (q0 + 1 < NW) o += p1;
        if (q0 + 2 < NW) o += p2;
        if (q0 + 3 < NW) o += p3;
      }
      const XsTile t = xs_tile(a, tiles, static_cast<int>(blockIdx.x) + G * i);
      const int n = t.col + 4 * g;
      if (4 * g < t.live && me < a.M) {
        if (t.mat == 0) {
          const u32x4_t w01 = tap[i][2 * g], w23 = tap[i][2 * g + 1];
          const u32x4_t bb = tap[i][8 + (g >> 1)];
          const uint64_t bias4 = (g & 1) ? (static_cast<uint64_t>(bb[3]) << 32 | bb[2])
                                         : (static_cast<uint64_t>(bb[1]) << 32 | bb[0]);
          const int woff = wbase >= 0 ? wbase + n * 8 : IP_OOB;
          conv_epilogue(a, o, w01, w23, bias4, win[i][wave][0][lane], win[i][wave][1][lane], woff, me, n);
        } else {
          uint16_t *ymat = t.mat == 1 ? a.y[1] : t.mat == 2 ? a.y[2] : a.y[3];
          const int nmat = t.mat == 1 ? a.n[1] : t.mat == 2 ? a.n[2] : a.n[3];
          uint2 *yp = reinterpret_cast<uint2 *>(ymat + static_cast<int64_t>(me) * nmat + n);
          *yp = make_uint2(pack2(o[0], o[1]), pack2(o[2], o[3]));
        }
      }
    }
    if (i == 0 && wave < 4) ba_partials();
    ip_lds_barrier();  // the partials are consumed: the next tile's may go in
  }
  if (nt == 0 && nbc > 0) {  // no tile: the b / a columns alone
    __builtin_amdgcn_s_waitcnt(ip_vmcnt(0));
    ip_lds_barrier();
    ba_partials();
    ip_lds_barrier();
  }
  if (nt <= 1 && wave == 4) ba_finish();
}

// One or two rows (the smallest decode batches): the projection is a GEMV stream.
// Workgroup = IN_GEMV_WAVES waves over 4 IN_GEMV_WAVES columns of one matrix (b and
// a: 8 waves each); wave w takes columns 4 w .. 4 w + 3 and reads
// each of its weight rows as K / 512 contiguous 1 KiB loads (lane l: 16
// bytes at 16 l of every KiB), all issued at the start; the rows of x sit in
// registers in the same lane layout.  Each lane sums its products in fp32,
// a wave reduction gives the dot products, and lane c + 4 m writes (row m,
// column c), through the same conv epilogue as the MFMA kernel.
template <int MR, int KB>  // MR rows (1, 2); KB = K / 512
__global__ __launch_bounds__(64 * IN_GEMV_WAVES, 4) void in_proj_gemv_kernel(InProjArgs a) {  // 4 waves per SIMD: <= 128 VGPRs
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int mat, col;
  const int bid = blockIdx.x;
  if (bid < a.blocks_qkv) {
    mat = 0;
    col = bid * IN_GEMV_COLS + 4 * wave;
  } else if (bid < a.blocks_qkv + a.blocks_z) {
    mat = 1;
    col = (bid - a.blocks_qkv) * IN_GEMV_COLS + 4 * wave;
  } else {  // b then a, 8 waves of 4 columns each
    const int w = (bid - a.blocks_qkv - a.blocks_z) * IN_GEMV_WAVES + wave;
    mat = 2 + (w >> 3);
    col = 4 * (w & 7);
  }
  mat = __builtin_amdgcn_readfirstlane(mat);
  col = __builtin_amdgcn_readfirstlane(col);
  const uint16_t *wmat = mat == 0 ? a.w[0] : mat == 1 ? a.w[1] : mat == 2 ? a.w[2] : a.w[3];
  const int nmat = mat == 0 ? a.n[0] : mat == 1 ? a.n[1] : mat == 2 ? a.n[2] : a.n[3];
  if (col >= nmat) return;  // (b / a narrower than 32 columns; nmat is a multiple of 4)
  const int K = KB * 512;
  const auto rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(wmat) + static_cast<int64_t>(col) * K, 0,
                                                    4 * K * 2, BUF_DWORD3);
  const auto rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(a.x), 0,
                                                    static_cast<int>(((a.M - 1) * a.xs + K) * 2), BUF_DWORD3);
  u32x4_t wv[4][KB], xv[MR][KB];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int i = 0; i < KB; ++i)
      xv[m][i] = __builtin_amdgcn_raw_buffer_load_b128(rx, static_cast<int>((m * a.xs + 512 * i + 8 * lane) * 2), 0, 0);
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int i = 0; i < KB; ++i)
      wv[c][i] = __builtin_amdgcn_raw_buffer_load_b128(rw, (c * K + 512 * i + 8 * lane) * 2, 0, 0);
  float dot[4][MR];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < KB; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t wp = wv[c][i][e], xp = xv[m][i][e];
          s += bf16_bits_to_f32(wp & 0xffffu) * bf16_bits_to_f32(xp & 0xffffu);
          s += bf16_bits_to_f32(wp >> 16) * bf16_bits_to_f32(xp >> 16);
        }
      dot[c][m] = wave_sum(s);
    }
  // lane c + 4 m finishes (row m, column col + c)
  const int c = lane & 3, m = lane >> 2;
  if (m >= MR || m >= a.M) return;
  float o = 0.f;
#pragma unroll
  for (int cc = 0; cc < 4; ++cc)
#pragma unroll
    for (int mm = 0; mm < MR; ++mm)
      if (cc == c && mm == m) o = dot[cc][mm];
  const int n = col + c;
  if (mat == 0) {
    const int64_t id = a.idx ? a.idx[m] : m;  // pool_row's rule
    const bool live = id >= 0 && id < a.rows && !(m == 1 && a.idx && a.idx[0] == id);  // (row 1 repeating row 0's slot: none)
    uint16_t win[4] = {0, 0, 0, 0};
    uint16_t *wp = a.pool + (live ? (id * a.n[0] + n) * 4 : 0);
    if (live)
#pragma unroll
      for (int j = 0; j < 4; ++j) win[j] = wp[j];
    const uint16_t xb = f32_to_bf16_bits(o);
    float acc_c = a.cb ? bf16_bits_to_f32(a.cb[n]) : 0.f;
#pragma unroll
    for (int j = 0; j < 3; ++j) acc_c += bf16_bits_to_f32(a.cw[n * 4 + j]) * bf16_bits_to_f32(win[j + 1]);
    acc_c += bf16_bits_to_f32(a.cw[n * 4 + 3]) * bf16_bits_to_f32(xb);
    const float y = a.silu ? silu_f(acc_c) : acc_c;
    if (live) {
      wp[0] = win[1];
      wp[1] = win[2];
      wp[2] = win[3];
      wp[3] = xb;
    }
    a.y[0][static_cast<int64_t>(m) * a.n[0] + n] = f32_to_bf16_bits(y);
  } else {
    uint16_t *ymat = mat == 1 ? a.y[1] : mat == 2 ? a.y[2] : a.y[3];
    ymat[static_cast<int64_t>(m) * nmat + n] = f32_to_bf16_bits(o);
  }
}

template <int MR>
void launch_gemv(const InProjArgs &args, unsigned gx, int kb, hipStream_t s) {
  if (kb == 2)
    hipLaunchKernelGGL((in_proj_gemv_kernel<MR, 2>), dim3(gx), dim3(64 * IN_GEMV_WAVES), 0, s, args);
  else
    hipLaunchKernelGGL((in_proj_gemv_kernel<MR, 4>), dim3(gx), dim3(64 * IN_GEMV_WAVES), 0, s, args);
}

struct OutProjArgs {
  const uint16_t *x;  // [M, K] bf16, row stride xs elements
  int64_t xs;
  const uint16_t *w;  // [N, K] bf16, rows contiguous
  int M, K, N;
  int split, ncb;     // workgroups per column block (K / 512 or K / 1024), column blocks (N / 64 or N / 32)
  float *part;        // [split][row blocks][64][N] fp32 partial sums
  uint16_t *y;        // [M, N] bf16, row stride ys elements
  int64_t ys;
};

// Partial block (64 rows x S::COLS columns, S::KQ S::KPART of K) of
// workgroup (column block cb, split sp, row block blockIdx.y).  A column
// block's split workgroups are bid = cb + ncb sp.
template <class S>
__global__ __launch_bounds__(64 * IP_WAVES) void out_proj_partial_kernel(OutProjArgs a) {
  constexpr int KSPAN = S::KQ * S::KPART;
  __shared__ u32x4_t xl[S::LDS_BLOCKS];  // the rows' KSPAN columns of K: 64 or 128 KiB
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cg = wave % S::CG, kq = wave / S::CG;
  const int cb = blockIdx.x % a.ncb, sp = blockIdx.x / a.ncb;
  const int mblk = blockIdx.y, nmb = gridDim.y;
  const int m0 = mblk * IP_ROWS;
  const int mb = min(IP_ROWS, a.M - m0);
  const int col = cb * S::COLS + 16 * cg;
  const int k0 = sp * KSPAN;
  const auto rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(a.w) + static_cast<int64_t>(col) * a.K, 0,
                                                    16 * a.K * 2, BUF_DWORD3);
  const uint16_t *xbase = a.x + static_cast<int64_t>(m0) * a.xs + k0;
  const int xbytes = static_cast<int>(((mb - 1) * a.xs + (a.K - k0)) * 2);  // rows past M read as zero

  dma_x<S>(xl, xbase, xbytes, a.xs, 0, wave, lane);
  __builtin_amdgcn_sched_barrier(0);
  u32x4_t wr[S::KS];
  load_w<S::KS>(wr, rw, k0 + kq * S::KPART, a.K, lane);
  __builtin_amdgcn_sched_barrier(0);
  const f32x4_t o = proj_phases<S, 0>(xl, wr, [](int) {}, wave, lane);

  // lane (c, g) of wave (cg, kq), kq < 4: row 16 kq + c, columns col + 4 g .. + 3
  // (waves of the further K parts hold no row tile: with KQ = 8 they would
  // address rows 64-127, the next block's)
  if (kq >= 4) return;
  const int c = lane & 15, g = lane >> 4;
  const int64_t prow = static_cast<int64_t>(sp * nmb + mblk) * IP_ROWS + 16 * kq + c;
  *reinterpret_cast<f32x4_t *>(a.part + prow * a.N + col + 4 * g) = o;
}

// y[m][4 i .. 4 i + 3] = bf16(sum over splits, in split order): one thread
// per 4 outputs.  SPLIT > 0: that many splits, all loads issued before the
// adds; SPLIT = 0: a.split of them, one at a time.
template <int SPLIT>
__global__ __launch_bounds__(OP_RED_NT) void out_proj_sum_kernel(OutProjArgs a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * OP_RED_NT + threadIdx.x;
  const int n4 = a.N / 4;
  if (i >= static_cast<int64_t>(a.M) * n4) return;
  const int m = static_cast<int>(i / n4), n = 4 * static_cast<int>(i % n4);
  const int64_t pstride = static_cast<int64_t>((a.M + IP_ROWS - 1) / IP_ROWS) * IP_ROWS * a.N;
  const float *p = a.part + static_cast<int64_t>(m) * a.N + n;
  f32x4_t t;
  if constexpr (SPLIT > 0) {
    f32x4_t v[SPLIT];
#pragma unroll
    for (int q = 0; q < SPLIT; ++q) v[q] = *reinterpret_cast<const f32x4_t *>(p + q * pstride);
    t = v[0];
#pragma unroll
    for (int q = 1; q < SPLIT; ++q) t += v[q];
  } else {
    t = *reinterpret_cast<const f32x4_t *>(p);
    for (int q = 1; q < a.split; ++q) t += *reinterpret_cast<const f32x4_t *>(p + q * pstride);
  }
  *reinterpret_cast<uint2 *>(a.y + static_cast<int64_t>(m) * a.ys + n) = make_uint2(pack2(t[0], t[1]), pack2(t[2], t[3]));
}

// One row: a GEMV stream in one kernel (no partial sums).  Workgroup =
// OUT_GEMV_WAVES waves over 2 OUT_GEMV_WAVES columns; wave w takes columns 2 w, 2 w + 1 and streams each
// weight row as K / 512 contiguous 1 KiB loads (all issued at the start),
// the row of x in registers in the same lane layout; a wave reduction per
// column, lanes 0 and 1 store.  KB = K / 512.
template <int KB>
__global__ __launch_bounds__(64 * OUT_GEMV_WAVES) void out_proj_gemv_kernel(OutProjArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int col = (blockIdx.x * OUT_GEMV_WAVES + wave) * 2;
  constexpr int K = KB * 512;
  const auto rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(a.w) + static_cast<int64_t>(col) * K, 0,
                                                    2 * K * 2, BUF_DWORD3);
  const auto rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(a.x), 0, K * 2, BUF_DWORD3);
  u32x4_t xv[KB], wv[2][KB];
#pragma unroll
  for (int i = 0; i < KB; ++i) xv[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, (512 * i + 8 * lane) * 2, 0, 0);
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int i = 0; i < KB; ++i)
      wv[c][i] = __builtin_amdgcn_raw_buffer_load_b128(rw, (c * K + 512 * i + 8 * lane) * 2, 0, 0);
  float dot[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < KB; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t wp = wv[c][i][e], xp = xv[i][e];
        s += bf16_bits_to_f32(wp & 0xffffu) * bf16_bits_to_f32(xp & 0xffffu);
        s += bf16_bits_to_f32(wp >> 16) * bf16_bits_to_f32(xp >> 16);
      }
    dot[c] = wave_sum(s);
  }
  if (lane < 2) a.y[col + lane] = f32_to_bf16_bits(lane == 0 ? dot[0] : dot[1]);
}

template <int KB>
void launch_out_gemv(const OutProjArgs &args, hipStream_t s) {
  hipLaunchKernelGGL((out_proj_gemv_kernel<KB>), dim3(static_cast<unsigned>(args.N / (2 * OUT_GEMV_WAVES))),
                     dim3(64 * OUT_GEMV_WAVES), 0, s, args);
}

}  // namespace
}  // namespace gdn

extern "C" size_t gdn_out_proj_workspace_bytes(int32_t M, int32_t K, int32_t N) {
  using namespace gdn;
  if (M <= 0 || K <= 0 || N <= 0) return 0;
  const int64_t nmb = (M + IP_ROWS - 1) / IP_ROWS;
  const int64_t split = (K + op_kspan(K) - 1) / op_kspan(K);
  return static_cast<size_t>(split * nmb * IP_ROWS * N * 4);
}

extern "C" int gdn_out_proj_decode(const void *x, int64_t x_stride, const void *w, int32_t M, int32_t K, int32_t N,
                                   void *y, int64_t y_stride, void *workspace, size_t workspace_bytes, void *stream) {
  using namespace gdn;
  if (!x || !w || !y || !workspace) return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_out_proj_decode: null pointer argument");
  if (M < 0 || N <= 0 || N % OutProjShape::COLS || K <= 0 || K % OP_KSPAN || K / OP_KSPAN > OP_MAX_SPLIT)
    return fail(GDN_ERR_UNSUPPORTED,
                "gdn_out_proj_decode: need N a multiple of %d and K a multiple of %d up to %d (got M=%d K=%d N=%d)",
                OutProjShape::COLS, OP_KSPAN, OP_KSPAN * OP_MAX_SPLIT, M, K, N);
  if (x_stride < K || x_stride % 8 || y_stride < N || y_stride % 4)
    return fail(GDN_ERR_INVALID_ARGUMENT,
                "gdn_out_proj_decode: row strides x %lld (>= K, multiple of 8), y %lld (>= N, multiple of 4)",
                static_cast<long long>(x_stride), static_cast<long long>(y_stride));
  // buffer offsets are 32-bit: one 64-row slice of x and one 16-row block of w
  if ((static_cast<int64_t>(IP_ROWS - 1) * x_stride + K) * 2 > INT32_MAX)
    return fail(GDN_ERR_UNSUPPORTED, "gdn_out_proj_decode: x stride %lld too large", static_cast<long long>(x_stride));
  auto al = [](const void *p, uintptr_t n) { return reinterpret_cast<uintptr_t>(p) % n == 0; };
  if (!al(x, 16) || !al(w, 16) || !al(y, 8) || !al(workspace, 16))
    return fail(GDN_ERR_INVALID_ARGUMENT,
                "gdn_out_proj_decode: x, w and the workspace must be 16-byte aligned, y 8-byte");
  if (M == 0) return ok();
  if ((M + IP_ROWS - 1) / IP_ROWS > 65535) return fail(GDN_ERR_UNSUPPORTED, "gdn_out_proj_decode: M=%d too large", M);
  const size_t need = gdn_out_proj_workspace_bytes(M, K, N);
  if (workspace_bytes < need)
    return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_out_proj_decode: workspace of %zu bytes, need %zu", workspace_bytes,
                need);
  OutProjArgs args{};
  args.x = static_cast<const uint16_t *>(x);
  args.xs = x_stride;
  args.w = static_cast<const uint16_t *>(w);
  args.M = M;
  args.K = K;
  args.N = N;
  const bool wide = op_kspan(K) == OP_KSPAN_WIDE;
  args.split = K / op_kspan(K);
  args.ncb = N / (wide ? OutProjShapeWide::COLS : OutProjShape::COLS);
  args.part = static_cast<float *>(workspace);
  args.y = static_cast<uint16_t *>(y);
  args.ys = y_stride;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int kb = K / 512;  // the GEMV kernel's 1 KiB row pieces
  if (M == 1 && (kb == 1 || kb == 2 || kb == 4 || kb == 8)) {  // one GEMV kernel
    switch (kb) {
      case 1: launch_out_gemv<1>(args, s); break;
      case 2: launch_out_gemv<2>(args, s); break;
      case 4: launch_out_gemv<4>(args, s); break;
      default: launch_out_gemv<8>(args, s); break;
    }
    return check_launch("gdn_out_proj_decode");
  }
  const dim3 grid(static_cast<unsigned>(args.ncb * args.split), static_cast<unsigned>((M + IP_ROWS - 1) / IP_ROWS));
  if (wide)
    hipLaunchKernelGGL(out_proj_partial_kernel<OutProjShapeWide>, grid, dim3(64 * IP_WAVES), 0, s, args);
  else
    hipLaunchKernelGGL(out_proj_partial_kernel<OutProjShape>, grid, dim3(64 * IP_WAVES), 0, s, args);
  const int64_t quads = static_cast<int64_t>(M) * (N / 4);
  const dim3 rgrid(static_cast<unsigned>((quads + OP_RED_NT - 1) / OP_RED_NT));
  switch (args.split) {
    case 1: hipLaunchKernelGGL(out_proj_sum_kernel<1>, rgrid, dim3(OP_RED_NT), 0, s, args); break;
    case 2: hipLaunchKernelGGL(out_proj_sum_kernel<2>, rgrid, dim3(OP_RED_NT), 0, s, args); break;
    case 4: hipLaunchKernelGGL(out_proj_sum_kernel<4>, rgrid, dim3(OP_RED_NT), 0, s, args); break;
    case 8: hipLaunchKernelGGL(out_proj_sum_kernel<8>, rgrid, dim3(OP_RED_NT), 0, s, args); break;
    default: hipLaunchKernelGGL(out_proj_sum_kernel<0>, rgrid, dim3(OP_RED_NT), 0, s, args); break;
  }
  return check_launch("gdn_out_proj_decode");
}

namespace gdn {
namespace {

// Scratch of gdn_out_proj_decode_noalloc: the split-K partial sums, in a
// file-scope device array instead of a caller workspace.  Each GPU the
// library runs on holds its own copy (one per loaded code object) until the
// process ends; every call on that GPU shares it, so calls that overlap on
// one GPU (two streams) race.  The partial kernel writes every partial the
// sum kernel reads, so nothing is cleared between calls.
constexpr size_t OP_SCRATCH_BYTES = GDN_OUT_PROJ_NOALLOC_MAX_BYTES;
__device__ __align__(256) float scratch[OP_SCRATCH_BYTES / sizeof(float)];

// `scratch` as a device address, per device: in host code the array's name
// is only a host-side stand-in, so kernels get the address that
// hipGetSymbolAddress returns with that device current (looked up on the
// first call on each device).
constexpr int OP_MAX_DEVICES = 64;
std::mutex scratch_mu;
void *scratch_addr[OP_MAX_DEVICES];

int scratch_on_current_device(void **out, const char *name) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= OP_MAX_DEVICES)
    return fail(GDN_ERR_LAUNCH, "%s: no current device (or device index %d beyond %d)", name, dev, OP_MAX_DEVICES);
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_addr[dev]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(GDN_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", name, dev,
                  hipGetErrorString(e));
    scratch_addr[dev] = p;
  }
  *out = scratch_addr[dev];
  return GDN_OK;
}

}  // namespace
}  // namespace gdn

extern "C" int gdn_out_proj_decode_noalloc(const void *x, int64_t x_stride, const void *w, int32_t M, int32_t K,
                                           int32_t N, void *y, int64_t y_stride, void *stream) {
  using namespace gdn;
  const size_t need = gdn_out_proj_workspace_bytes(M, K, N);
  if (need > OP_SCRATCH_BYTES)
    return fail(GDN_ERR_UNSUPPORTED,
                "gdn_out_proj_decode_noalloc: M=%d K=%d N=%d needs %zu bytes of partial sums, the built-in scratch "
                "holds %zu (use gdn_out_proj_decode with a workspace)",
                M, K, N, need, OP_SCRATCH_BYTES);
  void *ws = nullptr;
  const int st = scratch_on_current_device(&ws, "gdn_out_proj_decode_noalloc");
  if (st != GDN_OK) return st;
  return gdn_out_proj_decode(x, x_stride, w, M, K, N, y, y_stride, ws, OP_SCRATCH_BYTES, stream);
}

extern "C" int gdn_in_proj_decode(const void *x, int64_t x_stride, const void *w_qkv, const void *w_z,
                                  const void *w_b, const void *w_a, int32_t M, int32_t K, int32_t n_qkv,
                                  int32_t n_z, int32_t n_b, int32_t n_a, const void *conv_w, const void *conv_bias,
                                  void *conv_pool, const int64_t *slot_idx, int64_t pool_rows, void *y_qkv, void *z,
                                  void *b, void *a, int silu, void *stream) {
  using namespace gdn;
  if (!x || !w_qkv || !w_z || !conv_w || !conv_pool || !y_qkv || !z || ((n_b > 0) && (!w_b || !b)) ||
      ((n_a > 0) && (!w_a || !a)))
    return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_in_proj_decode: null pointer argument");
  if (M < 0 || n_qkv <= 0 || n_qkv % IP_COLS || n_z < 0 || n_z % IP_COLS || n_b < 0 || n_a < 0 || n_b % 4 ||
      n_a % 4 || n_b > 32 || n_a > 32)
    return fail(GDN_ERR_UNSUPPORTED,
                "gdn_in_proj_decode: need n_qkv and n_z multiples of %d, n_b and n_a multiples of 4 up to 32 "
                "(got M=%d n=%d/%d/%d/%d)",
                IP_COLS, M, n_qkv, n_z, n_b, n_a);
  if (K != 1024 && K != 2048)
    return fail(GDN_ERR_UNSUPPORTED, "gdn_in_proj_decode: K=%d (built for 1024 and 2048)", K);
  if (x_stride < K || x_stride % 8)
    return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_in_proj_decode: x row stride %lld must be >= K and a multiple of 8",
                static_cast<long long>(x_stride));
  // buffer offsets are 32-bit: one weight tile row block and one 64-row slice of x
  if (static_cast<int64_t>(16) * K * 2 > INT32_MAX || (static_cast<int64_t>(IP_ROWS - 1) * x_stride + K) * 2 > INT32_MAX)
    return fail(GDN_ERR_UNSUPPORTED, "gdn_in_proj_decode: K=%d / x stride %lld too large", K,
                static_cast<long long>(x_stride));
  auto al = [](const void *p, uintptr_t n) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % n == 0; };
  if (!al(x, 16) || !al(w_qkv, 16) || !al(w_z, 16) || !al(w_b, 16) || !al(w_a, 16) || !al(conv_w, 16) ||
      !al(conv_pool, 16) || !al(y_qkv, 8) || !al(z, 8) || !al(b, 8) || !al(a, 8) || !al(conv_bias, 2))
    return fail(GDN_ERR_INVALID_ARGUMENT,
                "gdn_in_proj_decode: x, weights, conv taps and pool must be 16-byte aligned, outputs 8-byte aligned");
  if (pool_rows * n_qkv * 8 >= IP_OOB)
    return fail(GDN_ERR_UNSUPPORTED, "gdn_in_proj_decode: conv pool of %lld rows x %d channels exceeds 1 GiB",
                static_cast<long long>(pool_rows), n_qkv);
  if (!rows_cover(conv_pool, slot_idx, pool_rows, M))
    return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_in_proj_decode: %lld pool rows do not cover %d rows",
                static_cast<long long>(pool_rows), M);
  if (M == 0) return ok();
  if ((M + IP_ROWS - 1) / IP_ROWS > 65535)
    return fail(GDN_ERR_UNSUPPORTED, "gdn_in_proj_decode: M=%d too large", M);
  InProjArgs args{};
  args.x = static_cast<const uint16_t *>(x);
  args.xs = x_stride;
  args.w[0] = static_cast<const uint16_t *>(w_qkv);
  args.w[1] = static_cast<const uint16_t *>(w_z);
  args.w[2] = static_cast<const uint16_t *>(w_b);
  args.w[3] = static_cast<const uint16_t *>(w_a);
  args.n[0] = n_qkv;
  args.n[1] = n_z;
  args.n[2] = n_b;
  args.n[3] = n_a;
  args.blocks_qkv = n_qkv / IN_GEMV_COLS;
  args.blocks_z = n_z / IN_GEMV_COLS;
  args.M = M;
  args.K = K;
  args.cw = static_cast<const uint16_t *>(conv_w);
  args.cb = static_cast<const uint16_t *>(conv_bias);
  args.pool = static_cast<uint16_t *>(conv_pool);
  args.idx = slot_idx;
  args.rows = pool_rows;
  args.y[0] = static_cast<uint16_t *>(y_qkv);
  args.y[1] = static_cast<uint16_t *>(z);
  args.y[2] = static_cast<uint16_t *>(b);
  args.y[3] = static_cast<uint16_t *>(a);
  args.silu = silu;
  const dim3 grid(static_cast<unsigned>(args.blocks_qkv + args.blocks_z + (n_b + n_a > 0 ? 16 / IN_GEMV_WAVES : 0)),
                  static_cast<unsigned>((M + IP_ROWS - 1) / IP_ROWS));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (M <= IP_GEMV_ROWS) {  // a GEMV stream of the weights (one row block)
    if (M == 1)
      launch_gemv<1>(args, grid.x, K / 512, s);
    else
      launch_gemv<2>(args, grid.x, K / 512, s);
    return check_launch("gdn_in_proj_decode");
  }
  const int ntiles = (n_qkv + 15) / 16 + (n_z + 15) / 16;  // b and a go by columns, XS_BA_MAX per workgroup
  const int gx = std::max(std::min(ntiles, std::max(XS_MIN_WGS, (ntiles + XS_MAX_TILES - 1) / XS_MAX_TILES)),
                          (n_b + n_a + XS_BA_MAX - 1) / XS_BA_MAX);
  const dim3 xgrid(static_cast<unsigned>(gx), grid.y);
  switch (K) {
    case 1024: hipLaunchKernelGGL((in_proj_xs_kernel<XS_WAVES, 2>), xgrid, dim3(64 * XS_WAVES), 0, s, args); break;
    case 2048: hipLaunchKernelGGL((in_proj_xs_kernel<XS_WAVES, 4>), xgrid, dim3(64 * XS_WAVES), 0, s, args); break;
    default: return fail(GDN_ERR_UNSUPPORTED, "gdn_in_proj_decode: K=%d unsupported", K);
  }
  return check_launch("gdn_in_proj_decode");
}
