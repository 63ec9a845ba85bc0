// Token recurrence of the gated delta rule (decode / spec-verify / small-T).
//
// One workgroup owns a [KD x VT] column slice of one (sequence, v-head)
// state (KD = 128 by default; 64 and 256 are also built, and any v head dim
// that is a multiple of VT) and keeps it in registers for all of the
// sequence's tokens: the
// state is read from HBM once and written once, so decode is a pure stream
// of the fp32 state (the HBM roofline).  Thread mapping (NT = 2*VT threads):
//   columns: 4 per thread (float4), TPR = VT/4 threads span the slice;
//   rows:    8 row groups, thread row group rg owns rows rg + 8r, r < KD / 8.
// Per token the two K-reductions k~^T S and q~^T S are done together: in
// registers over 16 rows, xor-shuffles across the row groups of a wave, and
// LDS across waves when VT > 32.  The output uses
//   o = q~^T (e^g S + k~ d^T) = e^g (q~^T S) + (q~ . k~) d,
// so no second reduction is needed after the rank-1 update.
//
// Semantics: transformers modeling_qwen3_5_moe.py:331-381 (the torch
// recurrence the reference imports at engine/runtime/cuda_graphs.py:126-135).
#include "gdn_common.h"

namespace gdn {
namespace {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) unsigned u32x4;

constexpr int KD_DEFAULT = 128;  // head dim of k (rows of the state) of the tuned build
constexpr int VD_DEFAULT = 128;  // head dim of v (columns of the state)

struct RecArgs {
  const void *q, *k, *v;
  int64_t qs, ks, vs;  // token strides (elements)
  GateArgs gate;
  const float *state_in;
  const int64_t *in_idx;
  int64_t in_rows;
  float *state_out;
  const int64_t *out_idx;
  int64_t out_rows;
  void *o;
  float *snap;
  const int32_t *cu;
  int n_seqs, T, Hk, Hv;
  int V;  // v head dim (a multiple of the workgroup's columns)
  int64_t total;
  float scale;
  int l2norm;
  int qkv_dt, o_dt;
  int head_major;  // workgroup order: v-head fastest (a capped decode grid) or column block fastest
};

// Workgroup shape: 32 state columns, 64 threads (one wave, 16 rows per
// thread, 149 VGPRs, 3 waves per SIMD; capped at 128 it spills and takes
// 64.3 us).  Measured at B=64 on MI355X, before the first token's inputs were
// requested ahead of the state: 56.0 us;
// 128 threads (8 rows per thread, 4 waves per SIMD) 58.5 us; 256 threads
// 62.7 us -- more waves per workgroup cost a cross-wave reduction per token.
constexpr int REC_VT = 32;
constexpr int REC_NT = 64;

// Resident workgroups per CU and their order.  The registers allow 12 of
// these one-wave workgroups per CU (3 waves per SIMD, 256 CUs: 3,072 at
// once).  A decode grid (one token per sequence) of more than 2,304
// workgroups (B > 18 at 32 v-heads) is launched
//   * with dynamic LDS reserved so that 6 share a CU: the state streams of
//     fewer resident workgroups reach HBM faster (B = 64, eager launches,
//     per CU: 3 / 4 / 5 / 6 / 7 / 8 / 12 workgroups 53.7 / 50.7 / 48.6 /
//     48.6 / 50.2 / 51.5 / 52.2 us with the order below);
//   * head-major: the v-heads of one (sequence, column block) in consecutive
//     workgroups, so that the 4 column blocks of a head are a multiple of 8
//     workgroups apart and run on one XCD (workgroups are dealt to the 8 XCDs
//     in turn): the two 64-byte halves of each 128-byte line of o meet in
//     that XCD's L2 and the head's q/k rows are fetched once (at 4 per CU:
//     49.9-50.3 us against 51.8-52.3 us column-block-major).
// From graphs: B = 20 / 24 / 25 / 32 / 64 17.7 / 20.4 / 21.9 / 26.4 / 48.7 us
// against 18.3 / 21.4 / 23.7 / 28.3 / 54.2 us at full occupancy, column-block-
// major.  A smaller grid (1.5 capped rounds or less) runs best with all of it
// resident and column-block-major (B = 16: 13.4 us; capped 15.4 us).
// A multi-token step that writes per-token snapshots (spec verify) is a
// write stream as much as a read stream: head-major with 4 per CU (B = 32 x
// T = 4: 66.4-67.9 us; full occupancy 71.4-71.6, head-major alone 69.4-70.3,
// at 3 / 5 / 6 per CU 81.0 / 71.6-72.3 / 68.9-69.5 us).  Without snapshots the
// tokens' arithmetic needs the resident waves: full occupancy, column-block-
// major (B = 32 / 64 x T = 4: 40.2-41.2 / 70.7-71.2 us; at 4 per CU 56.0-56.7 /
// 103.2-104.6 us).
constexpr int64_t REC_CAP_MIN_BLOCKS = 2304;   // 1.5 rounds of 6 per CU on 256 CUs
constexpr unsigned REC_CAP_LDS = 24 * 1024;    // + 1 KiB static: 6 per CU in 160 KiB
constexpr unsigned REC_SNAP_CAP_LDS = 36 * 1024;  // + 1 KiB static: 4 per CU

// KD: k head dim (64, 128 or 256); VDC: v head dim, or 0 for a.V
template <int VT, int NT, int KD, int VDC>
__global__ __launch_bounds__(NT) void recurrent_kernel(RecArgs a) {
  constexpr int NW = NT / 64;
  constexpr int TPR = VT / 4;     // threads per state row
  constexpr int NRG = NT / TPR;   // row groups
  constexpr int RPT = KD / NRG;   // rows per thread
  constexpr int QE = KD / 64;     // q and k elements per lane
  static_assert(KD % 64 == 0 && KD % NRG == 0, "k head dim");
  const int VD = VDC ? VDC : a.V;
  const int NSPLIT = VD / VT;

  __shared__ float qs_l[KD];
  __shared__ float ks_l[KD];
  __shared__ float red[NW > 1 ? NW : 1][2][VT];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int c4 = tid % TPR;
  const int rg = tid / TPR;

  int bid = blockIdx.x, vt, h;
  if (a.head_major) {
    h = bid % a.Hv;
    bid /= a.Hv;
    vt = bid % NSPLIT;
    bid /= NSPLIT;
  } else {
    vt = bid % NSPLIT;
    bid /= NSPLIT;
    h = bid % a.Hv;
    bid /= a.Hv;
  }
  const int n = bid;
  const int hk = h / (a.Hv / a.Hk);
  const int col0 = vt * VT + c4 * 4;

  int64_t t0;
  int len;
  seq_range(a.cu, n, a.T, a.total, &t0, &len);

  const int64_t in_row = a.state_in ? pool_row(a.in_idx, n, a.in_rows) : -1;
  int64_t out_row = a.state_out ? pool_row(a.out_idx, n, a.out_rows) : -1;

  // A token's inputs as raw bits: this lane's two elements of q and k, its
  // four columns of v, and the gates.
  struct TokIn {
    uint32_t q[QE], k[QE], v[4];
    GateRaw gate;
  };
  auto tok_load = [&](int64_t tok) {
    TokIn r;
    const int64_t qoff = tok * a.qs + (int64_t)hk * KD + QE * lane;
    const int64_t koff = tok * a.ks + (int64_t)hk * KD + QE * lane;
    const int64_t vo = tok * a.vs + (int64_t)h * VD + col0;
#pragma unroll
    for (int i = 0; i < QE; ++i) {
      r.q[i] = load_bits(a.q, qoff + i, a.qkv_dt);
      r.k[i] = load_bits(a.k, koff + i, a.qkv_dt);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) r.v[c] = load_bits(a.v, vo + c, a.qkv_dt);
    r.gate = load_gates_raw(a.gate, tok, h);
    return r;
  };

  // The first token's inputs and the earlier rows' slot ids are requested
  // before the state: vector loads complete in order, so the q/k prologue and
  // the repeated-slot test wait for these few loads only, while the state
  // stream is in flight, and nothing is left to fetch once the state is in.
  TokIn cur{};
  if (len > 0) cur = tok_load(t0);
  const int64_t in_lane_id = in_row >= 0 ? earlier_id_of_lane(a.in_idx, n, lane) : 0;
  const int64_t out_lane_id = out_row >= 0 ? earlier_id_of_lane(a.out_idx, n, lane) : 0;
  __builtin_amdgcn_sched_barrier(0);

  // The state is touched exactly once per launch: non-temporal loads and
  // stores keep it from displacing reusable lines in the caches.  One
  // (sequence, head) state is one 64 KiB buffer range; a thread's rows
  // rg + 8r sit 4 KiB apart, an offset carried in a scalar register, so the
  // 16 accesses share one vector offset.
  const int voff = (rg * VD + col0) * 4;
  const int ROW8 = NRG * VD * 4;  // bytes between a thread's rows
  // (a row with no slot gets an empty range: its loads read zeros without
  // touching memory, so the loads are issued on one path whatever the row)
  auto state_rsrc = [&](const float *pool, int64_t row) {
    return row >= 0 ? __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(pool) + (row * a.Hv + h) * (int64_t)(KD * VD),
                                                        0, KD * VD * 4, BUF_DWORD3)
                    : __builtin_amdgcn_make_buffer_rsrc(nullptr, 0, 0, BUF_DWORD3);
  };
  f32x4 s[RPT];
  {
    const auto rs = state_rsrc(a.state_in, in_row);
#pragma unroll
    for (int r = 0; r < RPT; ++r)
      s[r] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, r * ROW8, BUF_NT));
  }
  __builtin_amdgcn_sched_barrier(0);
  // A row whose slot id an earlier row already named: zero state, like a
  // padding row, and nothing written.
  const bool in_rep = in_row >= 0 && repeats_earlier_wave(a.in_idx, n, in_row, in_lane_id, lane);
  if (out_row >= 0 && repeats_earlier_wave(a.out_idx, n, out_row, out_lane_id, lane)) out_row = -1;

  for (int t = 0; t < len; ++t) {
    const int64_t tok = t0 + t;
    // ---- q/k prologue: every wave reduces the full KD-vectors itself
    float qv[QE], kv[QE], pqq = 0.f, pkk = 0.f, pqk = 0.f;
#pragma unroll
    for (int i = 0; i < QE; ++i) {
      qv[i] = bits_to_f32(cur.q[i], a.qkv_dt);
      kv[i] = bits_to_f32(cur.k[i], a.qkv_dt);
      pqq += qv[i] * qv[i];
      pkk += kv[i] * kv[i];
      pqk += qv[i] * kv[i];
    }
    const float sqq = wave_sum(pqq);
    const float skk = wave_sum(pkk);
    const float sqk = wave_sum(pqk);
    const float rq = a.l2norm ? rsqrtf(sqq + 1e-6f) : 1.f;
    const float rk = a.l2norm ? rsqrtf(skk + 1e-6f) : 1.f;
    const float qsc = rq * a.scale;
    if (wave == 0) {
#pragma unroll
      for (int i = 0; i < QE; ++i) {
        qs_l[QE * lane + i] = qv[i] * qsc;
        ks_l[QE * lane + i] = kv[i] * rk;
      }
    }
    const float qk = sqk * qsc * rk;
    float gl, bt;
    gates_from_raw(a.gate, cur.gate, &gl, &bt);
    const float eg = expf(gl);
    float vv[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) vv[c] = bits_to_f32(cur.v[c], a.qkv_dt);
    if (t + 1 < len) cur = tok_load(tok + 1);  // the next token's inputs, during this one's update
    if (t == 0 && in_rep) {
#pragma unroll
      for (int r = 0; r < RPT; ++r) s[r] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    __syncthreads();

    // ---- partial k~^T S and q~^T S over this thread's rows
    float pk[4] = {0.f, 0.f, 0.f, 0.f}, pq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
      const float kk = ks_l[rg + NRG * r], qq = qs_l[rg + NRG * r];
      pk[0] += kk * s[r].x; pk[1] += kk * s[r].y; pk[2] += kk * s[r].z; pk[3] += kk * s[r].w;
      pq[0] += qq * s[r].x; pq[1] += qq * s[r].y; pq[2] += qq * s[r].z; pq[3] += qq * s[r].w;
    }
#pragma unroll
    for (int m = TPR; m < 64; m <<= 1) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        pk[c] += __shfl_xor(pk[c], m, 64);
        pq[c] += __shfl_xor(pq[c], m, 64);
      }
    }
    if constexpr (NW > 1) {
      if (lane < TPR) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          red[wave][0][c4 * 4 + c] = pk[c];
          red[wave][1][c4 * 4 + c] = pq[c];
        }
      }
      __syncthreads();
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float sk = 0.f, sq = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          sk += red[w][0][c4 * 4 + c];
          sq += red[w][1][c4 * 4 + c];
        }
        pk[c] = sk;
        pq[c] = sq;
      }
    }

    // ---- delta, rank-1 update, output
    float d[4], out[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      d[c] = bt * (vv[c] - eg * pk[c]);
      out[c] = eg * pq[c] + qk * d[c];
    }
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
      const float kk = ks_l[rg + NRG * r];
      s[r].x = eg * s[r].x + kk * d[0];
      s[r].y = eg * s[r].y + kk * d[1];
      s[r].z = eg * s[r].z + kk * d[2];
      s[r].w = eg * s[r].w + kk * d[3];
    }
    if (rg == 0) {
      const int64_t ooff = (tok * a.Hv + h) * (int64_t)VD + col0;
#pragma unroll
      for (int c = 0; c < 4; ++c) store_elem(a.o, ooff + c, a.o_dt, out[c]);
    }
    // Snapshots take global stores: stores through a buffer range rebuilt
    // per token in this loop were compiled with a per-token term in the vector
    // offset and landed outside the range (dropped).  Non-temporal, as the
    // state stream: with ordinary stores the B = 32 x T = 4 verify step took
    // 75.2-75.6 us against 68.4-69.6 us.
    if (a.snap) {
      float *sb = a.snap + (((int64_t)n * a.T + t) * a.Hv + h) * (int64_t)(KD * VD) + col0;
#pragma unroll
      for (int r = 0; r < RPT; ++r)
        __builtin_nontemporal_store(s[r], reinterpret_cast<f32x4 *>(sb + (rg + NRG * r) * VD));
    }
    __syncthreads();
  }

  if (len <= 0 && in_rep) {
#pragma unroll
    for (int r = 0; r < RPT; ++r) s[r] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  if (out_row >= 0) {
    const auto rs = state_rsrc(a.state_out, out_row);
#pragma unroll
    for (int r = 0; r < RPT; ++r)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, s[r]), rs, voff, r * ROW8, BUF_NT);
  }
}

}  // namespace
}  // namespace gdn

namespace gdn {
namespace {

int recurrent_fwd(const void *q, const void *k, const void *v, int qkv_dtype,
                  int64_t q_stride_t, int64_t k_stride_t, int64_t v_stride_t, const GateArgs &gate,
                  const float *state_in, const int64_t *state_in_idx, int64_t state_in_rows,
                  float *state_out, const int64_t *state_out_idx, int64_t state_out_rows,
                  void *o, int o_dtype, float *snapshots,
                  const int32_t *cu_seqlens, int32_t n_seqs, int32_t T,
                  int32_t Hk, int32_t Hv, int32_t K, int32_t V,
                  float scale, int l2norm_qk, void *stream, const char *name) {
  if ((K != 64 && K != 128 && K != 256) || V <= 0 || V % REC_VT)
    return fail(GDN_ERR_UNSUPPORTED, "%s: K=%d V=%d; K must be 64, 128 or 256 and V a positive multiple of %d",
                name, K, V, REC_VT);
  if (n_seqs < 0 || T < 0 || Hk <= 0 || Hv <= 0 || Hv % Hk)
    return fail(GDN_ERR_INVALID_ARGUMENT, "%s: bad sizes n_seqs=%d T=%d Hk=%d Hv=%d", name, n_seqs, T, Hk, Hv);
  if (!valid_dtype(qkv_dtype) || !valid_dtype(gate.dt) || !valid_dtype(o_dtype))
    return fail(GDN_ERR_INVALID_ARGUMENT, "%s: bad dtype", name);
  if (n_seqs == 0) return ok();
  if (!q || !k || !v || !gate.g_or_a || !gate.beta_or_b || !o)
    return fail(GDN_ERR_INVALID_ARGUMENT, "%s: null q/k/v/gate/o", name);
  if (gate.A_log && !gate.dt_bias) return fail(GDN_ERR_INVALID_ARGUMENT, "%s: null dt_bias", name);
  if (gate.stride < Hv) return fail(GDN_ERR_INVALID_ARGUMENT, "%s: gate token stride smaller than Hv", name);
  if (snapshots && cu_seqlens)
    return fail(GDN_ERR_INVALID_ARGUMENT, "%s: snapshots need equal-length sequences", name);
  if (!rows_cover(state_in, state_in_idx, state_in_rows, n_seqs) ||
      !rows_cover(state_out, state_out_idx, state_out_rows, n_seqs))
    return fail(GDN_ERR_INVALID_ARGUMENT, "%s: state rows (%lld in, %lld out) do not cover %d sequences", name,
                static_cast<long long>(state_in_rows), static_cast<long long>(state_out_rows), n_seqs);
  if (q_stride_t < Hk * K || k_stride_t < Hk * K || v_stride_t < Hv * V)
    return fail(GDN_ERR_INVALID_ARGUMENT, "%s: token stride smaller than a row", name);
  const int64_t n_blocks = static_cast<int64_t>(n_seqs) * Hv * (V / REC_VT);
  if (n_blocks > 0x7fffffff) return fail(GDN_ERR_INVALID_ARGUMENT, "%s: grid too large", name);

  RecArgs a{q, k, v, q_stride_t, k_stride_t, v_stride_t, gate, state_in, state_in_idx, state_in_rows,
            state_out, state_out_idx, state_out_rows, o, snapshots, cu_seqlens, n_seqs, T, Hk, Hv, V,
            cu_seqlens ? static_cast<int64_t>(T) : static_cast<int64_t>(n_seqs) * T,
            scale, l2norm_qk, qkv_dtype, o_dtype};
  const bool capped = n_blocks > REC_CAP_MIN_BLOCKS && (T == 1 || snapshots);
  a.head_major = capped;
  const unsigned lds = !capped ? 0u : T == 1 ? REC_CAP_LDS : REC_SNAP_CAP_LDS;
  const dim3 grid(static_cast<unsigned>(n_blocks)), block(REC_NT);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (K == KD_DEFAULT && V == VD_DEFAULT)
    hipLaunchKernelGGL((recurrent_kernel<REC_VT, REC_NT, KD_DEFAULT, VD_DEFAULT>), grid, block, lds, st, a);
  else if (K == 64)
    hipLaunchKernelGGL((recurrent_kernel<REC_VT, REC_NT, 64, 0>), grid, block, lds, st, a);
  else if (K == 128)
    hipLaunchKernelGGL((recurrent_kernel<REC_VT, REC_NT, 128, 0>), grid, block, lds, st, a);
  else
    hipLaunchKernelGGL((recurrent_kernel<REC_VT, REC_NT, 256, 0>), grid, block, lds, st, a);
  return check_launch(name);
}

}  // namespace
}  // namespace gdn

extern "C" int gdn_recurrent_fwd(const void *q, const void *k, const void *v, int qkv_dtype,
                                 int64_t q_stride_t, int64_t k_stride_t, int64_t v_stride_t,
                                 const float *g, const void *beta, int beta_dtype,
                                 const float *state_in, const int64_t *state_in_idx, int64_t state_in_rows,
                                 float *state_out, const int64_t *state_out_idx, int64_t state_out_rows,
                                 void *o, int o_dtype, float *snapshots,
                                 const int32_t *cu_seqlens, int32_t n_seqs, int32_t T,
                                 int32_t Hk, int32_t Hv, int32_t K, int32_t V,
                                 float scale, int l2norm_qk, void *stream) {
  const gdn::GateArgs gate{g, beta, beta_dtype, Hv, nullptr, nullptr};
  return gdn::recurrent_fwd(q, k, v, qkv_dtype, q_stride_t, k_stride_t, v_stride_t, gate, state_in, state_in_idx,
                            state_in_rows, state_out, state_out_idx, state_out_rows, o, o_dtype, snapshots, cu_seqlens, n_seqs, T, Hk, Hv, K, V,
                            scale, l2norm_qk, stream, "gdn_recurrent_fwd");
}

extern "C" int gdn_recurrent_fwd_gated(const void *q, const void *k, const void *v, int qkv_dtype,
                                       int64_t q_stride_t, int64_t k_stride_t, int64_t v_stride_t,
                                       const void *a, const void *b, int ab_dtype, int64_t ab_stride_t,
                                       const float *A_log, const float *dt_bias,
                                       const float *state_in, const int64_t *state_in_idx, int64_t state_in_rows,
                                       float *state_out, const int64_t *state_out_idx, int64_t state_out_rows,
                                       void *o, int o_dtype, float *snapshots,
                                       const int32_t *cu_seqlens, int32_t n_seqs, int32_t T,
                                       int32_t Hk, int32_t Hv, int32_t K, int32_t V,
                                       float scale, int l2norm_qk, void *stream) {
  if (!A_log) return gdn::fail(GDN_ERR_INVALID_ARGUMENT, "gdn_recurrent_fwd_gated: null A_log");
  const gdn::GateArgs gate{a, b, ab_dtype, ab_stride_t, A_log, dt_bias};
  return gdn::recurrent_fwd(q, k, v, qkv_dtype, q_stride_t, k_stride_t, v_stride_t, gate, state_in, state_in_idx,
                            state_in_rows, state_out, state_out_idx, state_out_rows, o, o_dtype, snapshots, cu_seqlens, n_seqs, T, Hk, Hv, K, V,
                            scale, l2norm_qk, stream, "gdn_recurrent_fwd_gated");
}
