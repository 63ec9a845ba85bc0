// Speculative-verify commit: copy the snapshot of the last accepted draft
// token into the slot pool.  A pure 64 KiB-per-(sequence, head) copy, so
// each workgroup streams one state with 16-byte loads and stores.  The conv
// window commit does the same for the causal-conv state: the window after
// the accepted tokens is a slice of the verify step's history (the window
// before the step followed by the step's inputs), one thread per channel.
//
// No reference implementation: engine/runtime/spec_decode.py:81-87 and
// :99-103 record that GDN rollback "requires saving state snapshots".
#include "gdn_common.h"

namespace gdn {
namespace {

constexpr int COMMIT_NT = 256;

__global__ __launch_bounds__(COMMIT_NT) void commit_kernel(float *pool, const int64_t *slot_ids, int64_t rows,
                                                           const float *snaps, const int32_t *acc,
                                                           int T, int H, int64_t kv) {
  const int h = blockIdx.x % H;
  const int b = blockIdx.x / H;
  const int64_t slot = pool_row_first(slot_ids, b, rows);  // a repeated slot id commits nothing
  const int a = acc[b];
  if (slot < 0 || a <= 0) return;
  const int t = a > T ? T - 1 : a - 1;
  const float4 *src = reinterpret_cast<const float4 *>(snaps + (((int64_t)b * T + t) * H + h) * kv);
  float4 *dst = reinterpret_cast<float4 *>(pool + (slot * H + h) * kv);
  const int64_t n4 = kv / 4;
  for (int64_t i = threadIdx.x; i < n4; i += COMMIT_NT) dst[i] = src[i];
}

template <typename T>
__global__ __launch_bounds__(COMMIT_NT) void conv_commit_kernel(T *pool, const int64_t *slot_ids, int64_t rows,
                                                                const T *hist, const int32_t *acc, int C, int S, int L,
                                                                int steps) {
  const int b = blockIdx.y;
  const int c = blockIdx.x * COMMIT_NT + threadIdx.x;
  const int64_t slot = pool_row_first(slot_ids, b, rows);  // a repeated slot id commits nothing
  const int a = acc[b];
  if (c >= C || slot < 0 || a <= 0) return;
  const int first = a > steps ? steps : a;  // window after `first` tokens: history columns [first, first + S)
  const T *src = hist + (static_cast<int64_t>(b) * C + c) * L + first;
  T *dst = pool + (slot * C + c) * S;
  for (int j = 0; j < S; ++j) dst[j] = src[j];
}

}  // namespace
}  // namespace gdn

extern "C" int gdn_conv_state_commit(void *pool, const int64_t *slot_ids, int64_t pool_rows, const void *hist,
                                     const int32_t *accepted_len, int32_t n_seqs, int32_t C, int32_t S,
                                     int32_t L, int32_t dtype, void *stream) {
  using namespace gdn;
  if (n_seqs < 0 || C <= 0 || S <= 0 || L <= S || n_seqs > 65535)
    return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_conv_state_commit: bad sizes n_seqs=%d C=%d S=%d L=%d", n_seqs, C,
                S, L);
  if (!valid_dtype(dtype))
    return fail(GDN_ERR_UNSUPPORTED, "gdn_conv_state_commit: dtype %d (bf16, fp16 or fp32)", dtype);
  if (n_seqs == 0) return ok();
  if (!pool || !slot_ids || !hist || !accepted_len || pool_rows < 0)
    return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_conv_state_commit: null pointer or negative pool_rows");
  const dim3 grid((C + COMMIT_NT - 1) / COMMIT_NT, n_seqs);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype != GDN_DTYPE_F32)  // a 2-byte copy: bf16 and fp16 alike
    hipLaunchKernelGGL(conv_commit_kernel<uint16_t>, grid, dim3(COMMIT_NT), 0, st, static_cast<uint16_t *>(pool),
                       slot_ids, static_cast<int64_t>(pool_rows), static_cast<const uint16_t *>(hist), accepted_len,
                       C, S, L, L - S);
  else
    hipLaunchKernelGGL(conv_commit_kernel<float>, grid, dim3(COMMIT_NT), 0, st, static_cast<float *>(pool), slot_ids,
                       static_cast<int64_t>(pool_rows), static_cast<const float *>(hist), accepted_len, C, S, L, L - S);
  return check_launch("gdn_conv_state_commit");
}

extern "C" int gdn_state_commit(float *pool, const int64_t *slot_ids, int64_t pool_rows, const float *snapshots,
                                const int32_t *accepted_len, int32_t n_seqs, int32_t T,
                                int32_t H, int32_t K, int32_t V, void *stream) {
  using namespace gdn;
  if (n_seqs < 0 || T <= 0 || H <= 0 || K <= 0 || V <= 0 || (static_cast<int64_t>(K) * V) % 4)
    return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_state_commit: bad sizes n_seqs=%d T=%d H=%d K=%d V=%d",
                n_seqs, T, H, K, V);
  if (n_seqs == 0) return ok();
  if (!pool || !slot_ids || !snapshots || !accepted_len || pool_rows < 0)
    return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_state_commit: null pointer or negative pool_rows");
  const int64_t blocks = static_cast<int64_t>(n_seqs) * H;
  if (blocks > 0x7fffffff) return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_state_commit: grid too large");
  hipLaunchKernelGGL(commit_kernel, dim3(static_cast<unsigned>(blocks)), dim3(COMMIT_NT), 0,
                     static_cast<hipStream_t>(stream), pool, slot_ids, static_cast<int64_t>(pool_rows), snapshots,
                     accepted_len, T, H,
                     static_cast<int64_t>(K) * V);
  return check_launch("gdn_state_commit");
}
