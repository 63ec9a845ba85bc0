// Speculative-verify commit: copy the snapshot of the last accepted draft
// token into the slot pool.  A pure 64 KiB-per-(sequence, head) copy, so
// each workgroup streams one state with 16-byte loads and stores.
//
// No reference implementation: engine/runtime/spec_decode.py:81-87 and
// :99-103 record that GDN rollback "requires saving state snapshots".
#include "gdn_common.h"

namespace gdn {
namespace {

constexpr int COMMIT_NT = 256;

__global__ __launch_bounds__(COMMIT_NT) void commit_kernel(float *pool, const int64_t *slot_ids,
                                                           const float *snaps, const int32_t *acc,
                                                           int T, int H, int64_t kv) {
  const int h = blockIdx.x % H;
  const int b = blockIdx.x / H;
  const int64_t slot = slot_ids[b];
  const int a = acc[b];
  if (slot < 0 || a <= 0) return;
  const int t = a > T ? T - 1 : a - 1;
  const float4 *src = reinterpret_cast<const float4 *>(snaps + (((int64_t)b * T + t) * H + h) * kv);
  float4 *dst = reinterpret_cast<float4 *>(pool + (slot * H + h) * kv);
  const int64_t n4 = kv / 4;
  for (int64_t i = threadIdx.x; i < n4; i += COMMIT_NT) dst[i] = src[i];
}

}  // namespace
}  // namespace gdn

extern "C" int gdn_state_commit(float *pool, const int64_t *slot_ids, const float *snapshots,
                                const int32_t *accepted_len, int32_t n_seqs, int32_t T,
                                int32_t H, int32_t K, int32_t V, void *stream) {
  using namespace gdn;
  if (n_seqs < 0 || T <= 0 || H <= 0 || K <= 0 || V <= 0 || (static_cast<int64_t>(K) * V) % 4)
    return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_state_commit: bad sizes n_seqs=%d T=%d H=%d K=%d V=%d",
                n_seqs, T, H, K, V);
  if (n_seqs == 0) return ok();
  if (!pool || !slot_ids || !snapshots || !accepted_len)
    return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_state_commit: null pointer");
  const int64_t blocks = static_cast<int64_t>(n_seqs) * H;
  if (blocks > 0x7fffffff) return fail(GDN_ERR_INVALID_ARGUMENT, "gdn_state_commit: grid too large");
  hipLaunchKernelGGL(commit_kernel, dim3(static_cast<unsigned>(blocks)), dim3(COMMIT_NT), 0,
                     static_cast<hipStream_t>(stream), pool, slot_ids, snapshots, accepted_len, T, H,
                     static_cast<int64_t>(K) * V);
  return check_launch("gdn_state_commit");
}
