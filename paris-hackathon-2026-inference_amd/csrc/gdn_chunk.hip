// Chunk-64 gated delta rule prefill (placeholder until the MFMA kernels land).
#include "gdn_common.h"

extern "C" size_t gdn_chunk_workspace_bytes(int32_t n_seqs, int64_t total_tokens, int32_t Hv, int32_t K,
                                            int32_t V) {
  (void)n_seqs; (void)total_tokens; (void)Hv; (void)K; (void)V;
  return 0;
}

extern "C" int gdn_chunk_fwd(const void *, const void *, const void *, int, int64_t, int64_t, int64_t,
                             const float *, const void *, int, const float *, const int64_t *, float *,
                             const int64_t *, void *, int, const int32_t *, int32_t, int32_t, int32_t,
                             int32_t, int32_t, int32_t, float, int, void *, size_t, void *) {
  return gdn::fail(GDN_ERR_UNSUPPORTED, "gdn_chunk_fwd: not built yet");
}
