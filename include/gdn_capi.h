/*
 * gdn_capi.h -- C ABI of the MI355X (gfx950) Gated DeltaNet library.
 *
 * One shared library, libgdn_mi355x.so, exports the functions below with C
 * linkage.  They are what the reference's Python kernel boundary would bind
 * through ctypes (the reference has no compiled code of its own: its GDN
 * entry points are Python functions in engine/kernels/ that dispatch to
 * Helion/Triton/third-party kernels).  Each declaration names the reference
 * interface it replaces.
 *
 * Conventions shared by every entry point
 *   - Pointers are device pointers unless stated otherwise.  Nothing here
 *     allocates device memory or synchronises the device or the stream:
 *     every kernel is enqueued on `stream` (a hipStream_t passed as void*;
 *     NULL is the null stream), so calls are safe to record into a HIP graph.
 *     The library creates no streams or events.  Between calls it keeps
 *     the thread-local error string and, for gdn_out_proj_decode_noalloc
 *     only, a fixed per-GPU scratch array (GDN_OUT_PROJ_NOALLOC_MAX_BYTES)
 *     whose address is looked up once per device; every other entry point
 *     works only on the buffers its caller passes.
 *   - The return value is a gdn_status_t.  On failure nothing was launched
 *     and gdn_last_error_string() (thread-local) says why.
 *   - Token-major activations: element (token t, head h, dim d) of q/k/v lives
 *     at base + t*stride_t + h*D + d, so strided views of a packed
 *     [tokens, 2*Hk*K + Hv*V] projection can be passed without a copy.
 *     Batched inputs [B, T, ...] are addressed as token b*T + t.
 *   - State tensors are fp32 [*, Hv, K, V] with V contiguous.  A slot index
 *     array (int64, one entry per sequence) selects rows of a pool; a NULL
 *     index array means row n for sequence n.  A negative slot id means
 *     "no slot": the initial state is taken as zero and no state is written.
 *     An id equal to the id of an earlier sequence in the same index array
 *     also means "no slot" (only the first sequence naming a slot reads and
 *     writes it), so a batch padded by repeating a row -- what the
 *     reference's CUDA-graph runner does, engine/runtime/cuda_graphs.py:
 *     478-482 -- advances each slot exactly once.
 *   - v-head j uses q/k head j / (Hv / Hk) (HF's repeat_interleave GQA).
 */
#ifndef GDN_CAPI_H
#define GDN_CAPI_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GDN_ABI_VERSION 8

typedef enum {
  GDN_OK = 0,
  GDN_ERR_INVALID_ARGUMENT = 1,  /* bad shape, null pointer, bad dtype   */
  GDN_ERR_UNSUPPORTED = 2,       /* valid but not implemented (e.g. K!=128) */
  GDN_ERR_WORKSPACE = 3,         /* workspace missing or too small       */
  GDN_ERR_LAUNCH = 4             /* hipLaunchKernel / hipGetLastError failed */
} gdn_status_t;

typedef enum {
  GDN_DTYPE_F32 = 0,
  GDN_DTYPE_BF16 = 1,
  GDN_DTYPE_F16 = 2
} gdn_dtype_t;

/* Library ABI version (GDN_ABI_VERSION of the build). */
int gdn_abi_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char *gdn_last_error_string(void);

/*
 * Token recurrence: decode (T = 1), speculative verify (T > 1 with
 * snapshots) and small-T prefill.
 *
 * Replaces fla's fused_recurrent_gated_delta_rule, reached from HF's GDN
 * decode branch (transformers modeling_qwen3_5_moe.py:503-515) and held by
 * the reference as the torch path at engine/runtime/cuda_graphs.py:126-135,
 * 201-203; together with the reference cache's gather/scatter around it
 * (engine/runtime/kv_cache.py:189-208), which the slot indices make
 * unnecessary.
 *
 *   q, k      [tokens, Hk, K] (qkv_dtype, token stride q_stride_t/k_stride_t)
 *   v         [tokens, Hv, V] (qkv_dtype, token stride v_stride_t)
 *   g         [tokens, Hv] fp32 log-decay;  beta [tokens, Hv] (beta_dtype)
 *   state_in  fp32 pool of state_in_rows rows, rows selected by state_in_idx
 *             (may be NULL: zero state)
 *   state_out fp32 pool of state_out_rows rows, rows selected by
 *             state_out_idx (may be NULL: not written).  state_out ==
 *             state_in updates the pool in place.
 *   (every *_idx: int64 [n_seqs] on the device, or NULL for row n; an id
 *    outside [0, rows) -- negative ones included -- selects no row: zero
 *    state in, nothing written.  Without ids, rows must be >= n_seqs.)
 *   o         [tokens, Hv, V] (o_dtype, contiguous)
 *   snapshots fp32 [n_seqs, T, Hv, K, V] or NULL; snapshot t = state after
 *             token t (requires cu_seqlens == NULL)
 *   cu_seqlens int32 [n_seqs + 1] (device) or NULL for n_seqs x T tokens
 *   scale     multiplier of q after the optional l2norm (K^-1/2 by default)
 * Requires K in {64, 128, 256} and V a positive multiple of 32 (K == V == 128
 * is the build the decode figures are measured on).
 */
int gdn_recurrent_fwd(const void *q, const void *k, const void *v, int qkv_dtype,
                      int64_t q_stride_t, int64_t k_stride_t, int64_t v_stride_t,
                      const float *g, const void *beta, int beta_dtype,
                      const float *state_in, const int64_t *state_in_idx, int64_t state_in_rows,
                      float *state_out, const int64_t *state_out_idx, int64_t state_out_rows,
                      void *o, int o_dtype, float *snapshots,
                      const int32_t *cu_seqlens, int32_t n_seqs, int32_t T,
                      int32_t Hk, int32_t Hv, int32_t K, int32_t V,
                      float scale, int l2norm_qk, void *stream);

/*
 * gdn_recurrent_fwd with the gates computed in the kernel prologue from the
 * layer's raw projections instead of passed precomputed:
 *   beta = sigmoid(b),  g = -exp(A_log[h]) * softplus(a + dt_bias[h])
 * (softplus(x) = x for x > 20), replacing the torch glue of HF's GDN layer
 * forward (transformers modeling_qwen3_5_moe.py:495-497) and its extra
 * [tokens, Hv] round trips.
 *   a, b     [tokens, Hv] (ab_dtype, token stride ab_stride_t >= Hv)
 *   A_log, dt_bias  fp32 [Hv]
 * Every other argument as for gdn_recurrent_fwd.
 */
int gdn_recurrent_fwd_gated(const void *q, const void *k, const void *v, int qkv_dtype,
                            int64_t q_stride_t, int64_t k_stride_t, int64_t v_stride_t,
                            const void *a, const void *b, int ab_dtype, int64_t ab_stride_t,
                            const float *A_log, const float *dt_bias,
                            const float *state_in, const int64_t *state_in_idx, int64_t state_in_rows,
                            float *state_out, const int64_t *state_out_idx, int64_t state_out_rows,
                            void *o, int o_dtype, float *snapshots,
                            const int32_t *cu_seqlens, int32_t n_seqs, int32_t T,
                            int32_t Hk, int32_t Hv, int32_t K, int32_t V,
                            float scale, int l2norm_qk, void *stream);

/*
 * Chunk-64 prefill (WY/UT form).
 *
 * Replaces engine/kernels/delta_rule.py:352-438 (chunk_gated_delta_rule, the
 * fla-compatible entry) and the kernels behind it: the Helion kernel
 * (delta_rule.py:128-263), the torch fallback (:286-349) and fla's Triton
 * chunk kernels.  Unlike the reference entry, cu_seqlens is honoured.
 *
 *   q, k, v, g, beta as for gdn_recurrent_fwd; tokens = n_seqs*T, or
 *   cu_seqlens[n_seqs] when cu_seqlens (int32, device) is given.
 *   h0  fp32 initial states (h0_rows rows, selected by h0_idx) or NULL for zero
 *   hT  fp32 final states (hT_rows rows, selected by hT_idx) or NULL; hT may
 *       equal h0.  Ids as for gdn_recurrent_fwd.
 *   o   [tokens, Hv, V] o_dtype, contiguous
 *   workspace  device scratch of at least gdn_chunk_workspace_bytes(...),
 *              256-byte aligned (unused, may be NULL, when that is 0)
 * Requires K == V == 128 and q/k/v in bf16 (other head dims and fp16 / fp32
 * q/k/v: gdn_recurrent_fwd, the token recurrence, which the Python entry
 * chunk_gated_delta_rule calls for them).
 */
int gdn_chunk_fwd(const void *q, const void *k, const void *v, int qkv_dtype,
                  int64_t q_stride_t, int64_t k_stride_t, int64_t v_stride_t,
                  const float *g, const void *beta, int beta_dtype,
                  const float *h0, const int64_t *h0_idx, int64_t h0_rows,
                  float *hT, const int64_t *hT_idx, int64_t hT_rows,
                  void *o, int o_dtype,
                  const int32_t *cu_seqlens, int32_t n_seqs, int32_t T,
                  int32_t Hk, int32_t Hv, int32_t K, int32_t V,
                  float scale, int l2norm_qk,
                  void *workspace, size_t workspace_bytes, void *stream);

/*
 * gdn_chunk_fwd with the gates computed in the kernel prologue from the
 * layer's raw projections (a, b, A_log, dt_bias as for
 * gdn_recurrent_fwd_gated; transformers modeling_qwen3_5_moe.py:495-497).
 */
int gdn_chunk_fwd_gated(const void *q, const void *k, const void *v, int qkv_dtype,
                        int64_t q_stride_t, int64_t k_stride_t, int64_t v_stride_t,
                        const void *a, const void *b, int ab_dtype, int64_t ab_stride_t,
                        const float *A_log, const float *dt_bias,
                        const float *h0, const int64_t *h0_idx, int64_t h0_rows,
                        float *hT, const int64_t *hT_idx, int64_t hT_rows,
                        void *o, int o_dtype,
                        const int32_t *cu_seqlens, int32_t n_seqs, int32_t T,
                        int32_t Hk, int32_t Hv, int32_t K, int32_t V,
                        float scale, int l2norm_qk,
                        void *workspace, size_t workspace_bytes, void *stream);

/* Workspace bytes gdn_chunk_fwd(_gated) needs for `total_tokens` tokens in
 * `n_seqs` sequences (an upper bound that needs no knowledge of the lengths).
 * 0 when n_seqs * Hv >= 160: such a batch runs one workgroup per (sequence,
 * v-head) that keeps every chunk operand in LDS, and the workspace pointer
 * may then be NULL.  Batches whose longest sequence has one 64-token chunk,
 * or two at 96 pairs or more (with cu_seqlens: whose total tokens fit one
 * or two chunks), run that kernel too and leave the workspace they are
 * given unused. */
size_t gdn_chunk_workspace_bytes(int32_t n_seqs, int64_t total_tokens,
                                 int32_t Hv, int32_t K, int32_t V);

/*
 * Gated RMS norm of the GDN output, per (token, head) row of D values:
 *   y = weight * x / sqrt(mean(x^2) + eps) * silu(z)
 * in fp32, rounded once to y's dtype.  Replaces HF's RMSNormGated module
 * applied to the core output (transformers modeling_qwen3_5_moe.py:169-185,
 * called at :535-538), one pass instead of its chain of elementwise ops.
 *   x, z, y  [tokens, H, D] with token strides x/z/y_stride_t (elements),
 *            rows contiguous; dtypes bf16, fp16 or fp32 each
 *   weight   [D] (w_dtype)
 * Requires D == 128.
 */
int gdn_rmsnorm_gated_fwd(const void *x, int x_dtype, int64_t x_stride_t,
                          const void *z, int z_dtype, int64_t z_stride_t,
                          const void *weight, int w_dtype,
                          void *y, int y_dtype, int64_t y_stride_t,
                          int64_t n_tokens, int32_t H, int32_t D, float eps, void *stream);

/*
 * Causal depthwise conv, prefill.
 *
 * Replaces causal-conv1d's causal_conv1d_fn as HF's GDN prefill calls it
 * (transformers modeling_qwen3_5_moe.py:462-478 and :220-240; reference pool
 * layout engine/runtime/kv_cache.py:142-156), including the cache update HF
 * does before it (cache_utils.py:1032-1068).
 *
 *   dtype  bf16, fp16 or fp32 storage of x, w, bias, y and the windows
 *          (fp32 arithmetic, one rounding per stored value)
 *   x      [tokens, C] (dtype, token stride x_stride_t, channels contiguous)
 *   w      [C, width] (dtype);  bias [C] (dtype) or NULL
 *   y      [tokens, C] (dtype, token stride y_stride_t)
 *   state_in  [state_in_rows, C, state_len] (dtype) history rows by
 *             state_in_idx, or NULL for zero history
 *   state_out [state_out_rows, C, state_len] (dtype) rows by state_out_idx,
 *             or NULL: the last state_len inputs of cat(history, x) per
 *             sequence.  Ids as for gdn_recurrent_fwd.
 *   cu_seqlens int32 [n_seqs+1] or NULL for n_seqs x T tokens
 * Requires width <= state_len + 1, state_len <= 8, C % 8 == 0.
 */
int causal_conv1d_fwd(const void *x, int64_t x_stride_t, const void *w, const void *bias,
                      void *y, int64_t y_stride_t,
                      const void *state_in, const int64_t *state_in_idx, int64_t state_in_rows,
                      void *state_out, const int64_t *state_out_idx, int64_t state_out_rows,
                      const int32_t *cu_seqlens, int32_t n_seqs, int32_t T,
                      int32_t C, int32_t width, int32_t state_len,
                      int silu, int dtype, void *stream);

/*
 * Causal depthwise conv, decode / verify step (T new tokens per sequence,
 * window updated in place).
 *
 * Replaces causal-conv1d's causal_conv1d_update as HF's GDN decode calls it
 * (transformers modeling_qwen3_5_moe.py:452-461, :200-217), on the
 * reference's slot pool [slots, C, state_len] (engine/runtime/kv_cache.py:
 * 142-146) addressed by slot index instead of gathered.
 *
 *   x [n_seqs*T, C] (token stride x_stride_t), y likewise (y_stride_t);
 *   x, w, bias, y and conv_state share dtype: bf16, fp16 or fp32
 *   conv_state [state_rows, C, state_len], rows by state_idx (NULL: row n);
 *   updated in place.  Ids outside [0, state_rows): zero window, nothing
 *   written.
 */
int causal_conv1d_update(const void *x, int64_t x_stride_t, void *conv_state,
                         const int64_t *state_idx, int64_t state_rows, const void *w, const void *bias,
                         void *y, int64_t y_stride_t, int32_t n_seqs, int32_t T,
                         int32_t C, int32_t width, int32_t state_len,
                         int silu, int dtype, void *stream);

/*
 * Decode-step input projections of the GDN layer with the causal-conv update
 * fused into the epilogue:
 *   p       = x W_qkv^T  (rounded to bf16, as the nn.Linear output)
 *   y_qkv   = act(conv taps . (window[1..3], p) + bias)   per channel
 *   window  <- (window[1..3], p)                          in conv_pool[slot]
 *   z = x W_z^T,  b = x W_b^T,  a = x W_a^T               (bf16)
 *
 * Replaces, for one decode token per row, the four nn.Linear projections
 * of HF's GDN layer (transformers modeling_qwen3_5_moe.py:424-427, called at
 * :443-450) and the causal_conv1d_update that follows (:452-461), on the
 * reference's conv slot pool (engine/runtime/kv_cache.py:142-146).
 *
 *   x       [M, K] bf16, row stride x_stride (elements, >= K, multiple of 8)
 *   w_*     [n_*, K] bf16 nn.Linear weights, rows contiguous (16-byte aligned)
 *   conv_w  [n_qkv, 4] bf16 depthwise taps;  conv_bias [n_qkv] bf16 or NULL
 *   conv_pool [pool_rows, n_qkv, 4] bf16 windows (oldest first), rows by
 *           slot_idx (NULL: row m); ids outside [0, pool_rows): zero window,
 *           nothing written
 *   y_qkv [M, n_qkv], z [M, n_z], b [M, n_b], a [M, n_a] bf16, contiguous
 *   K in {1024, 2048}; n_qkv, n_z multiples of 64;
 *   n_b, n_a multiples of 4, at most 32.  silu: apply SiLU after the conv.
 */
int gdn_in_proj_decode(const void *x, int64_t x_stride, const void *w_qkv, const void *w_z,
                       const void *w_b, const void *w_a, int32_t M, int32_t K, int32_t n_qkv,
                       int32_t n_z, int32_t n_b, int32_t n_a, const void *conv_w, const void *conv_bias,
                       void *conv_pool, const int64_t *slot_idx, int64_t pool_rows, void *y_qkv, void *z,
                       void *b, void *a, int silu, void *stream);

/*
 * Decode-step output projection of the GDN layer:  y = x W^T  (bf16, fp32
 * sums), with K split over workgroups (1024 of K each when K is a multiple of
 * 1024, else 512); a second kernel adds
 * the fp32 partial sums in split order, so results do not depend on
 * scheduling.  One row with K / 512 in {1, 2, 4, 8} runs as a single GEMV
 * kernel (the workspace is then not touched).
 *
 * Replaces, for small M (decode rows), the out_proj nn.Linear of HF's GDN
 * layer (transformers modeling_qwen3_5_moe.py:428, called at :540).
 *
 *   x  [M, K] bf16, row stride x_stride (elements, >= K, multiple of 8), 16-byte aligned
 *   w  [N, K] bf16 nn.Linear weight, rows contiguous, 16-byte aligned
 *   y  [M, N] bf16, row stride y_stride (>= N, multiple of 4), 8-byte aligned
 *   N a multiple of 64; K a multiple of 512, at most 8192
 *   workspace: gdn_out_proj_workspace_bytes(M, K, N) bytes (the partial
 *     sums), 16-byte aligned, used until the second kernel has run
 */
size_t gdn_out_proj_workspace_bytes(int32_t M, int32_t K, int32_t N);
int gdn_out_proj_decode(const void *x, int64_t x_stride, const void *w, int32_t M, int32_t K, int32_t N,
                        void *y, int64_t y_stride, void *workspace, size_t workspace_bytes, void *stream);

/*
 * gdn_out_proj_decode without a workspace argument: allocates nothing.
 *
 * No counterpart in the reference.  It is for callers that cannot allocate
 * device memory at call time -- code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc: the split-K partial sums go to a
 * scratch array built into the library (GDN_OUT_PROJ_NOALLOC_MAX_BYTES per
 * GPU, held from the library's first use on that GPU until the process
 * ends), so the caller passes only x, w and y.  Calls that need more partial
 * sums than that (gdn_out_proj_workspace_bytes(M, K, N) > the maximum; 64
 * rows at K = 4096, N = 2048 need 2 MiB) fail with GDN_ERR_UNSUPPORTED.  All
 * calls on one GPU share the scratch: calls that overlap on one GPU (on two
 * streams) race.  The stream must belong to the current device.  Results are
 * bit-identical to gdn_out_proj_decode's.
 */
#define GDN_OUT_PROJ_NOALLOC_MAX_BYTES ((size_t)8 << 20)
int gdn_out_proj_decode_noalloc(const void *x, int64_t x_stride, const void *w, int32_t M, int32_t K, int32_t N,
                                void *y, int64_t y_stride, void *stream);

/*
 * Speculative-verify commit: pool[slot_ids[b]] = snapshots[b, accepted_len[b]-1].
 * accepted_len[b] <= 0 or slot_ids[b] outside [0, pool_rows) leaves the
 * slot untouched.
 *
 * No reference implementation exists; engine/runtime/spec_decode.py:81-87
 * and :99-103 document the missing GDN rollback this provides.
 *   pool fp32 [pool_rows, H, K, V];  snapshots fp32 [n_seqs, T, H, K, V]
 *   slot_ids int64 [n_seqs];  accepted_len int32 [n_seqs]
 */
int gdn_state_commit(float *pool, const int64_t *slot_ids, int64_t pool_rows, const float *snapshots,
                     const int32_t *accepted_len, int32_t n_seqs, int32_t T,
                     int32_t H, int32_t K, int32_t V, void *stream);

/*
 * Speculative-verify commit of the causal-conv window:
 *   pool[slot_ids[b]][c][j] = hist[b][c][a + j]   (j < S, a = min(accepted_len[b], L - S))
 * where hist[b] is the verify step's conv history: the S-column window
 * before the step followed by the step's L - S inputs, so columns
 * [a, a + S) are the window after the first a tokens.  accepted_len[b] <= 0
 * or slot_ids[b] outside [0, pool_rows) leaves the slot untouched.  Rolls back the conv state
 * that engine/runtime/spec_decode.py:81-87 leaves without a rollback.
 *   pool [pool_rows, C, S] and hist [n_seqs, C, L] of dtype (bf16, fp16 or fp32)
 *   slot_ids int64 [n_seqs];  accepted_len int32 [n_seqs]
 */
int gdn_conv_state_commit(void *pool, const int64_t *slot_ids, int64_t pool_rows, const void *hist,
                          const int32_t *accepted_len, int32_t n_seqs, int32_t C, int32_t S,
                          int32_t L, int32_t dtype, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* GDN_CAPI_H */
