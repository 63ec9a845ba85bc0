"""Numpy restatement of the Gated DeltaNet math -- test infrastructure only.

Layouts follow the fla / HF convention used by the reference:
  q, k      [B, T, Hk, K]   (Hk may be smaller than H: v-head j uses k-head j // (H // Hk))
  v         [B, T, H, V]
  g, beta   [B, T, H]       (g is the per-token log-decay, <= 0)
  state     [B, H, K, V]    (fp32 in the engine; K rows, V contiguous)
  o         [B, T, H, V]

Every function computes in ``dtype`` (float64 by default, float32 for the
CPU baseline) and returns arrays of that dtype.
"""
from __future__ import annotations

import numpy as np


def expand_heads(x: np.ndarray, h: int) -> np.ndarray:
    """GQA lift of q/k from Hk to H heads.

    Same as ``repeat_interleave(H // Hk, dim=2)`` in HF's GDN forward
    (transformers 5.15.0 modeling_qwen3_5_moe.py:498-500): repeated head j
    is source head j // (H // Hk).
    """
    hk = x.shape[2]
    if hk == h:
        return x
    if h % hk:
        raise ValueError(f"H={h} is not a multiple of Hk={hk}")
    return np.repeat(x, h // hk, axis=2)


def l2norm(x: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """x * rsqrt(sum(x^2) + eps) over the last axis.

    Follows engine/kernels/delta_rule.py:281-283 (``_l2norm``).
    """
    return x / np.sqrt((x * x).sum(axis=-1, keepdims=True) + eps)


def softplus(x: np.ndarray) -> np.ndarray:
    """torch.nn.functional.softplus with its default threshold: x for x > 20,
    log(1 + e^x) otherwise."""
    x = np.asarray(x)
    return np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20))))


def gdn_gates(a, b, A_log, dt_bias, dtype=np.float64):
    """The GDN layer's gates from its raw projections.

    Follows transformers 5.15.0 modeling_qwen3_5_moe.py:495-497 (the layer
    forward the reference runs): ``beta = b.sigmoid()``,
    ``g = -A_log.float().exp() * softplus(a.float() + dt_bias)``.
    a, b [..., H]; A_log, dt_bias [H].  Returns (g, beta).
    """
    a, b, A_log, dt_bias = (np.asarray(x, dtype=dtype) for x in (a, b, A_log, dt_bias))
    beta = 1.0 / (1.0 + np.exp(-b))
    g = -np.exp(A_log) * softplus(a + dt_bias)
    return g, beta


def rms_norm_gated(x, z, weight, eps=1e-6, dtype=np.float64):
    """Gated RMS norm over the last axis:
    ``weight * x / sqrt(mean(x^2) + eps) * silu(z)``.

    Follows transformers 5.15.0 ``Qwen3_5MoeRMSNormGated.forward``
    (modeling_qwen3_5_moe.py:169-185), applied to the GDN core output at
    :535-538, in one precision (the module rounds x * rsqrt(.) to the input
    dtype before the weight; in fp32 that rounding is the identity).
    """
    x, z, weight = (np.asarray(t, dtype=dtype) for t in (x, z, weight))
    r = 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    return weight * (x * r) * (z / (1.0 + np.exp(-z)))


def _prep(q, k, v, g, beta, use_qk_l2norm, dtype):
    q, k, v, g, beta = (np.asarray(a, dtype=dtype) for a in (q, k, v, g, beta))
    h = v.shape[2]
    if use_qk_l2norm:
        # the reference normalises before the GQA repeat; the result is the same
        q = l2norm(q)
        k = l2norm(k)
    return expand_heads(q, h), expand_heads(k, h), v, g, beta


def recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=None, output_final_state=True,
                               use_qk_l2norm_in_kernel=True, scale=None, dtype=np.float64,
                               return_snapshots=False):
    """Token-by-token gated delta rule.

    Follows transformers 5.15.0 ``torch_recurrent_gated_delta_rule``
    (models/qwen3_5_moe/modeling_qwen3_5_moe.py:331-381), which the reference
    imports at engine/runtime/cuda_graphs.py:126-135 and which fla's
    ``fused_recurrent_gated_delta_rule`` implements on the GPU:

        S <- exp(g_t) S ;  u = k_t^T S ;  d = beta_t (v_t - u) ;
        S <- S + k_t d^T ;  o_t = (scale q_t)^T S

    Returns ``(o, final_state_or_None)`` or, with ``return_snapshots``,
    ``(o, final_state, snapshots[B, T, H, K, V])`` where snapshot t is the
    state after token t.
    """
    q, k, v, g, beta = _prep(q, k, v, g, beta, use_qk_l2norm_in_kernel, dtype)
    b, t_len, h, dk = k.shape
    dv = v.shape[-1]
    if scale is None:
        scale = dk ** -0.5
    q = q * dtype(scale)
    s = (np.zeros((b, h, dk, dv), dtype) if initial_state is None
         else np.array(initial_state, dtype=dtype, copy=True))
    o = np.zeros((b, t_len, h, dv), dtype)
    snaps = np.zeros((b, t_len, h, dk, dv), dtype) if return_snapshots else None
    for t in range(t_len):
        s = s * np.exp(g[:, t])[:, :, None, None]
        kv_mem = np.einsum("bhk,bhkv->bhv", k[:, t], s)
        delta = (v[:, t] - kv_mem) * beta[:, t][:, :, None]
        s = s + k[:, t][:, :, :, None] * delta[:, :, None, :]
        o[:, t] = np.einsum("bhk,bhkv->bhv", q[:, t], s)
        if snaps is not None:
            snaps[:, t] = s
    if return_snapshots:
        return o, s, snaps
    return o, (s if output_final_state else None)


def forward_substitution_inverse(attn: np.ndarray) -> np.ndarray:
    """The reference's in-place row loop that turns -L into (I + L)^-1 - I.

    Follows engine/kernels/delta_rule.py:319-322: for i = 1..C-1,
    ``attn[i, :i] += attn[i, :i] @ attn[:i, :i]``.  ``attn`` holds
    ``-L`` (strictly lower) on entry; the caller adds the identity.
    """
    attn = attn.copy()
    c = attn.shape[-1]
    for i in range(1, c):
        row = attn[..., i, :i].copy()
        sub = attn[..., :i, :i].copy()
        attn[..., i, :i] = row + (row[..., :, None] * sub).sum(-2)
    return attn


def chunk_gated_delta_rule(q, k, v, g, beta, chunk_size=64, initial_state=None,
                           output_final_state=True, use_qk_l2norm_in_kernel=True,
                           scale=None, dtype=np.float64):
    """Chunked (WY/UT) gated delta rule, op for op.

    Follows engine/kernels/delta_rule.py:286-349 (``_torch_fallback``), a
    line-for-line copy of transformers' ``torch_chunk_gated_delta_rule``:
    zero-pad T to a multiple of the chunk, chunk-local cumsum of g, decay
    mask exp(gamma_i - gamma_j) masked before exp, forward substitution for
    T = (I + L)^-1, U = T (beta v), W = T (beta e^gamma k), then the serial
    chunk scan for the output and the state.
    """
    q, k, v, g, beta = _prep(q, k, v, g, beta, use_qk_l2norm_in_kernel, dtype)
    # [B, T, H, D] -> [B, H, T, D]    (delta_rule.py:295-297)
    q, k, v = (np.ascontiguousarray(x.transpose(0, 2, 1, 3)) for x in (q, k, v))
    g, beta = (np.ascontiguousarray(x.transpose(0, 2, 1)) for x in (g, beta))
    b, h, t_len, dk = k.shape
    dv = v.shape[-1]
    c = chunk_size
    pad = (c - t_len % c) % c                                        # :300
    if pad:
        q, k, v = (np.pad(x, ((0, 0), (0, 0), (0, pad), (0, 0))) for x in (q, k, v))
        g, beta = (np.pad(x, ((0, 0), (0, 0), (0, pad))) for x in (g, beta))
    tp = t_len + pad
    if scale is None:
        scale = dk ** -0.5
    q = q * dtype(scale)                                             # :307
    vb = v * beta[..., None]                                         # :309
    kb = k * beta[..., None]                                         # :310
    nc = tp // c
    q, k, v, kb, vb = (x.reshape(b, h, nc, c, x.shape[-1]) for x in (q, k, v, kb, vb))
    g = g.reshape(b, h, nc, c).cumsum(-1)                            # :314-316
    diff = g[..., :, None] - g[..., None, :]
    lower = np.tril(np.ones((c, c), dtype=bool))
    decay = np.where(lower, np.exp(np.where(lower, diff, 0.0)), 0.0).astype(dtype)  # :317
    upper = ~np.tril(np.ones((c, c), dtype=bool), -1)                # triu(diagonal=0)
    attn = -np.where(upper, 0.0, (kb @ np.swapaxes(k, -1, -2)) * decay).astype(dtype)  # :318
    attn = forward_substitution_inverse(attn)                        # :319-322
    attn = attn + np.eye(c, dtype=dtype)                             # :323
    u = attn @ vb                                                    # :324
    w = attn @ (kb * np.exp(g)[..., None])                           # :325
    s = (np.zeros((b, h, dk, dv), dtype) if initial_state is None
         else np.array(initial_state, dtype=dtype, copy=True))      # :326-330
    o = np.zeros_like(u)
    strict_upper = ~np.tril(np.ones((c, c), dtype=bool))             # triu(diagonal=1)
    for i in range(nc):                                              # :333-343
        q_i, k_i, u_i = q[:, :, i], k[:, :, i], u[:, :, i]
        a = np.where(strict_upper, 0.0, (q_i @ np.swapaxes(k_i, -1, -2)) * decay[:, :, i])
        v_new = u_i - w[:, :, i] @ s
        inter = (q_i * np.exp(g[:, :, i])[..., None]) @ s
        o[:, :, i] = inter + a @ v_new
        g_last = g[:, :, i, -1]
        kd = k_i * np.exp(g_last[..., None] - g[:, :, i])[..., None]
        s = s * np.exp(g_last)[..., None, None] + np.swapaxes(kd, -1, -2) @ v_new
    o = o.reshape(b, h, tp, dv)[:, :, :t_len]                        # :347
    o = np.ascontiguousarray(o.transpose(0, 2, 1, 3))                # :348
    return o, (s if output_final_state else None)


def _split_varlen(x, cu_seqlens, i):
    return x[:, int(cu_seqlens[i]):int(cu_seqlens[i + 1])]


def chunk_gated_delta_rule_varlen(q, k, v, g, beta, cu_seqlens, initial_state=None,
                                  chunk_size=64, use_qk_l2norm_in_kernel=True, scale=None,
                                  dtype=np.float64):
    """Packed-varlen prefill: B=1, sequences delimited by ``cu_seqlens`` [N+1].

    The reference entry swallows ``cu_seqlens`` (delta_rule.py:362), so its
    meaning here is fla's: each sequence is an independent call with its own
    initial state ``initial_state[n]``; chunks never straddle a boundary.
    Returns ``(o[1, sum L, H, V], final_states[N, H, K, V])``.
    """
    n = len(cu_seqlens) - 1
    h = np.asarray(v).shape[2]
    dk, dv = np.asarray(k).shape[-1], np.asarray(v).shape[-1]
    o = np.zeros(np.asarray(v).shape, dtype)
    finals = np.zeros((n, h, dk, dv), dtype)
    for i in range(n):
        h0 = None if initial_state is None else np.asarray(initial_state)[i:i + 1]
        parts = [_split_varlen(np.asarray(a), cu_seqlens, i) for a in (q, k, v, g, beta)]
        if parts[0].shape[1] == 0:
            finals[i] = 0.0 if h0 is None else h0[0]
            continue
        oi, si = chunk_gated_delta_rule(*parts, chunk_size=chunk_size, initial_state=h0,
                                        output_final_state=True,
                                        use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel,
                                        scale=scale, dtype=dtype)
        o[:, int(cu_seqlens[i]):int(cu_seqlens[i + 1])] = oi
        finals[i] = si[0]
    return o, finals


def recurrent_gated_delta_rule_varlen(q, k, v, g, beta, cu_seqlens, initial_state=None,
                                      use_qk_l2norm_in_kernel=True, scale=None, dtype=np.float64):
    """Packed-varlen token recurrence (fla ``cu_seqlens`` meaning, as above)."""
    n = len(cu_seqlens) - 1
    h = np.asarray(v).shape[2]
    dk, dv = np.asarray(k).shape[-1], np.asarray(v).shape[-1]
    o = np.zeros(np.asarray(v).shape, dtype)
    finals = np.zeros((n, h, dk, dv), dtype)
    for i in range(n):
        h0 = None if initial_state is None else np.asarray(initial_state)[i:i + 1]
        parts = [_split_varlen(np.asarray(a), cu_seqlens, i) for a in (q, k, v, g, beta)]
        oi, si = recurrent_gated_delta_rule(*parts, initial_state=h0,
                                            use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel,
                                            scale=scale, dtype=dtype)
        o[:, int(cu_seqlens[i]):int(cu_seqlens[i + 1])] = oi
        finals[i] = si[0]
    return o, finals


def slot_recurrent_step(pool, slot_ids, q, k, v, g, beta, use_qk_l2norm_in_kernel=True,
                        scale=None, dtype=np.float64):
    """Decode against a slot pool: gather rows, run the recurrence, scatter back.

    Restates what the reference cache does around each forward
    (engine/runtime/kv_cache.py:189-208: ``index_select(...).clone()`` then
    ``index_copy_``).  A negative slot id means "no slot": zero initial
    state and nothing written back.  Returns ``(o, new_pool)``.
    """
    pool = np.array(pool, dtype=dtype, copy=True)
    slot_ids = np.asarray(slot_ids)
    h, dk, dv = pool.shape[1:]
    h0 = np.zeros((len(slot_ids), h, dk, dv), dtype)
    live = slot_ids >= 0
    h0[live] = pool[slot_ids[live]]
    o, s = recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=h0,
                                      use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel,
                                      scale=scale, dtype=dtype)
    pool[slot_ids[live]] = s[live]
    return o, pool


def spec_verify(pool, slot_ids, q, k, v, g, beta, accepted_len, use_qk_l2norm_in_kernel=True,
                scale=None, dtype=np.float64):
    """Speculative-verify: T draft tokens per sequence with per-step snapshots.

    There is no reference implementation; engine/runtime/spec_decode.py:81-87
    and :99-103 state the need ("requires saving state snapshots").  Defined by
    the recurrence: snapshot[b, t] is the state after t+1 tokens, and the
    commit writes snapshot[b, accepted_len[b] - 1] into pool[slot_ids[b]].
    Returns ``(o, snapshots, committed_pool)``.
    """
    pool = np.array(pool, dtype=dtype, copy=True)
    h0 = pool[np.asarray(slot_ids)]
    o, _, snaps = recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=h0,
                                             use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel,
                                             scale=scale, dtype=dtype, return_snapshots=True)
    for b, (slot, acc) in enumerate(zip(np.asarray(slot_ids), np.asarray(accepted_len))):
        if slot >= 0 and acc > 0:
            pool[slot] = snaps[b, acc - 1]
    return o, snaps, pool


def state_rel_err(got, ref) -> float:
    """Norm-wise relative error ||got - ref||_F / ||ref||_F per (seq, head), max over all."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    num = np.sqrt(((got - ref) ** 2).sum(axis=(-1, -2)))
    den = np.sqrt((ref ** 2).sum(axis=(-1, -2)))
    return float((num / np.maximum(den, 1e-30)).max())
