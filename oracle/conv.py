"""Numpy restatement of the GDN causal depthwise conv -- test infrastructure only.

Layout follows HF: x [B, C, T] (channels, then time), weight [C, W].
The engine's GDN layers use W = 4, no bias, SiLU (transformers 5.15.0
modeling_qwen3_5_moe.py:403-410; configuration_qwen3_5_moe.py:95).
"""
from __future__ import annotations

import numpy as np


def silu(x):
    return x / (1.0 + np.exp(-x))


def causal_conv1d_fn(x, weight, bias=None, activation="silu", initial_state=None,
                     dtype=np.float64):
    """y[c, t] = act(sum_i w[c, i] x[c, t - (W-1) + i] + bias[c]), x[c, <0] = history.

    Follows transformers 5.15.0 ``causal_conv1d_fn`` (modeling_qwen3_5_moe.py:
    220-240): a grouped ``F.conv1d`` with left zero padding W-1, truncated to T.
    ``initial_state`` [B, C, S] (S >= W-1) supplies the history instead of
    zeros, which is what HF does for a prefill continuation
    (cache_utils.py:1049-1068 concatenates the cached window in front of x).
    Returns ``(y [B, C, T], final_state [B, C, S])`` where the final state is
    the last S inputs of cat(history, x) (cache_utils.py:1062-1064).
    """
    x = np.asarray(x, dtype)
    w = np.asarray(weight, dtype)
    b_, c, t_len = x.shape
    width = w.shape[-1]
    s_len = width if initial_state is None else np.asarray(initial_state).shape[-1]
    hist = (np.zeros((b_, c, s_len), dtype) if initial_state is None
            else np.asarray(initial_state, dtype))
    full = np.concatenate([hist, x], axis=-1)               # [B, C, S + T]
    y = np.zeros((b_, c, t_len), dtype)
    for i in range(width):
        # output t uses full[s_len + t - (width-1) + i]
        start = s_len - (width - 1) + i
        y += w[None, :, i, None] * full[:, :, start:start + t_len]
    if bias is not None:
        y += np.asarray(bias, dtype)[None, :, None]
    if activation in ("silu", "swish"):
        y = silu(y)
    final = full[:, :, -s_len:].copy()
    return y, final


def causal_conv1d_update(x, conv_state, weight, bias=None, activation="silu", dtype=np.float64):
    """Decode step(s) of the conv with an in-place window.

    Follows transformers 5.15.0 ``causal_conv1d_update`` (modeling_qwen3_5_moe.py:
    200-217): cat(state, x) along time, keep the last S columns as the new
    state, grouped conv without padding, keep the last T outputs.
    Returns ``(y [B, C, T], new_state [B, C, S])``.
    """
    x = np.asarray(x, dtype)
    st = np.asarray(conv_state, dtype)
    w = np.asarray(weight, dtype)
    t_len = x.shape[-1]
    width = w.shape[-1]
    full = np.concatenate([st, x], axis=-1)
    new_state = full[:, :, -st.shape[-1]:].copy()
    n_out = full.shape[-1] - width + 1
    y = np.zeros(x.shape[:2] + (n_out,), dtype)
    for i in range(width):
        y += w[None, :, i, None] * full[:, :, i:i + n_out]
    y = y[:, :, -t_len:]
    if bias is not None:
        y += np.asarray(bias, dtype)[None, :, None]
    if activation in ("silu", "swish"):
        y = silu(y)
    return y, new_state


def causal_conv1d_varlen(x_tc, weight, cu_seqlens, bias=None, activation="silu",
                         initial_states=None, state_len=None, dtype=np.float64):
    """Packed-varlen conv over a token-major stream x [sum L, C].

    Each sequence restarts its window (zero history, or ``initial_states[n]``
    [C, S]).  Returns ``(y [sum L, C], final_states [N, C, S])``.
    """
    x_tc = np.asarray(x_tc, dtype)
    width = np.asarray(weight).shape[-1]
    s_len = state_len or width
    n = len(cu_seqlens) - 1
    y = np.zeros_like(x_tc)
    finals = np.zeros((n, x_tc.shape[1], s_len), dtype)
    for i in range(n):
        a, b = int(cu_seqlens[i]), int(cu_seqlens[i + 1])
        h0 = None if initial_states is None else np.asarray(initial_states)[i:i + 1]
        yi, fi = causal_conv1d_fn(x_tc[a:b].T[None], weight, bias, activation,
                                  initial_state=h0, dtype=dtype)
        y[a:b] = yi[0].T
        finals[i] = fi[0]
    return y, finals

