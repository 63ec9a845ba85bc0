"""Numpy restatement of the GDN layer's projections around the path -- test
infrastructure only.

The decode step's input side (four bias-free ``nn.Linear`` and the conv
window update, transformers 5.15.0 modeling_qwen3_5_moe.py:424-427,
443-461) and its output projection (:420, applied at :540), on bf16-valued
inputs in float64.
"""
from __future__ import annotations

import numpy as np

from . import conv


def round_bf16(x) -> np.ndarray:
    """Round to the nearest bfloat16 (ties to even), returned as float64.

    The value an ``nn.Linear`` with bf16 output stores: fp32 bits rounded
    by adding 0x7FFF plus the lowest kept bit, then truncating the low 16
    bits (finite inputs)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    return u.astype(np.uint32).view(np.float32).astype(np.float64)


def in_proj_decode(x, w_qkv, w_z, w_b, w_a, conv_weight, conv_state, conv_bias=None, activation="silu",
                   dtype=np.float64):
    """One decode token per row through HF's GDN input side.

    Follows transformers 5.15.0 ``Qwen3_5MoeGatedDeltaNet.forward``
    (modeling_qwen3_5_moe.py:443-461): the four bias-free ``nn.Linear``
    projections of the hidden rows x [M, K] (weights [n, K]), the qkv one
    stored in bf16 (the layer's dtype) before ``causal_conv1d_update``
    (:200-217, restated above) advances each row's window [M, C, S].
    Returns ``(y [M, C], z [M, n_z], b [M, n_b], a [M, n_a], new_state)``;
    z, b, a unrounded (dtype), y and the state as the conv update gives them.
    """
    x = np.asarray(x, dtype)
    p = x @ np.asarray(w_qkv, dtype).T
    z = x @ np.asarray(w_z, dtype).T
    b = x @ np.asarray(w_b, dtype).T
    a = x @ np.asarray(w_a, dtype).T
    y, new_state = conv.causal_conv1d_update(round_bf16(p)[:, :, None], conv_state, conv_weight, conv_bias,
                                        activation=activation, dtype=dtype)
    return y[:, :, 0], z, b, a, new_state


def out_proj(x, w, dtype=np.float64):
    """The layer's ``out_proj`` over decode rows: a bias-free ``nn.Linear``
    (transformers 5.15.0 modeling_qwen3_5_moe.py:420, applied at :540),
    x [M, K] @ w [N, K]^T, unrounded (the module stores it in bf16)."""
    return np.asarray(x, dtype) @ np.asarray(w, dtype).T
