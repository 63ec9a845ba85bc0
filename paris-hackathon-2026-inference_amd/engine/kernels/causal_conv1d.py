"""Causal depthwise conv1d (+ SiLU) on the MI355X: GDN prefill and decode.

Drop-ins for causal-conv1d's ``causal_conv1d_fn`` / ``causal_conv1d_update``
with the signatures HF's GDN layer uses (transformers
modeling_qwen3_5_moe.py:200-240, called at :452-478), extended with packed
varlen (``cu_seqlens``) and slot-indexed window pools (the reference holds
them as ``_pool_conv_states [slots, conv_dim, 4]`` bf16,
engine/runtime/kv_cache.py:142-146, 175-178).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib


def _act(activation) -> int:
    if activation in (None, False):
        return 0
    if activation in ("silu", "swish", True):
        return 1
    raise ValueError(f"unsupported activation {activation!r} (None or 'silu')")


def _stream_view(x: torch.Tensor) -> tuple[torch.Tensor, int, int, int, bool]:
    """Token-major view of x: returns (xt, token stride, B, T, was_bct).

    The kernel addresses token i (= b*T + t) at ``xt + i*stride`` with the
    channels contiguous and 16-byte aligned; anything else is copied.
    """
    if x.dim() == 2:                      # [tokens, C]
        n, c = x.shape
        st = x.stride(0) if n > 1 else c
        if x.stride(1) != 1 or st % 8 or x.storage_offset() % 8:
            x = x.contiguous()
            st = c
        return x, st, 1, n, False
    if x.dim() != 3:
        raise ValueError(f"x must be [B, C, T] or [tokens, C], got {tuple(x.shape)}")
    b, c, t = x.shape
    xt = x.transpose(1, 2)                # [B, T, C]
    st = xt.stride(1) if t > 1 else (xt.stride(0) if b > 1 else c)
    if xt.stride(2) != 1 or st % 8 or xt.storage_offset() % 8 or (b > 1 and t > 1 and xt.stride(0) != t * st):
        xt = xt.contiguous()
        st = c
    return xt, st, b, t, True


def causal_conv1d_fn(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    activation=None,
    *,
    cu_seqlens: Optional[torch.Tensor] = None,
    initial_states: Optional[torch.Tensor] = None,
    conv_states: Optional[torch.Tensor] = None,
    cache_indices: Optional[torch.Tensor] = None,
    has_initial_state: Optional[torch.Tensor] = None,
    return_final_states: bool = False,
    final_states_out: Optional[torch.Tensor] = None,
    **_ignored,
):
    """y = act(causal depthwise conv(x, weight) + bias), zero or cached history.

    x: ``[B, C, T]`` (HF layout, usually a transposed view of ``[B, T, C]``)
    or a token-major ``[tokens, C]`` stream.  weight ``[C, W]`` (W <= 4).
    With ``cu_seqlens`` [N+1] the tokens are N packed sequences (B = 1) and
    every sequence restarts its window.

    History / final windows (width S = 4 as HF caches, or the shape's last dim):
      * ``initial_states`` [N, C, S]: history per sequence (default zeros);
      * ``conv_states`` pool [slots, C, S] + ``cache_indices`` [N]: history is
        read from and the final window written back to ``pool[idx]`` (rows
        with ``has_initial_state`` False start from zeros; negative indices
        are skipped);
      * ``return_final_states`` / ``final_states_out`` [N, C, S]: final windows.
    Returns y (same layout as x), or ``(y, final_states)``.
    """
    dev = _lib.require_gpu(x, weight, bias, initial_states, conv_states, final_states_out)
    dt = x.dtype
    if dt not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"causal_conv1d_fn: dtype {dt} unsupported (bf16, fp16 or fp32)")
    w = weight.to(dt).contiguous()
    bb = None if bias is None else bias.to(dt).contiguous()
    xt, xs, b, t, was_bct = _stream_view(x)
    c = xt.shape[-1]
    if w.dim() != 2 or w.shape[0] != c:
        raise ValueError(f"weight must be [C={c}, W], got {tuple(weight.shape)}")
    cu = _lib.as_cu_seqlens(cu_seqlens, dev)
    if cu is not None and b != 1:
        raise ValueError("cu_seqlens requires B == 1")
    n_seqs = cu.numel() - 1 if cu is not None else b

    state_in = state_out = None
    in_idx = out_idx = None
    s_len = 4 if w.shape[1] > 1 else 3
    if conv_states is not None:
        if conv_states.dtype != dt or not conv_states.is_contiguous() or conv_states.shape[1] != c:
            raise ValueError("conv_states must be a contiguous [slots, C, S] pool of x's dtype")
        s_len = conv_states.shape[2]
        idx = _lib.as_index(cache_indices, dev)
        if idx is None and conv_states.shape[0] != n_seqs:
            raise ValueError("conv_states without cache_indices needs one row per sequence")
        state_in = state_out = conv_states
        out_idx = idx
        in_idx = idx
        if has_initial_state is not None:
            base = idx if idx is not None else torch.arange(n_seqs, device=dev)
            has = has_initial_state.to(dev).bool().reshape(-1)
            if idx is not None:  # a repeated slot id neither reads nor writes: decide it on the unmasked ids
                has = has & ~(base[:, None] == base[None, :]).tril(-1).any(dim=1)
            in_idx = torch.where(has, base, torch.full_like(base, -1))
    if initial_states is not None:
        if initial_states.shape[:2] != (n_seqs, c):
            raise ValueError(f"initial_states must be [{n_seqs}, {c}, S]")
        state_in, in_idx = initial_states.to(dt).contiguous(), None
        s_len = state_in.shape[2]
    final = None
    if final_states_out is not None or return_final_states:
        final = final_states_out if final_states_out is not None else torch.empty(
            (n_seqs, c, s_len), dtype=dt, device=dev)
        if final.shape != (n_seqs, c, s_len) or final.dtype != dt or not final.is_contiguous():
            raise ValueError(f"final_states_out must be contiguous [{n_seqs}, {c}, {s_len}] {dt}")
        state_out, out_idx = final, None

    y = torch.empty((b * t, c), dtype=dt, device=dev)
    lib = _lib.load()
    st = lib.causal_conv1d_fwd(
        _lib.ptr(xt), xs, _lib.ptr(w), _lib.ptr(bb), _lib.ptr(y), c,
        _lib.ptr(state_in), _lib.ptr(in_idx), _lib.rows_of(state_in),
        _lib.ptr(state_out), _lib.ptr(out_idx), _lib.rows_of(state_out),
        _lib.ptr(cu), n_seqs, b * t if cu is not None else t,
        c, w.shape[1], s_len, _act(activation), _lib.GDN_DTYPE[dt], _lib.stream_of(y))
    _lib.check(st, "causal_conv1d_fwd")
    y = y.view(b, t, c).transpose(1, 2) if was_bct else y
    return (y, final) if (return_final_states or final_states_out is not None) else y


def causal_conv1d_update(
    x: torch.Tensor,
    conv_state: torch.Tensor,
    weight: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    activation=None,
    conv_state_indices: Optional[torch.Tensor] = None,
    **_ignored,
) -> torch.Tensor:
    """One (or T) decode step(s): shift ``conv_state`` in place, return the conv.

    x ``[B, C, T]`` (or ``[B, C]`` for T = 1); conv_state ``[B, C, S]``, or a
    pool ``[slots, C, S]`` addressed by ``conv_state_indices`` [B]
    (negative = zero window, not written).  Matches HF's
    ``causal_conv1d_update`` (modeling_qwen3_5_moe.py:200-217).
    """
    dev = _lib.require_gpu(x, conv_state, weight, bias)
    squeeze = x.dim() == 2
    x3 = x.unsqueeze(-1) if squeeze else x
    b, c, t = x3.shape
    dt = x.dtype
    if dt not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"causal_conv1d_update: dtype {dt} unsupported (bf16, fp16 or fp32)")
    if conv_state.dtype != dt or not conv_state.is_contiguous() or conv_state.shape[1] != c:
        raise ValueError("conv_state must be a contiguous [*, C, S] tensor of x's dtype")
    idx = _lib.as_index(conv_state_indices, dev)
    if idx is None and conv_state.shape[0] != b:
        raise ValueError("conv_state has a row count different from the batch and no indices")
    w = weight.to(dt).contiguous()
    bb = None if bias is None else bias.to(dt).contiguous()
    xt = x3.transpose(1, 2)                       # [B, T, C]
    if xt.stride(2) != 1 or (b > 1 and xt.stride(0) != t * xt.stride(1)):
        xt = xt.contiguous()
    xs = xt.stride(1) if t > 1 else (xt.stride(0) if b > 1 else c)
    y = torch.empty((b, t, c), dtype=dt, device=dev)
    lib = _lib.load()
    st = lib.causal_conv1d_update(
        _lib.ptr(xt), xs, _lib.ptr(conv_state), _lib.ptr(idx), _lib.rows_of(conv_state), _lib.ptr(w), _lib.ptr(bb),
        _lib.ptr(y), c, b, t, c, w.shape[1], conv_state.shape[2], _act(activation),
        _lib.GDN_DTYPE[dt], _lib.stream_of(y))
    _lib.check(st, "causal_conv1d_update")
    y = y.transpose(1, 2)
    return y.squeeze(-1) if squeeze else y
