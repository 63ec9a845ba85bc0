"""Slot-indexed GDN state pools and the speculative-verify commit.

The reference keeps one GDN layer's state as two slot pools
(``_LinearAttentionSlotLayer``, engine/runtime/kv_cache.py:134-212):
recurrent ``[slots, Hv, K, V]`` fp32 and conv ``[slots, conv_dim, 4]`` bf16,
gathered with ``index_select(...).clone()`` before each forward and
scattered back with ``index_copy_`` after it (:189-208).  Here the kernels
address the pools by slot id (engine/runtime/slot_pools.py owns the tensors);
decode, prefill and the spec-verify commits of both the recurrent state and
the conv window update them in place.
"""
from __future__ import annotations

import torch

from . import _lib


def gdn_state_commit(pool: torch.Tensor, slot_ids: torch.Tensor, snapshots: torch.Tensor,
                     accepted_len: torch.Tensor) -> torch.Tensor:
    """``pool[slot_ids[b]] = snapshots[b, accepted_len[b] - 1]`` on the GPU, in place.

    ``accepted_len[b] <= 0`` or a slot outside the pool leaves that slot untouched;
    values above T are clamped to T.  There is no reference implementation:
    engine/runtime/spec_decode.py:81-87 and :99-103 document the missing
    GDN rollback ("requires saving state snapshots").
    """
    dev = _lib.require_gpu(pool, snapshots)
    if pool.dtype != torch.float32 or snapshots.dtype != torch.float32:
        raise TypeError("pool and snapshots must be fp32")
    if not pool.is_contiguous() or not snapshots.is_contiguous():
        raise ValueError("pool and snapshots must be contiguous")
    n, t, h, k, v = snapshots.shape
    if pool.shape[1:] != (h, k, v):
        raise ValueError(f"pool {tuple(pool.shape)} does not match snapshots {tuple(snapshots.shape)}")
    idx = _lib.as_index(slot_ids, dev)
    acc = accepted_len.to(device=dev, dtype=torch.int32).contiguous()
    if idx.numel() != n or acc.numel() != n:
        raise ValueError("slot_ids and accepted_len need one entry per sequence")
    st = _lib.load().gdn_state_commit(_lib.ptr(pool), _lib.ptr(idx), _lib.rows_of(pool), _lib.ptr(snapshots), _lib.ptr(acc),
                                      n, t, h, k, v, _lib.stream_of(pool))
    _lib.check(st, "gdn_state_commit")
    return pool


def gdn_conv_state_commit(pool: torch.Tensor, slot_ids: torch.Tensor, hist: torch.Tensor,
                          accepted_len: torch.Tensor) -> torch.Tensor:
    """Roll a causal-conv state pool back to the window after each
    sequence's accepted tokens, on the GPU, in place.

    ``hist`` ``[N, C, S + T]`` is a verify step's conv history: the S-column
    window before the step, then the step's T inputs; the window after the
    first ``a = accepted_len[b]`` tokens is ``hist[b, :, a:a + S]`` (a clamped
    to T).  ``accepted_len[b] <= 0`` or a negative slot leaves that slot
    untouched.  The conv half of the rollback that
    engine/runtime/spec_decode.py:81-87 leaves unimplemented.
    """
    dev = _lib.require_gpu(pool, hist)
    if pool.dtype != hist.dtype or pool.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError("pool and hist must share a dtype, bf16, fp16 or fp32")
    if not pool.is_contiguous() or not hist.is_contiguous():
        raise ValueError("pool and hist must be contiguous")
    n, c, length = hist.shape
    s = pool.shape[2]
    if pool.shape[1] != c or length <= s:
        raise ValueError(f"hist {tuple(hist.shape)} does not extend pool windows {tuple(pool.shape)}")
    idx = _lib.as_index(slot_ids, dev)
    acc = accepted_len.to(device=dev, dtype=torch.int32).contiguous()
    if idx.numel() != n or acc.numel() != n:
        raise ValueError("slot_ids and accepted_len need one entry per sequence")
    st = _lib.load().gdn_conv_state_commit(_lib.ptr(pool), _lib.ptr(idx), _lib.rows_of(pool), _lib.ptr(hist), _lib.ptr(acc),
                                           n, c, s, length, _lib.GDN_DTYPE[pool.dtype], _lib.stream_of(pool))
    _lib.check(st, "gdn_conv_state_commit")
    return pool
