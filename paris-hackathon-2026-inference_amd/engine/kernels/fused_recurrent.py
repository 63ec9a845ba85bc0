"""Token-recurrent gated delta rule on the MI355X (decode and spec-verify).

Drop-in for fla's ``fused_recurrent_gated_delta_rule`` as HF's GDN decode
branch calls it (transformers modeling_qwen3_5_moe.py:503-515; the reference
holds the torch equivalent at engine/runtime/cuda_graphs.py:126-135 and
swaps it in at :201-203), extended with the slot-pool contract the reference
cache needs (engine/runtime/kv_cache.py:134-212): pass the pool as
``initial_state`` with ``ssm_state_indices`` and ``inplace_final_state=True``
and the kernel reads and writes ``pool[slot]`` directly, with no
gather/clone/index_copy around it (kv_cache.py:189-208).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib


def fused_recurrent_gated_delta_rule(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
    initial_state: Optional[torch.Tensor] = None,
    output_final_state: bool = False,
    cu_seqlens: Optional[torch.Tensor] = None,
    use_qk_l2norm_in_kernel: bool = False,
    ssm_state_indices: Optional[torch.Tensor] = None,
    inplace_final_state: bool = False,
    snapshots: Optional[torch.Tensor] = None,
    **_ignored,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Gated delta rule, one token at a time, state kept in registers.

    Shapes (fla convention): q, k ``[B, T, Hk, K]``; v ``[B, T, Hv, V]``;
    g, beta ``[B, T, Hv]``; states ``[N, Hv, K, V]`` fp32, N = B (or the
    number of sequences when ``cu_seqlens`` [N+1] packs them into B = 1).
    Hk may divide Hv (v-head j uses k-head j // (Hv // Hk)).

    Modes
      * fla: ``initial_state`` [N, ...] (or None), returns a NEW final state
        when ``output_final_state``.
      * slot pool: ``initial_state`` is the pool [slots, Hv, K, V] fp32,
        ``ssm_state_indices`` [N] selects rows (negative = no slot: zero
        state, nothing written) and ``inplace_final_state=True`` writes the
        final state back into the pool; the pool is returned.
      * spec-verify: ``snapshots`` fp32 [N, T, Hv, K, V] receives the state
        after every token; combine with ``output_final_state=False`` and
        commit with :func:`engine.kernels.state_pool.gdn_state_commit`.

    Returns ``(o [B, T, Hv, V] in q's dtype, final_state or None)``.
    """
    _lib.require_gpu(q, g, beta)
    if beta is None:
        beta = torch.ones_like(g)
    bsz, t, hv = v.shape[0], v.shape[1], v.shape[2]
    g32, _ = _lib.per_token(g.to(torch.float32), bsz, t, hv, "g")
    if beta.dtype not in _lib.GDN_DTYPE:
        beta = beta.float()
    beta_c, _ = _lib.per_token(beta, bsz, t, hv, "beta")
    g32, beta_c = g32.contiguous(), beta_c.contiguous()  # the precomputed-gate ABI takes token stride Hv
    gates = ("gdn_recurrent_fwd", [_lib.ptr(g32), _lib.ptr(beta_c), _lib.dtype_code(beta_c, "beta")])
    return _recurrent(q, k, v, gates, scale, initial_state, output_final_state, cu_seqlens,
                      use_qk_l2norm_in_kernel, ssm_state_indices, inplace_final_state, snapshots)


def fused_recurrent_gated_delta_rule_from_projections(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    A_log: torch.Tensor,
    dt_bias: torch.Tensor,
    scale: Optional[float] = None,
    initial_state: Optional[torch.Tensor] = None,
    output_final_state: bool = False,
    cu_seqlens: Optional[torch.Tensor] = None,
    use_qk_l2norm_in_kernel: bool = True,
    ssm_state_indices: Optional[torch.Tensor] = None,
    inplace_final_state: bool = False,
    snapshots: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """:func:`fused_recurrent_gated_delta_rule` with the gates computed in
    the kernel from the GDN layer's raw projections: ``a``, ``b``
    ``[B, T, Hv]``, ``A_log``, ``dt_bias`` ``[Hv]``; beta = sigmoid(b),
    g = -exp(A_log) * softplus(a + dt_bias) (transformers
    modeling_qwen3_5_moe.py:495-497)."""
    bsz, t, hv = v.shape[0], v.shape[1], v.shape[2]
    _lib.require_gpu(q, a, b, A_log, dt_bias)
    if a.dtype not in _lib.GDN_DTYPE:
        a = a.float()
    if b.dtype != a.dtype:
        b = b.to(a.dtype)
    ax, ast = _lib.per_token(a, bsz, t, hv, "a")
    bx, bst = _lib.per_token(b, bsz, t, hv, "b")
    if ast != bst:
        ax, bx, ast = ax.contiguous(), bx.contiguous(), hv
    alog, dtb = _lib.f32_vector(A_log), _lib.f32_vector(dt_bias)
    if alog.numel() != hv or dtb.numel() != hv:
        raise ValueError(f"A_log / dt_bias must have {hv} entries")
    gates = ("gdn_recurrent_fwd_gated", [_lib.ptr(ax), _lib.ptr(bx), _lib.dtype_code(ax, "a"), ast,
                                         _lib.ptr(alog), _lib.ptr(dtb)])
    keep = (ax, bx, alog, dtb)  # alive until the launch is enqueued
    out = _recurrent(q, k, v, gates, scale, initial_state, output_final_state, cu_seqlens,
                     use_qk_l2norm_in_kernel, ssm_state_indices, inplace_final_state, snapshots)
    del keep
    return out


def _recurrent(q, k, v, gates, scale, initial_state, output_final_state, cu_seqlens,
               use_qk_l2norm_in_kernel, ssm_state_indices, inplace_final_state, snapshots):
    """Shared body: shape checks, state plumbing and the launch.
    ``gates`` = (entry point, its gate arguments)."""
    dev = _lib.require_gpu(q, k, v, initial_state, snapshots)
    b, t, hk, dk = q.shape
    hv, dv = v.shape[2], v.shape[3]
    if k.shape != q.shape or v.shape[:2] != (b, t):
        raise ValueError(f"shape mismatch: q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)}")
    if hv % hk:
        raise ValueError(f"Hv={hv} is not a multiple of Hk={hk}")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError(f"q/k/v dtypes differ: {q.dtype} {k.dtype} {v.dtype}")
    if scale is None:
        scale = dk ** -0.5
    cu = _lib.as_cu_seqlens(cu_seqlens, dev)
    if cu is not None and b != 1:
        raise ValueError(f"cu_seqlens requires B == 1, got B={b}")
    n_seqs = (cu.numel() - 1) if cu is not None else b
    total = b * t

    qx, qs = _lib.token_major(q, "q")
    kx, ks = _lib.token_major(k, "k")
    vx, vs = _lib.token_major(v, "v")

    idx = _lib.as_index(ssm_state_indices, dev)
    state_in = state_out = None
    in_idx = out_idx = None
    final = None
    if initial_state is not None:
        if initial_state.dtype != torch.float32:
            if inplace_final_state:
                raise TypeError("in-place state update needs an fp32 state tensor")
            initial_state = initial_state.float()
        if not initial_state.is_contiguous():
            if inplace_final_state:
                raise ValueError("in-place state update needs a contiguous state tensor")
            initial_state = initial_state.contiguous()
        if initial_state.shape[1:] != (hv, dk, dv):
            raise ValueError(f"state shape {tuple(initial_state.shape)} != [*, {hv}, {dk}, {dv}]")
        if idx is None and initial_state.shape[0] != n_seqs:
            raise ValueError(f"initial_state has {initial_state.shape[0]} rows for {n_seqs} sequences")
        state_in, in_idx = initial_state, idx
    elif idx is not None:
        raise ValueError("ssm_state_indices given without a state pool (initial_state)")
    if inplace_final_state:
        if initial_state is None:
            raise ValueError("inplace_final_state needs initial_state (the pool)")
        state_out, out_idx, final = initial_state, idx, initial_state
    elif output_final_state:
        final = torch.empty((n_seqs, hv, dk, dv), dtype=torch.float32, device=dev)
        state_out = final
    if snapshots is not None:
        if snapshots.dtype != torch.float32 or not snapshots.is_contiguous() or \
                snapshots.shape != (n_seqs, t, hv, dk, dv):
            raise ValueError(f"snapshots must be contiguous fp32 [{n_seqs}, {t}, {hv}, {dk}, {dv}]")

    o = torch.empty((b, t, hv, dv), dtype=q.dtype, device=dev)
    lib = _lib.load()
    name, gate_args = gates
    st = getattr(lib, name)(
        _lib.ptr(qx), _lib.ptr(kx), _lib.ptr(vx), _lib.dtype_code(q, "q"), qs, ks, vs,
        *gate_args,
        _lib.ptr(state_in), _lib.ptr(in_idx), _lib.rows_of(state_in),
        _lib.ptr(state_out), _lib.ptr(out_idx), _lib.rows_of(state_out),
        _lib.ptr(o), _lib.dtype_code(o, "o"), _lib.ptr(snapshots),
        _lib.ptr(cu), n_seqs, total if cu is not None else t,
        hk, hv, dk, dv, float(scale), int(bool(use_qk_l2norm_in_kernel)), _lib.stream_of(q))
    _lib.check(st, name)
    return o, final


def recurrent_gated_delta_rule(query, key, value, g, beta, initial_state, output_final_state,
                               use_qk_l2norm_in_kernel=False, **kwargs):
    """HF-signature adapter (``torch_recurrent_gated_delta_rule``,
    transformers modeling_qwen3_5_moe.py:331-342) over the HIP kernel."""
    return fused_recurrent_gated_delta_rule(
        query, key, value, g, beta, initial_state=initial_state,
        output_final_state=output_final_state, use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel,
        **kwargs)
