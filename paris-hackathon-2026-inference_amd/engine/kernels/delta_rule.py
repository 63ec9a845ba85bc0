"""Chunked gated delta rule prefill on the MI355X (chunk size 64).

Drop-in for the reference's ``chunk_gated_delta_rule``
(engine/kernels/delta_rule.py:352-438), which mirrors fla's
``chunk_gated_delta_rule`` signature; the HIP kernels replace the Helion
kernel (:128-263), the torch fallback (:286-349) and fla's Triton chunk
kernels.  Differences from the reference entry, all additive:

* ``cu_seqlens`` is honoured (the reference swallows it, :362): packed
  sequences with per-sequence initial/final states, chunks never straddle a
  sequence boundary;
* q/k may carry fewer heads than v (native GQA, v-head j uses k-head
  j // (Hv // Hk)), so HF's ``repeat_interleave`` copy is optional;
* ``initial_state`` may be a slot pool addressed by ``ssm_state_indices``,
  and ``inplace_final_state=True`` writes the final states back into it;
  ``has_initial_state`` [N] bool starts the sequences marked False from a
  zero state (a fresh prefill into its slot) while their final states still
  land in the pool.

Like the reference entry, any ``chunk_size`` and any float q/k/v dtype is
accepted: the reference falls back to its torch chunk path for
``chunk_size != 64`` (:383-388) and upcasts q/k/v to fp32 (:396-400).  The
result of the chunk algorithm does not depend on the chunk size, so the
kernels always run with 64.  bf16 q/k/v take the MFMA chunk kernels; fp32 and
fp16 q/k/v take the token-recurrence kernel, which computes in fp32 from the
inputs as given (bf16 MFMA operands would round them).

The reference's opt-out variable ``PARIS_DISABLE_HELION_DELTA=1`` keeps its
meaning for :func:`install_delta_rule_monkeypatch` (nothing is patched);
the functions here always run the HIP kernels and raise if the library is
missing -- there is no CPU fallback.
"""
from __future__ import annotations

import logging
import os
from typing import Optional, Tuple

import torch

from . import _lib

log = logging.getLogger(__name__)

CHUNK_SIZE = 64


def chunk_gated_delta_rule(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    chunk_size: int = 64,
    initial_state: Optional[torch.Tensor] = None,
    output_final_state: bool = False,
    use_qk_l2norm_in_kernel: bool = False,
    cu_seqlens: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
    ssm_state_indices: Optional[torch.Tensor] = None,
    inplace_final_state: bool = False,
    has_initial_state: Optional[torch.Tensor] = None,
    **_ignored,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Chunk-64 (WY/UT) gated delta rule forward.

    Shapes: query, key ``[B, T, Hk, K]``; value ``[B, T, Hv, V]``; g, beta
    ``[B, T, Hv]``; ``initial_state`` ``[N, Hv, K, V]`` fp32 (N = B, or the
    number of sequences with ``cu_seqlens`` [N+1], B = 1).  bf16 q/k/v with
    K = V = 128 run the MFMA chunk kernels; fp16 or fp32 q/k/v, and K = 64 or
    256 or V another multiple of 32, run the token recurrence (exact in the
    inputs as given, one token after another); ``chunk_size`` any positive
    value (computed with 64).

    Returns ``(core_attn_out [B, T, Hv, V] in query's dtype,
    last_recurrent_state [N, Hv, K, V] fp32 or None)`` as the reference does
    (delta_rule.py:366-374).
    """
    b, t, hv = value.shape[0], value.shape[1], value.shape[2]
    _lib.require_gpu(g, beta)
    g32, _ = _lib.per_token(g.to(torch.float32), b, t, hv, "g")
    if beta.dtype not in _lib.GDN_DTYPE:
        beta = beta.float()
    beta_c, _ = _lib.per_token(beta, b, t, hv, "beta")
    g32, beta_c = g32.contiguous(), beta_c.contiguous()  # the precomputed-gate ABI takes token stride Hv
    gates = ("gdn_chunk_fwd", [_lib.ptr(g32), _lib.ptr(beta_c), _lib.dtype_code(beta_c, "beta")])
    return _chunk(query, key, value, gates, chunk_size, initial_state, output_final_state,
                  use_qk_l2norm_in_kernel, cu_seqlens, scale, ssm_state_indices, inplace_final_state,
                  has_initial_state)


def chunk_gated_delta_rule_from_projections(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    A_log: torch.Tensor,
    dt_bias: torch.Tensor,
    initial_state: Optional[torch.Tensor] = None,
    output_final_state: bool = False,
    use_qk_l2norm_in_kernel: bool = True,
    cu_seqlens: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
    ssm_state_indices: Optional[torch.Tensor] = None,
    inplace_final_state: bool = False,
    has_initial_state: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """:func:`chunk_gated_delta_rule` with the gates computed inside the
    kernel from the GDN layer's raw projections (``a``, ``b`` ``[B, T, Hv]``,
    ``A_log``, ``dt_bias`` ``[Hv]``): beta = sigmoid(b),
    g = -exp(A_log) * softplus(a + dt_bias), the glue of HF's layer forward
    (transformers modeling_qwen3_5_moe.py:495-497)."""
    bsz, t, hv = value.shape[0], value.shape[1], value.shape[2]
    _lib.require_gpu(a, b, A_log, dt_bias)
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
    gates = ("gdn_chunk_fwd_gated", [_lib.ptr(ax), _lib.ptr(bx), _lib.dtype_code(ax, "a"), ast,
                                     _lib.ptr(alog), _lib.ptr(dtb)])
    keep = (ax, bx, alog, dtb)  # alive until the launch is enqueued
    out = _chunk(query, key, value, gates, CHUNK_SIZE, initial_state, output_final_state,
                 use_qk_l2norm_in_kernel, cu_seqlens, scale, ssm_state_indices, inplace_final_state,
                 has_initial_state)
    del keep
    return out


def _chunk(query, key, value, gates, chunk_size, initial_state, output_final_state,
           use_qk_l2norm_in_kernel, cu_seqlens, scale, ssm_state_indices, inplace_final_state,
           has_initial_state=None):
    """Shared body: shape checks, state / workspace plumbing and the launch.
    ``gates`` = (entry point, its gate arguments)."""
    if int(chunk_size) <= 0:
        raise ValueError(f"chunk_size={chunk_size} must be positive")
    if chunk_size != CHUNK_SIZE:  # the chunk algorithm's result does not depend on it
        log.debug("chunk_size=%s requested; computing with %d", chunk_size, CHUNK_SIZE)
    dev = _lib.require_gpu(query, key, value, initial_state)
    b, t, hk, dk = query.shape
    hv, dv = value.shape[2], value.shape[3]
    if key.shape != query.shape or value.shape[:2] != (b, t):
        raise ValueError(f"shape mismatch: q{tuple(query.shape)} k{tuple(key.shape)} v{tuple(value.shape)}")
    if hv % hk:
        raise ValueError(f"Hv={hv} is not a multiple of Hk={hk}")
    if not (query.dtype == key.dtype == value.dtype):
        raise TypeError(f"q/k/v dtypes differ: {query.dtype} {key.dtype} {value.dtype}")
    if scale is None:
        scale = dk ** -0.5
    cu = _lib.as_cu_seqlens(cu_seqlens, dev)
    if cu is not None and b != 1:
        raise ValueError(f"cu_seqlens requires B == 1, got B={b}")
    n_seqs = cu.numel() - 1 if cu is not None else b
    total = b * t

    qx, qs = _lib.token_major(query, "query")
    kx, ks = _lib.token_major(key, "key")
    vx, vs = _lib.token_major(value, "value")

    idx = _lib.as_index(ssm_state_indices, dev)
    h0 = h0_idx = None
    if initial_state is not None:
        if initial_state.dtype != torch.float32 or not initial_state.is_contiguous():
            if inplace_final_state:
                raise ValueError("in-place final state needs a contiguous fp32 state tensor")
            initial_state = initial_state.float().contiguous()
        if initial_state.shape[1:] != (hv, dk, dv):
            raise ValueError(f"initial_state {tuple(initial_state.shape)} != [*, {hv}, {dk}, {dv}]")
        if idx is None and initial_state.shape[0] != n_seqs:
            raise ValueError(f"initial_state has {initial_state.shape[0]} rows for {n_seqs} sequences")
        h0, h0_idx = initial_state, idx
    elif idx is not None:
        raise ValueError("ssm_state_indices given without initial_state (the pool)")
    final = hT = hT_idx = None
    if inplace_final_state:
        if h0 is None:
            raise ValueError("inplace_final_state needs initial_state (the pool)")
        final, hT, hT_idx = h0, h0, idx
    if has_initial_state is not None:
        if h0 is None:
            raise ValueError("has_initial_state needs initial_state")
        has = has_initial_state.to(device=dev, dtype=torch.bool).reshape(-1)
        if has.numel() != n_seqs:
            raise ValueError(f"has_initial_state has {has.numel()} entries for {n_seqs} sequences")
        rows = idx if idx is not None else torch.arange(n_seqs, device=dev, dtype=torch.int64)
        if idx is not None:
            # a row repeating an earlier row's slot id is "no slot" for both the
            # read and the write: decide the repeats on the unmasked ids, so the
            # masked read ids cannot turn a later repeat into the slot's reader
            # while the first row writes it
            rep = (rows[:, None] == rows[None, :]).tril(-1).any(dim=1)
            has = has & ~rep
        h0_idx = torch.where(has, rows, torch.full_like(rows, -1))
    if output_final_state and not inplace_final_state:
        final = hT = torch.empty((n_seqs, hv, dk, dv), dtype=torch.float32, device=dev)
        hT_idx = None

    lib = _lib.load()
    o = torch.empty((b, t, hv, dv), dtype=query.dtype, device=dev)
    name, gate_args = gates
    if query.dtype != torch.bfloat16 or dk != 128 or dv != 128:
        # fp32 / fp16 q, k, v, or head dims the chunk kernels are not built for:
        # the token recurrence, fp32 math on the inputs as given
        rec = {"gdn_chunk_fwd": "gdn_recurrent_fwd", "gdn_chunk_fwd_gated": "gdn_recurrent_fwd_gated"}[name]
        st = getattr(lib, rec)(
            _lib.ptr(qx), _lib.ptr(kx), _lib.ptr(vx), _lib.dtype_code(query, "query"), qs, ks, vs,
            *gate_args,
            _lib.ptr(h0), _lib.ptr(h0_idx), _lib.rows_of(h0), _lib.ptr(hT), _lib.ptr(hT_idx), _lib.rows_of(hT),
            _lib.ptr(o), _lib.dtype_code(o, "o"), None,
            _lib.ptr(cu), n_seqs, total if cu is not None else t,
            hk, hv, dk, dv, float(scale), int(bool(use_qk_l2norm_in_kernel)), _lib.stream_of(query))
        _lib.check(st, rec)
        return o, final
    ws_bytes = lib.gdn_chunk_workspace_bytes(n_seqs, total, hv, dk, dv)
    ws = torch.empty(max(int(ws_bytes), 1), dtype=torch.uint8, device=dev)
    st = getattr(lib, name)(
        _lib.ptr(qx), _lib.ptr(kx), _lib.ptr(vx), _lib.dtype_code(query, "query"), qs, ks, vs,
        *gate_args,
        _lib.ptr(h0), _lib.ptr(h0_idx), _lib.rows_of(h0), _lib.ptr(hT), _lib.ptr(hT_idx), _lib.rows_of(hT),
        _lib.ptr(o), _lib.dtype_code(o, "o"),
        _lib.ptr(cu), n_seqs, total if cu is not None else t,
        hk, hv, dk, dv, float(scale), int(bool(use_qk_l2norm_in_kernel)),
        _lib.ptr(ws), int(ws_bytes), _lib.stream_of(query))
    _lib.check(st, name)
    return o, final


def install_delta_rule_monkeypatch() -> bool:
    """Point HF's / fla's GDN entry points at the MI355X kernels.

    Same contract as the reference's installer (delta_rule.py:446-480): call
    it after transformers is imported and BEFORE the model is constructed;
    returns True if anything was patched; ``PARIS_DISABLE_HELION_DELTA=1``
    makes it a no-op.  Unlike the reference (which patched the qwen3_next
    module only, so Qwen3.5-MoE layers never saw it), it patches every HF
    module that defines the GDN torch paths, including qwen3_5_moe, plus fla
    when it is importable.
    """
    if os.environ.get("PARIS_DISABLE_HELION_DELTA", "") == "1":
        log.info("PARIS_DISABLE_HELION_DELTA=1 -- skipping delta_rule monkeypatch")
        return False
    from .causal_conv1d import causal_conv1d_fn, causal_conv1d_update
    from .fused_recurrent import fused_recurrent_gated_delta_rule, recurrent_gated_delta_rule

    hf_names = {
        "torch_chunk_gated_delta_rule": chunk_gated_delta_rule,
        "chunk_gated_delta_rule": chunk_gated_delta_rule,
        "torch_recurrent_gated_delta_rule": recurrent_gated_delta_rule,
        "fused_recurrent_gated_delta_rule": fused_recurrent_gated_delta_rule,
        "causal_conv1d_fn": causal_conv1d_fn,
        "causal_conv1d_update": causal_conv1d_update,
    }
    patched = False
    import importlib

    for mod_name in ("transformers.models.qwen3_5_moe.modeling_qwen3_5_moe",
                     "transformers.models.qwen3_5.modeling_qwen3_5",
                     "transformers.models.qwen3_next.modeling_qwen3_next"):
        try:
            mod = importlib.import_module(mod_name)
        except Exception:  # model family not present in this transformers
            continue
        for attr, fn in hf_names.items():
            if hasattr(mod, attr):
                setattr(mod, attr, fn)
                patched = True
        if hasattr(mod, "is_fast_path_available"):
            mod.is_fast_path_available = True
        log.info("patched %s GDN entry points -> MI355X HIP kernels", mod_name)
    try:
        import fla.ops.gated_delta_rule as fla_mod  # type: ignore
        fla_mod.chunk_gated_delta_rule = chunk_gated_delta_rule
        fla_mod.fused_recurrent_gated_delta_rule = fused_recurrent_gated_delta_rule
        patched = True
    except Exception:
        pass
    return patched
