"""The GDN layer glue fused into the MI355X kernels.

HF's ``Qwen3_5MoeGatedDeltaNet.forward`` (transformers
modeling_qwen3_5_moe.py:430-541, the layer the reference runs for its 30
hybrid layers) computes, around the core kernel, in separate torch ops:

* the gates ``beta = sigmoid(b)``, ``g = -exp(A_log) * softplus(a + dt_bias)``
  (:495-497), two extra [tokens, Hv] round trips;
* ``repeat_interleave`` of q and k to the 32 v-heads (:498-500), a copy of
  2 x [tokens, 16, 128] that doubles the k/q bytes the core kernel reads;
* ``RMSNormGated(o, z)`` (:535-538, module at :169-185), a chain of
  elementwise ops over the core output.

:func:`gated_delta_net_forward` is that forward with the gates computed in
the kernel prologues (``*_from_projections``), q/k passed at their 16 heads
(native GQA), and the norm as one HIP pass (:func:`rms_norm_gated`).  A
one-token decode step runs the four input projections and the conv update
as one HIP kernel (:func:`engine.kernels.in_proj.gdn_in_proj_decode`);
otherwise the projections are torch matmuls (hipBLASLt) and the conv runs
the HIP ``causal_conv1d`` kernels on their output in place.  The cache calls
are HF's own, in HF's order, so the layer works with the transformers cache
unchanged.  With an engine
slot-pool cache (``cache_params.gdn_slot_pools``, see
:mod:`engine.runtime.slot_pools`) the kernels address the pools by slot id
instead.  :func:`install_gdn_layer_patch` swaps it in for the HF layer
classes.
"""
from __future__ import annotations

import importlib
import logging
import os
import sys
from typing import Optional

import torch

from . import _lib
from .causal_conv1d import causal_conv1d_fn, causal_conv1d_update
from .delta_rule import chunk_gated_delta_rule_from_projections
from .fused_recurrent import fused_recurrent_gated_delta_rule_from_projections
from .in_proj import OUT_PROJ_MAX_M, fused_in_proj_supported, fused_out_proj_supported, gdn_in_proj_decode, gdn_out_proj_decode

log = logging.getLogger(__name__)


def rms_norm_gated(x: torch.Tensor, z: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
                   out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """``weight * x / sqrt(mean(x^2, -1) + eps) * silu(z)`` per row of the
    last dim (D = 128), in fp32 with one rounding to the output dtype
    (default x's).  x, z ``[..., H, D]``; rows of a token may be strided
    views (token stride a multiple of 8 elements).  Replaces HF's
    RMSNormGated (transformers modeling_qwen3_5_moe.py:169-185)."""
    dev = _lib.require_gpu(x, z, weight)
    if x.shape != z.shape:
        raise ValueError(f"x{tuple(x.shape)} and z{tuple(z.shape)} differ")
    if x.dim() < 2:
        raise ValueError("expected [..., H, D]")
    d = x.shape[-1]
    if weight.numel() != d:
        raise ValueError(f"weight has {weight.numel()} entries for D={d}")
    out_dtype = out_dtype or x.dtype
    x4 = x.reshape(1, -1, x.shape[-2], d)
    z4 = z.reshape(1, -1, z.shape[-2], d)
    xx, xs = _lib.token_major(x4, "x")
    zz, zs = _lib.token_major(z4, "z")
    w = weight.detach()
    if w.dtype not in _lib.GDN_DTYPE:
        w = w.float()
    w = w.contiguous()
    if w.data_ptr() % 32:  # the kernel reads the weight as 16-byte (fp32: 32-byte) vectors
        w = w.clone()
    n_tok, h = x4.shape[1], x4.shape[2]
    y = torch.empty((n_tok, h, d), dtype=out_dtype, device=dev)
    lib = _lib.load()
    st = lib.gdn_rmsnorm_gated_fwd(
        _lib.ptr(xx), _lib.dtype_code(xx, "x"), xs, _lib.ptr(zz), _lib.dtype_code(zz, "z"), zs,
        _lib.ptr(w), _lib.dtype_code(w, "weight"), _lib.ptr(y), _lib.dtype_code(y, "y"), h * d,
        n_tok, h, d, float(eps), _lib.stream_of(x))
    _lib.check(st, "gdn_rmsnorm_gated_fwd")
    return y.view(x.shape)


def _fused_decode_fits(self, hidden_states: torch.Tensor, conv_state: torch.Tensor) -> bool:
    """Whether this one-token step can take :func:`gdn_in_proj_decode`: bf16
    bias-free projections of a supported shape and a bf16 [rows, C, 4] window
    pool."""
    lins = (self.in_proj_qkv, self.in_proj_z, self.in_proj_b, self.in_proj_a)
    if hidden_states.dtype != torch.bfloat16 or hidden_states.shape[1] != 1:
        return False
    if any(l.bias is not None or l.weight.dtype != torch.bfloat16 for l in lins):
        return False
    if self.conv1d.weight.dtype != torch.bfloat16 or self.activation not in ("silu", "swish", None):
        return False
    n = [l.weight.shape[0] for l in lins]
    if not fused_in_proj_supported(hidden_states.shape[-1], *n, self.conv1d.weight.shape[-1]):
        return False
    return (conv_state.dtype == torch.bfloat16 and conv_state.dim() == 3 and conv_state.is_contiguous()
            and tuple(conv_state.shape[1:]) == (n[0], 4))


def _fused_decode(self, hidden_states: torch.Tensor, conv_state: torch.Tensor,
                  slots: Optional[torch.Tensor]) -> tuple[torch.Tensor, ...]:
    """(mixed_qkv after the conv [B, 1, C], z [B, 1, Hv*V], b, a [B, 1, Hv])
    of a one-token step, conv windows advanced in place."""
    batch_size = hidden_states.shape[0]
    y, z, b, a = gdn_in_proj_decode(hidden_states.reshape(batch_size, -1), self.in_proj_qkv.weight,
                                    self.in_proj_z.weight, self.in_proj_b.weight, self.in_proj_a.weight,
                                    self.conv1d.weight, self.conv1d.bias, conv_state, slots, self.activation)
    return tuple(t.view(batch_size, 1, -1) for t in (y, z, b, a))


def _out_proj_fits(self, out: torch.Tensor) -> bool:
    """Whether ``out_proj`` over these rows can take :func:`gdn_out_proj_decode`:
    one token per row, at most OUT_PROJ_MAX_M rows, a plain bias-free bf16
    ``nn.Linear`` of a supported shape."""
    lin = self.out_proj
    return (type(lin) is torch.nn.Linear and out.shape[1] == 1 and out.shape[0] <= OUT_PROJ_MAX_M
            and out.dtype == torch.bfloat16 and lin.bias is None and lin.weight.dtype == torch.bfloat16
            and fused_out_proj_supported(lin.weight.shape[1], lin.weight.shape[0]))


def _out_proj(self, out: torch.Tensor) -> torch.Tensor:
    """``self.out_proj(out)`` for ``out`` [B, L, Hv*V]; decode rows through the kernel."""
    if _out_proj_fits(self, out):
        return gdn_out_proj_decode(out, self.out_proj.weight)
    return self.out_proj(out)


def gated_delta_net_forward(self, hidden_states: torch.Tensor, cache_params=None,
                            attention_mask: Optional[torch.Tensor] = None, **kwargs) -> torch.Tensor:
    """Forward of HF's GDN layer (``self`` is a ``*GatedDeltaNet`` module of
    transformers qwen3_5_moe / qwen3_5 / qwen3_next) on the MI355X kernels.
    Same inputs, cache protocol and output as the HF method
    (modeling_qwen3_5_moe.py:430-541)."""
    pools = getattr(cache_params, "gdn_slot_pools", None) if cache_params is not None else None
    if pools is not None:
        return _forward_on_pools(self, hidden_states, pools, attention_mask)
    hf = sys.modules[type(self).__module__]
    hidden_states = hf.apply_mask_to_padding_states(hidden_states, attention_mask)
    batch_size, seq_len, _ = hidden_states.shape
    use_precomputed_states = cache_params is not None and cache_params.has_previous_state(self.layer_idx)

    layer = cache_params.layers[self.layer_idx] if cache_params is not None else None
    decode_step = use_precomputed_states and seq_len == 1 and not layer.record_past
    if decode_step and layer.conv_states[0].shape[0] == batch_size and _fused_decode_fits(
            self, hidden_states, layer.conv_states[0]):
        mixed_qkv, z, b, a = _fused_decode(self, hidden_states, layer.conv_states[0], None)
    else:
        mixed_qkv = self.in_proj_qkv(hidden_states).transpose(1, 2)
        z = self.in_proj_z(hidden_states)
        b = self.in_proj_b(hidden_states)
        a = self.in_proj_a(hidden_states)
        conv_w = self.conv1d.weight.squeeze(1)
        if decode_step:
            mixed_qkv = causal_conv1d_update(mixed_qkv, layer.conv_states[0], conv_w, self.conv1d.bias,
                                             self.activation)
        else:
            if cache_params is not None:
                mixed_qkv = cache_params.update_conv_state(mixed_qkv, self.layer_idx,
                                                           conv_kernel_size=self.conv_kernel_size)
            mixed_qkv = causal_conv1d_fn(mixed_qkv, conv_w, self.conv1d.bias, activation=self.activation)
            if cache_params is not None:
                mixed_qkv = mixed_qkv[:, :, -seq_len:]
        mixed_qkv = mixed_qkv.transpose(1, 2)
    query, key, value = torch.split(mixed_qkv, [self.key_dim, self.key_dim, self.value_dim], dim=-1)
    query = query.reshape(batch_size, seq_len, -1, self.head_k_dim)  # 16 heads: no repeat_interleave
    key = key.reshape(batch_size, seq_len, -1, self.head_k_dim)
    value = value.reshape(batch_size, seq_len, -1, self.head_v_dim)

    cu = kwargs.pop("cu_seq_lens_q", None)
    recurrent_state = layer.recurrent_states[0] if use_precomputed_states else None
    if use_precomputed_states and seq_len == 1:
        # decode: the cache's state tensor is updated in place by the kernel
        inplace = (recurrent_state is not None and recurrent_state.dtype == torch.float32
                   and recurrent_state.is_contiguous())
        core, last = fused_recurrent_gated_delta_rule_from_projections(
            query, key, value, a, b, self.A_log, self.dt_bias, initial_state=recurrent_state,
            output_final_state=not inplace, use_qk_l2norm_in_kernel=True, cu_seqlens=cu,
            inplace_final_state=inplace)
        if not inplace:
            cache_params.update_recurrent_state(last, self.layer_idx)
    else:
        core, last = chunk_gated_delta_rule_from_projections(
            query, key, value, a, b, self.A_log, self.dt_bias, initial_state=recurrent_state,
            output_final_state=cache_params is not None, use_qk_l2norm_in_kernel=True, cu_seqlens=cu)
        if cache_params is not None:
            cache_params.update_recurrent_state(last, self.layer_idx)

    z = z.reshape(batch_size, seq_len, -1, self.head_v_dim)
    out = rms_norm_gated(core, z, self.norm.weight, self.norm.variance_epsilon)
    return _out_proj(self, out.reshape(batch_size, seq_len, -1))


# decode steps longer than this (a continued prefill) take the chunk kernels
_RECURRENT_MAX_T = 16


def _forward_on_pools(self, hidden_states: torch.Tensor, pools, attention_mask: Optional[torch.Tensor]) -> torch.Tensor:
    """The layer forward on slot pools (:class:`engine.runtime.slot_pools.GDNSlotPools`):
    conv and recurrent state are read from and written to ``pool[slot]`` by
    the kernels, rows as bound by ``pools.bind``.  Prefill rows start from
    a zero state and leave their final state and conv window in their slot;
    decode rows continue from their slot; a bound verify step also records
    the snapshots and conv history that ``pools.commit_verify`` rolls back to."""
    hf = sys.modules[type(self).__module__]
    hidden_states = hf.apply_mask_to_padding_states(hidden_states, attention_mask)
    batch_size, seq_len, _ = hidden_states.shape
    conv_pool, rec_pool = pools.layer(self.layer_idx)
    slots = pools.slots()
    if slots.numel() != batch_size:
        raise ValueError(f"pools bound for {slots.numel()} rows, forward has {batch_size}")
    verify = pools.verify_tokens
    if verify and seq_len != verify:
        raise ValueError(f"verify step bound for {verify} tokens, forward has {seq_len}")

    # a verify step of any length (one token included) keeps its conv history
    # and per-token state snapshots for commit_verify, so it never takes the
    # fused decode input side (which moves the window on) or the chunk kernels
    # (which keep no snapshots)
    step = pools.decode and seq_len == 1 and not verify
    if step and _fused_decode_fits(self, hidden_states, conv_pool):
        mixed_qkv, z, b, a = _fused_decode(self, hidden_states, conv_pool, slots)
    else:
        mixed_qkv = self.in_proj_qkv(hidden_states).transpose(1, 2)  # [B, conv_dim, L]
        z = self.in_proj_z(hidden_states)
        b = self.in_proj_b(hidden_states)
        a = self.in_proj_a(hidden_states)
        conv_w = self.conv1d.weight.squeeze(1)
        if step:
            mixed_qkv = causal_conv1d_update(mixed_qkv, conv_pool, conv_w, self.conv1d.bias, self.activation,
                                             conv_state_indices=slots)
        else:
            if verify:
                pools.record_conv(self.layer_idx, mixed_qkv)
            mixed_qkv = causal_conv1d_fn(mixed_qkv, conv_w, self.conv1d.bias, activation=self.activation,
                                         conv_states=conv_pool, cache_indices=slots,
                                         has_initial_state=pools.has_state())
        mixed_qkv = mixed_qkv.transpose(1, 2)
    query, key, value = torch.split(mixed_qkv, [self.key_dim, self.key_dim, self.value_dim], dim=-1)
    query = query.reshape(batch_size, seq_len, -1, self.head_k_dim)
    key = key.reshape(batch_size, seq_len, -1, self.head_k_dim)
    value = value.reshape(batch_size, seq_len, -1, self.head_v_dim)
    if verify or (pools.decode and seq_len <= _RECURRENT_MAX_T):
        core, _ = fused_recurrent_gated_delta_rule_from_projections(
            query, key, value, a, b, self.A_log, self.dt_bias, initial_state=rec_pool,
            use_qk_l2norm_in_kernel=True, ssm_state_indices=slots, inplace_final_state=True,
            snapshots=pools.snapshots(self.layer_idx) if verify else None)
    else:
        core, _ = chunk_gated_delta_rule_from_projections(
            query, key, value, a, b, self.A_log, self.dt_bias, initial_state=rec_pool,
            use_qk_l2norm_in_kernel=True, ssm_state_indices=slots, inplace_final_state=True,
            has_initial_state=pools.has_state())

    z = z.reshape(batch_size, seq_len, -1, self.head_v_dim)
    out = rms_norm_gated(core, z, self.norm.weight, self.norm.variance_epsilon)
    return _out_proj(self, out.reshape(batch_size, seq_len, -1))


_LAYER_CLASSES = (
    ("transformers.models.qwen3_5_moe.modeling_qwen3_5_moe", "Qwen3_5MoeGatedDeltaNet"),
    ("transformers.models.qwen3_5.modeling_qwen3_5", "Qwen3_5GatedDeltaNet"),
    ("transformers.models.qwen3_next.modeling_qwen3_next", "Qwen3NextGatedDeltaNet"),
)


def install_gdn_layer_patch() -> bool:
    """Replace ``forward`` of the HF GDN layer classes with
    :func:`gated_delta_net_forward`.  Returns True if a class was patched.
    ``PARIS_DISABLE_HELION_DELTA=1`` makes it a no-op, like
    :func:`engine.kernels.install_delta_rule_monkeypatch`."""
    if os.environ.get("PARIS_DISABLE_HELION_DELTA", "") == "1":
        log.info("PARIS_DISABLE_HELION_DELTA=1 -- skipping GDN layer patch")
        return False
    patched = False
    for mod_name, cls_name in _LAYER_CLASSES:
        try:
            cls = getattr(importlib.import_module(mod_name), cls_name)
        except Exception:  # model family not present in this transformers
            continue
        needed = ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a")
        if not all(n in cls.__init__.__code__.co_names for n in needed):
            log.info("%s.%s has a different projection layout; not patched", mod_name, cls_name)
            continue
        cls.forward = gated_delta_net_forward
        patched = True
        log.info("patched %s.%s.forward -> fused MI355X GDN layer", mod_name, cls_name)
    return patched
