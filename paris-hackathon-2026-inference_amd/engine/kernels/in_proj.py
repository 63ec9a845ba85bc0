"""Decode-step projections of the GDN layer: the input side (conv update
fused) and the output projection.

HF's GDN decode step (transformers modeling_qwen3_5_moe.py:443-461) runs
``in_proj_qkv``, ``in_proj_z``, ``in_proj_b``, ``in_proj_a`` (four
``nn.Linear``, :424-427) over the same hidden rows and then
``causal_conv1d_update`` over the qkv projection.  :func:`gdn_in_proj_decode`
does all of it in one HIP kernel (``gdn_in_proj_decode`` in
include/gdn_capi.h): each weight row is read once from HBM, and the qkv
projection goes through the conv window update in registers, so it is never
written out before the conv.  :func:`gdn_out_proj_decode` runs ``out_proj``
(:428, called at :540) for decode rows with K split over 256 workgroups (the
2048 output columns alone would occupy 32).  Prefill keeps the library GEMMs
(hipBLASLt via ``torch.nn.functional.linear``): there the projections are
compute-bound and the conv kernels read their output in place.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib

SUPPORTED_K = (1024, 2048)  # hidden sizes the kernel is instantiated for


def _weight(w: torch.Tensor, k: int, what: str) -> torch.Tensor:
    if w.dtype != torch.bfloat16 or w.dim() != 2 or w.shape[1] != k:
        raise ValueError(f"{what}: expected a bf16 [n, {k}] weight, got {tuple(w.shape)} {w.dtype}")
    w = w.detach().contiguous()
    return w.clone() if w.data_ptr() % 16 else w


def fused_in_proj_supported(hidden_size: int, n_qkv: int, n_z: int, n_b: int, n_a: int, conv_width: int) -> bool:
    """Shapes :func:`gdn_in_proj_decode` is built for (the Qwen3.5 / Qwen3-Next
    GDN layers: K = 2048, n = 8192 / 4096 / 32 / 32, conv width 4)."""
    return (hidden_size in SUPPORTED_K and n_qkv % 64 == 0 and n_z % 64 == 0 and n_b % 4 == 0
            and n_a % 4 == 0 and n_b <= 32 and n_a <= 32 and conv_width == 4)


def gdn_in_proj_decode(hidden: torch.Tensor, w_qkv: torch.Tensor, w_z: torch.Tensor, w_b: torch.Tensor,
                       w_a: torch.Tensor, conv_weight: torch.Tensor, conv_bias: Optional[torch.Tensor],
                       conv_state: torch.Tensor, conv_state_indices: Optional[torch.Tensor] = None,
                       activation="silu") -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """One decode token per row: returns ``(conv(qkv), z, b, a)``, each
    ``[M, n]`` bf16, and advances ``conv_state`` in place.

    hidden ``[M, K]`` (or ``[M, 1, K]``) bf16; ``w_*`` the ``nn.Linear``
    weights ``[n, K]`` bf16; ``conv_weight`` ``[n_qkv, 4]`` (or the module's
    ``[n_qkv, 1, 4]``) and ``conv_bias`` ``[n_qkv]`` or None, bf16;
    ``conv_state`` ``[rows, n_qkv, 4]`` bf16 windows, row
    ``conv_state_indices[m]`` (default m) for hidden row m; ids outside
    ``[0, rows)`` (the engine's padding rows) read a zero window and write
    nothing.  ``activation``: ``"silu"`` or None, as ``causal_conv1d_update``.
    """
    dev = _lib.require_gpu(hidden, w_qkv, w_z, w_b, w_a, conv_weight, conv_state)
    x = hidden.reshape(-1, hidden.shape[-1]) if hidden.dim() == 3 else hidden
    if x.dim() != 2 or x.dtype != torch.bfloat16:
        raise ValueError(f"hidden: expected bf16 [M, K] or [M, 1, K], got {tuple(hidden.shape)} {hidden.dtype}")
    if hidden.dim() == 3 and hidden.shape[1] != 1:
        raise ValueError(f"hidden: one token per row, got {tuple(hidden.shape)}")
    m, k = x.shape
    if x.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    ws = [_weight(w, k, n) for w, n in ((w_qkv, "w_qkv"), (w_z, "w_z"), (w_b, "w_b"), (w_a, "w_a"))]
    n_qkv, n_z, n_b, n_a = (w.shape[0] for w in ws)
    cw = conv_weight.detach().reshape(conv_weight.shape[0], -1)
    if cw.shape != (n_qkv, 4) or cw.dtype != torch.bfloat16:
        raise ValueError(f"conv_weight: expected bf16 [{n_qkv}, 4], got {tuple(conv_weight.shape)} {conv_weight.dtype}")
    cw = cw.contiguous()
    cb = None
    if conv_bias is not None:
        if conv_bias.numel() != n_qkv or conv_bias.dtype != torch.bfloat16:
            raise ValueError("conv_bias: expected bf16 [n_qkv]")
        cb = conv_bias.detach().contiguous()
    if (conv_state.dtype != torch.bfloat16 or conv_state.dim() != 3 or conv_state.shape[1:] != (n_qkv, 4)
            or not conv_state.is_contiguous()):
        raise ValueError(f"conv_state: expected a contiguous bf16 [rows, {n_qkv}, 4] pool, "
                         f"got {tuple(conv_state.shape)} {conv_state.dtype}")
    idx = _lib.as_index(conv_state_indices, dev)
    if idx is not None and idx.numel() != m:
        raise ValueError(f"conv_state_indices: {idx.numel()} ids for {m} rows")
    silu = 1 if activation in ("silu", "swish", True) else 0
    if activation not in (None, False, "silu", "swish", True):
        raise ValueError(f"unsupported activation {activation!r}")
    outs = [torch.empty((m, n), dtype=torch.bfloat16, device=dev) for n in (n_qkv, n_z, n_b, n_a)]
    lib = _lib.load()
    st = lib.gdn_in_proj_decode(
        _lib.ptr(x), x.stride(0) if m > 1 else k, *(_lib.ptr(w) for w in ws), m, k, n_qkv, n_z, n_b, n_a,
        _lib.ptr(cw), _lib.ptr(cb), _lib.ptr(conv_state), _lib.ptr(idx), _lib.rows_of(conv_state),
        *(_lib.ptr(o) for o in outs), silu, _lib.stream_of(x))
    _lib.check(st, "gdn_in_proj_decode")
    return tuple(outs)


OUT_PROJ_MAX_M = 64  # rows up to which the decode out_proj kernel is used (above: hipBLASLt, measured faster at 128)


def fused_out_proj_supported(k: int, n: int) -> bool:
    """Shapes :func:`gdn_out_proj_decode` takes: K a multiple of 512 up to
    8192 (Hv*V = 4096 for Qwen3.5), N a multiple of 64 (hidden 2048)."""
    return k % 512 == 0 and 0 < k <= 8192 and n % 64 == 0 and n > 0


def gdn_out_proj_decode(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """``x @ weight.T`` for decode rows: x ``[M, K]`` (or ``[M, 1, K]``) bf16,
    weight the ``nn.Linear`` weight ``[N, K]`` bf16; returns ``[M, N]`` bf16
    (``[M, 1, N]`` for a 3-d x).  The partial sums over K are added in a
    fixed order, so the result does not depend on scheduling."""
    dev = _lib.require_gpu(x, weight)
    x2 = x.reshape(-1, x.shape[-1]) if x.dim() == 3 else x
    if x2.dim() != 2 or x2.dtype != torch.bfloat16:
        raise ValueError(f"x: expected bf16 [M, K] or [M, 1, K], got {tuple(x.shape)} {x.dtype}")
    if x.dim() == 3 and x.shape[1] != 1:
        raise ValueError(f"x: one token per row, got {tuple(x.shape)}")
    m, k = x2.shape
    if x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    w = _weight(weight, k, "weight")
    n = w.shape[0]
    if not fused_out_proj_supported(k, n):
        raise ValueError(f"out_proj of {k} -> {n}: the kernel needs K a multiple of 512 up to 8192 and N of 64")
    y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    lib = _lib.load()
    ws_bytes = int(lib.gdn_out_proj_workspace_bytes(m, k, n))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    st = lib.gdn_out_proj_decode(_lib.ptr(x2), x2.stride(0) if m > 1 else k, _lib.ptr(w), m, k, n,
                                 _lib.ptr(y), n, _lib.ptr(ws), ws.numel(), _lib.stream_of(x2))
    _lib.check(st, "gdn_out_proj_decode")
    return y.view(m, 1, n) if x.dim() == 3 else y


def gdn_out_proj_decode_noalloc(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """:func:`gdn_out_proj_decode` into a caller's ``out`` ``[M, N]`` bf16
    (row stride a multiple of 4, 8-byte aligned), with the partial sums in the
    library's built-in per-GPU scratch: the call allocates nothing, so it can
    run where allocation is not allowed (under graph capture, in a serving
    loop).  x ``[M, K]`` bf16 with unit column stride, row stride a multiple
    of 8 and 16-byte alignment, weight ``[N, K]`` contiguous bf16.  At most
    GDN_OUT_PROJ_NOALLOC_MAX_BYTES of partial sums (64 rows at K = 4096,
    N = 2048 need 4 MiB); calls that overlap on one GPU race.  Same bits as
    :func:`gdn_out_proj_decode`."""
    _lib.require_gpu(x, weight, out)
    if x.dim() != 2 or x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16 or out.dtype != torch.bfloat16:
        raise ValueError("x [M, K], weight [N, K] and out [M, N] must be bf16 2-d tensors")
    m, k = x.shape
    n = weight.shape[0]
    if weight.shape != (n, k) or not weight.is_contiguous() or out.shape != (m, n):
        raise ValueError(f"shapes x{tuple(x.shape)} weight{tuple(weight.shape)} out{tuple(out.shape)}")
    if x.stride(1) != 1 or out.stride(1) != 1:
        raise ValueError("x and out need unit column stride (no copy is made)")
    st = _lib.load().gdn_out_proj_decode_noalloc(
        _lib.ptr(x), x.stride(0) if m > 1 else k, _lib.ptr(weight), m, k, n, _lib.ptr(out),
        out.stride(0) if m > 1 else n, _lib.stream_of(x))
    _lib.check(st, "gdn_out_proj_decode_noalloc")
    return out
