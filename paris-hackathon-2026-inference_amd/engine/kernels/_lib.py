"""ctypes binding of libgdn_mi355x.so and the tensor plumbing around it.

The library is loaded after ``torch`` so that its HIP runtime dependency
(``libamdhip64.so.7``) resolves to the copy torch already mapped: one HIP
runtime per process, and torch's streams and allocations are valid handles
inside the library.  There is no fallback: if the library is missing the
first call raises, naming the build command.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch

LIB_NAME = "libgdn_mi355x.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
ABI_VERSION = 8

GDN_DTYPE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}

_c_void_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float
_size = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/gdn_capi.h
SIGNATURES = {
    "gdn_abi_version": (_int, []),
    "gdn_last_error_string": (ctypes.c_char_p, []),
    "gdn_recurrent_fwd": (_int, [
        _c_void_p, _c_void_p, _c_void_p, _int,      # q k v qkv_dtype
        _i64, _i64, _i64,                           # token strides
        _c_void_p, _c_void_p, _int,                 # g beta beta_dtype
        _c_void_p, _c_void_p, _i64,                 # state_in, state_in_idx, rows
        _c_void_p, _c_void_p, _i64,                 # state_out, state_out_idx, rows
        _c_void_p, _int, _c_void_p,                 # o, o_dtype, snapshots
        _c_void_p, _i32, _i32,                      # cu_seqlens n_seqs T
        _i32, _i32, _i32, _i32,                     # Hk Hv K V
        _f32, _int, _c_void_p]),                    # scale l2norm stream
    "gdn_chunk_fwd": (_int, [
        _c_void_p, _c_void_p, _c_void_p, _int,
        _i64, _i64, _i64,
        _c_void_p, _c_void_p, _int,
        _c_void_p, _c_void_p, _i64,                 # h0, h0_idx, rows
        _c_void_p, _c_void_p, _i64,                 # hT, hT_idx, rows
        _c_void_p, _int,                            # o, o_dtype
        _c_void_p, _i32, _i32,
        _i32, _i32, _i32, _i32,
        _f32, _int,
        _c_void_p, _size, _c_void_p]),              # workspace, bytes, stream
    "gdn_chunk_workspace_bytes": (_size, [_i32, _i64, _i32, _i32, _i32]),
    "gdn_recurrent_fwd_gated": (_int, [
        _c_void_p, _c_void_p, _c_void_p, _int,      # q k v qkv_dtype
        _i64, _i64, _i64,                           # token strides
        _c_void_p, _c_void_p, _int, _i64,           # a b ab_dtype ab_stride
        _c_void_p, _c_void_p,                       # A_log dt_bias
        _c_void_p, _c_void_p, _i64,                 # state_in, state_in_idx, rows
        _c_void_p, _c_void_p, _i64,                 # state_out, state_out_idx, rows
        _c_void_p, _int, _c_void_p,                 # o, o_dtype, snapshots
        _c_void_p, _i32, _i32,                      # cu_seqlens n_seqs T
        _i32, _i32, _i32, _i32,                     # Hk Hv K V
        _f32, _int, _c_void_p]),                    # scale l2norm stream
    "gdn_chunk_fwd_gated": (_int, [
        _c_void_p, _c_void_p, _c_void_p, _int,
        _i64, _i64, _i64,
        _c_void_p, _c_void_p, _int, _i64,           # a b ab_dtype ab_stride
        _c_void_p, _c_void_p,                       # A_log dt_bias
        _c_void_p, _c_void_p, _i64,                 # h0, h0_idx, rows
        _c_void_p, _c_void_p, _i64,                 # hT, hT_idx, rows
        _c_void_p, _int,                            # o, o_dtype
        _c_void_p, _i32, _i32,
        _i32, _i32, _i32, _i32,
        _f32, _int,
        _c_void_p, _size, _c_void_p]),              # workspace, bytes, stream
    "gdn_rmsnorm_gated_fwd": (_int, [
        _c_void_p, _int, _i64,                      # x x_dtype x_stride
        _c_void_p, _int, _i64,                      # z z_dtype z_stride
        _c_void_p, _int,                            # weight w_dtype
        _c_void_p, _int, _i64,                      # y y_dtype y_stride
        _i64, _i32, _i32, _f32, _c_void_p]),        # n_tokens H D eps stream
    "gdn_in_proj_decode": (_int, [
        _c_void_p, _i64,                            # x x_stride
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, # w_qkv w_z w_b w_a
        _i32, _i32, _i32, _i32, _i32, _i32,         # M K n_qkv n_z n_b n_a
        _c_void_p, _c_void_p,                       # conv_w conv_bias
        _c_void_p, _c_void_p, _i64,                 # conv_pool slot_idx pool_rows
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, # y_qkv z b a
        _int, _c_void_p]),                          # silu stream
    "gdn_out_proj_workspace_bytes": (_size, [_i32, _i32, _i32]),  # M K N
    "gdn_out_proj_decode": (_int, [
        _c_void_p, _i64, _c_void_p,                 # x x_stride w
        _i32, _i32, _i32,                           # M K N
        _c_void_p, _i64,                            # y y_stride
        _c_void_p, _size, _c_void_p]),              # workspace bytes stream
    "gdn_out_proj_decode_noalloc": (_int, [
        _c_void_p, _i64, _c_void_p,                 # x x_stride w
        _i32, _i32, _i32,                           # M K N
        _c_void_p, _i64, _c_void_p]),               # y y_stride stream
    "causal_conv1d_fwd": (_int, [
        _c_void_p, _i64, _c_void_p, _c_void_p,      # x x_stride w bias
        _c_void_p, _i64,                            # y y_stride
        _c_void_p, _c_void_p, _i64,                 # state_in idx rows
        _c_void_p, _c_void_p, _i64,                 # state_out idx rows
        _c_void_p, _i32, _i32,                      # cu n_seqs T
        _i32, _i32, _i32,                           # C width state_len
        _int, _int, _c_void_p]),                    # silu dtype stream
    "causal_conv1d_update": (_int, [
        _c_void_p, _i64, _c_void_p, _c_void_p,      # x x_stride conv_state idx
        _i64,                                       # conv_state rows
        _c_void_p, _c_void_p, _c_void_p, _i64,      # w bias y y_stride
        _i32, _i32, _i32, _i32, _i32,               # n_seqs T C width state_len
        _int, _int, _c_void_p]),
    "gdn_state_commit": (_int, [
        _c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p,  # pool slot_ids pool_rows snapshots accepted_len
        _i32, _i32, _i32, _i32, _i32, _c_void_p]),
    "gdn_conv_state_commit": (_int, [
        _c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p,  # pool slot_ids pool_rows hist accepted_len
        _i32, _i32, _i32, _i32, _int, _c_void_p]),   # n_seqs C S L dtype stream
}

_LIB: Optional[ctypes.CDLL] = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load (once) and type the shared library; raises if it is missing or stale."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise RuntimeError(
            f"{LIB_NAME} not found at {path}; build it with "
            "`python paris-hackathon-2026-inference_amd/build_lib.py` (hipcc, gfx950)")
    lib = ctypes.CDLL(path, mode=ctypes.RTLD_LOCAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.gdn_abi_version()
    if ver != ABI_VERSION:
        raise RuntimeError(f"{LIB_NAME} ABI {ver} != expected {ABI_VERSION}; rebuild it")
    _LIB = lib
    return lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().gdn_last_error_string().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {status}): {msg}")


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def require_gpu(*tensors: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(f"expected a GPU tensor, got one on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise ValueError("no tensor given")
    return dev


def dtype_code(t: torch.Tensor, what: str) -> int:
    try:
        return GDN_DTYPE[t.dtype]
    except KeyError:
        raise TypeError(f"{what}: unsupported dtype {t.dtype}") from None


def token_major(x: torch.Tensor, what: str) -> tuple[torch.Tensor, int]:
    """View [B, T, H, D] as a token-major stream; returns (tensor, token stride).

    Heads and dims must be packed (stride(3) == 1, stride(2) == D) and the
    batch stride must equal T * token stride; otherwise a contiguous copy is
    made.
    """
    if x.dim() != 4:
        raise ValueError(f"{what}: expected [B, T, H, D], got shape {tuple(x.shape)}")
    b, t, h, d = x.shape
    # token b*T + t: with one token per sequence the batch stride is the token stride
    st = x.stride(1) if t > 1 else (x.stride(0) if b > 1 else h * d)
    ok = (x.stride(3) == 1 and (h == 1 or x.stride(2) == d) and st >= h * d and st % 8 == 0
          and (b == 1 or x.stride(0) == t * st) and x.storage_offset() % 8 == 0)
    if not ok:
        x = x.contiguous()
        st = h * d
    return x, st


def per_token(x: torch.Tensor, b: int, t: int, h: int, what: str) -> tuple[torch.Tensor, int]:
    """View a [B, T, H] per-token, per-head tensor (gates, gate projections)
    as token-major rows; returns (tensor, token stride).  Heads must be
    contiguous and batches evenly spaced, otherwise a contiguous copy is made."""
    if tuple(x.shape) != (b, t, h):
        raise ValueError(f"{what}: expected shape {(b, t, h)}, got {tuple(x.shape)}")
    st = x.stride(1) if t > 1 else (x.stride(0) if b > 1 else h)
    if not (x.stride(2) == 1 or h == 1) or st < h or (b > 1 and x.stride(0) != t * st):
        x = x.contiguous()
        st = h
    return x, st


def f32_vector(t: torch.Tensor) -> torch.Tensor:
    """``t`` as a contiguous fp32 vector.  A conversion is kept on the tensor
    itself (the layer's ``A_log``, ``dt_bias`` parameters) and redone when it
    is modified or replaced, so a layer step launches no conversion kernel
    (and a captured graph records none) once the parameter was seen."""
    if t.dtype == torch.float32 and t.is_contiguous():
        return t.detach().reshape(-1)
    key = (t.data_ptr(), t._version, t.dtype, t.numel(), t.device)
    hit = getattr(t, "_gdn_f32", None)
    if hit is not None and hit[0] == key:
        return hit[1]
    out = t.detach().to(torch.float32).reshape(-1).contiguous()
    t._gdn_f32 = (key, out)
    return out


def rows_of(t: Optional[torch.Tensor]) -> int:
    """Row count of a state tensor as the C ABI takes it (0 when absent)."""
    return 0 if t is None else int(t.shape[0])


def as_index(idx: Optional[torch.Tensor], device: torch.device) -> Optional[torch.Tensor]:
    if idx is None:
        return None
    if idx.device != device or idx.dtype != torch.int64 or not idx.is_contiguous():
        idx = idx.to(device=device, dtype=torch.int64).contiguous()
    return idx


def as_cu_seqlens(cu: Optional[torch.Tensor], device: torch.device) -> Optional[torch.Tensor]:
    if cu is None:
        return None
    if cu.device != device or cu.dtype != torch.int32 or not cu.is_contiguous():
        cu = cu.to(device=device, dtype=torch.int32).contiguous()
    return cu
