"""Seeded synthetic inputs for the five benchmark / parity configurations.

Tensors are generated on the CPU with ``torch.Generator().manual_seed(seed)``
(config i uses seed i unless told otherwise) so that the HIP kernels and the
CPU checker see bit-identical inputs.  Shapes are the real Qwen3.5-35B-A3B GDN
layer: 16 q/k heads, 32 v heads, head dim 128, conv width 4 over the
8192-wide q|k|v projection.

  0  recurrent, fp32, B=1 T=256, zero initial state
  1  decode, B=64 T=1, bf16 q/k/v, fp32 state pool [128 slots] ~N(0, 0.1)
  2  chunked prefill, B=1 T=4096, bf16 q/k/v, fp32 g/beta, zero initial state
  3  varlen prefill, 16 sequences L~U[128, 2048], conv1d(width 4, silu) over
     the 8192-wide projection, nonzero initial states ~N(0, 0.1)
  4  spec-verify, B=32 T=4, bf16, per-step snapshots, accepted ~U{1..4}
"""
from __future__ import annotations

from typing import Dict

import torch

HK, HV, D = 16, 32, 128
CONV_DIM = 2 * HK * D + HV * D  # 8192
CONV_WIDTH = 4


def _gates(gen: torch.Generator, shape) -> tuple[torch.Tensor, torch.Tensor]:
    beta = torch.sigmoid(torch.randn(shape, generator=gen))
    g = -torch.nn.functional.softplus(torch.randn(shape, generator=gen)) * torch.exp(
        torch.empty(shape).uniform_(-2.0, 0.0, generator=gen))
    return g, beta


def _l2n(x: torch.Tensor) -> torch.Tensor:
    return x / x.norm(dim=-1, keepdim=True)


def _qkv(gen, b, t, dtype, hk=HK, hv=HV, d=D):
    q = _l2n(torch.randn(b, t, hk, d, generator=gen)).to(dtype)
    k = _l2n(torch.randn(b, t, hk, d, generator=gen)).to(dtype)
    v = torch.randn(b, t, hv, d, generator=gen).to(dtype)
    return q, k, v


def config0(seed: int = 0, t: int = 256) -> Dict[str, torch.Tensor]:
    gen = torch.Generator().manual_seed(seed)
    q, k, v = _qkv(gen, 1, t, torch.float32)
    g, beta = _gates(gen, (1, t, HV))
    return dict(q=q, k=k, v=v, g=g, beta=beta)


def config1(seed: int = 1, batch: int = 64, num_slots: int = 128, state_std: float = 0.1
            ) -> Dict[str, torch.Tensor]:
    gen = torch.Generator().manual_seed(seed)
    q, k, v = _qkv(gen, batch, 1, torch.bfloat16)
    g, beta = _gates(gen, (batch, 1, HV))
    pool = torch.randn(num_slots, HV, D, D, generator=gen) * state_std
    slots = torch.randperm(num_slots, generator=gen)[:batch]
    return dict(q=q, k=k, v=v, g=g, beta=beta, pool=pool, slots=slots)


def config2(seed: int = 2, t: int = 4096) -> Dict[str, torch.Tensor]:
    gen = torch.Generator().manual_seed(seed)
    q, k, v = _qkv(gen, 1, t, torch.bfloat16)
    g, beta = _gates(gen, (1, t, HV))
    return dict(q=q, k=k, v=v, g=g, beta=beta)


def config3(seed: int = 3, n_seqs: int = 16, lo: int = 128, hi: int = 2048, state_std: float = 0.1,
            weight_std: float = 0.5) -> Dict[str, torch.Tensor]:
    gen = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (n_seqs,), generator=gen)
    cu = torch.zeros(n_seqs + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(lens, 0)
    total = int(cu[-1])
    x = torch.randn(total, CONV_DIM, generator=gen).to(torch.bfloat16)
    w = (torch.randn(CONV_DIM, CONV_WIDTH, generator=gen) * weight_std).to(torch.bfloat16)
    g, beta = _gates(gen, (1, total, HV))
    h0 = torch.randn(n_seqs, HV, D, D, generator=gen) * state_std
    return dict(x=x, conv_w=w, cu_seqlens=cu, g=g, beta=beta, h0=h0)


def config4(seed: int = 4, batch: int = 32, t: int = 4, num_slots: int = 64, state_std: float = 0.1
            ) -> Dict[str, torch.Tensor]:
    gen = torch.Generator().manual_seed(seed)
    q, k, v = _qkv(gen, batch, t, torch.bfloat16)
    g, beta = _gates(gen, (batch, t, HV))
    pool = torch.randn(num_slots, HV, D, D, generator=gen) * state_std
    slots = torch.randperm(num_slots, generator=gen)[:batch]
    accepted = torch.randint(1, t + 1, (batch,), generator=gen, dtype=torch.int32)
    return dict(q=q, k=k, v=v, g=g, beta=beta, pool=pool, slots=slots, accepted=accepted)


def split_qkv(y: torch.Tensor):
    """Split a token-major conv output [tokens, 8192] into q|k|v views [1, tokens, H, D]
    (HF's split order, transformers modeling_qwen3_5_moe.py:481-493)."""
    n = y.shape[0]
    q = y[:, : HK * D].view(1, n, HK, D)
    k = y[:, HK * D: 2 * HK * D].view(1, n, HK, D)
    v = y[:, 2 * HK * D:].view(1, n, HV, D)
    return q, k, v
