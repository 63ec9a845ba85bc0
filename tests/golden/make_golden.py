"""Write the golden vectors in this folder (run once, in the build container).

The reference (TheJDen/paris-hackathon-2026-inference) ships no tests or
fixtures for the GDN path.  Its math is reached through third-party code:

* ``torch_chunk_gated_delta_rule`` -- the reference's own ``_torch_fallback``
  (engine/kernels/delta_rule.py:286-349) is a line-for-line copy of it;
* ``torch_recurrent_gated_delta_rule`` -- imported by the reference at
  engine/runtime/cuda_graphs.py:126-135 as the torch decode path;
* ``causal_conv1d_fn`` / ``causal_conv1d_update`` -- the torch conv paths HF's
  GDN layer falls back to (reference call sites kv_cache.py:153-156,
  cuda_graphs.py:202);
* ``Qwen3_5MoeRMSNormGated`` -- the GDN output norm of the same layer.

All of them live in transformers' ``models/qwen3_5_moe/modeling_qwen3_5_moe.py``.
The container has transformers 5.15.0 installed (the reference's uv.lock pins
4.57.6, but its code needs >= 5.5, engine/model/qwen3_next.py:4-5).  This
script calls those functions on small seeded inputs and saves inputs and
outputs as ``golden_gdn.npz``.  Inputs are rounded to bf16-representable
values and passed as fp32, so the vectors serve the fp32 oracle and the bf16
GPU path alike, and HF's l2norm runs in fp32 (as fla's in-kernel l2norm does).

Usage:  HF_HUB_OFFLINE=1 python tests/golden/make_golden.py
"""
from __future__ import annotations

import os

import numpy as np
import torch

from transformers.models.qwen3_5_moe import modeling_qwen3_5_moe as hf

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden_gdn.npz")


def bf16r(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).to(torch.float32)


def gates(gen, shape):
    beta = torch.sigmoid(torch.randn(shape, generator=gen))
    g = -torch.nn.functional.softplus(torch.randn(shape, generator=gen)) * torch.exp(
        torch.empty(shape).uniform_(-2, 0, generator=gen))
    return g, beta


def gdn_case(name, seed, b, t, hk, h, d, h0_std, out, chunk):
    gen = torch.Generator().manual_seed(seed)
    q = bf16r(torch.randn(b, t, hk, d, generator=gen))
    k = bf16r(torch.randn(b, t, hk, d, generator=gen))
    v = bf16r(torch.randn(b, t, h, d, generator=gen))
    g, beta = gates(gen, (b, t, h))
    h0 = torch.randn(b, h, d, d, generator=gen) * h0_std if h0_std else None
    rep = h // hk
    qr, kr = q.repeat_interleave(rep, dim=2), k.repeat_interleave(rep, dim=2)
    fn = hf.torch_chunk_gated_delta_rule if chunk else hf.torch_recurrent_gated_delta_rule
    kw = dict(chunk_size=64) if chunk else {}
    o, s = fn(qr, kr, v, g=g, beta=beta, initial_state=None if h0 is None else h0.clone(),
              output_final_state=True, use_qk_l2norm_in_kernel=True, **kw)
    out.update({f"{name}.q": q, f"{name}.k": k, f"{name}.v": v, f"{name}.g": g,
                f"{name}.beta": beta, f"{name}.o": o, f"{name}.state": s})
    if h0 is not None:
        out[f"{name}.h0"] = h0


def conv_cases(out):
    gen = torch.Generator().manual_seed(7)
    c, w = 24, 4
    x = bf16r(torch.randn(2, c, 7, generator=gen))
    wt = bf16r(torch.randn(c, w, generator=gen) * 0.5)
    y = hf.causal_conv1d_fn(x, wt, None, activation="silu")
    out.update({"conv_fn.x": x, "conv_fn.w": wt, "conv_fn.y": y})
    # short prompt (T < W): the cached window is zero-padded on the left
    xs = bf16r(torch.randn(1, c, 2, generator=gen))
    out.update({"conv_fn_short.x": xs, "conv_fn_short.y": hf.causal_conv1d_fn(xs, wt, None, activation="silu")})
    st = bf16r(torch.randn(3, c, w, generator=gen))
    xu = bf16r(torch.randn(3, c, 1, generator=gen))
    st_after = st.clone()
    yu = hf.causal_conv1d_update(xu, st_after, wt, None, "silu")
    out.update({"conv_upd.x": xu, "conv_upd.state": st, "conv_upd.w": wt, "conv_upd.y": yu,
                "conv_upd.state_after": st_after})


def norm_case(out):
    """HF's RMSNormGated module (the GDN output norm) on fp32 inputs."""
    gen = torch.Generator().manual_seed(21)
    mod = hf.Qwen3_5MoeRMSNormGated(128, eps=1e-6)
    with torch.no_grad():
        mod.weight.copy_(bf16r(1.0 + 0.3 * torch.randn(128, generator=gen)))
    x = bf16r(torch.randn(6, 4, 128, generator=gen))
    z = bf16r(2.0 * torch.randn(6, 4, 128, generator=gen))
    with torch.no_grad():
        y = mod(x, z)
    out.update({"norm_gated.x": x, "norm_gated.z": z, "norm_gated.w": mod.weight.detach(), "norm_gated.y": y})


def main():
    torch.manual_seed(0)
    out: dict[str, torch.Tensor] = {}
    gdn_case("rec_small", 11, b=2, t=9, hk=2, h=4, d=32, h0_std=0.1, out=out, chunk=False)
    gdn_case("rec_d128", 12, b=1, t=5, hk=1, h=1, d=128, h0_std=0.1, out=out, chunk=False)
    gdn_case("chunk_small", 13, b=1, t=100, hk=2, h=4, d=32, h0_std=0.1, out=out, chunk=True)
    gdn_case("chunk_d128", 14, b=1, t=70, hk=1, h=2, d=128, h0_std=0.1, out=out, chunk=True)
    gdn_case("chunk_zero_h0", 15, b=2, t=64, hk=2, h=2, d=16, h0_std=0.0, out=out, chunk=True)
    conv_cases(out)
    x = bf16r(torch.randn(3, 5, 128))
    out["l2norm.x"] = x
    out["l2norm.y"] = hf.l2norm(x, dim=-1, eps=1e-6)
    norm_case(out)
    np.savez_compressed(OUT, **{k: v.detach().cpu().numpy().astype(np.float32) for k, v in out.items()})
    print(f"wrote {OUT}: {len(out)} arrays")


if __name__ == "__main__":
    main()
