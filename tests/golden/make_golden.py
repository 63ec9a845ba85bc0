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

It also writes ``golden_layer.npz``: the expected values of the layer-level
GPU tests, from transformers' ``Qwen3_5MoeGatedDeltaNet.forward`` (fp32, CPU,
with its own torch GDN paths and ``DynamicCache``) on the seeded layers of
``tests/layer_cases.py`` -- prefill, cached decode, sequences decoded side by
side (each through its own cache, as the reference engine's slot cache
gathers them), a slot reset and reused, and speculative verify of T = 1, 4
and 17 tokens followed by the decode of only the accepted tokens.  The GPU
tests rebuild the same weights and compare.  The expected values always come
from HF's forward on its own torch paths, here; on the GPU box HF's forward
runs only as the caller of the installed GPU kernels (test_gpu_binding.py),
never as the source of expected values.

Usage:  HF_HUB_OFFLINE=1 python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

from transformers.models.qwen3_5_moe import modeling_qwen3_5_moe as hf

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import layer_cases as lc  # noqa: E402  (tests/layer_cases.py)

OUT = os.path.join(HERE, "golden_gdn.npz")
OUT_LAYER = os.path.join(HERE, lc.GOLDEN_LAYER)


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
    layer_fixtures()


class Seq:
    """One sequence through HF's GDN module with its own DynamicCache."""

    def __init__(self, cfg, module):
        from transformers.cache_utils import DynamicCache
        self.m, self.cache = module, DynamicCache(config=cfg)

    def __call__(self, x):
        with torch.no_grad():
            return self.m(x, cache_params=self.cache)

    def state(self, heads=None):
        s = self.cache.layers[0].recurrent_states[0]
        return s if heads is None else s[:, heads]

    def conv(self):
        return self.cache.layers[0].conv_states[0]


def layer_fixtures():
    """Expected values of the layer-level GPU tests (see the module docstring).
    States are stored as fp16 for the heads in STATE_HEADS (fp16 keeps 11
    bits; the tests compare states to 1e-2 relative)."""
    out: dict[str, np.ndarray] = {}
    gen = torch.Generator().manual_seed(4321)
    tiny_heads = [0, 3]

    def put(key, t, dtype=np.float32):
        out[key] = (t.detach().cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t)).astype(dtype)

    def put_seq(prefix, seq, heads):
        put(prefix + ".state", seq.state(heads), np.float16)
        put(prefix + ".conv", seq.conv())

    cfg, m = lc.layer("tiny")
    put("tiny.sig", lc.weight_signature(m), np.float64)
    # one prefill without a cache
    x = lc.bf16_inputs(gen, 1, 150, 64)
    with torch.no_grad():
        put("prefill.x", x)
        put("prefill.y", m(x))
    # B = 2: prefill then three cached decode steps
    s = Seq(cfg, m)
    steps = [lc.bf16_inputs(gen, 2, 70, 64)] + [lc.bf16_inputs(gen, 2, 1, 64) for _ in range(3)]
    for i, xs in enumerate(steps):
        put(f"cache.x{i}", xs)
        put(f"cache.y{i}", s(xs))
    put("cache.state", s.state(), np.float16)
    put("cache.conv", s.conv())
    # slot pools: A, B, C prefilled one at a time, decoded side by side; then
    # B's slot reset and reused by D, decoded in another row order
    seqs = {n: Seq(cfg, m) for n in "ABC"}
    for n, length in zip("ABC", (70, 5, 130)):
        x = lc.bf16_inputs(gen, 1, length, 64)
        put(f"pools.pre{n}.x", x)
        put(f"pools.pre{n}.y", seqs[n](x))
    for i in range(3):
        x = lc.bf16_inputs(gen, 3, 1, 64)
        put(f"pools.dec{i}.x", x)
        put(f"pools.dec{i}.y", torch.cat([seqs[n](x[r:r + 1]) for r, n in enumerate("ABC")]))
    for n in "ABC":
        put_seq(f"pools.after1.{n}", seqs[n], tiny_heads)
    seqs["D"] = Seq(cfg, m)
    x = lc.bf16_inputs(gen, 1, 40, 64)
    put("pools.preD.x", x)
    put("pools.preD.y", seqs["D"](x))
    for i in range(2):
        x = lc.bf16_inputs(gen, 3, 1, 64)
        put(f"pools.redec{i}.x", x)
        put(f"pools.redec{i}.y", torch.cat([seqs[n](x[r:r + 1]) for r, n in enumerate("CDA")]))
    for n in "ACD":
        put_seq(f"pools.after2.{n}", seqs[n], tiny_heads)
    # speculative verify of T tokens, then only the accepted ones decoded by HF
    pre = {n: lc.bf16_inputs(gen, 1, length, 64) for n, length in zip("ABC", (70, 5, 130))}
    for n in "ABC":
        put(f"verify.pre{n}.x", pre[n])
    for t, acc in ((4, [1, 3, 4]), (1, [1, 1, 1]), (17, [1, 9, 17])):
        seqs = {n: Seq(cfg, m) for n in "ABC"}
        for n in "ABC":
            seqs[n](pre[n])
        xv = lc.bf16_inputs(gen, 3, t, 64)
        y = torch.zeros(3, t, 64)
        for r, (n, a) in enumerate(zip("ABC", acc)):
            y[r, :a] = torch.cat([seqs[n](xv[r:r + 1, i:i + 1]) for i in range(a)], dim=1)[0]
        put(f"verify{t}.x", xv)
        put(f"verify{t}.acc", np.array(acc), np.int32)
        put(f"verify{t}.y", y)
        for n in "ABC":
            put_seq(f"verify{t}.{n}", seqs[n], tiny_heads)
        xn = lc.bf16_inputs(gen, 3, 1, 64)
        put(f"verify{t}.xn", xn)
        put(f"verify{t}.yn", torch.cat([seqs[n](xn[r:r + 1]) for r, n in enumerate("ABC")]))

    # hidden 1024 (the fused decode input kernel's smallest K): three sequences, three decode steps
    cfg, m = lc.layer("w1024")
    put("w1024.sig", lc.weight_signature(m), np.float64)
    seqs = [Seq(cfg, m) for _ in range(3)]
    for i, length in enumerate((40, 7, 70)):
        x = lc.bf16_inputs(gen, 1, length, 1024)
        put(f"w1024.pre{i}.x", x)
        put(f"w1024.pre{i}.y", seqs[i](x))
    for step in range(3):
        x = lc.bf16_inputs(gen, 3, 1, 1024)
        put(f"w1024.dec{step}.x", x)
        put(f"w1024.dec{step}.y", torch.cat([seqs[r](x[r:r + 1]) for r in range(3)]))
    for i in range(3):
        put_seq(f"w1024.seq{i}", seqs[i], [0, 3])

    # the Qwen3.5-MoE GDN layer shape (hidden 2048, 16 / 32 heads): two sequences, two decode steps
    cfg, m = lc.layer("model")
    put("model.sig", lc.weight_signature(m), np.float64)
    seqs = [Seq(cfg, m) for _ in range(2)]
    for i, length in enumerate((20, 9)):
        x = lc.bf16_inputs(gen, 1, length, 2048)
        put(f"model.pre{i}.x", x)
        put(f"model.pre{i}.y", seqs[i](x))
    for step in range(2):
        x = lc.bf16_inputs(gen, 2, 1, 2048)
        put(f"model.dec{step}.x", x)
        put(f"model.dec{step}.y", torch.cat([seqs[r](x[r:r + 1]) for r in range(2)]))
    for i in range(2):
        put_seq(f"model.seq{i}", seqs[i], lc.MODEL_STATE_HEADS)

    np.savez_compressed(OUT_LAYER, **out)
    print(f"wrote {OUT_LAYER}: {len(out)} arrays")


if __name__ == "__main__":
    main()
