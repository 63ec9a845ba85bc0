"""Seeded GDN layers for the layer-level parity tests.

The expected values of the layer tests (rows f-1 to f-4 end to end) come
from transformers' own ``Qwen3_5MoeGatedDeltaNet.forward`` -- the module the
reference runs for its GDN layers -- executed in fp32 on the CPU by
``tests/golden/make_golden.py`` in the build container, and stored in
``tests/golden/golden_layer.npz``.  The GPU tests never run that forward: they
use the HF class only as a container for the same weights, which this module
rebuilds bit for bit on any machine.

Weights are integer draws of numpy's PCG64 generator scaled by powers of two,
so every value is exact in bf16 and independent of the host's floating-point
libraries (no transcendental functions are involved).  Inputs are stored in
the fixture itself.
"""
from __future__ import annotations

import math

import numpy as np
import torch

GOLDEN_LAYER = "golden_layer.npz"


def config(hidden=64, hk=2, hv=4):
    """A Qwen3.5-MoE text config with one GDN layer of the given width."""
    from transformers.models.qwen3_5_moe.configuration_qwen3_5_moe import Qwen3_5MoeTextConfig
    return Qwen3_5MoeTextConfig(hidden_size=hidden, num_hidden_layers=1, layer_types=["linear_attention"],
                                linear_num_key_heads=hk, linear_num_value_heads=hv, linear_key_head_dim=128,
                                linear_value_head_dim=128, linear_conv_kernel_dim=4, rms_norm_eps=1e-6)


def _ints(rng, shape, lo, hi):
    return rng.integers(lo, hi, size=shape, dtype=np.int64).astype(np.float64)


def _tensor(x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))


def make_layer(cfg, seed):
    """``Qwen3_5MoeGatedDeltaNet`` (fp32, CPU, eval) holding seeded bf16-exact weights.

    Linear weights are k / 128 * 2^-e with k in [-128, 128) and 2^-e the power
    of two nearest 1 / sqrt(fan_in); conv taps k / 256; norm weight
    1 + k / 128 (k in [-32, 32)); dt_bias k / 64 (k in [-128, 128)); A_log
    k / 32 (k in [-22, 44), so exp(A_log) spans about [0.5, 4])."""
    from transformers.models.qwen3_5_moe import modeling_qwen3_5_moe as hf
    rng = np.random.Generator(np.random.PCG64(seed))
    m = hf.Qwen3_5MoeGatedDeltaNet(cfg, layer_idx=0).eval()
    with torch.no_grad():
        for lin in (m.in_proj_qkv, m.in_proj_z, m.in_proj_b, m.in_proj_a, m.out_proj):
            fan_in = lin.weight.shape[1]
            scale = 2.0 ** -round(math.log2(math.sqrt(fan_in)))
            lin.weight.copy_(_tensor(_ints(rng, lin.weight.shape, -128, 128) / 128 * scale))
        m.conv1d.weight.copy_(_tensor(_ints(rng, m.conv1d.weight.shape, -128, 128) / 256))
        m.norm.weight.copy_(_tensor(1.0 + _ints(rng, m.norm.weight.shape, -32, 32) / 128))
        m.dt_bias.copy_(_tensor(_ints(rng, m.dt_bias.shape, -128, 128) / 64))
        m.A_log.copy_(_tensor(_ints(rng, m.A_log.shape, -22, 44) / 32))
    for p in m.parameters():
        assert torch.equal(p, p.to(torch.bfloat16).float()), "weights must be bf16-exact"
    return m


def weight_signature(m) -> np.ndarray:
    """Sum and sum of squares of every parameter (fp64): stored next to the
    expected values so a test can tell that it rebuilt the same weights."""
    return np.array([[p.detach().double().sum().item(), (p.detach().double() ** 2).sum().item()]
                     for _, p in sorted(m.named_parameters())])


def bf16_inputs(gen, *shape):
    """Layer inputs: N(0, 1) rounded to bf16 (stored in the fixture)."""
    return torch.randn(*shape, generator=gen).to(torch.bfloat16).float()


# Layers of the fixture: name -> (config kwargs, weight seed)
LAYERS = {
    "tiny": (dict(hidden=64, hk=2, hv=4), 1234),
    "w1024": (dict(hidden=1024, hk=2, hv=4), 1235),
    "model": (dict(hidden=2048, hk=16, hv=32), 1236),
}

# State heads kept in the fixture for the model-shape layer (all 32 would be 4 MiB per sequence)
MODEL_STATE_HEADS = [0, 13, 31]


def layer(name):
    kw, seed = LAYERS[name]
    cfg = config(**kw)
    return cfg, make_layer(cfg, seed)


# ---------------------------------------------------------------- test side
TINY_STATE_HEADS = [0, 3]  # state heads stored for the tiny layer


def load_golden() -> dict:
    import os
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", GOLDEN_LAYER))
    return {k: z[k] for k in z.files}


def gpu_layer(name, golden, device="cuda"):
    """(config, layer in bf16 on the device) with the fixture's weights --
    checked against the stored signature, so a drift in the generator would
    fail here rather than as a tolerance miss."""
    cfg, m = layer(name)
    np.testing.assert_array_equal(weight_signature(m), golden[f"{name}.sig"])
    return cfg, m.to(device, torch.bfloat16)


def f64(t) -> np.ndarray:
    if isinstance(t, torch.Tensor):
        t = t.detach().float().cpu().numpy()
    return np.asarray(t, dtype=np.float64)


def layer_close(y, ref, tol=3e-2) -> bool:
    """Layer outputs: max abs error <= tol * max |ref| (bf16 projections and
    intermediates on the GPU path against an fp32 forward)."""
    y, ref = f64(y), f64(ref)
    return y.shape == ref.shape and np.abs(y - ref).max() <= tol * np.abs(ref).max()


def state_close(state, ref, heads, tol=1e-2) -> bool:
    """A pool row [Hv, K, V] against a stored [1, len(heads), K, V] state:
    relative error, norm-wise per head, <= tol."""
    s = f64(state)[heads]
    r = f64(ref)[0]
    err = np.sqrt(((s - r) ** 2).sum(axis=(1, 2))) / np.maximum(np.sqrt((r ** 2).sum(axis=(1, 2))), 1e-30)
    return err.max() <= tol


def conv_close(window, ref, tol=2e-2) -> bool:
    """A conv window [C, S] (bf16) against a stored [1, C, S] one."""
    return np.abs(f64(window)[None] - f64(ref)).max() <= tol
