"""CPU checks of the layer fixture (tests/golden/golden_layer.npz).

The layer-level GPU tests compare with values that transformers'
``Qwen3_5MoeGatedDeltaNet.forward`` produced in the build container.  Here
that fixture is pinned independently of HF: the weights rebuilt by
tests/layer_cases.py must match the stored signatures bit for bit, and the
stored outputs must equal the layer forward composed from this repository's
oracle (projections, conv, gates, chunk rule, gated norm, out projection;
transformers modeling_qwen3_5_moe.py:430-541 step by step) in fp64.
"""
import numpy as np
import pytest

import layer_cases as lc
from oracle import conv, gdn


@pytest.fixture(scope="module")
def golden():
    return lc.load_golden()


@pytest.mark.parametrize("name", sorted(lc.LAYERS))
def test_weights_rebuild_bit_for_bit(golden, name):
    _, m = lc.layer(name)
    np.testing.assert_array_equal(lc.weight_signature(m), golden[f"{name}.sig"])


def oracle_layer(m, x, h0=None, conv0=None):
    """HF's GDN layer forward restated with the oracle, fp64: x [B, T, H]."""
    f = lambda t: t.detach().double().numpy()  # noqa: E731
    hk, hv = m.num_k_heads, m.num_v_heads
    b, t, _ = x.shape
    p = x @ f(m.in_proj_qkv.weight).T                          # [B, T, C]
    y, conv_final = conv.causal_conv1d_fn(p.transpose(0, 2, 1), f(m.conv1d.weight)[:, 0], None,
                                          activation="silu", initial_state=conv0)
    y = y.transpose(0, 2, 1)
    kd = hk * 128
    q = y[..., :kd].reshape(b, t, hk, 128)
    k = y[..., kd:2 * kd].reshape(b, t, hk, 128)
    v = y[..., 2 * kd:].reshape(b, t, hv, 128)
    g, beta = gdn.gdn_gates(x @ f(m.in_proj_a.weight).T, x @ f(m.in_proj_b.weight).T, f(m.A_log), f(m.dt_bias))
    o, s = gdn.chunk_gated_delta_rule(q, k, v, g, beta, initial_state=h0)
    z = (x @ f(m.in_proj_z.weight).T).reshape(b, t, hv, 128)
    out = gdn.rms_norm_gated(o, z, f(m.norm.weight), eps=1e-6).reshape(b, t, hv * 128)
    return out @ f(m.out_proj.weight).T, s, conv_final


def test_prefill_fixture_matches_the_oracle_layer(golden):
    _, m = lc.layer("tiny")
    y, _, _ = oracle_layer(m, golden["prefill.x"].astype(np.float64))
    ref = golden["prefill.y"].astype(np.float64)
    assert np.abs(y - ref).max() <= 1e-4 * np.abs(ref).max()


def test_cached_steps_fixture_matches_the_oracle_layer(golden):
    """The B = 2 prefill and three cached decode steps (state and conv window
    carried from step to step), then the final states and conv windows."""
    _, m = lc.layer("tiny")
    s = c = None
    for i in range(4):
        y, s, c = oracle_layer(m, golden[f"cache.x{i}"].astype(np.float64), h0=s, conv0=c)
        ref = golden[f"cache.y{i}"].astype(np.float64)
        assert np.abs(y - ref).max() <= 1e-4 * np.abs(ref).max(), i
    assert gdn.state_rel_err(s, golden["cache.state"].astype(np.float64)) < 2e-3  # (stored in fp16)
    assert np.abs(c - golden["cache.conv"]).max() <= 1e-5 * np.abs(c).max()
