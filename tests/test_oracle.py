"""Pins the CPU oracle: golden vectors from transformers' torch reference
functions, closed forms, and agreement between independent algorithms.

None of these retypes the oracle's formula: each compares it with a
different computation (HF's torch code, numpy.linalg.solve, np.convolve,
the recurrence vs the chunk form, algebraic special cases)."""
import numpy as np
import pytest

from conftest import golden_case
from oracle import conv, gdn, proj

RNG = np.random.default_rng(1234)


def rand_inputs(b, t, hk, h, d, rng=RNG, h0_std=0.1):
    q = rng.standard_normal((b, t, hk, d))
    k = rng.standard_normal((b, t, hk, d))
    v = rng.standard_normal((b, t, h, d))
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((b, t, h))))
    g = -np.log1p(np.exp(rng.standard_normal((b, t, h)))) * np.exp(rng.uniform(-2, 0, (b, t, h)))
    h0 = rng.standard_normal((b, h, d, d)) * h0_std if h0_std else None
    return q, k, v, g, beta, h0


# --------------------------------------------------------------------- golden vectors

@pytest.mark.parametrize("name,chunk", [("rec_small", False), ("rec_d128", False),
                                        ("chunk_small", True), ("chunk_d128", True),
                                        ("chunk_zero_h0", True)])
def test_gdn_matches_hf_golden(golden, name, chunk):
    a = golden_case(golden, name)
    fn = gdn.chunk_gated_delta_rule if chunk else gdn.recurrent_gated_delta_rule
    o, s = fn(a["q"], a["k"], a["v"], a["g"], a["beta"], initial_state=a.get("h0"))
    assert np.abs(o - a["o"]).max() < 1e-5
    assert gdn.state_rel_err(s, a["state"]) < 1e-5


@pytest.mark.parametrize("name", ["rec_small", "chunk_small", "chunk_d128"])
def test_other_algorithm_matches_golden(golden, name):
    """The recurrence reproduces HF's chunk vectors and vice versa."""
    a = golden_case(golden, name)
    fn = gdn.recurrent_gated_delta_rule if name.startswith("chunk") else gdn.chunk_gated_delta_rule
    o, s = fn(a["q"], a["k"], a["v"], a["g"], a["beta"], initial_state=a.get("h0"))
    assert np.abs(o - a["o"]).max() < 1e-5
    assert gdn.state_rel_err(s, a["state"]) < 1e-5


def test_conv_matches_hf_golden(golden):
    y, _ = conv.causal_conv1d_fn(golden["conv_fn.x"], golden["conv_fn.w"], activation="silu")
    assert np.abs(y - golden["conv_fn.y"]).max() < 1e-6
    y, _ = conv.causal_conv1d_fn(golden["conv_fn_short.x"], golden["conv_fn.w"], activation="silu")
    assert np.abs(y - golden["conv_fn_short.y"]).max() < 1e-6
    y, st = conv.causal_conv1d_update(golden["conv_upd.x"], golden["conv_upd.state"], golden["conv_upd.w"],
                                      activation="silu")
    assert np.abs(y - golden["conv_upd.y"]).max() < 1e-6
    assert np.array_equal(st.astype(np.float32), golden["conv_upd.state_after"])


def test_l2norm_matches_hf_golden(golden):
    assert np.abs(gdn.l2norm(golden["l2norm.x"].astype(np.float64)) - golden["l2norm.y"]).max() < 1e-6


# --------------------------------------------------------------------- closed forms

def test_l2norm_closed_form():
    x = RNG.standard_normal((7, 128)) * RNG.uniform(1e-3, 10, (7, 1))
    s = (x * x).sum(-1)
    assert np.allclose(np.linalg.norm(gdn.l2norm(x), axis=-1), np.sqrt(s / (s + 1e-6)), rtol=1e-12)


def test_beta_zero_is_pure_decay():
    q, k, v, g, beta, h0 = rand_inputs(2, 9, 2, 4, 16)
    beta[:] = 0.0
    o, s = gdn.recurrent_gated_delta_rule(q, k, v, g, beta, h0)
    decay = np.exp(np.cumsum(g, axis=1))                      # [B, T, H]
    assert np.allclose(s, np.exp(g.sum(1))[:, :, None, None] * h0, rtol=1e-12, atol=1e-14)
    qn = gdn.expand_heads(gdn.l2norm(q), 4) * 16 ** -0.5
    o_ref = np.einsum("bthk,bhkv->bthv", qn * decay[..., None], h0)
    assert np.allclose(o, o_ref, rtol=1e-12, atol=1e-14)


def test_single_token_rank1_write():
    q, k, v, g, beta, _ = rand_inputs(1, 1, 2, 2, 16)
    g[:] = 0.0
    beta[:] = 1.0
    o, s = gdn.recurrent_gated_delta_rule(q, k, v, g, beta, None)
    kn = gdn.expand_heads(gdn.l2norm(k), 2)[:, 0]
    qn = gdn.expand_heads(gdn.l2norm(q), 2)[:, 0] * 16 ** -0.5
    assert np.allclose(s, kn[..., :, None] * v[:, 0][..., None, :], rtol=1e-12)
    assert np.allclose(o[:, 0], (qn * kn).sum(-1)[..., None] * v[:, 0], rtol=1e-12)


def test_delta_write_then_read():
    """With beta=1, g=0 the written value is read back exactly: k^T S = v."""
    q, k, v, g, beta, h0 = rand_inputs(1, 1, 2, 2, 16)
    g[:] = 0.0
    beta[:] = 1.0
    _, s = gdn.recurrent_gated_delta_rule(q, k, v, g, beta, h0)
    kn = gdn.expand_heads(gdn.l2norm(k, eps=0.0), 2)[:, 0]
    # eps makes ||k~|| slightly below 1; use the unit vector the step used (eps=1e-6)
    kn_used = gdn.expand_heads(gdn.l2norm(k), 2)[:, 0]
    read = np.einsum("bhk,bhkv->bhv", kn_used, s)
    nrm2 = (kn_used ** 2).sum(-1)[..., None]
    # k~^T S = (1 - |k~|^2) k~^T S0 + |k~|^2 v  (exact algebra of one delta step)
    expect = (1 - nrm2) * np.einsum("bhk,bhkv->bhv", kn_used, h0) + nrm2 * v[:, 0]
    assert np.allclose(read, expect, rtol=1e-10, atol=1e-12)
    assert np.allclose(kn, kn_used, rtol=1e-5)


def test_linearity_in_v_at_zero_state():
    q, k, v, g, beta, _ = rand_inputs(1, 12, 2, 2, 8)
    v2 = RNG.standard_normal(v.shape)
    o1, s1 = gdn.recurrent_gated_delta_rule(q, k, v, g, beta, None)
    o2, s2 = gdn.recurrent_gated_delta_rule(q, k, v2, g, beta, None)
    o3, s3 = gdn.recurrent_gated_delta_rule(q, k, 2.0 * v - 3.0 * v2, g, beta, None)
    assert np.allclose(o3, 2 * o1 - 3 * o2, atol=1e-12)
    assert np.allclose(s3, 2 * s1 - 3 * s2, atol=1e-12)


# --------------------------------------------------------------------- independent algorithms

@pytest.mark.parametrize("t", [1, 63, 64, 65, 127, 256])
def test_chunk_equals_recurrence(t):
    q, k, v, g, beta, h0 = rand_inputs(1, t, 2, 4, 16)
    o1, s1 = gdn.recurrent_gated_delta_rule(q, k, v, g, beta, h0)
    o2, s2 = gdn.chunk_gated_delta_rule(q, k, v, g, beta, initial_state=h0)
    assert np.abs(o1 - o2).max() < 1e-11
    assert gdn.state_rel_err(s2, s1) < 1e-11


@pytest.mark.parametrize("d", [4, 8, 16])
def test_chunk_equals_recurrence_small_dims(d):
    q, k, v, g, beta, h0 = rand_inputs(2, 100, 1, 2, d)
    o1, s1 = gdn.recurrent_gated_delta_rule(q, k, v, g, beta, h0)
    o2, s2 = gdn.chunk_gated_delta_rule(q, k, v, g, beta, initial_state=h0)
    assert np.abs(o1 - o2).max() < 1e-11 and gdn.state_rel_err(s2, s1) < 1e-11


@pytest.mark.parametrize("dk,dv", [(64, 96), (32, 160), (256, 32)])
def test_chunk_equals_recurrence_unequal_dims(dk, dv):
    """Pins the oracle at the head dims the recurrence kernel also builds
    (K 64 / 256, V a multiple of 32, K != V)."""
    rng = np.random.default_rng(dk * 1000 + dv)
    q, k, _, g, beta, _ = rand_inputs(1, 70, 1, 2, dk, rng=rng, h0_std=0)
    v = rng.standard_normal((1, 70, 2, dv))
    h0 = rng.standard_normal((1, 2, dk, dv)) * 0.1
    o1, s1 = gdn.recurrent_gated_delta_rule(q, k, v, g, beta, h0)
    o2, s2 = gdn.chunk_gated_delta_rule(q, k, v, g, beta, initial_state=h0)
    assert o1.shape == (1, 70, 2, dv) and s1.shape == (1, 2, dk, dv)
    assert np.abs(o1 - o2).max() < 1e-10 and gdn.state_rel_err(s2, s1) < 1e-10


def test_chunk_equals_recurrence_at_extreme_gates():
    """g in {0, -40, ordinary} (e^{-40} = 4e-18; a chunk's cumsum reaches
    -2560 and its exponentials underflow) and beta in {0, 1, ordinary}: the
    chunk form exps only non-positive cumsum differences, so it stays finite
    and equal to the recurrence (the GPU tests' comparator at these gates)."""
    rng = np.random.default_rng(77)
    q, k, v, g, beta, h0 = rand_inputs(1, 150, 2, 4, 16, rng=rng)
    pick = rng.integers(0, 3, g.shape)
    g = np.where(pick == 0, 0.0, np.where(pick == 1, -40.0, g))
    pick = rng.integers(0, 3, beta.shape)
    beta = np.where(pick == 0, 0.0, np.where(pick == 1, 1.0, beta))
    o1, s1 = gdn.recurrent_gated_delta_rule(q, k, v, g, beta, h0)
    o2, s2 = gdn.chunk_gated_delta_rule(q, k, v, g, beta, initial_state=h0)
    assert np.isfinite(o2).all() and np.isfinite(s2).all()
    assert np.abs(o1 - o2).max() < 1e-11 and gdn.state_rel_err(s2, s1) < 1e-11


def test_full_decay_forgets_the_state():
    """g = -40 on every token: the state carried into a token is ~4e-18 of
    itself, so o_t = beta_t (q~_t . k~_t) v_t to that precision."""
    q, k, v, g, beta, h0 = rand_inputs(1, 70, 2, 4, 16)
    g[:] = -40.0
    o, _ = gdn.chunk_gated_delta_rule(q, k, v, g, beta, initial_state=h0)
    qn = gdn.expand_heads(gdn.l2norm(q), 4) * 16 ** -0.5
    kn = gdn.expand_heads(gdn.l2norm(k), 4)
    expect = (beta * (qn * kn).sum(-1))[..., None] * v
    assert np.allclose(o, expect, rtol=1e-12, atol=1e-14)


def test_forward_substitution_is_the_inverse():
    c = 64
    lower = np.tril(RNG.standard_normal((3, c, c)) * 0.3, -1)
    t_mat = gdn.forward_substitution_inverse(-lower) + np.eye(c)
    ref = np.stack([np.linalg.solve(np.eye(c) + lower[i], np.eye(c)) for i in range(3)])
    assert np.allclose(t_mat, ref, rtol=1e-9, atol=1e-11)


def test_state_passing_split():
    q, k, v, g, beta, h0 = rand_inputs(1, 150, 2, 2, 16)
    o, s = gdn.chunk_gated_delta_rule(q, k, v, g, beta, initial_state=h0)
    cut = 77
    oa, sa = gdn.chunk_gated_delta_rule(q[:, :cut], k[:, :cut], v[:, :cut], g[:, :cut], beta[:, :cut],
                                        initial_state=h0)
    ob, sb = gdn.chunk_gated_delta_rule(q[:, cut:], k[:, cut:], v[:, cut:], g[:, cut:], beta[:, cut:],
                                        initial_state=sa)
    assert np.abs(np.concatenate([oa, ob], 1) - o).max() < 1e-11
    assert gdn.state_rel_err(sb, s) < 1e-11


def test_zero_padding_invariance():
    """Zero q/k/v/beta/g tail tokens change neither S nor o[:T]."""
    q, k, v, g, beta, h0 = rand_inputs(1, 70, 2, 2, 16)
    pad = lambda x: np.concatenate([x, np.zeros((1, 30) + x.shape[2:])], 1)
    o, s = gdn.chunk_gated_delta_rule(q, k, v, g, beta, initial_state=h0)
    op, sp = gdn.chunk_gated_delta_rule(pad(q), pad(k), pad(v), pad(g), pad(beta), initial_state=h0,
                                        use_qk_l2norm_in_kernel=True)
    assert np.abs(op[:, :70] - o).max() < 1e-11 and gdn.state_rel_err(sp, s) < 1e-11


def test_varlen_equals_per_sequence():
    lens = [5, 64, 0, 130]
    cu = np.concatenate([[0], np.cumsum(lens)])
    q, k, v, g, beta, _ = rand_inputs(1, int(cu[-1]), 2, 4, 8)
    h0 = RNG.standard_normal((len(lens), 4, 8, 8)) * 0.1
    o, s = gdn.chunk_gated_delta_rule_varlen(q, k, v, g, beta, cu, h0)
    o2, s2 = gdn.recurrent_gated_delta_rule_varlen(q, k, v, g, beta, cu, h0)
    assert np.abs(o - o2).max() < 1e-11 and gdn.state_rel_err(s, s2) < 1e-11
    for i in range(len(lens)):
        a, b = cu[i], cu[i + 1]
        if a == b:
            continue
        oi, si = gdn.recurrent_gated_delta_rule(q[:, a:b], k[:, a:b], v[:, a:b], g[:, a:b], beta[:, a:b],
                                                h0[i:i + 1])
        assert np.abs(o[:, a:b] - oi).max() < 1e-11
        assert np.abs(s[i] - si[0]).max() < 1e-11
    assert np.array_equal(s[2], h0[2])  # empty sequence keeps its state


def test_spec_snapshots_and_commit():
    q, k, v, g, beta, _ = rand_inputs(3, 4, 2, 2, 8)
    pool = RNG.standard_normal((6, 2, 8, 8))
    slots = np.array([4, 1, 5])
    acc = np.array([2, 4, 1])
    o, snaps, committed = gdn.spec_verify(pool, slots, q, k, v, g, beta, acc)
    for b in range(3):
        for t in range(4):
            _, st = gdn.recurrent_gated_delta_rule(q[b:b + 1, :t + 1], k[b:b + 1, :t + 1], v[b:b + 1, :t + 1],
                                                   g[b:b + 1, :t + 1], beta[b:b + 1, :t + 1], pool[slots[b]][None])
            assert np.allclose(snaps[b, t], st[0], atol=1e-13)
        assert np.allclose(committed[slots[b]], snaps[b, acc[b] - 1])
    untouched = [i for i in range(6) if i not in slots]
    assert np.array_equal(committed[untouched], pool[untouched])


def test_slot_step_negative_slot():
    q, k, v, g, beta, _ = rand_inputs(3, 1, 2, 2, 8)
    pool = RNG.standard_normal((5, 2, 8, 8))
    o, new = gdn.slot_recurrent_step(pool, np.array([3, -1, 0]), q, k, v, g, beta)
    o_ref, s_ref = gdn.recurrent_gated_delta_rule(q, k, v, g, beta,
                                                  np.stack([pool[3], np.zeros_like(pool[0]), pool[0]]))
    assert np.allclose(o, o_ref)
    assert np.allclose(new[3], s_ref[0]) and np.allclose(new[0], s_ref[2])
    assert np.array_equal(new[[1, 2, 4]], pool[[1, 2, 4]])


# --------------------------------------------------------------------- conv

def test_conv_equals_numpy_convolve():
    x = RNG.standard_normal((2, 8, 20))
    w = RNG.standard_normal((8, 4))
    y, fin = conv.causal_conv1d_fn(x, w, activation=None)
    for b in range(2):
        for c in range(8):
            ref = np.convolve(x[b, c], w[c, ::-1])[:20]
            assert np.allclose(y[b, c], ref, atol=1e-12)
    assert np.array_equal(fin, x[:, :, -4:])


def test_conv_update_is_last_column_of_fn():
    x = RNG.standard_normal((2, 8, 10))
    w = RNG.standard_normal((8, 4))
    y_full, _ = conv.causal_conv1d_fn(x, w, activation="silu")
    _, state = conv.causal_conv1d_fn(x[:, :, :9], w, activation="silu")
    y1, new_state = conv.causal_conv1d_update(x[:, :, 9:], state, w, activation="silu")
    assert np.allclose(y1[:, :, 0], y_full[:, :, 9], atol=1e-12)
    assert np.array_equal(new_state, x[:, :, -4:])


def test_conv_history_continuation():
    """fn over [a; b] equals fn over a, then fn over b with a's final window."""
    x = RNG.standard_normal((1, 8, 30))
    w = RNG.standard_normal((8, 4))
    y, fin = conv.causal_conv1d_fn(x, w, activation="silu")
    ya, fa = conv.causal_conv1d_fn(x[:, :, :11], w, activation="silu")
    yb, fb = conv.causal_conv1d_fn(x[:, :, 11:], w, activation="silu", initial_state=fa)
    assert np.allclose(np.concatenate([ya, yb], -1), y, atol=1e-12)
    assert np.array_equal(fb, fin)


def test_conv_varlen_equals_per_sequence():
    lens = [3, 40, 1]
    cu = np.concatenate([[0], np.cumsum(lens)])
    x = RNG.standard_normal((int(cu[-1]), 16))
    w = RNG.standard_normal((16, 4))
    h0 = RNG.standard_normal((3, 16, 4))
    y, fin = conv.causal_conv1d_varlen(x, w, cu, initial_states=h0)
    for i in range(3):
        yi, fi = conv.causal_conv1d_fn(x[cu[i]:cu[i + 1]].T[None], w, initial_state=h0[i:i + 1])
        assert np.allclose(y[cu[i]:cu[i + 1]], yi[0].T)
        assert np.array_equal(fin[i], fi[0])


# --------------------------------------------------------------------- layer glue (row f-1)
def test_rms_norm_gated_matches_hf_golden(golden):
    a = golden_case(golden, "norm_gated")
    y = gdn.rms_norm_gated(a["x"], a["z"], a["w"], eps=1e-6)
    assert np.abs(y - a["y"]).max() < 2e-6 * max(1.0, np.abs(a["y"]).max())


def test_rms_norm_gated_invariants():
    rng = np.random.default_rng(3)
    x, z, w = rng.standard_normal((5, 128)), rng.standard_normal((5, 128)), rng.standard_normal(128)
    y = gdn.rms_norm_gated(x, z, w, eps=0.0)
    assert np.allclose(gdn.rms_norm_gated(7.5 * x, z, w, eps=0.0), y)   # scale-free in x
    ones = gdn.rms_norm_gated(x, np.full_like(z, 40.0), np.ones(128), eps=0.0)
    assert np.allclose(np.sqrt((ones * ones).mean(-1)), 40.0)           # silu(40) = 40: rms = 40
    assert np.allclose(gdn.rms_norm_gated(x, np.zeros_like(z), w), 0.0)  # silu(0) = 0


def test_gates_closed_forms():
    A_log = np.log(np.array([1.0, 2.0, 0.5]))
    dt = np.array([0.0, 1.0, -1.0])
    g, beta = gdn.gdn_gates(np.array([[0.0, -1.0, 1.0]]), np.array([[0.0, 100.0, -100.0]]), A_log, dt)
    assert np.allclose(g, -np.exp(A_log) * np.log(2.0))   # a + dt_bias = 0 everywhere
    assert np.allclose(beta, [[0.5, 1.0, 0.0]])
    big = gdn.gdn_gates(np.array([30.0]), np.array([0.0]), np.array([0.0]), np.array([0.0]))[0]
    assert np.allclose(big, -30.0)                         # softplus threshold: identity above 20
    small = gdn.gdn_gates(np.array([-30.0]), np.array([0.0]), np.array([0.0]), np.array([0.0]))[0]
    assert np.allclose(small, -np.exp(-30.0), rtol=1e-9)   # softplus(x) ~ e^x far below 0
    a = np.linspace(-5, 5, 11)
    g_line = gdn.gdn_gates(a, np.zeros_like(a), np.zeros(1), np.zeros(1))[0]
    assert np.all(np.diff(g_line) < 0) and np.all(g_line < 0)   # decay strengthens with a


# ------------------------------------------------------ decode in-projection

def test_round_bf16_matches_torch():
    import torch
    x = np.random.default_rng(61).standard_normal(4096) * 10.0 ** np.random.default_rng(62).integers(-6, 6, 4096)
    ref = torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16).double().numpy()
    assert np.array_equal(proj.round_bf16(x.astype(np.float32)), ref)


def test_in_proj_decode_matches_hf_layer_on_cpu():
    """The decode input side of HF's own module (its four projections in
    bf16 and its torch causal_conv1d_update) on bf16 weights and inputs."""
    import torch
    from transformers.models.qwen3_5_moe import modeling_qwen3_5_moe as hf
    from transformers.models.qwen3_5_moe.configuration_qwen3_5_moe import Qwen3_5MoeTextConfig
    cfg = Qwen3_5MoeTextConfig(hidden_size=64, num_hidden_layers=1, layer_types=["linear_attention"],
                               linear_num_key_heads=2, linear_num_value_heads=4, linear_key_head_dim=16,
                               linear_value_head_dim=16, linear_conv_kernel_dim=4)
    torch.manual_seed(63)
    layer = hf.Qwen3_5MoeGatedDeltaNet(cfg, layer_idx=0).eval().to(torch.bfloat16)
    x = torch.randn(3, 64).to(torch.bfloat16)
    c = layer.conv1d.weight.shape[0]
    st = torch.randn(3, c, 4).to(torch.bfloat16)
    cw = layer.conv1d.weight.squeeze(1)
    with torch.no_grad():
        qkv = layer.in_proj_qkv(x)
        hf_st = st.clone()
        y_hf = hf.causal_conv1d_update(qkv[:, :, None], hf_st, cw, None, "silu")[:, :, 0]
        z_hf, b_hf, a_hf = layer.in_proj_z(x), layer.in_proj_b(x), layer.in_proj_a(x)
    f = lambda t: t.detach().double().numpy()
    y, z, b, a, new_st = proj.in_proj_decode(f(x), f(layer.in_proj_qkv.weight), f(layer.in_proj_z.weight),
                                             f(layer.in_proj_b.weight), f(layer.in_proj_a.weight), f(cw), f(st))
    # HF runs in bf16 (fp32 sums, one rounding per op): allow two bf16 ulps of
    # the terms' magnitudes, the projection's ulp carried through the last tap
    ulp = 2.0 ** -7
    terms = np.abs(f(cw))[None, :, :3] * np.abs(f(st))[:, :, 1:]
    y_scale = terms.sum(-1) + np.abs(f(cw))[None, :, 3] * np.abs(f(qkv))
    assert (np.abs(y - f(y_hf)) <= 2 * ulp * y_scale + 1e-6).all()
    for got, ref in ((z, z_hf), (b, b_hf), (a, a_hf)):
        assert (np.abs(got - f(ref)) <= ulp * np.abs(f(ref)) + 1e-3).all()
    # the new window: the three shifted taps exactly, then the bf16 projection
    assert np.array_equal(new_st[:, :, :3], f(st)[:, :, 1:])
    assert (np.abs(new_st[:, :, 3] - f(hf_st)[:, :, 3]) <= ulp * np.abs(f(hf_st)[:, :, 3])).all()


def test_in_proj_decode_is_the_matmul_then_the_conv_update():
    """Brute force on tiny shapes: every output entry as an explicit sum."""
    rng = np.random.default_rng(64)
    m, k = 2, 8
    x, wq, wz, wb, wa = (rng.standard_normal(s) for s in ((m, k), (4, k), (3, k), (2, k), (2, k)))
    cw, st = rng.standard_normal((4, 4)), rng.standard_normal((m, 4, 4))
    y, z, b, a, new_st = proj.in_proj_decode(x, wq, wz, wb, wa, cw, st, activation=None)
    for r in range(m):
        for c in range(4):
            p = proj.round_bf16(sum(x[r, i] * wq[c, i] for i in range(k)))
            ref = sum(cw[c, j] * st[r, c, j + 1] for j in range(3)) + cw[c, 3] * p
            assert abs(y[r, c] - ref) < 1e-12
            assert list(new_st[r, c]) == [st[r, c, 1], st[r, c, 2], st[r, c, 3], p]
        assert np.allclose(z[r], [sum(x[r, i] * wz[j, i] for i in range(k)) for j in range(3)], atol=1e-12)
        assert np.allclose(b[r], [sum(x[r, i] * wb[j, i] for i in range(k)) for j in range(2)], atol=1e-12)
        assert np.allclose(a[r], [sum(x[r, i] * wa[j, i] for i in range(k)) for j in range(2)], atol=1e-12)


def test_out_proj_matches_hf_module_on_cpu():
    """HF's out_proj module (bf16 weights, bf16 output) against the exact sum
    rounded to bf16: equal up to the fp32 summation of the module (one ulp
    of the rounding plus 2^-16 of the terms' magnitudes)."""
    import torch
    from transformers.models.qwen3_5_moe import modeling_qwen3_5_moe as hf
    from transformers.models.qwen3_5_moe.configuration_qwen3_5_moe import Qwen3_5MoeTextConfig
    cfg = Qwen3_5MoeTextConfig(hidden_size=64, num_hidden_layers=1, layer_types=["linear_attention"],
                               linear_num_key_heads=2, linear_num_value_heads=4, linear_key_head_dim=16,
                               linear_value_head_dim=32, linear_conv_kernel_dim=4)
    torch.manual_seed(65)
    layer = hf.Qwen3_5MoeGatedDeltaNet(cfg, layer_idx=0).eval().to(torch.bfloat16)
    x = torch.randn(5, 1, 128).to(torch.bfloat16)
    with torch.no_grad():
        y_hf = layer.out_proj(x)[:, 0]
    f = lambda t: t.detach().double().numpy()
    w = f(layer.out_proj.weight)
    assert w.shape == (64, 128)
    ref = proj.out_proj(f(x[:, 0]), w)
    scale = np.abs(f(x[:, 0])) @ np.abs(w).T
    assert (np.abs(proj.round_bf16(ref) - f(y_hf)) <= 2.0 ** -7 * np.abs(ref) + 2.0 ** -16 * scale).all()


def test_out_proj_is_the_explicit_sum():
    rng = np.random.default_rng(66)
    x, w = rng.standard_normal((3, 7)), rng.standard_normal((5, 7))
    y = proj.out_proj(x, w)
    for r in range(3):
        for c in range(5):
            assert abs(y[r, c] - sum(x[r, i] * w[c, i] for i in range(7))) < 1e-12
