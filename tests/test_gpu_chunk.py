"""GPU parity of the chunk-64 prefill (MFMA path) with the CPU oracle.

Tolerances (north star): bf16 outputs max abs error <= 2e-2; fp32 final
states relative error <= 1e-3, norm-wise per (sequence, head).  Inputs are
bf16 (the MFMA operand type); the oracle sees the same bf16 values in fp64.
"""
import numpy as np
import pytest
import torch

from conftest import golden_case
from engine import configs
from engine.kernels import causal_conv1d_fn, chunk_gated_delta_rule, fused_recurrent_gated_delta_rule
from oracle import conv, gdn

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

DEV = "cuda"
O_TOL = 2e-2
S_TOL = 1e-3


def np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def run_chunk(c, h0=None, **kw):
    args = [c[x].to(DEV) for x in ("q", "k", "v", "g", "beta")]
    return chunk_gated_delta_rule(*args, initial_state=None if h0 is None else h0.to(DEV),
                                  output_final_state=True, use_qk_l2norm_in_kernel=True, **kw)


def oracle_chunk(c, h0=None):
    return gdn.chunk_gated_delta_rule(*(c[x].float().numpy() for x in ("q", "k", "v", "g", "beta")),
                                      initial_state=None if h0 is None else h0.numpy())


def test_chunk_matches_hf_golden(golden):
    a = {k: torch.from_numpy(v) for k, v in golden_case(golden, "chunk_d128").items()}
    c = {x: a[x].to(torch.bfloat16) for x in ("q", "k", "v")}
    c.update(g=a["g"], beta=a["beta"])
    o, s = run_chunk(c, a["h0"])
    assert o.dtype == torch.bfloat16
    assert np.abs(np64(o) - a["o"].numpy()).max() < O_TOL
    assert gdn.state_rel_err(np64(s), a["state"].numpy()) < S_TOL


def test_config2_t4096():
    c = configs.config2()
    o_ref, s_ref = oracle_chunk(c)
    o, s = run_chunk(c)
    err_o = np.abs(np64(o) - o_ref).max()
    err_s = gdn.state_rel_err(np64(s), s_ref)
    print(f"config2: max|o-o_ref|={err_o:.3e} state rel={err_s:.3e}")
    assert err_o < O_TOL and err_s < S_TOL


@pytest.mark.parametrize("t", [1, 17, 63, 64, 65, 127, 200])
def test_ragged_lengths_with_initial_state(t):
    c = configs.config2(seed=100 + t, t=t)
    h0 = torch.randn(1, 32, 128, 128, generator=torch.Generator().manual_seed(t)) * 0.1
    o_ref, s_ref = oracle_chunk(c, h0)
    o, s = run_chunk(c, h0)
    assert np.abs(np64(o) - o_ref).max() < O_TOL
    assert gdn.state_rel_err(np64(s), s_ref) < S_TOL


def test_batched_b2_and_gqa_native_equals_repeated():
    c = configs.config2(seed=7, t=150)
    cb = {x: torch.cat([c[x], c[x].flip(1)], 0) for x in c}
    o, s = run_chunk(cb)
    o_ref, s_ref = oracle_chunk(cb)
    assert np.abs(np64(o) - o_ref).max() < O_TOL and gdn.state_rel_err(np64(s), s_ref) < S_TOL
    rep = dict(cb)
    rep["q"] = cb["q"].repeat_interleave(2, 2)
    rep["k"] = cb["k"].repeat_interleave(2, 2)
    o2, s2 = run_chunk(rep)
    assert torch.equal(o2, o) and torch.equal(s2, s)


@pytest.mark.parametrize("t", [300, 4200])
def test_repeated_qk_single_sequence_equals_native(t):
    """q and k given per v-head (Hk == Hv) as repeat_interleave makes them: the
    prep finds every pair of v-heads repeated and the scan reads one copy of
    each pair; the results are the GQA call's bits (4200 tokens: two workspace
    segments)."""
    c = configs.config2(seed=11, t=t)
    o, s = run_chunk(c)
    rep = dict(c)
    rep["q"] = c["q"].repeat_interleave(2, 2)
    rep["k"] = c["k"].repeat_interleave(2, 2)
    o2, s2 = run_chunk(rep)
    assert torch.equal(o2, o) and torch.equal(s2, s)


def test_per_v_head_qk_with_partly_repeated_pairs():
    """Hk == Hv with pairs that repeat in every chunk, pairs that differ in
    one row of one chunk (q of head 5, k of head 9), and independent heads
    (20-31): each v-head's own q and k rows are used wherever its pair differs."""
    c = configs.config2(seed=12, t=300)
    gen = torch.Generator().manual_seed(13)
    q = c["q"].repeat_interleave(2, 2).clone()
    k = c["k"].repeat_interleave(2, 2).clone()
    q[0, 130, 5] = torch.randn(128, generator=gen).to(torch.bfloat16)
    k[0, 200, 9] = torch.randn(128, generator=gen).to(torch.bfloat16)
    q[:, :, 20:] = torch.randn(1, 300, 12, 128, generator=gen).to(torch.bfloat16)
    k[:, :, 20:] = torch.randn(1, 300, 12, 128, generator=gen).to(torch.bfloat16)
    mixed = dict(c, q=q, k=k)
    o, s = run_chunk(mixed)
    o_ref, s_ref = oracle_chunk(mixed)
    assert np.abs(np64(o) - o_ref).max() < O_TOL
    assert gdn.state_rel_err(np64(s), s_ref) < S_TOL



def test_per_v_head_qk_pairs_on_the_persistent_scan():
    """A batch of three (the persistent scan walks all of their chunks) with
    q and k given per v-head: pairs repeated in every chunk of every
    sequence, a pair whose odd head differs in one row of the second
    sequence (q of head 7), a pair whose even head differs in one row of the
    third (k of head 12), and independent heads (24-31)."""
    c = configs.config2(seed=14, t=150)
    cb = {x: torch.cat([c[x], c[x].flip(1), c[x].roll(7, 1)], 0) for x in c}
    gen = torch.Generator().manual_seed(15)
    q = cb["q"].repeat_interleave(2, 2).clone()
    k = cb["k"].repeat_interleave(2, 2).clone()
    q[1, 77, 7] = torch.randn(128, generator=gen).to(torch.bfloat16)
    k[2, 140, 12] = torch.randn(128, generator=gen).to(torch.bfloat16)
    q[:, :, 24:] = torch.randn(3, 150, 8, 128, generator=gen).to(torch.bfloat16)
    k[:, :, 24:] = torch.randn(3, 150, 8, 128, generator=gen).to(torch.bfloat16)
    mixed = dict(cb, q=q, k=k)
    o, s = run_chunk(mixed)
    o_ref, s_ref = oracle_chunk(mixed)
    assert np.abs(np64(o) - o_ref).max() < O_TOL
    assert gdn.state_rel_err(np64(s), s_ref) < S_TOL

def test_slot_pool_in_place():
    c = configs.config2(seed=8, t=100)
    cb = {x: torch.cat([c[x], c[x].flip(1)], 0) for x in c}
    gen = torch.Generator().manual_seed(3)
    pool0 = torch.randn(5, 32, 128, 128, generator=gen) * 0.1
    slots = torch.tensor([3, 1])
    o_ref, s_ref = oracle_chunk(cb, pool0[slots])
    pool = pool0.to(DEV)
    o, ret = chunk_gated_delta_rule(*(cb[x].to(DEV) for x in ("q", "k", "v", "g", "beta")), initial_state=pool,
                                    ssm_state_indices=slots.to(DEV), inplace_final_state=True,
                                    use_qk_l2norm_in_kernel=True)
    assert ret is pool
    assert np.abs(np64(o) - o_ref).max() < O_TOL
    assert gdn.state_rel_err(np64(pool[slots.to(DEV)]), s_ref) < S_TOL
    assert torch.equal(pool[[0, 2, 4]].cpu(), pool0[[0, 2, 4]])


def test_config3_varlen_after_conv():
    """conv1d over the packed 8192-wide projection, q|k|v split as strided views,
    chunk prefill with cu_seqlens and per-sequence initial states."""
    c = configs.config3()
    cu = c["cu_seqlens"]
    x, w = c["x"], c["conv_w"]
    y_ref, _ = conv.causal_conv1d_varlen(x.float().numpy(), w.float().numpy(), cu.numpy(), activation="silu",
                                         dtype=np.float32)
    y = causal_conv1d_fn(x.to(DEV), w.to(DEV), None, activation="silu", cu_seqlens=cu.to(DEV))
    q, k, v = configs.split_qkv(y)
    assert q.stride(1) == configs.CONV_DIM
    o, s = chunk_gated_delta_rule(q, k, v, c["g"].to(DEV), c["beta"].to(DEV), initial_state=c["h0"].to(DEV),
                                  output_final_state=True, use_qk_l2norm_in_kernel=True, cu_seqlens=cu.to(DEV))
    # oracle on the GPU's own conv output (bf16), so the GDN check is isolated from the conv rounding
    yq, yk, yv = (np64(t) for t in (q, k, v))
    o_ref, s_ref = gdn.chunk_gated_delta_rule_varlen(yq, yk, yv, c["g"].numpy(), c["beta"].numpy(), cu.numpy(),
                                                     c["h0"].numpy())
    err_o = np.abs(np64(o) - o_ref).max()
    err_s = gdn.state_rel_err(np64(s), s_ref)
    err_c = (np.abs(np64(y) - y_ref) / np.maximum(1.0, np.abs(y_ref))).max()
    print(f"config3: max|o-o_ref|={err_o:.3e} state rel={err_s:.3e} conv max err (rel to max(1,|y|))={err_c:.3e}")
    assert err_c <= 2e-2  # conv of the bf16 projection with zero history: bf16 output rounding
    assert err_o < O_TOL and err_s < S_TOL


def test_varlen_with_empty_and_tiny_sequences():
    lens = [0, 1, 64, 0, 70, 3]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    c = configs.config2(seed=55, t=int(cu[-1]))
    h0 = torch.randn(len(lens), 32, 128, 128, generator=torch.Generator().manual_seed(1)) * 0.1
    o_ref, s_ref = gdn.chunk_gated_delta_rule_varlen(*(c[x].float().numpy() for x in ("q", "k", "v", "g", "beta")),
                                                     cu.numpy(), h0.numpy())
    o, s = chunk_gated_delta_rule(*(c[x].to(DEV) for x in ("q", "k", "v", "g", "beta")), initial_state=h0.to(DEV),
                                  output_final_state=True, use_qk_l2norm_in_kernel=True, cu_seqlens=cu.to(DEV))
    assert np.abs(np64(o) - o_ref).max() < O_TOL
    assert gdn.state_rel_err(np64(s), s_ref) < S_TOL
    assert torch.equal(s[0].cpu(), h0[0]) and torch.equal(s[3].cpu(), h0[3])


def test_chunk_agrees_with_recurrent_kernel():
    c = configs.config2(seed=9, t=300)
    h0 = torch.randn(1, 32, 128, 128, generator=torch.Generator().manual_seed(2)) * 0.1
    o1, s1 = run_chunk(c, h0)
    o2, s2 = fused_recurrent_gated_delta_rule(*(c[x].to(DEV) for x in ("q", "k", "v", "g", "beta")),
                                              initial_state=h0.to(DEV), output_final_state=True,
                                              use_qk_l2norm_in_kernel=True)
    assert (o1.float() - o2.float()).abs().max().item() < O_TOL
    assert gdn.state_rel_err(np64(s1), np64(s2)) < S_TOL


def test_state_passing_split_on_gpu():
    """Prefill [0, 130) then [130, 260) with the state threaded equals one call."""
    c = configs.config2(seed=10, t=260)
    o, s = run_chunk(c)
    first = {x: c[x][:, :130] for x in c}
    second = {x: c[x][:, 130:] for x in c}
    oa, sa = run_chunk(first)
    ob, sb = run_chunk(second, sa.cpu())
    assert (torch.cat([oa, ob], 1).float() - o.float()).abs().max().item() < O_TOL
    assert gdn.state_rel_err(np64(sb), np64(s)) < S_TOL


def test_segments_equal_split_calls():
    """Inputs over 64 chunks run as several prep + scan segments, the state
    carried between them in fp32: the same bits as splitting the input at a
    segment boundary into two calls threaded through h0 / hT, dense and
    varlen (both sequences span a segment boundary; several sequences take
    the persistent scan, which walks them in one workgroup)."""
    print("chunk segments: dense T=9000", flush=True)
    c = configs.config2(seed=21, t=9000)
    q, k, v, g, beta = (c[x].to(DEV) for x in ("q", "k", "v", "g", "beta"))
    h0 = torch.randn(1, 32, 128, 128, generator=torch.Generator().manual_seed(22)).mul(0.1).to(DEV)
    kw = dict(output_final_state=True, use_qk_l2norm_in_kernel=True)
    o, s = chunk_gated_delta_rule(q, k, v, g, beta, initial_state=h0, **kw)
    cut = 64 * 64
    o1, s1 = chunk_gated_delta_rule(q[:, :cut], k[:, :cut], v[:, :cut], g[:, :cut], beta[:, :cut],
                                    initial_state=h0, **kw)
    o2, s2 = chunk_gated_delta_rule(q[:, cut:], k[:, cut:], v[:, cut:], g[:, cut:], beta[:, cut:],
                                    initial_state=s1, **kw)
    assert torch.equal(o[:, :cut], o1) and torch.equal(o[:, cut:], o2) and torch.equal(s, s2)

    print("chunk segments: varlen 5000 + 4000", flush=True)
    lens = [5000, 4000]
    cu = torch.tensor([0, lens[0], sum(lens)], dtype=torch.int32, device=DEV)
    c = configs.config2(seed=23, t=sum(lens))
    q, k, v, g, beta = (c[x].to(DEV) for x in ("q", "k", "v", "g", "beta"))
    h0 = torch.randn(2, 32, 128, 128, generator=torch.Generator().manual_seed(24)).mul(0.1).to(DEV)
    o, s = chunk_gated_delta_rule(q, k, v, g, beta, initial_state=h0, cu_seqlens=cu, **kw)
    for i, (a, b) in enumerate(((0, lens[0]), (lens[0], sum(lens)))):
        oi, si = chunk_gated_delta_rule(q[:, a:b], k[:, a:b], v[:, a:b], g[:, a:b], beta[:, a:b],
                                        initial_state=h0[i:i + 1], **kw)
        assert torch.equal(o[:, a:b], oi) and torch.equal(s[i:i + 1], si), i

    print("chunk segments: slot pool, varlen 4500 + 0 + 100 + 4000", flush=True)
    lens = [4500, 0, 100, 4000]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=DEV)
    c = configs.config2(seed=25, t=sum(lens))
    q, k, v, g, beta = (c[x].to(DEV) for x in ("q", "k", "v", "g", "beta"))
    pool0 = torch.randn(7, 32, 128, 128, generator=torch.Generator().manual_seed(26)).mul(0.1).to(DEV)
    slots = torch.tensor([5, 2, 0, 3], device=DEV)
    pool = pool0.clone()
    o, ret = chunk_gated_delta_rule(q, k, v, g, beta, initial_state=pool, ssm_state_indices=slots,
                                    inplace_final_state=True, cu_seqlens=cu, use_qk_l2norm_in_kernel=True)
    assert ret is pool
    starts = np.concatenate([[0], np.cumsum(lens)])
    for i, slot in enumerate(slots.tolist()):
        a, b = int(starts[i]), int(starts[i + 1])
        if a == b:
            assert torch.equal(pool[slot], pool0[slot]), i
            continue
        oi, si = chunk_gated_delta_rule(q[:, a:b], k[:, a:b], v[:, a:b], g[:, a:b], beta[:, a:b],
                                        initial_state=pool0[slot:slot + 1], **kw)
        assert torch.equal(o[:, a:b], oi) and torch.equal(pool[slot:slot + 1], si), i
    untouched = [r for r in range(pool.shape[0]) if r not in slots.tolist()]
    assert torch.equal(pool[untouched], pool0[untouched])


@pytest.mark.parametrize("dtype,t", [(torch.float32, 256), (torch.float16, 200)])
def test_chunk_entry_accepts_fp32_and_fp16_inputs(dtype, t):
    """The reference entry upcasts any float q/k/v (delta_rule.py:396-400):
    fp32 at configuration 0's shape and fp16 at a ragged length, with an
    initial state, against the oracle.  fp32 / fp16 inputs run the token
    recurrence in fp32 (bf16 MFMA operands would round them), so the
    tolerance is the fp32 one of configuration 0."""
    print(f"chunk entry dtype={dtype} T={t}", flush=True)
    c = configs.config0(seed=61, t=t)
    h0 = torch.randn(1, 32, 128, 128, generator=torch.Generator().manual_seed(62)) * 0.1
    q, k, v = (c[x].to(dtype) for x in ("q", "k", "v"))
    o, s = chunk_gated_delta_rule(q.to(DEV), k.to(DEV), v.to(DEV), c["g"].to(DEV), c["beta"].to(DEV),
                                  initial_state=h0.to(DEV), output_final_state=True, use_qk_l2norm_in_kernel=True)
    assert o.dtype == dtype and s.dtype == torch.float32
    o_ref, s_ref = gdn.chunk_gated_delta_rule(*(np64(x) for x in (q, k, v)), c["g"].numpy(), c["beta"].numpy(),
                                              initial_state=h0.numpy())
    err_o = np.abs(np64(o) - o_ref).max()
    err_s = gdn.state_rel_err(np64(s), s_ref)
    print(f"  max|o-o_ref|={err_o:.3e} state rel={err_s:.3e}")
    assert err_o < (1e-4 if dtype == torch.float32 else 2e-3)  # fp16 output rounding
    assert err_s < 1e-5


def test_chunk_size_other_than_64_gives_the_same_result():
    """The reference falls back to its torch path for chunk_size != 64
    (delta_rule.py:383-388); the chunk algorithm's result does not depend on
    the chunk size, so the kernels compute with 64: bit-identical results."""
    c = configs.config2(seed=63, t=300)
    args = [c[x].to(DEV) for x in ("q", "k", "v", "g", "beta")]
    o64, s64 = chunk_gated_delta_rule(*args, output_final_state=True, use_qk_l2norm_in_kernel=True)
    for cs in (32, 16, 128):
        o, s = chunk_gated_delta_rule(*args, chunk_size=cs, output_final_state=True, use_qk_l2norm_in_kernel=True)
        assert torch.equal(o, o64) and torch.equal(s, s64), cs
    o_ref, s_ref = oracle_chunk(c)
    assert np.abs(np64(o64) - o_ref).max() < O_TOL and gdn.state_rel_err(np64(s64), s_ref) < S_TOL


def test_has_initial_state_with_a_new_final_state():
    """has_initial_state with output_final_state (not in place) returns a new
    final-state tensor: rows marked False start from zero, the pool is left
    as it was."""
    c = configs.config2(seed=64, t=2 * 70)
    cu = torch.tensor([0, 70, 140], dtype=torch.int32)
    pool = torch.randn(4, 32, 128, 128, generator=torch.Generator().manual_seed(65)) * 0.1
    ids = torch.tensor([3, 1])
    has = torch.tensor([True, False])
    pool_d = pool.to(DEV)
    o, s = chunk_gated_delta_rule(*(c[x].to(DEV) for x in ("q", "k", "v", "g", "beta")), initial_state=pool_d,
                                  ssm_state_indices=ids.to(DEV), has_initial_state=has.to(DEV),
                                  output_final_state=True, use_qk_l2norm_in_kernel=True, cu_seqlens=cu.to(DEV))
    assert s is not None and s.shape == (2, 32, 128, 128)
    assert torch.equal(pool_d.cpu(), pool)
    h0 = np.stack([pool[3].numpy(), np.zeros((32, 128, 128), np.float32)])
    o_ref, s_ref = gdn.chunk_gated_delta_rule_varlen(*(c[x].float().numpy() for x in ("q", "k", "v", "g", "beta")),
                                                     cu.numpy(), h0)
    assert np.abs(np64(o) - o_ref).max() < O_TOL and gdn.state_rel_err(np64(s), s_ref) < S_TOL


def test_repeated_slot_ids_advance_a_slot_once():
    """ids [s, s, t] with identical rows 0 and 1 (a bucket padded by
    repeating row 0, cuda_graphs.py:478-482): slot s advances exactly once,
    to the oracle's state for row 0, row 1 runs as a padding row (zero
    state, nothing written), slot t as usual; the same for the prefill
    (chunk) and decode (recurrent) kernels."""
    c = configs.config2(seed=66, t=3 * 50)
    x = {k: c[k].view(1, 3, 50, *c[k].shape[2:])[0] for k in ("q", "k", "v", "g", "beta")}
    x = {k: torch.stack([v[0], v[0], v[2]]) for k, v in x.items()}  # rows 0 and 1 identical
    pool = torch.randn(5, 32, 128, 128, generator=torch.Generator().manual_seed(67)) * 0.1
    ids = torch.tensor([2, 2, 4])
    s_ref_rows = []
    for r, row in ((0, 2), (2, 4)):
        _, sr = gdn.chunk_gated_delta_rule(*(x[k][r:r + 1].float().numpy() for k in ("q", "k", "v", "g", "beta")),
                                           initial_state=pool[row:row + 1].numpy())
        s_ref_rows.append(sr[0])
    o0_pad, _ = gdn.chunk_gated_delta_rule(*(x[k][1:2].float().numpy() for k in ("q", "k", "v", "g", "beta")))
    for fn in ("chunk", "recurrent"):
        pd = pool.to(DEV)
        args = [x[k].to(DEV) for k in ("q", "k", "v", "g", "beta")]
        if fn == "chunk":
            o, _ = chunk_gated_delta_rule(*args, initial_state=pd, ssm_state_indices=ids.to(DEV),
                                          inplace_final_state=True, use_qk_l2norm_in_kernel=True)
        else:
            o, _ = fused_recurrent_gated_delta_rule(*args, initial_state=pd, ssm_state_indices=ids.to(DEV),
                                                    inplace_final_state=True, use_qk_l2norm_in_kernel=True)
        assert gdn.state_rel_err(np64(pd[2])[None], s_ref_rows[0][None]) < S_TOL, fn
        assert gdn.state_rel_err(np64(pd[4])[None], s_ref_rows[1][None]) < S_TOL, fn
        assert torch.equal(pd[[0, 1, 3]].cpu(), pool[[0, 1, 3]]), fn
        assert np.abs(np64(o[1]) - o0_pad[0]).max() < O_TOL, fn  # the repeated row: zero initial state


@pytest.mark.parametrize("has_first", [False, True])
def test_repeated_slot_id_with_mismatched_has_initial_state(has_first):
    """ids [5, 5] with has_initial_state [has_first, not has_first], in place,
    varlen: the repeat is decided on the slot ids themselves, so row 0 alone
    reads (when its flag is set) and writes slot 5, and row 1 runs from a zero
    state and writes nothing -- the read of one row never races the write of
    the other."""
    c = configs.config2(seed=68, t=2 * 90)
    cu = torch.tensor([0, 90, 180], dtype=torch.int32)
    pool = torch.randn(6, 32, 128, 128, generator=torch.Generator().manual_seed(69)) * 0.1
    ids = torch.tensor([5, 5])
    has = torch.tensor([has_first, not has_first])
    pd = pool.to(DEV)
    o, _ = chunk_gated_delta_rule(*(c[x].to(DEV) for x in ("q", "k", "v", "g", "beta")), initial_state=pd,
                                  ssm_state_indices=ids.to(DEV), has_initial_state=has.to(DEV),
                                  inplace_final_state=True, use_qk_l2norm_in_kernel=True, cu_seqlens=cu.to(DEV))
    zero = np.zeros((32, 128, 128), np.float32)
    h0 = np.stack([pool[5].numpy() if has_first else zero, zero])
    o_ref, s_ref = gdn.chunk_gated_delta_rule_varlen(*(c[x].float().numpy() for x in ("q", "k", "v", "g", "beta")),
                                                     cu.numpy(), h0)
    assert np.abs(np64(o) - o_ref).max() < O_TOL
    assert gdn.state_rel_err(np64(pd[5])[None], s_ref[0:1]) < S_TOL
    assert torch.equal(pd[:5].cpu(), pool[:5])


@pytest.mark.parametrize("b,t,seed", [(8, 130, 5), (16, 64, 6), (5, 200, 7)])
def test_per_pair_kernel_batches_match_the_oracle(b, t, seed):
    """A batch of 160 or more (sequence, v-head) pairs runs one workgroup per
    pair (chunk_local_kernel, no workspace): B = 8 x T = 130 (a partial last
    chunk), B = 16 x T = 64 (one chunk each) and B = 5 x T = 200 (160 pairs,
    fewer workgroups than CUs), zero h0, final states out, against the oracle
    sequence by sequence."""
    from engine.kernels import _lib
    assert _lib.load().gdn_chunk_workspace_bytes(b, b * t, 32, 128, 128) == 0  # the per-pair kernel's batch
    c = configs.config2(t=b * t, seed=seed)
    x = {k: c[k].reshape(b, t, *c[k].shape[2:]) for k in ("q", "k", "v", "g", "beta")}
    print(f"per-pair kernel B={b} T={t}", flush=True)
    o, s = chunk_gated_delta_rule(*(x[k].to(DEV) for k in ("q", "k", "v", "g", "beta")), output_final_state=True,
                                  use_qk_l2norm_in_kernel=True)
    for i in range(b):
        o_ref, s_ref = gdn.chunk_gated_delta_rule(*(x[k][i:i + 1].float().numpy() for k in ("q", "k", "v", "g", "beta")))
        assert np.abs(np64(o[i:i + 1]) - o_ref).max() < O_TOL, i
        assert gdn.state_rel_err(np64(s[i:i + 1]), s_ref) < S_TOL, i


def test_per_pair_kernel_varlen_on_a_slot_pool():
    """8 packed sequences (256 pairs: the per-pair kernel) of 4,500 (71 chunks,
    past the two-kernel path's 64-chunk segment), 0, 1, 130, 64, 700, 65 and 17
    tokens on a 12-slot pool, in place, with slot ids [7, 2, 9, 2, -1, 0, 11, 5]
    (row 3 repeats row 1's slot, row 4 has none) and has_initial_state False
    for row 5: rows 3 and 4 start from zero and write nothing, row 5 starts
    from zero and writes slot 0, the empty row 1 passes slot 2 through."""
    lens = [4500, 0, 1, 130, 64, 700, 65, 17]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    c = configs.config2(seed=77, t=int(cu[-1]))
    pool0 = torch.randn(12, 32, 128, 128, generator=torch.Generator().manual_seed(78)) * 0.1
    ids = torch.tensor([7, 2, 9, 2, -1, 0, 11, 5])
    has = torch.tensor([True, True, True, True, True, False, True, True])
    h0 = torch.zeros(len(lens), 32, 128, 128)
    for r in (0, 1, 2, 6, 7):
        h0[r] = pool0[ids[r]]
    print("per-pair kernel varlen on a pool", flush=True)
    pool = pool0.to(DEV)
    o, _ = chunk_gated_delta_rule(*(c[x].to(DEV) for x in ("q", "k", "v", "g", "beta")), initial_state=pool,
                                  ssm_state_indices=ids.to(DEV), has_initial_state=has.to(DEV),
                                  inplace_final_state=True, use_qk_l2norm_in_kernel=True, cu_seqlens=cu.to(DEV))
    o_ref, s_ref = gdn.chunk_gated_delta_rule_varlen(*(c[x].float().numpy() for x in ("q", "k", "v", "g", "beta")),
                                                     cu.numpy(), h0.numpy())
    assert np.abs(np64(o) - o_ref).max() < O_TOL
    for r in (0, 1, 2, 5, 6, 7):  # the rows that own their slot
        assert gdn.state_rel_err(np64(pool[int(ids[r])])[None], s_ref[r:r + 1]) < S_TOL, r
    assert torch.equal(pool[2].cpu(), pool0[2])  # the empty row passed its state through
    untouched = [i for i in range(12) if i not in (7, 2, 9, 0, 11, 5)]
    assert torch.equal(pool[untouched].cpu(), pool0[untouched])


@pytest.mark.parametrize("n_seqs", [300, 520])
def test_per_pair_kernel_many_varlen_sequences(n_seqs):
    """Many packed sequences of 0..90 tokens (some empty) on the per-pair
    kernel, final states out: with 300 the workgroups take the sequences
    longest first (the workgroup for slot n ranks the lengths and takes the
    n-th longest), with 520 (more than one per thread of the ranking) in
    sequence order.  Every 9th sequence, the longest and the first empty ones
    against the oracle (each sequence is independent)."""
    from engine.kernels import _lib
    rng = np.random.default_rng(n_seqs)
    lens = rng.integers(0, 91, n_seqs)
    lens[::37] = 0
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    total = int(cu[-1])
    assert _lib.load().gdn_chunk_workspace_bytes(n_seqs, total, 32, 128, 128) == 0  # the per-pair kernel
    c = configs.config2(seed=n_seqs, t=total)
    print(f"per-pair kernel, {n_seqs} varlen sequences", flush=True)
    o, s = chunk_gated_delta_rule(*(c[x].to(DEV) for x in ("q", "k", "v", "g", "beta")), output_final_state=True,
                                  use_qk_l2norm_in_kernel=True, cu_seqlens=torch.from_numpy(cu).to(DEV))
    empty = np.nonzero(lens == 0)[0]
    check = sorted(set(range(0, n_seqs, 9)) | {int(np.argmax(lens))} | {int(i) for i in empty[:3]})
    for i in check:
        a, b = int(cu[i]), int(cu[i + 1])
        if a == b:
            assert torch.count_nonzero(s[i]).item() == 0, i  # zero initial state, no tokens
            continue
        o_ref, s_ref = gdn.chunk_gated_delta_rule(*(c[x][:, a:b].float().numpy() for x in ("q", "k", "v", "g", "beta")))
        assert np.abs(np64(o[:, a:b]) - o_ref).max() < O_TOL, i
        assert gdn.state_rel_err(np64(s[i:i + 1]), s_ref) < S_TOL, i


@pytest.mark.parametrize("b,t", [(1, 200), (2, 150), (8, 130)])
def test_fp32_output_through_the_c_abi(b, t):
    """o in fp32 from bf16 q/k/v (the C ABI's o_dtype; the Python entry
    returns o in q's dtype): the prep + scan path (B = 1), the persistent scan
    (B = 2) and the per-pair kernel (B = 8 x 32 v-heads), against the oracle,
    and rounded to bf16 equal to the bf16-output call."""
    from engine.kernels import _lib
    lib = _lib.load()
    c = configs.config2(t=b * t, seed=90 + b)
    x = {k: c[k].reshape(b, t, *c[k].shape[2:]).to(DEV) for k in ("q", "k", "v", "g", "beta")}
    hk, hv = x["q"].shape[2], x["v"].shape[2]
    g32, beta32 = x["g"].float().contiguous(), x["beta"].float().contiguous()
    ws_bytes = int(lib.gdn_chunk_workspace_bytes(b, b * t, hv, 128, 128))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
    outs = {}
    for odt in (torch.float32, torch.bfloat16):
        o = torch.empty(b, t, hv, 128, dtype=odt, device=DEV)
        hT = torch.empty(b, hv, 128, 128, dtype=torch.float32, device=DEV)
        st = lib.gdn_chunk_fwd(
            _lib.ptr(x["q"]), _lib.ptr(x["k"]), _lib.ptr(x["v"]), _lib.dtype_code(x["q"], "q"),
            hk * 128, hk * 128, hv * 128, _lib.ptr(g32), _lib.ptr(beta32), _lib.dtype_code(beta32, "beta"),
            None, None, 0, _lib.ptr(hT), None, b, _lib.ptr(o), _lib.dtype_code(o, "o"),
            None, b, t, hk, hv, 128, 128, 128 ** -0.5, 1, _lib.ptr(ws), ws_bytes, _lib.stream_of(x["q"]))
        _lib.check(st, "gdn_chunk_fwd")
        outs[odt] = (o, hT)
    o32, s32 = outs[torch.float32]
    assert torch.equal(o32.to(torch.bfloat16), outs[torch.bfloat16][0])
    assert torch.equal(s32, outs[torch.bfloat16][1])
    for i in range(b):
        o_ref, s_ref = gdn.chunk_gated_delta_rule(*(c[k].reshape(b, t, *c[k].shape[2:])[i:i + 1].float().numpy()
                                                    for k in ("q", "k", "v", "g", "beta")))
        assert np.abs(np64(o32[i:i + 1]) - o_ref).max() < O_TOL, i
        assert gdn.state_rel_err(np64(s32[i:i + 1]), s_ref) < S_TOL, i


def test_per_pair_kernel_repeated_qk_equals_native():
    """The per-pair kernel with q/k repeated to the 32 v-heads (HF's layout:
    one k-head per v-head) gives the bits of native GQA (16 k-heads), B = 8 x
    T = 130, with an initial state and final states out."""
    b, t = 8, 130
    c = configs.config2(t=b * t, seed=97)
    x = {k: c[k].reshape(b, t, *c[k].shape[2:]).to(DEV) for k in ("q", "k", "v", "g", "beta")}
    h0 = torch.randn(b, 32, 128, 128, generator=torch.Generator().manual_seed(98)).to(DEV) * 0.1
    o1, s1 = chunk_gated_delta_rule(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=h0,
                                    output_final_state=True, use_qk_l2norm_in_kernel=True)
    o2, s2 = chunk_gated_delta_rule(x["q"].repeat_interleave(2, 2), x["k"].repeat_interleave(2, 2), x["v"], x["g"],
                                    x["beta"], initial_state=h0, output_final_state=True, use_qk_l2norm_in_kernel=True)
    assert torch.equal(o1, o2) and torch.equal(s1, s2)


@pytest.mark.parametrize("hk,hv", [(8, 32), (4, 32), (16, 48), (8, 16)])
@pytest.mark.parametrize("b,t", [(1, 200), (8, 130)])
def test_gqa_ratios_other_than_two(hk, hv, b, t):
    """v-heads over k-heads at ratios 4, 8 and 3 and at 16 v-heads, on the
    prep + scan path (B = 1), at B = 8 on the per-pair kernel (256 or 384
    pairs) or the persistent scan (128 pairs), and the decode recurrence,
    against the oracle (which repeats the k-heads)."""
    from engine.kernels import fused_recurrent_gated_delta_rule
    gen = torch.Generator().manual_seed(60 + hk + hv + b)
    q = torch.randn(b, t, hk, 128, generator=gen).to(torch.bfloat16)
    k = torch.randn(b, t, hk, 128, generator=gen).to(torch.bfloat16)
    v = torch.randn(b, t, hv, 128, generator=gen).to(torch.bfloat16)
    g = -torch.nn.functional.softplus(torch.randn(b, t, hv, generator=gen)) * 0.3
    beta = torch.sigmoid(torch.randn(b, t, hv, generator=gen))
    h0 = torch.randn(b, hv, 128, 128, generator=gen) * 0.1
    o, s = chunk_gated_delta_rule(q.to(DEV), k.to(DEV), v.to(DEV), g.to(DEV), beta.to(DEV), initial_state=h0.to(DEV),
                                  output_final_state=True, use_qk_l2norm_in_kernel=True)
    od, sd = fused_recurrent_gated_delta_rule(q[:, :1].to(DEV), k[:, :1].to(DEV), v[:, :1].to(DEV), g[:, :1].to(DEV),
                                              beta[:, :1].to(DEV), initial_state=h0.to(DEV), output_final_state=True,
                                              use_qk_l2norm_in_kernel=True)
    for i in range(b):
        args = [np64(x[i:i + 1]) for x in (q, k, v, g, beta)]
        o_ref, s_ref = gdn.chunk_gated_delta_rule(*args, initial_state=np64(h0[i:i + 1]))
        assert np.abs(np64(o[i:i + 1]) - o_ref).max() < O_TOL, i
        assert gdn.state_rel_err(np64(s[i:i + 1]), s_ref) < S_TOL, i
        od_ref, sd_ref = gdn.recurrent_gated_delta_rule(*(x[:, :1] for x in args), initial_state=np64(h0[i:i + 1]))
        assert np.abs(np64(od[i:i + 1]) - od_ref).max() < O_TOL, i
        assert gdn.state_rel_err(np64(sd[i:i + 1]), sd_ref) < S_TOL, i


@pytest.mark.parametrize("lens", [[0, 17, 30, 0, 12], [40, 50, 0, 30]])
def test_short_packed_batches_on_the_per_pair_kernel(lens):
    """Packed batches whose total tokens fit one chunk (any pair count) or
    two chunks at 96 pairs or more run the per-pair kernel, empty sequences
    included (an empty one keeps its initial state), against the oracle."""
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    c = configs.config2(seed=57, t=int(cu[-1]))
    h0 = torch.randn(len(lens), 32, 128, 128, generator=torch.Generator().manual_seed(2)) * 0.1
    o_ref, s_ref = gdn.chunk_gated_delta_rule_varlen(*(c[x].float().numpy() for x in ("q", "k", "v", "g", "beta")),
                                                     cu.numpy(), h0.numpy())
    o, s = chunk_gated_delta_rule(*(c[x].to(DEV) for x in ("q", "k", "v", "g", "beta")), initial_state=h0.to(DEV),
                                  output_final_state=True, use_qk_l2norm_in_kernel=True, cu_seqlens=cu.to(DEV))
    assert np.abs(np64(o) - o_ref).max() < O_TOL
    assert gdn.state_rel_err(np64(s), s_ref) < S_TOL
    for i, n in enumerate(lens):
        if n == 0:
            assert torch.equal(s[i].cpu(), h0[i]), i
