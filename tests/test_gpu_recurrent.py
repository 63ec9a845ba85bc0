"""GPU parity of the token recurrence (decode / spec-verify / small T) with the
CPU oracle on identical seeded inputs, through the C ABI.

Tolerances (north star): bf16 outputs max abs error <= 2e-2; fp32 final
states relative error <= 1e-3, norm-wise per (sequence, head).  The
recurrence is pure fp32 on the GPU, so fp32-output cases use tighter bounds.
"""
import numpy as np
import pytest
import torch

from conftest import golden_case
from engine import configs
from engine.kernels import fused_recurrent_gated_delta_rule, gdn_state_commit
from oracle import gdn

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

DEV = "cuda"
O_TOL_BF16 = 2e-2
S_TOL = 1e-3


def np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def cuda(*ts):
    return [t.to(DEV) for t in ts]


@pytest.mark.parametrize("name", ["rec_d128", "chunk_d128"])
def test_recurrent_matches_hf_golden(golden, name):
    a = {k: torch.from_numpy(v) for k, v in golden_case(golden, name).items()}
    q, k, v, g, beta, h0 = cuda(a["q"], a["k"], a["v"], a["g"], a["beta"], a["h0"])
    o, s = fused_recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=h0, output_final_state=True,
                                            use_qk_l2norm_in_kernel=True)
    assert np.abs(np64(o) - a["o"].numpy()).max() < 1e-4
    assert gdn.state_rel_err(np64(s), a["state"].numpy()) < 1e-5


def test_config0_fp32_t256():
    c = configs.config0()
    o_ref, s_ref = gdn.recurrent_gated_delta_rule(*(c[x].numpy() for x in ("q", "k", "v", "g", "beta")))
    q, k, v, g, beta = cuda(*(c[x] for x in ("q", "k", "v", "g", "beta")))
    o, s = fused_recurrent_gated_delta_rule(q, k, v, g, beta, output_final_state=True,
                                            use_qk_l2norm_in_kernel=True)
    assert o.dtype == torch.float32 and o.shape == (1, 256, 32, 128)
    assert np.abs(np64(o) - o_ref).max() < 1e-4
    assert gdn.state_rel_err(np64(s), s_ref) < 1e-5
    # HF passes q/k already repeated to 32 heads: same result
    o2, s2 = fused_recurrent_gated_delta_rule(q.repeat_interleave(2, 2), k.repeat_interleave(2, 2), v, g, beta,
                                              output_final_state=True, use_qk_l2norm_in_kernel=True)
    assert torch.allclose(o2, o, atol=1e-6) and torch.allclose(s2, s, atol=1e-6)


def test_config1_decode_slot_pool_in_place():
    c = configs.config1()
    pool0 = c["pool"]
    slots = c["slots"]
    h0 = pool0[slots].numpy()
    o_ref, s_ref = gdn.recurrent_gated_delta_rule(*(c[x].float().numpy() for x in ("q", "k", "v", "g", "beta")),
                                                  initial_state=h0)
    q, k, v, g, beta = cuda(*(c[x] for x in ("q", "k", "v", "g", "beta")))
    pool = pool0.to(DEV)
    o, ret = fused_recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=pool,
                                              ssm_state_indices=slots.to(DEV), inplace_final_state=True,
                                              use_qk_l2norm_in_kernel=True)
    assert ret is pool and o.dtype == torch.bfloat16
    assert np.abs(np64(o) - o_ref).max() < O_TOL_BF16
    assert gdn.state_rel_err(np64(pool[slots.to(DEV)]), s_ref) < S_TOL
    untouched = torch.ones(pool0.shape[0], dtype=torch.bool)
    untouched[slots] = False
    assert torch.equal(pool[untouched.to(DEV)].cpu(), pool0[untouched])


def test_negative_slot_means_fresh_state_and_no_write():
    c = configs.config1(batch=4, num_slots=8)
    slots = torch.tensor([5, -1, 0, -1])
    h0 = np.zeros((4, 32, 128, 128))
    h0[0], h0[2] = c["pool"][5].numpy(), c["pool"][0].numpy()
    o_ref, s_ref = gdn.recurrent_gated_delta_rule(*(c[x].float().numpy() for x in ("q", "k", "v", "g", "beta")),
                                                  initial_state=h0)
    q, k, v, g, beta = cuda(*(c[x] for x in ("q", "k", "v", "g", "beta")))
    pool = c["pool"].to(DEV)
    o, _ = fused_recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=pool, ssm_state_indices=slots.to(DEV),
                                            inplace_final_state=True, use_qk_l2norm_in_kernel=True)
    assert np.abs(np64(o) - o_ref).max() < O_TOL_BF16
    assert gdn.state_rel_err(np64(pool[[5, 0]]), s_ref[[0, 2]]) < S_TOL
    keep = [1, 2, 3, 4, 6, 7]
    assert torch.equal(pool[keep].cpu(), c["pool"][keep])


def test_out_of_range_slot_is_no_slot_in_every_pool_kernel():
    # An id past the pool (or negative) selects no row: zero state in, nothing
    # written -- in the recurrence, the conv update, the chunk kernel and the
    # commits -- so a bad id can never address memory outside a pool.
    from engine.kernels import causal_conv1d_update, chunk_gated_delta_rule, gdn_conv_state_commit, gdn_state_commit
    c = configs.config1(batch=4, num_slots=8)
    q, k, v, g, beta = cuda(*(c[x] for x in ("q", "k", "v", "g", "beta")))
    bad = torch.tensor([5, 8, 0, 1 << 40], device=DEV)   # rows 1 and 3 outside the 8-slot pool
    ref = torch.tensor([5, -1, 0, -1], device=DEV)
    gen = torch.Generator().manual_seed(5)
    cpool0 = torch.randn(8, 64, 4, generator=gen).to(DEV, torch.bfloat16)
    x = torch.randn(4, 64, 1, generator=gen).to(DEV, torch.bfloat16)
    w = torch.randn(64, 4, generator=gen).to(DEV, torch.bfloat16)
    outs = []
    for ids in (bad, ref):
        pool = c["pool"].to(DEV)
        o, _ = fused_recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=pool, ssm_state_indices=ids,
                                                inplace_final_state=True, use_qk_l2norm_in_kernel=True)
        cpool = cpool0.clone()
        y = causal_conv1d_update(x, cpool, w, None, "silu", conv_state_indices=ids)
        outs.append((o, pool, y, cpool))
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b)
    assert torch.equal(outs[0][3][[1, 2, 3, 4, 6, 7]], cpool0[[1, 2, 3, 4, 6, 7]])
    t = 70  # the chunk kernel, initial and final states by id
    qc, kc = (torch.randn(4, t, 16, 128, device=DEV).to(torch.bfloat16) for _ in range(2))
    vc = torch.randn(4, t, 32, 128, device=DEV).to(torch.bfloat16)
    gc, bc = -0.1 * torch.rand(4, t, 32, device=DEV), torch.rand(4, t, 32, device=DEV)
    snaps = torch.randn(4, 2, 32, 128, 128, device=DEV)
    hist = torch.randn(4, 64, 6, generator=torch.Generator().manual_seed(6)).to(DEV, torch.bfloat16)
    res = []
    for ids in (bad, ref):
        pool = c["pool"].to(DEV)
        o, _ = chunk_gated_delta_rule(qc, kc, vc, gc, bc, initial_state=pool, ssm_state_indices=ids,
                                      inplace_final_state=True, use_qk_l2norm_in_kernel=True)
        gdn_state_commit(pool, ids, snaps, torch.tensor([1, 2, 2, 1]))
        cp = torch.zeros(8, 64, 4, device=DEV, dtype=torch.bfloat16)
        gdn_conv_state_commit(cp, ids, hist, torch.tensor([1, 2, 2, 1]))
        res.append((o, pool, cp))
    for a, b in zip(res[0], res[1]):
        assert torch.equal(a, b)


def test_fla_mode_returns_new_state_and_keeps_input():
    c = configs.config4(batch=3, t=3, num_slots=3)
    h0 = c["pool"].to(DEV)
    h0_copy = h0.clone()
    q, k, v, g, beta = cuda(*(c[x] for x in ("q", "k", "v", "g", "beta")))
    o, s = fused_recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=h0, output_final_state=True,
                                            use_qk_l2norm_in_kernel=True)
    assert torch.equal(h0, h0_copy) and s.data_ptr() != h0.data_ptr()
    o_ref, s_ref = gdn.recurrent_gated_delta_rule(*(c[x].float().numpy() for x in ("q", "k", "v", "g", "beta")),
                                                  initial_state=c["pool"].numpy())
    assert np.abs(np64(o) - o_ref).max() < O_TOL_BF16
    assert gdn.state_rel_err(np64(s), s_ref) < S_TOL
    _, none = fused_recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=h0)
    assert none is None


def test_varlen_cu_seqlens():
    lens = [1, 7, 0, 3]
    cu = torch.tensor([0, 1, 8, 8, 11], dtype=torch.int32)
    c = configs.config0(seed=21, t=11)
    h0 = torch.randn(4, 32, 128, 128, generator=torch.Generator().manual_seed(5)) * 0.1
    o_ref, s_ref = gdn.recurrent_gated_delta_rule_varlen(*(c[x].numpy() for x in ("q", "k", "v", "g", "beta")),
                                                         cu.numpy(), h0.numpy())
    q, k, v, g, beta = cuda(*(c[x] for x in ("q", "k", "v", "g", "beta")))
    o, s = fused_recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=h0.to(DEV), output_final_state=True,
                                            cu_seqlens=cu.to(DEV), use_qk_l2norm_in_kernel=True)
    assert np.abs(np64(o) - o_ref).max() < 1e-4
    assert gdn.state_rel_err(np64(s), s_ref) < 1e-5
    assert sum(lens) == 11


def test_config4_spec_verify_snapshots_and_commit():
    c = configs.config4()
    pool0 = c["pool"]
    slots, acc = c["slots"], c["accepted"]
    o_ref, snap_ref, pool_ref = gdn.spec_verify(pool0.numpy(), slots.numpy(),
                                                *(c[x].float().numpy() for x in ("q", "k", "v", "g", "beta")),
                                                acc.numpy())
    q, k, v, g, beta = cuda(*(c[x] for x in ("q", "k", "v", "g", "beta")))
    pool = pool0.to(DEV)
    snaps = torch.empty(32, 4, 32, 128, 128, device=DEV)
    o, none = fused_recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=pool,
                                               ssm_state_indices=slots.to(DEV), snapshots=snaps,
                                               use_qk_l2norm_in_kernel=True)
    assert none is None
    assert torch.equal(pool.cpu(), pool0)          # verify does not touch the pool
    assert np.abs(np64(o) - o_ref).max() < O_TOL_BF16
    for t in range(4):
        assert gdn.state_rel_err(np64(snaps[:, t]), snap_ref[:, t]) < S_TOL
    gdn_state_commit(pool, slots.to(DEV), snaps, acc.to(DEV))
    assert gdn.state_rel_err(np64(pool), pool_ref) < S_TOL
    untouched = torch.ones(pool0.shape[0], dtype=torch.bool)
    untouched[slots] = False
    assert torch.equal(pool[untouched.to(DEV)].cpu(), pool0[untouched])
    # commit picks exactly the snapshot (bit copy)
    b = 3
    assert torch.equal(pool[slots[b]], snaps[b, acc[b] - 1])


def test_strided_views_of_packed_projection():
    """q/k/v passed as views of one [tokens, 8192] projection (token stride 8192)."""
    gen = torch.Generator().manual_seed(9)
    n = 6
    y = torch.randn(n, configs.CONV_DIM, generator=gen).to(torch.bfloat16)
    g = -torch.rand(1, n, 32, generator=gen)
    beta = torch.rand(1, n, 32, generator=gen)
    qv, kv, vv = configs.split_qkv(y.to(DEV))
    o, s = fused_recurrent_gated_delta_rule(qv, kv, vv, g.to(DEV), beta.to(DEV), output_final_state=True,
                                            use_qk_l2norm_in_kernel=True)
    qc, kc, vc = (x.contiguous() for x in (qv, kv, vv))
    o2, s2 = fused_recurrent_gated_delta_rule(qc, kc, vc, g.to(DEV), beta.to(DEV), output_final_state=True,
                                              use_qk_l2norm_in_kernel=True)
    assert torch.equal(o, o2) and torch.equal(s, s2)
    q_np, k_np, v_np = (np64(x) for x in (qv, kv, vv))
    o_ref, s_ref = gdn.recurrent_gated_delta_rule(q_np, k_np, v_np, g.numpy(), beta.numpy())
    assert np.abs(np64(o) - o_ref).max() < O_TOL_BF16
    assert gdn.state_rel_err(np64(s), s_ref) < S_TOL


def test_bf16_beta_and_no_l2norm():
    c = configs.config4(batch=2, t=2, num_slots=2)
    q, k, v, g = cuda(*(c[x] for x in ("q", "k", "v", "g")))
    beta = c["beta"].to(torch.bfloat16)
    o, s = fused_recurrent_gated_delta_rule(q, k, v, g, beta.to(DEV), initial_state=c["pool"].to(DEV),
                                            output_final_state=True, use_qk_l2norm_in_kernel=False, scale=0.3)
    o_ref, s_ref = gdn.recurrent_gated_delta_rule(*(c[x].float().numpy() for x in ("q", "k", "v", "g")),
                                                  beta.float().numpy(), c["pool"].numpy(),
                                                  use_qk_l2norm_in_kernel=False, scale=0.3)
    assert np.abs(np64(o) - o_ref).max() < O_TOL_BF16
    assert gdn.state_rel_err(np64(s), s_ref) < S_TOL


@pytest.mark.parametrize("dtype,gated", [(torch.bfloat16, False), (torch.float32, False), (torch.bfloat16, True)])
def test_decode_b37_on_a_slot_pool_with_bad_and_repeated_ids(dtype, gated):
    """Single-token decode at B = 37 (4,736 column slices, not a whole number
    of rounds of the grid) on a 48-slot pool whose ids hold a negative, an
    out-of-range and a repeated id (each selects no row: zero state in,
    nothing written).  q / k / v in bf16 or fp32; gates given as g / beta or as
    the raw a / b projections (A_log, dt_bias)."""
    from engine.kernels import fused_recurrent_gated_delta_rule_from_projections
    gen = torch.Generator().manual_seed(61)
    bsz, n_slots = 37, 48
    q = torch.randn(bsz, 1, 16, 128, generator=gen).to(dtype)
    k = torch.randn(bsz, 1, 16, 128, generator=gen).to(dtype)
    v = torch.randn(bsz, 1, 32, 128, generator=gen).to(dtype)
    pool = torch.randn(n_slots, 32, 128, 128, generator=gen) * 0.1
    ids = torch.randperm(n_slots, generator=gen)[:bsz]
    ids[5], ids[9], ids[20] = -1, n_slots, ids[3]
    live = [i for i in range(bsz) if 0 <= int(ids[i]) < n_slots and int(ids[i]) not in ids[:i].tolist()]
    h0 = np.zeros((bsz, 32, 128, 128))
    h0[live] = pool[ids[live]].numpy()
    pool_gpu = pool.to(DEV)
    if gated:
        a = torch.randn(bsz, 1, 32, generator=gen).to(torch.bfloat16)
        b = torch.randn(bsz, 1, 32, generator=gen).to(torch.bfloat16)
        A_log = torch.log(torch.empty(32).uniform_(0.5, 16.0, generator=gen))
        dt_bias = torch.randn(32, generator=gen)
        o, _ = fused_recurrent_gated_delta_rule_from_projections(
            *cuda(q, k, v, a, b, A_log, dt_bias), initial_state=pool_gpu, ssm_state_indices=ids.to(DEV),
            inplace_final_state=True)
        g, beta = gdn.gdn_gates(np64(a), np64(b), np64(A_log), np64(dt_bias))
    else:
        g = -torch.rand(bsz, 1, 32, generator=gen) * 2
        beta = torch.rand(bsz, 1, 32, generator=gen)
        o, _ = fused_recurrent_gated_delta_rule(*cuda(q, k, v, g, beta), initial_state=pool_gpu,
                                                ssm_state_indices=ids.to(DEV), inplace_final_state=True,
                                                use_qk_l2norm_in_kernel=True)
        g, beta = np64(g), np64(beta)
    o_ref, s_ref = gdn.recurrent_gated_delta_rule(np64(q), np64(k), np64(v), g, beta, initial_state=h0)
    tol = O_TOL_BF16 if o.dtype == torch.bfloat16 else 1e-4
    assert np.abs(np64(o) - o_ref).max() < tol
    assert gdn.state_rel_err(np64(pool_gpu[ids[live].to(DEV)]), s_ref[live]) < (S_TOL if dtype != torch.float32 else 1e-5)
    untouched = np.setdiff1d(np.arange(n_slots), ids[live].numpy())
    assert torch.equal(pool_gpu[untouched].cpu(), pool[untouched])


@pytest.mark.parametrize("t", [1, 3])
def test_repeated_ids_beyond_the_first_64_rows(t):
    """B = 100 rows on a 128-slot pool.  The repeated-slot test compares a
    row's id with the first 64 rows' ids held one per lane and reads the
    ids of rows 64 .. n-1 in a loop: row 70 repeats row 10 (found among the
    lanes), row 90 repeats row 80 and row 99 repeats row 66 (found in the
    loop).  Each repeat selects no row (zero state in, nothing written), so
    the pool's repeated slots hold the first row's result."""
    gen = torch.Generator().manual_seed(71)
    bsz, n_slots = 100, 128
    q = torch.randn(bsz, t, 16, 128, generator=gen).to(torch.bfloat16)
    k = torch.randn(bsz, t, 16, 128, generator=gen).to(torch.bfloat16)
    v = torch.randn(bsz, t, 32, 128, generator=gen).to(torch.bfloat16)
    g = -torch.rand(bsz, t, 32, generator=gen) * 2
    beta = torch.rand(bsz, t, 32, generator=gen)
    pool = torch.randn(n_slots, 32, 128, 128, generator=gen) * 0.1
    ids = torch.randperm(n_slots, generator=gen)[:bsz]
    ids[70], ids[90], ids[99] = ids[10], ids[80], ids[66]
    live = [i for i in range(bsz) if int(ids[i]) not in ids[:i].tolist()]
    assert len(live) == bsz - 3
    h0 = np.zeros((bsz, 32, 128, 128))
    h0[live] = pool[ids[live]].numpy()
    pool_gpu = pool.to(DEV)
    o, _ = fused_recurrent_gated_delta_rule(*cuda(q, k, v, g, beta), initial_state=pool_gpu,
                                            ssm_state_indices=ids.to(DEV), inplace_final_state=True,
                                            use_qk_l2norm_in_kernel=True)
    o_ref, s_ref = gdn.recurrent_gated_delta_rule(np64(q), np64(k), np64(v), np64(g), np64(beta), initial_state=h0)
    assert np.abs(np64(o) - o_ref).max() < O_TOL_BF16
    assert gdn.state_rel_err(np64(pool_gpu[ids[live].to(DEV)]), s_ref[live]) < S_TOL
    untouched = np.setdiff1d(np.arange(n_slots), ids[live].numpy())
    assert torch.equal(pool_gpu[untouched].cpu(), pool[untouched])
