"""Seeded random sweep of the token recurrence entry (decode, multi-token
steps, spec-verify snapshots) against the CPU oracle.

Each case draws its own call: B of 1-100 rows, T of 1-4 tokens per row, Hv
of 16 or 32 with Hk = Hv, Hv / 2 or Hv / 4, q/k/v in bf16, fp16 or fp32,
beta in fp32 or bf16, and one of three modes: per-row initial states with
the final states returned; a slot pool updated in place with random slot
ids (some repeated, some negative); or spec-verify on a pool (distinct ids
and negatives, snapshots of the state after every token, the pool read but
not written).

Pool semantics checked (the reference cache's gather / scatter,
engine/runtime/kv_cache.py:189-208, with fla's slot-id convention): a row
owns its slot when its id is non-negative and no earlier row has the same
id; it starts from the slot's state and writes its final state back; other
rows start from zero and write nothing; slots no row owns keep their bits.

Tolerances: 16-bit outputs max abs error 2e-2 and states 1e-3 relative
(norm-wise per row and head); fp32 inputs and outputs 1e-4 and 1e-5.
"""
import numpy as np
import pytest
import torch

from engine.kernels import fused_recurrent_gated_delta_rule
from oracle import gdn

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

DEV = "cuda"
D = 128


@pytest.mark.parametrize("seed", range(12))
def test_random_recurrence_against_the_oracle(seed):
    rng = np.random.default_rng(500 + seed)
    hv = int(rng.choice([16, 32]))
    hk = hv // int(rng.choice([1, 2, 4]))
    bsz = int(rng.integers(1, 101))
    t = int(rng.choice([1, 1, 2, 3, 4]))
    dt = [torch.bfloat16, torch.bfloat16, torch.float16, torch.float32][int(rng.integers(0, 4))]
    mode = ["states", "pool", "verify"][int(rng.integers(0, 3))]
    if mode == "verify" and t == 1:
        t = 4
    print(f"case {seed}: B={bsz} T={t} Hv={hv} Hk={hk} {dt} {mode}", flush=True)
    gen = torch.Generator().manual_seed(2000 + seed)
    q = torch.randn(bsz, t, hk, D, generator=gen).to(dt)
    k = torch.randn(bsz, t, hk, D, generator=gen).to(dt)
    v = torch.randn(bsz, t, hv, D, generator=gen).to(dt)
    g = -torch.nn.functional.softplus(torch.randn(bsz, t, hv, generator=gen)) * torch.exp(
        torch.empty(bsz, t, hv).uniform_(-2, 0, generator=gen))
    beta = torch.sigmoid(torch.randn(bsz, t, hv, generator=gen))
    if rng.random() < 0.5:
        beta = beta.bfloat16()
    args = [x.to(DEV) for x in (q, k, v, g, beta)]
    ref_in = [x.float().numpy() for x in (q, k, v, g, beta)]
    o_tol, s_tol = (1e-4, 1e-5) if dt == torch.float32 else (2e-2, 1e-3)

    if mode == "states":
        h0 = torch.randn(bsz, hv, D, D, generator=gen) * 0.1
        o, s = fused_recurrent_gated_delta_rule(*args, initial_state=h0.to(DEV), output_final_state=True,
                                                use_qk_l2norm_in_kernel=True)
        o_ref, s_ref = gdn.recurrent_gated_delta_rule(*ref_in, initial_state=h0.numpy())
        assert np.abs(o.double().cpu().numpy() - o_ref).max() < o_tol
        assert gdn.state_rel_err(s.cpu().numpy(), s_ref) < s_tol
        return

    slots = bsz + 5
    pool0 = torch.randn(slots, hv, D, D, generator=gen) * 0.1
    if mode == "pool":
        ids = rng.integers(-1, slots, bsz)
        if bsz > 2:
            ids[int(rng.integers(1, bsz))] = ids[0]  # a repeated id
    else:
        ids = rng.permutation(slots)[:bsz]
        ids[rng.random(bsz) < 0.1] = -1
    owner = np.array([ids[r] >= 0 and ids[r] not in ids[:r] for r in range(bsz)])
    h0 = np.zeros((bsz, hv, D, D))
    for r in range(bsz):
        if owner[r]:
            h0[r] = pool0[int(ids[r])].numpy()
    pool = pool0.to(DEV)
    o_ref, s_ref, snaps_ref = gdn.recurrent_gated_delta_rule(*ref_in, initial_state=h0, return_snapshots=True)
    if mode == "pool":
        o, ret = fused_recurrent_gated_delta_rule(*args, initial_state=pool, ssm_state_indices=torch.tensor(ids, device=DEV),
                                                  inplace_final_state=True, use_qk_l2norm_in_kernel=True)
        assert ret is pool
    else:
        snaps = torch.empty((bsz, t, hv, D, D), dtype=torch.float32, device=DEV)
        o, _ = fused_recurrent_gated_delta_rule(*args, initial_state=pool, ssm_state_indices=torch.tensor(ids, device=DEV),
                                                use_qk_l2norm_in_kernel=True, snapshots=snaps)
        got = snaps.cpu().numpy()
        assert gdn.state_rel_err(got[owner], snaps_ref[owner]) < s_tol
    assert o.dtype == dt
    assert np.abs(o.double().cpu().numpy() - o_ref).max() < o_tol
    after = pool.cpu().numpy()
    written = {int(ids[r]) for r in range(bsz) if owner[r]} if mode == "pool" else set()
    for r in range(bsz):
        if mode == "pool" and owner[r]:
            assert gdn.state_rel_err(after[int(ids[r])][None], s_ref[r:r + 1]) < s_tol, r
    kept = [i for i in range(slots) if i not in written]
    assert np.array_equal(after[kept], pool0.numpy()[kept])
