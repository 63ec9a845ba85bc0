"""Seeded random sweep of the chunk prefill entry against the CPU oracle.

Each case draws its own batch: 1-14 sequences of 0-350 tokens (some empty
or of one to three tokens), packed with ``cu_seqlens`` or as a dense batch,
Hv of 16 or 32 with Hk = Hv, Hv / 2 or Hv / 4, and one of three state
modes: no initial state; per-sequence initial states with the final states
returned; a slot pool updated in place with random slot ids (some repeated,
some negative) and ``has_initial_state``.  Together the cases reach every
prefill path -- prep + scan, the persistent scan, the per-pair kernel
(from 160 (sequence, v-head) pairs) and the short batches on it.

Pool semantics checked (the reference cache's gather / scatter,
engine/runtime/kv_cache.py:189-208, with fla's slot-id convention): a row
owns its slot when its id is non-negative and no earlier row has the same
id; it starts from the slot's state when ``has_initial_state`` is true (else
from zero) and writes its final state back; other rows start from zero and
write nothing, and every slot no row owns keeps its bits.

Tolerances (north star): bf16 outputs max abs error 2e-2, fp32 final states
relative error 1e-3 norm-wise per (sequence, head).  The oracle is the
fp64 chunk form, pinned against the recurrence in tests/test_oracle.py.
"""
import numpy as np
import pytest
import torch

from engine.kernels import chunk_gated_delta_rule
from oracle import gdn

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

DEV = "cuda"
D = 128


def draw_case(seed):
    rng = np.random.default_rng(seed)
    hv = int(rng.choice([16, 32]))
    hk = hv // int(rng.choice([1, 2, 4]))
    n = int(rng.integers(1, 15))
    dense = n > 1 and rng.random() < 0.25
    if dense:
        lens = [int(rng.integers(1, 351))] * n
    else:
        lens = []
        for _ in range(n):
            u = rng.random()
            lens.append(0 if u < 0.15 else int(rng.integers(1, 4)) if u < 0.25 else int(rng.integers(4, 351)))
    mode = ["none", "states", "pool"][int(rng.integers(0, 3))]
    return rng, hv, hk, lens, dense, mode


@pytest.mark.parametrize("seed", range(12))
def test_random_prefill_against_the_oracle(seed):
    rng, hv, hk, lens, dense, mode = draw_case(seed)
    n, total = len(lens), sum(lens)
    print(f"case {seed}: Hv={hv} Hk={hk} lens={lens} dense={dense} mode={mode}", flush=True)
    gen = torch.Generator().manual_seed(1000 + seed)
    q = torch.randn(1, total, hk, D, generator=gen).bfloat16()
    k = torch.randn(1, total, hk, D, generator=gen).bfloat16()
    v = torch.randn(1, total, hv, D, generator=gen).bfloat16()
    g = -torch.nn.functional.softplus(torch.randn(1, total, hv, generator=gen)) * torch.exp(
        torch.empty(1, total, hv).uniform_(-2, 0, generator=gen))
    beta = torch.sigmoid(torch.randn(1, total, hv, generator=gen))
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)

    h0_rows = np.zeros((n, hv, D, D))
    kw = {}
    if dense:
        t = lens[0]
        args = [x.reshape(n, t, *x.shape[2:]) for x in (q, k, v, g, beta)]
    else:
        args = [q, k, v, g, beta]
        kw["cu_seqlens"] = torch.tensor(cu, dtype=torch.int32, device=DEV)
    owner = np.zeros(n, bool)
    if mode == "states":
        h0 = torch.randn(n, hv, D, D, generator=gen) * 0.1
        h0_rows[:] = h0.numpy()
        kw.update(initial_state=h0.to(DEV), output_final_state=True)
    elif mode == "pool":
        slots = n + 3
        pool0 = torch.randn(slots, hv, D, D, generator=gen) * 0.1
        ids = rng.integers(-1, slots, n)
        if n > 2:
            ids[int(rng.integers(1, n))] = ids[0]  # a repeated id
        has = rng.random(n) < 0.8
        for r in range(n):
            owner[r] = ids[r] >= 0 and ids[r] not in ids[:r]
            if owner[r] and has[r]:
                h0_rows[r] = pool0[int(ids[r])].numpy()
        pool = pool0.to(DEV)
        kw.update(initial_state=pool, ssm_state_indices=torch.tensor(ids, device=DEV),
                  has_initial_state=torch.tensor(has, device=DEV), inplace_final_state=True)
    else:
        kw.update(output_final_state=True)

    o, s = chunk_gated_delta_rule(*(x.to(DEV) for x in args), use_qk_l2norm_in_kernel=True, **kw)
    o_ref, s_ref = gdn.chunk_gated_delta_rule_varlen(*(x.float().numpy() for x in (q, k, v, g, beta)), cu,
                                                     initial_state=h0_rows)
    o_got = o.float().cpu().numpy().reshape(o_ref.shape).astype(np.float64)
    assert np.abs(o_got - o_ref).max() < 2e-2
    if mode == "pool":
        got = pool.cpu().numpy().astype(np.float64)
        for r in range(n):
            if owner[r]:
                assert gdn.state_rel_err(got[int(ids[r])][None], s_ref[r:r + 1]) < 1e-3, r
        kept = [i for i in range(slots) if i not in set(int(ids[r]) for r in range(n) if owner[r])]
        assert np.array_equal(got[kept], pool0.numpy()[kept])
    else:
        assert s.shape == (n, hv, D, D)
        assert gdn.state_rel_err(s.cpu().numpy().astype(np.float64), s_ref) < 1e-3
