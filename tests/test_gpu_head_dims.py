"""GPU parity at head dims other than 128, through the C ABI, with the CPU
oracle on identical seeded inputs.

The token recurrence is built for K in {64, 128, 256} and V any positive
multiple of 32 (K = V = 128 is the tuned build the decode figures use); the
chunk entry routes other head dims to it.  The oracle at these dims is
pinned by the chunk form = recurrence identity (tests/test_oracle.py).

Tolerances as for the K = V = 128 recurrence tests: fp32 inputs and outputs
max abs error 1e-4 on o and 1e-5 norm-wise relative on states; bf16 outputs
2e-2 abs, states 1e-3 relative.
"""
import numpy as np
import pytest
import torch

from engine.kernels import chunk_gated_delta_rule, fused_recurrent_gated_delta_rule
from oracle import gdn

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

DEV = "cuda"


def np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def inputs(b, t, hk, hv, dk, dv, seed, dtype=torch.float32):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(b, t, hk, dk, generator=gen).to(dtype)
    k = torch.randn(b, t, hk, dk, generator=gen).to(dtype)
    v = torch.randn(b, t, hv, dv, generator=gen).to(dtype)
    g = -torch.nn.functional.softplus(torch.randn(b, t, hv, generator=gen)) * 0.5
    beta = torch.sigmoid(torch.randn(b, t, hv, generator=gen))
    return q, k, v, g, beta


@pytest.mark.parametrize("dk,dv", [(64, 64), (256, 128), (128, 96), (64, 160)])
def test_recurrence_fp32_multi_token(dk, dv):
    q, k, v, g, beta = inputs(2, 37, 2, 4, dk, dv, seed=dk + dv)
    h0 = torch.randn(2, 4, dk, dv, generator=torch.Generator().manual_seed(7)) * 0.1
    o_ref, s_ref = gdn.recurrent_gated_delta_rule(*(x.numpy() for x in (q, k, v, g, beta)), initial_state=h0.numpy())
    o, s = fused_recurrent_gated_delta_rule(*(x.to(DEV) for x in (q, k, v, g, beta)), initial_state=h0.to(DEV),
                                            output_final_state=True, use_qk_l2norm_in_kernel=True)
    assert o.shape == (2, 37, 4, dv) and s.shape == (2, 4, dk, dv)
    assert np.abs(np64(o) - o_ref).max() < 1e-4
    assert gdn.state_rel_err(np64(s), s_ref) < 1e-5


@pytest.mark.parametrize("dk,dv", [(256, 64), (64, 128)])
def test_decode_slot_pool_in_place_bf16(dk, dv):
    q, k, v, g, beta = inputs(4, 1, 2, 4, dk, dv, seed=3 * dk + dv, dtype=torch.bfloat16)
    pool0 = torch.randn(6, 4, dk, dv, generator=torch.Generator().manual_seed(11)) * 0.1
    slots = torch.tensor([3, -1, 0, 5])
    o_ref, pool_ref = gdn.slot_recurrent_step(pool0.numpy(), slots.numpy(),
                                              *(x.float().numpy() for x in (q, k, v, g, beta)))
    pool = pool0.to(DEV)
    o, ret = fused_recurrent_gated_delta_rule(*(x.to(DEV) for x in (q, k, v, g, beta)), initial_state=pool,
                                             ssm_state_indices=slots.to(DEV), inplace_final_state=True,
                                             use_qk_l2norm_in_kernel=True)
    assert ret is pool and o.dtype == torch.bfloat16
    assert np.abs(np64(o) - o_ref).max() < 2e-2
    assert gdn.state_rel_err(np64(pool[[3, 0, 5]]), pool_ref[[3, 0, 5]]) < 1e-3
    assert torch.equal(pool[[1, 2, 4]].cpu(), pool0[[1, 2, 4]])  # slots no row names are untouched


def test_snapshots_at_v96():
    dk, dv = 64, 96
    q, k, v, g, beta = inputs(2, 5, 1, 2, dk, dv, seed=21)
    h0 = torch.randn(2, 2, dk, dv, generator=torch.Generator().manual_seed(22)) * 0.1
    o_ref, _, snaps_ref = gdn.recurrent_gated_delta_rule(*(x.numpy() for x in (q, k, v, g, beta)),
                                                         initial_state=h0.numpy(), return_snapshots=True)
    snaps = torch.empty((2, 5, 2, dk, dv), dtype=torch.float32, device=DEV)
    o, _ = fused_recurrent_gated_delta_rule(*(x.to(DEV) for x in (q, k, v, g, beta)), initial_state=h0.to(DEV),
                                            use_qk_l2norm_in_kernel=True, snapshots=snaps)
    assert np.abs(np64(o) - o_ref).max() < 1e-4
    assert gdn.state_rel_err(np64(snaps), snaps_ref) < 1e-5


def test_chunk_entry_routes_other_dims_varlen():
    dk, dv = 64, 64
    cu = [0, 50, 50, 173]  # an empty middle sequence
    q, k, v, g, beta = inputs(1, 173, 2, 4, dk, dv, seed=31, dtype=torch.bfloat16)
    h0 = torch.randn(3, 4, dk, dv, generator=torch.Generator().manual_seed(32)) * 0.1
    o_ref, s_ref = gdn.chunk_gated_delta_rule_varlen(*(x.float().numpy() for x in (q, k, v, g, beta)), cu,
                                                     initial_state=h0.numpy())
    o, s = chunk_gated_delta_rule(*(x.to(DEV) for x in (q, k, v, g, beta)), initial_state=h0.to(DEV),
                                  output_final_state=True, use_qk_l2norm_in_kernel=True,
                                  cu_seqlens=torch.tensor(cu, dtype=torch.int32, device=DEV))
    assert o.dtype == torch.bfloat16 and s.shape == (3, 4, dk, dv)
    assert np.abs(np64(o) - o_ref).max() < 2e-2
    assert gdn.state_rel_err(np64(s), s_ref) < 1e-3
    assert torch.equal(s[1].cpu(), h0[1])  # the empty sequence keeps its initial state
