"""Row f-1 on the MI355X: the GDN layer glue fused into the kernels.

* gates from raw projections (beta = sigmoid(b), g = -exp(A_log) softplus(a +
  dt_bias), transformers modeling_qwen3_5_moe.py:495-497) inside the chunk and
  recurrent kernels, against the oracle's gates + recurrence;
* the gated RMS norm kernel against the oracle (pinned by HF's module);
* the whole layer forward (``gated_delta_net_forward``: native GQA, fused
  gates, HIP conv / core / norm) against HF's own ``Qwen3_5MoeGatedDeltaNet``
  forward in fp32 with the same (bf16-exact) weights and inputs, for a
  prefill and for cached decode steps; HF's values are fixtures written in
  the build container (tests/golden/make_golden.py, golden_layer.npz).

Tolerances: core outputs bf16 max abs error <= 2e-2 and fp32 states relative
error <= 1e-3 (north star); the layer output, after five bf16 roundings of
intermediate tensors on the GPU path, max abs error <= 3e-2 * max|ref|.
"""
import numpy as np
import pytest
import torch

from oracle import gdn

import layer_cases as lc

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

DEV = "cuda"
O_TOL, S_TOL, LAYER_TOL = 2e-2, 1e-3, 3e-2


def np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def bf16r(t):
    return t.to(torch.bfloat16).to(torch.float32)


def raw_gates(gen, b, t, hv):
    a = bf16r(torch.randn(b, t, hv, generator=gen))
    bb = bf16r(torch.randn(b, t, hv, generator=gen))
    A_log = torch.log(torch.empty(hv).uniform_(0.5, 16.0, generator=gen))
    dt_bias = torch.randn(hv, generator=gen)
    return a, bb, A_log, dt_bias


@pytest.mark.parametrize("bsz,t", [(1, 200), (8, 130)])
def test_chunk_from_projections_matches_oracle(bsz, t):
    """Gates computed in the kernel from the raw projections: one sequence
    (prep + scan) and B = 8 x T = 130 (256 (sequence, v-head) pairs: the
    per-pair kernel, where a chain wave forms the gates), against the oracle
    sequence by sequence."""
    from engine.kernels import chunk_gated_delta_rule_from_projections
    gen = torch.Generator().manual_seed(31)
    hk, hv = 16, 32
    q = torch.randn(bsz, t, hk, 128, generator=gen).to(torch.bfloat16)
    k = torch.randn(bsz, t, hk, 128, generator=gen).to(torch.bfloat16)
    v = torch.randn(bsz, t, hv, 128, generator=gen).to(torch.bfloat16)
    a, b, A_log, dt_bias = raw_gates(gen, bsz, t, hv)
    a = a * 0.5 - 3.0  # moderate decays so the state carries across chunks
    h0 = torch.randn(bsz, hv, 128, 128, generator=gen) * 0.1
    o, s = chunk_gated_delta_rule_from_projections(
        q.to(DEV), k.to(DEV), v.to(DEV), a.to(torch.bfloat16).to(DEV), b.to(torch.bfloat16).to(DEV),
        A_log.to(DEV), dt_bias.to(DEV), initial_state=h0.to(DEV), output_final_state=True)
    g, beta = gdn.gdn_gates(np64(a.to(torch.bfloat16)), np64(b.to(torch.bfloat16)), np64(A_log), np64(dt_bias))
    for i in range(bsz):
        o_ref, s_ref = gdn.chunk_gated_delta_rule(np64(q[i:i + 1]), np64(k[i:i + 1]), np64(v[i:i + 1]),
                                                  g[i:i + 1], beta[i:i + 1], initial_state=np64(h0[i:i + 1]))
        err_o, err_s = np.abs(np64(o[i:i + 1]) - o_ref).max(), gdn.state_rel_err(np64(s[i:i + 1]), s_ref)
        print(f"chunk gated B={bsz} row {i}: max|o-o_ref|={err_o:.3e} state rel={err_s:.3e}")
        assert err_o < O_TOL and err_s < S_TOL, i


def test_recurrent_from_projections_matches_oracle_on_a_slot_pool():
    from engine.kernels import fused_recurrent_gated_delta_rule_from_projections
    gen = torch.Generator().manual_seed(32)
    bsz, hk, hv, slots = 8, 16, 32, 12
    q = torch.randn(bsz, 1, hk, 128, generator=gen).to(torch.bfloat16)
    k = torch.randn(bsz, 1, hk, 128, generator=gen).to(torch.bfloat16)
    v = torch.randn(bsz, 1, hv, 128, generator=gen).to(torch.bfloat16)
    a, b, A_log, dt_bias = raw_gates(gen, bsz, 1, hv)
    pool = torch.randn(slots, hv, 128, 128, generator=gen) * 0.1
    slot_ids = torch.randperm(slots, generator=gen)[:bsz]
    pool_gpu = pool.to(DEV)
    o, _ = fused_recurrent_gated_delta_rule_from_projections(
        q.to(DEV), k.to(DEV), v.to(DEV), a.to(DEV), b.to(DEV), A_log.to(DEV), dt_bias.to(DEV),
        initial_state=pool_gpu, ssm_state_indices=slot_ids.to(DEV), inplace_final_state=True)
    g, beta = gdn.gdn_gates(np64(a), np64(b), np64(A_log), np64(dt_bias))
    o_ref, s_ref = gdn.recurrent_gated_delta_rule(np64(q), np64(k), np64(v), g, beta,
                                                  initial_state=np64(pool)[slot_ids.numpy()])
    assert np.abs(np64(o) - o_ref).max() < O_TOL
    assert gdn.state_rel_err(np64(pool_gpu[slot_ids.to(DEV)]), s_ref) < S_TOL
    untouched = np.setdiff1d(np.arange(slots), slot_ids.numpy())
    assert torch.equal(pool_gpu[untouched].cpu(), pool[untouched])


@pytest.mark.parametrize("dtype,w_dtype,h", [(torch.bfloat16, torch.bfloat16, 32), (torch.float32, torch.float32, 32),
                                               (torch.bfloat16, torch.float32, 32), (torch.float16, torch.float16, 20)])
def test_rms_norm_gated_matches_oracle(dtype, w_dtype, h):
    """2-byte x / z / y take the kernel that issues all loads first (bf16 or
    fp32 weight; H = 20 leaves a partial group of 16 rows), fp32 the
    general one."""
    from engine.kernels import rms_norm_gated
    gen = torch.Generator().manual_seed(33)
    t = 37
    x = (torch.randn(t, h, 128, generator=gen) * 3.0).to(dtype)
    zz = torch.randn(t, 2 * h * 128, generator=gen).to(dtype)   # z as a strided view of a packed projection
    z = zz[:, h * 128:].view(t, h, 128)
    w = (1.0 + 0.3 * torch.randn(128, generator=gen)).to(w_dtype)
    y = rms_norm_gated(x.to(DEV), zz.to(DEV)[:, h * 128:].view(t, h, 128), w.to(DEV), eps=1e-6)
    assert y.dtype == dtype and y.shape == x.shape
    y_ref = gdn.rms_norm_gated(np64(x), np64(z), np64(w), eps=1e-6)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert np.abs(np64(y) - y_ref).max() < tol * max(1.0, np.abs(y_ref).max())


# ---------------------------------------------------------------- the HF layer
def test_layer_prefill_matches_hf_module():
    """The layer forward without a cache against HF's forward (fixture)."""
    from engine.kernels import gated_delta_net_forward
    golden = lc.load_golden()
    _, gpu = lc.gpu_layer("tiny", golden)
    x = torch.from_numpy(golden["prefill.x"])
    with torch.no_grad():
        y = gated_delta_net_forward(gpu, x.to(DEV, torch.bfloat16))
    y_ref = golden["prefill.y"]
    err = np.abs(np64(y) - y_ref).max()
    print(f"layer prefill: max|y-y_ref|={err:.3e} max|y_ref|={np.abs(y_ref).max():.3e}")
    assert lc.layer_close(y, y_ref, LAYER_TOL)


def test_layer_decode_with_cache_matches_hf_module():
    """Prefill then three cached decode steps through transformers' own
    DynamicCache (HF's cache protocol, the kernels updating its tensors),
    against HF's forward with its own cache (fixture): outputs, the final
    recurrent states and conv windows."""
    from transformers.cache_utils import DynamicCache
    from engine.kernels import gated_delta_net_forward
    golden = lc.load_golden()
    cfg, gpu = lc.gpu_layer("tiny", golden)
    cache = DynamicCache(config=cfg)
    with torch.no_grad():
        for i in range(4):
            y = gated_delta_net_forward(gpu, torch.from_numpy(golden[f"cache.x{i}"]).to(DEV, torch.bfloat16),
                                        cache_params=cache)
            err = np.abs(np64(y) - golden[f"cache.y{i}"]).max()
            print(f"layer step {i}: max|y-y_ref|={err:.3e}")
            assert lc.layer_close(y, golden[f"cache.y{i}"], LAYER_TOL), i
    s_ref = golden["cache.state"].astype(np.float64)
    s_gpu = np64(cache.layers[0].recurrent_states[0])
    assert gdn.state_rel_err(s_gpu, s_ref) < 1e-2   # states after bf16 projections and conv
    assert np.abs(np64(cache.layers[0].conv_states[0]) - golden["cache.conv"]).max() < 2e-2
