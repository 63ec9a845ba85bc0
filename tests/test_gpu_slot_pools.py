"""Rows f-2 / f-3 on the MI355X: the GDN layer on engine slot pools.

The layer forward (``gated_delta_net_forward``) with a slot-pool cache
(``engine.runtime.slot_pools.GDNSlotPools``) must give every sequence what
HF's own ``Qwen3_5MoeGatedDeltaNet`` gives it when run alone with its own
``DynamicCache`` (fp32, CPU): sequences prefilled one at a time into their
slots, then decoded together in any row order, slots reset and reused.
The reference engine's semantics are the same by construction (its cache
gathers each sequence's slot rows, runs HF's layer, scatters them back,
engine/runtime/kv_cache.py:189-208); here the kernels update the slots in
place.  Spec verify (no reference implementation): after a verify step of
T tokens and ``commit_verify(accepted)``, each slot must hold the state HF
reaches by decoding only the accepted tokens.

Tolerances as in test_gpu_layer: layer outputs max abs error <= 3e-2 *
max|ref| (bf16 projections and intermediates on the GPU path), states
relative error <= 1e-2, conv windows max abs error <= 2e-2.
"""
import types

import numpy as np
import pytest
import torch

from oracle import gdn

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

DEV = "cuda"
LAYER_TOL, STATE_TOL, CONV_TOL = 3e-2, 1e-2, 2e-2


def np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def bf16r(t):
    return t.to(torch.bfloat16).to(torch.float32)


def tiny_layer():
    from transformers.models.qwen3_5_moe.configuration_qwen3_5_moe import Qwen3_5MoeTextConfig
    from transformers.models.qwen3_5_moe import modeling_qwen3_5_moe as hf
    cfg = Qwen3_5MoeTextConfig(hidden_size=64, num_hidden_layers=1, layer_types=["linear_attention"],
                               linear_num_key_heads=2, linear_num_value_heads=4, linear_key_head_dim=128,
                               linear_value_head_dim=128, linear_conv_kernel_dim=4, rms_norm_eps=1e-6)
    torch.manual_seed(44)
    layer = hf.Qwen3_5MoeGatedDeltaNet(cfg, layer_idx=0).eval()
    with torch.no_grad():
        for p in layer.parameters():
            p.copy_(bf16r(p))
        layer.norm.weight.copy_(bf16r(1.0 + 0.2 * torch.randn(128)))
        layer.dt_bias.copy_(bf16r(torch.randn(4)))
        layer.A_log.copy_(bf16r(torch.log(torch.empty(4).uniform_(0.5, 4.0))))
    gpu = hf.Qwen3_5MoeGatedDeltaNet(cfg, layer_idx=0).eval()
    gpu.load_state_dict(layer.state_dict())
    return cfg, layer, gpu.to(DEV, torch.bfloat16)


def new_pools(num_slots=6, max_batch=None):
    from engine.runtime import GDNSlotPools
    return GDNSlotPools.allocate([0], num_slots, conv_dim=2 * 2 * 128 + 4 * 128, num_v_heads=4,
                                 device=torch.device(DEV), max_batch=max_batch)


class HFSeq:
    """One sequence through HF's module with its own cache (the ground truth)."""

    def __init__(self, cfg, layer):
        from transformers.cache_utils import DynamicCache
        self.layer, self.cache = layer, DynamicCache(config=cfg)

    def __call__(self, x):
        with torch.no_grad():
            return self.layer(x, cache_params=self.cache)

    def state(self):
        return np64(self.cache.layers[0].recurrent_states[0])

    def conv(self):
        return np64(self.cache.layers[0].conv_states[0])


def run(gpu, pools, x, slots, prefill, verify=0):
    from engine.kernels import gated_delta_net_forward
    pools.bind(torch.tensor(slots), is_prefill=prefill, verify_tokens=verify)
    with torch.no_grad():
        return gated_delta_net_forward(gpu, x.to(DEV, torch.bfloat16),
                                       cache_params=types.SimpleNamespace(gdn_slot_pools=pools))


def close(y, ref):
    return np.abs(np64(y) - np64(ref)).max() <= LAYER_TOL * np.abs(np64(ref)).max()


def check_slot(pools, slot, seq):
    conv, rec = pools.layer(0)
    assert gdn.state_rel_err(np64(rec[slot])[None], seq.state()) < STATE_TOL
    assert np.abs(np64(conv[slot])[None] - seq.conv()).max() < CONV_TOL


def test_prefill_decode_reset_reuse_match_hf_per_sequence():
    cfg, layer, gpu = tiny_layer()
    gen = torch.Generator().manual_seed(45)
    pools = new_pools()
    lens, slot_of = {"A": 70, "B": 5, "C": 130}, {"A": 4, "B": 1, "C": 2}
    seqs = {n: HFSeq(cfg, layer) for n in lens}
    for n, length in lens.items():  # prefill one sequence at a time (B = 1), as the reference engine does
        x = bf16r(torch.randn(1, length, 64, generator=gen))
        assert close(run(gpu, pools, x, [slot_of[n]], prefill=True), seqs[n](x)), n
    for _ in range(3):  # batched decode, rows A, B, C
        x = bf16r(torch.randn(3, 1, 64, generator=gen))
        y = run(gpu, pools, x, [slot_of[n] for n in "ABC"], prefill=False)
        for r, n in enumerate("ABC"):
            assert close(y[r:r + 1], seqs[n](x[r:r + 1])), n
    for n in "ABC":
        check_slot(pools, slot_of[n], seqs[n])
    conv, rec = pools.layer(0)
    for s in (0, 3, 5):  # slots no sequence used
        assert not rec[s].any() and not conv[s].any()

    pools.reset_slot(1)  # B finished; D takes its slot
    seqs["D"], slot_of["D"] = HFSeq(cfg, layer), 1
    x = bf16r(torch.randn(1, 40, 64, generator=gen))
    assert close(run(gpu, pools, x, [1], prefill=True), seqs["D"](x))
    for _ in range(2):  # a different row order
        x = bf16r(torch.randn(3, 1, 64, generator=gen))
        y = run(gpu, pools, x, [slot_of[n] for n in "CDA"], prefill=False)
        for r, n in enumerate("CDA"):
            assert close(y[r:r + 1], seqs[n](x[r:r + 1])), n
    for n in "ACD":
        check_slot(pools, slot_of[n], seqs[n])


def test_padding_row_repeating_a_slot_is_isolated():
    _, _, gpu = tiny_layer()
    gen = torch.Generator().manual_seed(46)
    pools = new_pools()
    x = bf16r(torch.randn(1, 33, 64, generator=gen))
    run(gpu, pools, x, [4], prefill=True)
    conv, rec = pools.layer(0)
    conv0, rec0 = conv.clone(), rec.clone()
    xd = bf16r(torch.randn(1, 1, 64, generator=gen)).expand(2, 1, 64)
    # reference: the second row in slot 5, which holds a zero state, like a padding row
    y_ref = run(gpu, pools, xd, [4, 5], prefill=False)
    conv_ref, rec_ref = conv.clone(), rec.clone()
    conv.copy_(conv0)
    rec.copy_(rec0)
    # the graph runner pads a bucket by repeating row 0 (cuda_graphs.py:473-497)
    y_pad = run(gpu, pools, xd, [4, 4], prefill=False)
    assert pools.slots().tolist() == [4, -1]
    assert torch.equal(y_pad, y_ref)
    assert torch.equal(rec[4], rec_ref[4]) and torch.equal(conv[4], conv_ref[4])  # slot 4 advanced exactly once
    assert torch.equal(rec[5], rec0[5]) and torch.equal(conv[5], conv0[5])  # the padding row wrote nothing
    others = [0, 1, 2, 3]
    assert torch.equal(rec[others], rec0[others]) and torch.equal(conv[others], conv0[others])


def test_decode_step_captured_in_a_graph_matches_eager():
    from engine.kernels import gated_delta_net_forward
    _, _, gpu = tiny_layer()
    gen = torch.Generator().manual_seed(47)
    pools = new_pools(max_batch=4)
    for s, length in ((4, 50), (1, 9), (2, 70)):
        run(gpu, pools, bf16r(torch.randn(1, length, 64, generator=gen)), [s], prefill=True)
    conv, rec = pools.layer(0)
    slots = [4, 1, 2, 4]  # bucket of 4, last row padding
    cache = types.SimpleNamespace(gdn_slot_pools=pools)
    static_x = torch.zeros(4, 1, 64, device=DEV, dtype=torch.bfloat16)
    pools.bind(torch.tensor(slots), is_prefill=False)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side), torch.no_grad():  # warm up outside the capture, then undo its update
        c0, r0 = conv.clone(), rec.clone()
        gated_delta_net_forward(gpu, static_x, cache_params=cache)
        conv.copy_(c0)
        rec.copy_(r0)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph), torch.no_grad():
        static_y = gated_delta_net_forward(gpu, static_x, cache_params=cache)
    conv.copy_(c0)  # the capture does not run the kernels, but keep the pools exact regardless
    rec.copy_(r0)
    for step in range(4):
        x = bf16r(torch.randn(4, 1, 64, generator=gen)).to(DEV, torch.bfloat16)
        ce, re_ = conv.clone(), rec.clone()
        y_eager = run(gpu, pools, x, slots, prefill=False)  # eager step on the current pools
        conv_e, rec_e = conv.clone(), rec.clone()
        conv.copy_(ce)
        rec.copy_(re_)
        torch.cuda.synchronize()
        pools.bind(torch.tensor(slots), is_prefill=False)  # outside the graph, as the runner does
        static_x.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_y[:3], y_eager[:3]), step
        assert torch.equal(rec, rec_e) and torch.equal(conv, conv_e), step


def test_spec_verify_commit_keeps_the_accepted_prefix():
    cfg, layer, gpu = tiny_layer()
    gen = torch.Generator().manual_seed(48)
    pools = new_pools()
    names, slots, accepted = "ABC", [4, 1, 2], [1, 3, 4]
    seqs = {n: HFSeq(cfg, layer) for n in names}
    for n, s, length in zip(names, slots, (70, 5, 130)):
        x = bf16r(torch.randn(1, length, 64, generator=gen))
        run(gpu, pools, x, [s], prefill=True)
        seqs[n](x)
    t = 4
    xv = bf16r(torch.randn(3, t, 64, generator=gen))  # last real token + 3 drafts per row
    y = run(gpu, pools, xv, slots, prefill=False, verify=t)
    pools.commit_verify(torch.tensor(accepted))
    for r, (n, a) in enumerate(zip(names, accepted)):
        ref = torch.cat([seqs[n](xv[r:r + 1, i:i + 1]) for i in range(a)], dim=1)  # decode the accepted tokens only
        assert close(y[r:r + 1, :a], ref), n
        check_slot(pools, slots[r], seqs[n])
    xn = bf16r(torch.randn(3, 1, 64, generator=gen))  # decoding continues from the accepted prefix
    y = run(gpu, pools, xn, slots, prefill=False)
    for r, n in enumerate(names):
        assert close(y[r:r + 1], seqs[n](xn[r:r + 1])), n
