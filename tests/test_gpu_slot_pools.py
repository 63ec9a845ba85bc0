"""Rows f-2 / f-3 on the MI355X: the GDN layer on engine slot pools.

The layer forward (``gated_delta_net_forward``) with a slot-pool cache
(``engine.runtime.slot_pools.GDNSlotPools``) must give every sequence what
transformers' own ``Qwen3_5MoeGatedDeltaNet`` gives it when run alone with
its own ``DynamicCache`` (fp32, CPU): sequences prefilled one at a time into
their slots, then decoded together in any row order, slots reset and
reused.  The reference engine's semantics are the same by construction (its
cache gathers each sequence's slot rows, runs HF's layer, scatters them back,
engine/runtime/kv_cache.py:189-208); here the kernels update the slots in
place.  Spec verify (no reference implementation; spec_decode.py:81-87):
after a verify step of T tokens and ``commit_verify(accepted)``, each slot
must hold the state HF reaches by decoding only the accepted tokens.

The expected values were written by tests/golden/make_golden.py from HF's
forward in the build container (``golden_layer.npz``); the layer's weights
are rebuilt here from tests/layer_cases.py.  Tolerances: layer outputs max
abs error <= 3e-2 * max|ref| (bf16 projections and intermediates on the GPU
path), states relative error <= 1e-2, conv windows max abs error <= 2e-2.
"""
import types

import pytest
import torch

import layer_cases as lc

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

DEV = "cuda"
HEADS = lc.TINY_STATE_HEADS


@pytest.fixture(scope="module")
def golden():
    return lc.load_golden()


def tensor(golden, key):
    return torch.from_numpy(golden[key])


def new_pools(num_slots=6, max_batch=None):
    from engine.runtime import GDNSlotPools
    return GDNSlotPools.allocate([0], num_slots, conv_dim=2 * 2 * 128 + 4 * 128, num_v_heads=4,
                                 device=torch.device(DEV), max_batch=max_batch)


def run(gpu, pools, x, slots, prefill, verify=0):
    from engine.kernels import gated_delta_net_forward
    pools.bind(torch.tensor(slots), is_prefill=prefill, verify_tokens=verify)
    with torch.no_grad():
        return gated_delta_net_forward(gpu, x.to(DEV, torch.bfloat16),
                                       cache_params=types.SimpleNamespace(gdn_slot_pools=pools))


def check_slot(pools, slot, golden, prefix):
    conv, rec = pools.layer(0)
    assert lc.state_close(rec[slot], golden[prefix + ".state"], HEADS), prefix
    assert lc.conv_close(conv[slot], golden[prefix + ".conv"]), prefix


def test_prefill_decode_reset_reuse_match_hf_per_sequence(golden):
    _, gpu = lc.gpu_layer("tiny", golden)
    pools = new_pools()
    slot_of = {"A": 4, "B": 1, "C": 2}
    print("slot pools: prefill A, B, C one at a time", flush=True)
    for n in "ABC":  # prefill one sequence at a time (B = 1), as the reference engine does
        y = run(gpu, pools, tensor(golden, f"pools.pre{n}.x"), [slot_of[n]], prefill=True)
        assert lc.layer_close(y, golden[f"pools.pre{n}.y"]), n
    for i in range(3):  # batched decode, rows A, B, C
        y = run(gpu, pools, tensor(golden, f"pools.dec{i}.x"), [slot_of[n] for n in "ABC"], prefill=False)
        assert lc.layer_close(y, golden[f"pools.dec{i}.y"]), i
    for n in "ABC":
        check_slot(pools, slot_of[n], golden, f"pools.after1.{n}")
    conv, rec = pools.layer(0)
    for s in (0, 3, 5):  # slots no sequence used
        assert not rec[s].any() and not conv[s].any()

    pools.reset_slot(1)  # B finished; D takes its slot
    slot_of["D"] = 1
    y = run(gpu, pools, tensor(golden, "pools.preD.x"), [1], prefill=True)
    assert lc.layer_close(y, golden["pools.preD.y"])
    for i in range(2):  # a different row order
        y = run(gpu, pools, tensor(golden, f"pools.redec{i}.x"), [slot_of[n] for n in "CDA"], prefill=False)
        assert lc.layer_close(y, golden[f"pools.redec{i}.y"]), i
    for n in "ACD":
        check_slot(pools, slot_of[n], golden, f"pools.after2.{n}")


def test_padding_row_repeating_a_slot_is_isolated(golden):
    _, gpu = lc.gpu_layer("tiny", golden)
    gen = torch.Generator().manual_seed(46)
    pools = new_pools()
    x = lc.bf16_inputs(gen, 1, 33, 64)
    run(gpu, pools, x, [4], prefill=True)
    conv, rec = pools.layer(0)
    conv0, rec0 = conv.clone(), rec.clone()
    xd = lc.bf16_inputs(gen, 1, 1, 64).expand(2, 1, 64)
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


def test_decode_step_captured_in_a_graph_matches_eager(golden):
    from engine.kernels import gated_delta_net_forward
    _, gpu = lc.gpu_layer("tiny", golden)
    gen = torch.Generator().manual_seed(47)
    pools = new_pools(max_batch=4)
    for s, length in ((4, 50), (1, 9), (2, 70)):
        run(gpu, pools, lc.bf16_inputs(gen, 1, length, 64), [s], prefill=True)
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
        x = lc.bf16_inputs(gen, 4, 1, 64).to(DEV, torch.bfloat16)
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


@pytest.mark.parametrize("t", [4, 1, 17])
def test_spec_verify_commit_keeps_the_accepted_prefix(golden, t):
    """A verify step of T tokens (1: only the last real token; 17: longer than
    the decode path's recurrent cut-over, so the step must still keep its
    snapshots and conv history), then commit_verify: every slot holds what
    HF's sequential decode of only the accepted tokens leaves, and decoding
    continues from there."""
    print(f"spec verify T={t}", flush=True)
    _, gpu = lc.gpu_layer("tiny", golden)
    pools = new_pools()
    names, slots = "ABC", [4, 1, 2]
    accepted = golden[f"verify{t}.acc"].tolist()
    for n, s in zip(names, slots):
        run(gpu, pools, tensor(golden, f"verify.pre{n}.x"), [s], prefill=True)
    y = run(gpu, pools, tensor(golden, f"verify{t}.x"), slots, prefill=False, verify=t)
    pools.commit_verify(torch.tensor(accepted))
    ref = golden[f"verify{t}.y"]
    for r, (n, a) in enumerate(zip(names, accepted)):
        assert lc.layer_close(y[r:r + 1, :a], ref[r:r + 1, :a]), n
        check_slot(pools, slots[r], golden, f"verify{t}.{n}")
    y = run(gpu, pools, tensor(golden, f"verify{t}.xn"), slots, prefill=False)
    assert lc.layer_close(y, golden[f"verify{t}.yn"])
