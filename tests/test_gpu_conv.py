"""GPU parity of the causal depthwise conv (prefill fn and decode update)
with the CPU oracle and with HF's golden vectors, through the C ABI.

fp32 cases are checked to 1e-5.  bf16 outputs are checked to
|y - y_ref| <= 2e-2 * max(1, |y_ref|): the north star's 2e-2 abs bound, widened
to one bf16 ulp (2^-7 relative) for the |y| > 1 values SiLU produces here.
fp16 outputs (one rounding of an fp32 result, 2^-11 relative) are checked to
|y - y_ref| <= 1e-3 * max(1, |y_ref|).  Window/state tensors are copies of
inputs, so they are checked bit-exactly."""
import numpy as np
import pytest
import torch

from engine import configs
from engine.kernels import causal_conv1d_fn, causal_conv1d_update
from oracle import conv

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

DEV = "cuda"


def np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def bf16_close(y, y_ref):
    err = np.abs(np64(y) - y_ref) / np.maximum(1.0, np.abs(y_ref))
    return err.max() <= 2e-2


def f16_close(y, y_ref):
    err = np.abs(np64(y) - y_ref) / np.maximum(1.0, np.abs(y_ref))
    return err.max() <= 1e-3


def close_for(dtype):
    return f16_close if dtype == torch.float16 else bf16_close


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_fn_matches_hf_golden(golden, dtype):
    x = torch.from_numpy(golden["conv_fn.x"]).to(DEV, dtype)
    w = torch.from_numpy(golden["conv_fn.w"]).to(DEV, dtype)
    close = (lambda a, b: np.abs(np64(a) - b).max() < 1e-5) if dtype == torch.float32 else bf16_close
    # (the golden input is fp32: rounding it to fp16 moves y by more than
    # fp16's own output bound, so fp16 is held to the bf16 bound here and to
    # its own bound on fp16 inputs below)
    y = causal_conv1d_fn(x, w, None, activation="silu")
    assert y.shape == x.shape and y.dtype == dtype
    assert close(y, golden["conv_fn.y"])
    xs = torch.from_numpy(golden["conv_fn_short.x"]).to(DEV, dtype)
    ys = causal_conv1d_fn(xs, w, None, activation="silu")
    assert close(ys, golden["conv_fn_short.y"])


def test_update_matches_hf_golden(golden):
    x = torch.from_numpy(golden["conv_upd.x"]).to(DEV)
    st = torch.from_numpy(golden["conv_upd.state"]).to(DEV)
    w = torch.from_numpy(golden["conv_upd.w"]).to(DEV)
    y = causal_conv1d_update(x, st, w, None, "silu")
    assert np.abs(np64(y) - golden["conv_upd.y"]).max() < 1e-5
    assert np.array_equal(st.cpu().numpy(), golden["conv_upd.state_after"])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_config3_varlen_conv_with_history_and_pool(dtype):
    c = configs.config3()
    cu = c["cu_seqlens"]
    n = cu.numel() - 1
    gen = torch.Generator().manual_seed(33)
    hist = torch.randn(n, configs.CONV_DIM, 4, generator=gen).to(dtype)
    num_slots = 24
    slots = torch.randperm(num_slots, generator=gen)[:n]
    pool0 = torch.randn(num_slots, configs.CONV_DIM, 4, generator=gen).to(dtype)
    pool0[slots] = hist
    x, cw = c["x"].to(dtype), c["conv_w"].to(dtype)
    y_ref, fin_ref = conv.causal_conv1d_varlen(x.float().numpy(), cw.float().numpy(), cu.numpy(),
                                               activation="silu", initial_states=hist.float().numpy(),
                                               dtype=np.float32)
    pool = pool0.to(DEV)
    y = causal_conv1d_fn(x.to(DEV), cw.to(DEV), None, activation="silu", cu_seqlens=cu.to(DEV),
                         conv_states=pool, cache_indices=slots.to(DEV))
    assert y.shape == x.shape and y.dtype == dtype and pool.dtype == dtype
    assert close_for(dtype)(y, y_ref)
    assert np.abs(np64(y) - y_ref).mean() < (2e-3 if dtype == torch.bfloat16 else 2e-4)
    assert np.array_equal(np64(pool[slots.to(DEV)]), fin_ref)
    keep = torch.ones(num_slots, dtype=torch.bool)
    keep[slots] = False
    assert torch.equal(pool[keep.to(DEV)].cpu(), pool0[keep])


def test_varlen_short_and_empty_sequences_fp32():
    lens = [2, 0, 37, 1, 64, 3]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    gen = torch.Generator().manual_seed(2)
    x = torch.randn(int(cu[-1]), 64, generator=gen)
    w = torch.randn(64, 4, generator=gen)
    hist = torch.randn(len(lens), 64, 4, generator=gen)
    y_ref, fin_ref = conv.causal_conv1d_varlen(x.numpy(), w.numpy(), cu.numpy(), activation="silu",
                                               initial_states=hist.numpy())
    y, fin = causal_conv1d_fn(x.to(DEV), w.to(DEV), activation="silu", cu_seqlens=cu.to(DEV),
                              initial_states=hist.to(DEV), return_final_states=True)
    assert np.abs(np64(y) - y_ref).max() < 1e-5
    assert np.array_equal(np64(fin), fin_ref.astype(np.float32).astype(np.float64))


def test_has_initial_state_false_starts_from_zeros():
    gen = torch.Generator().manual_seed(4)
    x = torch.randn(2, 16, 5, generator=gen).to(torch.bfloat16)
    w = torch.randn(16, 4, generator=gen).to(torch.bfloat16)
    pool = torch.randn(2, 16, 4, generator=gen).to(torch.bfloat16).to(DEV)
    pool_before = pool.clone()
    y = causal_conv1d_fn(x.to(DEV), w.to(DEV), activation="silu", conv_states=pool,
                         has_initial_state=torch.tensor([False, True], device=DEV))
    y0, f0 = conv.causal_conv1d_fn(x[:1].float().numpy(), w.float().numpy())
    y1, f1 = conv.causal_conv1d_fn(x[1:].float().numpy(), w.float().numpy(),
                                   initial_state=pool_before[1:].float().cpu().numpy())
    assert bf16_close(y[:1], y0) and bf16_close(y[1:], y1)
    assert np.array_equal(np64(pool[0]), f0[0]) and np.array_equal(np64(pool[1]), f1[0])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("t", [1, 2, 4])
def test_update_pool_indices_and_negative_slot(t, dtype):
    gen = torch.Generator().manual_seed(10 + t)
    b, c = 4, configs.CONV_DIM
    x = torch.randn(b, c, t, generator=gen).to(dtype)
    w = torch.randn(c, 4, generator=gen).to(dtype)
    pool0 = torch.randn(6, c, 4, generator=gen).to(dtype)
    idx = torch.tensor([4, -1, 0, 2])
    states = torch.zeros(b, c, 4)
    states[[0, 2, 3]] = pool0[[4, 0, 2]].float()
    y_ref, st_ref = conv.causal_conv1d_update(x.float().numpy(), states.numpy(), w.float().numpy(),
                                              activation="silu")
    pool = pool0.to(DEV)
    y = causal_conv1d_update(x.to(DEV), pool, w.to(DEV), None, "silu", conv_state_indices=idx.to(DEV))
    assert y.dtype == dtype and close_for(dtype)(y, y_ref)
    assert np.array_equal(np64(pool[[4, 0, 2]]), st_ref[[0, 2, 3]])
    assert torch.equal(pool[[1, 3, 5]].cpu(), pool0[[1, 3, 5]])


def test_prefill_then_decode_continuation():
    """fn over a prompt (pool window written) then update steps == fn over the whole stream."""
    gen = torch.Generator().manual_seed(6)
    c, t = 256, 45
    x = torch.randn(1, c, t + 3, generator=gen)
    w = torch.randn(c, 4, generator=gen)
    y_full = causal_conv1d_fn(x.to(DEV), w.to(DEV), activation="silu")
    pool = torch.zeros(3, c, 4, device=DEV)
    slot = torch.tensor([1], device=DEV)
    y_pre = causal_conv1d_fn(x[:, :, :t].to(DEV), w.to(DEV), activation="silu", conv_states=pool,
                             cache_indices=slot)
    outs = [causal_conv1d_update(x[:, :, t + i:t + i + 1].to(DEV), pool, w.to(DEV), None, "silu",
                                 conv_state_indices=slot) for i in range(3)]
    y_cat = torch.cat([y_pre] + outs, dim=-1)
    assert torch.allclose(y_cat, y_full, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_tile_lengths_agree(dtype):
    """The tile length follows the input's length (64, 56, 48 or 32 tokens:
    13,794 tokens run 56-token tiles, 5,000 run 48, 4,096 run 64 and 4,000
    run 32): the same tokens give the same bits whatever the tiling (and
    match the oracle), in each activation dtype."""
    gen = torch.Generator().manual_seed(12)
    c = configs.CONV_DIM
    x = torch.randn(1, 13794, c, generator=gen).to(dtype)
    w = torch.randn(c, 4, generator=gen).to(dtype)
    xd, wd = x.to(DEV), w.to(DEV)
    y_short = causal_conv1d_fn(xd[:, :4000].transpose(1, 2), wd, None, activation="silu")
    for t in (13794, 5000, 4096):
        y = causal_conv1d_fn(xd[:, :t].transpose(1, 2), wd, None, activation="silu")
        assert torch.equal(y[:, :, :4000], y_short), t
    y_ref, _ = conv.causal_conv1d_fn(x[:, :300].transpose(1, 2).float().numpy(), w.float().numpy(),
                                     activation="silu")
    assert bf16_close(y_short[:, :, :300], y_ref)


def test_conv_state_commit_matches_update_over_the_accepted_prefix():
    """gdn_conv_state_commit against the oracle: a verify step's history is
    the window before the step followed by its T inputs; after committing
    ``a`` accepted tokens a slot must hold the window that
    causal_conv1d_update over exactly those ``a`` tokens leaves (the conv
    half of the rollback spec_decode.py:81-87 leaves unimplemented).
    a <= 0 and a repeated slot id leave the slot untouched."""
    from engine.kernels import gdn_conv_state_commit
    gen = torch.Generator().manual_seed(71)
    n, c, s, t = 5, 256, 4, 6
    win0 = torch.randn(n, c, s, generator=gen).to(torch.bfloat16)
    x = torch.randn(n, c, t, generator=gen).to(torch.bfloat16)
    w = torch.randn(c, 4, generator=gen).to(torch.bfloat16)
    hist = torch.cat([win0, x], dim=2)
    slots = torch.tensor([3, 0, 6, 3, 2])  # row 3 repeats row 0's slot
    acc = torch.tensor([2, 6, 1, 4, 0])
    pool0 = torch.randn(7, c, s, generator=gen).to(torch.bfloat16)
    pool = pool0.to(DEV)
    gdn_conv_state_commit(pool, slots.to(DEV), hist.to(DEV), acc.to(DEV))
    for r in (0, 1, 2):
        a = int(acc[r])
        _, st_ref = conv.causal_conv1d_update(np64(x[r:r + 1, :, :a]), np64(win0[r:r + 1]), np64(w))
        assert np.array_equal(np64(pool[int(slots[r])])[None], st_ref), r
    assert torch.equal(pool[[1, 2, 4, 5]].cpu(), pool0[[1, 2, 4, 5]])  # a = 0 (row 4), unused slots


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_update_with_repeated_slot_ids_advances_a_slot_once(dtype):
    """ids [s, s, t] with identical rows 0 and 1: slot s's window moves by one
    token, row 1 runs as a padding row (zero window, nothing written)."""
    gen = torch.Generator().manual_seed(72)
    c = 512
    pool0 = torch.randn(4, c, 4, generator=gen).to(dtype)
    x = torch.randn(2, c, 1, generator=gen).to(dtype)
    x = torch.cat([x[:1], x[:1], x[1:]])  # rows 0 and 1 identical
    w = torch.randn(c, 4, generator=gen).to(dtype)
    close = close_for(dtype)
    pool = pool0.to(DEV)
    y = causal_conv1d_update(x.to(DEV), pool, w.to(DEV), None, "silu", conv_state_indices=torch.tensor([2, 2, 0]).to(DEV))
    y0, st0 = conv.causal_conv1d_update(np64(x[:1]), np64(pool0[2:3]), np64(w))
    y1, _ = conv.causal_conv1d_update(np64(x[1:2]), np.zeros((1, c, 4)), np64(w))
    y2, st2 = conv.causal_conv1d_update(np64(x[2:3]), np64(pool0[0:1]), np64(w))
    assert close(y[0:1], y0) and close(y[1:2], y1) and close(y[2:3], y2)
    assert np.array_equal(np64(pool[2])[None], st0) and np.array_equal(np64(pool[0])[None], st2)
    assert torch.equal(pool[[1, 3]].cpu(), pool0[[1, 3]])


def test_fn_repeated_slot_id_with_mismatched_has_initial_state():
    """Prefill conv on a pool with ids [3, 3] and has_initial_state [False,
    True]: row 0 alone owns slot 3 (zero history, its final window written),
    row 1 runs from a zero window and writes nothing."""
    gen = torch.Generator().manual_seed(74)
    c = 256
    x = torch.randn(2, c, 6, generator=gen).to(torch.bfloat16)
    w = torch.randn(c, 4, generator=gen).to(torch.bfloat16)
    pool0 = torch.randn(4, c, 4, generator=gen).to(torch.bfloat16)
    pool = pool0.to(DEV)
    y = causal_conv1d_fn(x.to(DEV), w.to(DEV), activation="silu", conv_states=pool,
                         cache_indices=torch.tensor([3, 3], device=DEV),
                         has_initial_state=torch.tensor([False, True], device=DEV))
    y0, f0 = conv.causal_conv1d_fn(np64(x[:1]), np64(w))
    y1, _ = conv.causal_conv1d_fn(np64(x[1:]), np64(w))
    assert bf16_close(y[:1], y0) and bf16_close(y[1:], y1)
    assert np.array_equal(np64(pool[3]), f0[0])
    assert torch.equal(pool[:3].cpu(), pool0[:3])
