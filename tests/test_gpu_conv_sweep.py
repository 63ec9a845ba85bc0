"""Seeded random sweep of the causal conv (prefill over packed sequences,
then decode steps on the same windows) against the CPU oracle.

Each case draws: dtype bf16, fp16 or fp32; C of 8192, 1024, 264 or 64
channels; kernel width 2, 3 or 4; with or without bias and SiLU; 1-8
packed sequences of 0-200 tokens; history from zeros, from per-sequence
initial windows, or from a slot pool (random ids with one repeated and
possibly a negative one, ``has_initial_state`` random).  The prefill's
final windows then feed 1-3 decode tokens through ``causal_conv1d_update``
(on the pool, or on the returned windows).

Pool semantics (the reference cache's gather / scatter,
engine/runtime/kv_cache.py:189-208, fla's slot-id convention): a row owns
its slot when its id is non-negative and no earlier row has the same id;
it reads the slot's window when ``has_initial_state`` is true (else zeros)
and writes its final window back; other rows run from zeros and write
nothing; every other slot keeps its bits.

Tolerances: fp32 1e-5 absolute; bf16 2e-2 x max(1, |y|) (the north star's
2e-2, widened to a bf16 ulp above 1); fp16 1e-3 x max(1, |y|) (one rounding
of an fp32 result).  Windows are copies of inputs: compared bit-exactly.
"""
import numpy as np
import pytest
import torch

from engine.kernels import causal_conv1d_fn, causal_conv1d_update
from oracle import conv

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

DEV = "cuda"
S = 4  # cached window length, as HF keeps it


def close(y, y_ref, dt):
    err = np.abs(y.detach().double().cpu().numpy() - y_ref)
    if dt == torch.float32:
        return err.max() < 1e-5
    rel = err / np.maximum(1.0, np.abs(y_ref))
    return rel.max() <= (2e-2 if dt == torch.bfloat16 else 1e-3)


@pytest.mark.parametrize("seed", range(10))
def test_random_conv_prefill_then_decode(seed):
    rng = np.random.default_rng(700 + seed)
    dt = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(0, 3))]
    c = int(rng.choice([8192, 1024, 264, 64]))
    width = int(rng.choice([2, 3, 4]))
    act = "silu" if rng.random() < 0.7 else None
    with_bias = rng.random() < 0.4
    n = int(rng.integers(1, 9))
    lens = [0 if rng.random() < 0.15 else int(rng.integers(1, 201)) for _ in range(n)]
    mode = ["zeros", "states", "pool"][int(rng.integers(0, 3))]
    print(f"case {seed}: {dt} C={c} W={width} act={act} bias={with_bias} lens={lens} {mode}", flush=True)
    gen = torch.Generator().manual_seed(3000 + seed)
    total = sum(lens)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    x = torch.randn(total, c, generator=gen).to(dt)
    w = torch.randn(c, width, generator=gen).to(dt)
    bias = torch.randn(c, generator=gen).to(dt) if with_bias else None
    args = dict(cu_seqlens=torch.tensor(cu, dtype=torch.int32, device=DEV))
    hist = np.zeros((n, c, S))
    if mode == "states":
        h = torch.randn(n, c, S, generator=gen).to(dt)
        hist[:] = h.double().numpy()
        args.update(initial_states=h.to(DEV), return_final_states=True)
    elif mode == "pool":
        slots = n + 3
        pool0 = torch.randn(slots, c, S, generator=gen).to(dt)
        ids = rng.permutation(slots)[:n]
        if n > 2:
            ids[int(rng.integers(1, n))] = ids[0]
        if n > 1 and rng.random() < 0.5:
            ids[int(rng.integers(0, n))] = -1
        has = rng.random(n) < 0.8
        owner = np.array([ids[r] >= 0 and ids[r] not in ids[:r] for r in range(n)])
        for r in range(n):
            if owner[r] and has[r]:
                hist[r] = pool0[int(ids[r])].double().numpy()
        pool = pool0.to(DEV)
        args.update(conv_states=pool, cache_indices=torch.tensor(ids, device=DEV),
                    has_initial_state=torch.tensor(has, device=DEV))
    else:
        args.update(return_final_states=True)

    out = causal_conv1d_fn(x.to(DEV), w.to(DEV), None if bias is None else bias.to(DEV), activation=act, **args)
    y = out[0] if isinstance(out, tuple) else out
    y_ref, fin_ref = conv.causal_conv1d_varlen(x.double().numpy(), w.double().numpy(), cu,
                                               None if bias is None else bias.double().numpy(), act,
                                               initial_states=hist, state_len=S)
    assert y.shape == x.shape and y.dtype == dt
    assert close(y, y_ref, dt)

    # decode steps on the windows the prefill left
    t = int(rng.integers(1, 4))
    xd = torch.randn(n, c, t, generator=gen).to(dt)
    if mode == "pool":
        after = pool.double().cpu().numpy()
        for r in range(n):
            if owner[r]:
                assert np.array_equal(after[int(ids[r])], fin_ref[r]), r
        kept = [i for i in range(slots) if i not in {int(ids[r]) for r in range(n) if owner[r]}]
        assert torch.equal(pool[kept].cpu(), pool0[kept])
        win = np.zeros((n, c, S))
        for r in range(n):
            if owner[r]:
                win[r] = after[int(ids[r])]
        yd = causal_conv1d_update(xd.to(DEV), pool, w.to(DEV), None if bias is None else bias.to(DEV), act,
                                  conv_state_indices=torch.tensor(ids, device=DEV))
    else:
        fin = out[1]
        assert np.array_equal(fin.double().cpu().numpy(), fin_ref)
        win = fin_ref
        yd = causal_conv1d_update(xd.to(DEV), fin, w.to(DEV), None if bias is None else bias.to(DEV), act)
    yd_ref, win_ref = conv.causal_conv1d_update(xd.double().numpy(), win, w.double().numpy(),
                                                None if bias is None else bias.double().numpy(), act)
    assert close(yd, yd_ref, dt)
    if mode == "pool":
        after2 = pool.double().cpu().numpy()
        for r in range(n):
            if owner[r]:
                assert np.array_equal(after2[int(ids[r])], win_ref[r]), r
    else:
        assert np.array_equal(fin.double().cpu().numpy(), win_ref)
