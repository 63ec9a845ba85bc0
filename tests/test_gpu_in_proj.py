"""GPU parity of the fused decode input projections (gdn_in_proj_decode:
four projections + causal conv update) and of the decode output projection
(gdn_out_proj_decode) with the CPU oracle, with the unfused / hipBLASLt GPU
path, under graph capture, and inside the GDN layer against HF's module (a
small layer and one at the model's shapes).

Tolerances: bf16 outputs |y - y_ref| <= 2e-2 * max(1, |y_ref|) (the north
star's 2e-2 abs bound, widened to one bf16 ulp for |y| > 1); window taps
that are copies are compared bit-exactly, the new tap (the bf16-rounded
projection) to one bf16 ulp plus the fp32 summation error of a 2048-term
dot product, 2^-16 * sum_i |x_i w_i| (the oracle sums exactly; where the
sum cancels, fp32 rounding moves the bf16 result by more than one ulp)."""
import types

import numpy as np
import pytest
import torch

from oracle import proj

import layer_cases as lc

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

DEV = "cuda"
K, NQKV, NZ, NB, NA = 2048, 8192, 4096, 32, 32  # the Qwen3.5-MoE GDN layer


def np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def bf16_close(y, y_ref):
    return (np.abs(np64(y) - y_ref) / np.maximum(1.0, np.abs(y_ref))).max() <= 2e-2


def weights(gen, k=K, n=(NQKV, NZ, NB, NA), bias=False):
    ws = [(0.02 * torch.randn(m, k, generator=gen)).to(torch.bfloat16).to(DEV) for m in n]
    cw = (0.5 * torch.randn(n[0], 4, generator=gen)).to(torch.bfloat16).to(DEV)
    cb = (0.1 * torch.randn(n[0], generator=gen)).to(torch.bfloat16).to(DEV) if bias else None
    return ws, cw, cb


def tap_close(got, ref, x, w):
    """New window tap vs its reference: one bf16 ulp + fp32 sum error."""
    scale = np.abs(np64(x)) @ np.abs(np64(w)).T
    return (np.abs(got - ref) <= 2.0 ** -7 * np.abs(ref) + 2.0 ** -16 * scale).all()


def run_fused(x, ws, cw, cb, pool, slots):
    from engine.kernels.in_proj import gdn_in_proj_decode
    return gdn_in_proj_decode(x, *ws, cw, cb, pool, slots)


@pytest.mark.parametrize("m,bias", [(64, False), (5, True), (1, False), (100, False)])
def test_matches_oracle_at_model_shape(m, bias):
    print(f"in_proj_decode oracle case M={m} bias={bias}", flush=True)
    gen = torch.Generator().manual_seed(71 + m)
    ws, cw, cb = weights(gen, bias=bias)
    rows = 128
    pool = torch.randn(rows, NQKV, 4, generator=gen).to(torch.bfloat16).to(DEV)
    slots = torch.randperm(rows, generator=gen)[:m]
    if m >= 5:
        slots[3] = -1  # a padding row
    x = torch.randn(m, K, generator=gen).to(torch.bfloat16).to(DEV)
    pool0 = pool.clone()
    y, z, b, a = run_fused(x, ws, cw, cb, pool, slots.to(DEV))

    s = slots.numpy()
    hist = np.zeros((m, NQKV, 4))
    live = s >= 0
    hist[live] = np64(pool0)[s[live]]
    y_ref, z_ref, b_ref, a_ref, st_ref = proj.in_proj_decode(
        np64(x), *(np64(w) for w in ws), np64(cw), hist, None if cb is None else np64(cb))
    assert bf16_close(y, y_ref)
    for got, ref in ((z, z_ref), (b, b_ref), (a, a_ref)):
        assert bf16_close(got, ref)
    new = np64(pool)
    assert np.array_equal(new[s[live]][:, :, :3], st_ref[live][:, :, :3])
    assert tap_close(new[s[live]][:, :, 3], st_ref[live][:, :, 3], x[torch.from_numpy(live).to(DEV)], ws[0])
    untouched = np.setdiff1d(np.arange(rows), s[live])
    assert torch.equal(pool[untouched], pool0[untouched])


@pytest.mark.parametrize("m,k,ids", [(1, 2048, True), (2, 2048, True), (2, 2048, False), (1, 1024, False),
                                     (2, 1024, True)])
def test_small_batches_gemv_path(m, k, ids):
    """One or two rows take the GEMV kernel: against the oracle (a padding id
    for two rows with ids), narrow b / a at K = 1024; its graph replays are
    bit-identical to eager calls."""
    print(f"in_proj_decode gemv case M={m} K={k} ids={ids}", flush=True)
    gen = torch.Generator().manual_seed(101 + m + k)
    n = (NQKV, NZ, NB, NA) if k == 2048 else (1024, 512, 4, 8)
    ws, cw, cb = weights(gen, k=k, n=n, bias=ids)
    rows = 16
    pool = torch.randn(rows, n[0], 4, generator=gen).to(torch.bfloat16).to(DEV)
    slots = torch.randperm(rows, generator=gen)[:m] if ids else torch.arange(m)
    if ids and m == 2:
        slots[1] = -1
    x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(DEV)
    pool0 = pool.clone()
    y, z, b, a = run_fused(x, ws, cw, cb, pool, slots.to(DEV) if ids else None)
    s = slots.numpy()
    live = s >= 0
    hist = np.zeros((m, n[0], 4))
    hist[live] = np64(pool0)[s[live]]
    y_ref, z_ref, b_ref, a_ref, st_ref = proj.in_proj_decode(
        np64(x), *(np64(w) for w in ws), np64(cw), hist, None if cb is None else np64(cb))
    for got, ref in ((y, y_ref), (z, z_ref), (b, b_ref), (a, a_ref)):
        assert bf16_close(got, ref)
    new = np64(pool)
    assert np.array_equal(new[s[live]][:, :, :3], st_ref[live][:, :, :3])
    assert tap_close(new[s[live]][:, :, 3], st_ref[live][:, :, 3], x[torch.from_numpy(live).to(DEV)], ws[0])
    untouched = np.setdiff1d(np.arange(rows), s[live])
    assert torch.equal(pool[untouched], pool0[untouched])
    # graph replay of the same call
    pool.copy_(pool0)
    eager = run_fused(x, ws, cw, cb, pool, slots.to(DEV) if ids else None)
    after = pool.clone()
    pool.copy_(pool0)
    sl = slots.to(DEV) if ids else None
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run_fused(x, ws, cw, cb, pool, sl)
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(graph):
        outs = run_fused(x, ws, cw, cb, pool, sl)
    pool.copy_(pool0)
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    for got, ref in zip(outs, eager):
        assert torch.equal(got, ref)
    assert torch.equal(pool, after)


def test_matches_the_unfused_gpu_path():
    """Four hipBLASLt projections (torch F.linear) then the conv update kernel."""
    import torch.nn.functional as F
    from engine.kernels import causal_conv1d_update
    gen = torch.Generator().manual_seed(81)
    ws, cw, cb = weights(gen)
    pool = torch.randn(96, NQKV, 4, generator=gen).to(torch.bfloat16).to(DEV)
    slots = torch.randperm(96, generator=gen)[:64].to(DEV)
    x = torch.randn(64, K, generator=gen).to(torch.bfloat16).to(DEV)
    pool_ref = pool.clone()
    y, z, b, a = run_fused(x, ws, cw, cb, pool, slots)
    qkv, z2, b2, a2 = (F.linear(x, w) for w in ws)
    y2 = causal_conv1d_update(qkv[:, :, None], pool_ref, cw, None, "silu", conv_state_indices=slots)[:, :, 0]
    for got, ref in ((y, y2), (z, z2), (b, b2), (a, a2)):
        assert bf16_close(got, np64(ref))
    assert torch.equal(pool[:, :, :3], pool_ref[:, :, :3])
    sl = slots.cpu()
    assert tap_close(np64(pool[sl, :, 3]), np64(pool_ref[sl, :, 3]), x, ws[0])
    others = np.setdiff1d(np.arange(96), sl.numpy())
    assert torch.equal(pool[others], pool_ref[others])


def test_rows_without_ids_use_row_m_and_small_shapes():
    """NULL ids (HF's per-batch cache [B, C, 4]) and small shapes: K = 1024
    (one round per quarter), b / a narrower than a wave's 16 columns."""
    gen = torch.Generator().manual_seed(82)
    n = (1024, 512, 4, 8)
    ws, cw, cb = weights(gen, k=1024, n=n)
    pool = torch.randn(3, n[0], 4, generator=gen).to(torch.bfloat16).to(DEV)
    x = torch.randn(3, 1024, generator=gen).to(torch.bfloat16).to(DEV)
    pool0 = pool.clone()
    y, z, b, a = run_fused(x, ws, cw, cb, pool, None)
    y_ref, z_ref, b_ref, a_ref, st_ref = proj.in_proj_decode(np64(x), *(np64(w) for w in ws), np64(cw), np64(pool0))
    assert b.shape == (3, 4) and a.shape == (3, 8)
    for got, ref in ((y, y_ref), (z, z_ref), (b, b_ref), (a, a_ref)):
        assert bf16_close(got, ref)
    assert np.array_equal(np64(pool)[:, :, :3], st_ref[:, :, :3])


def test_graph_replays_match_eager():
    gen = torch.Generator().manual_seed(83)
    ws, cw, cb = weights(gen)
    pool = torch.randn(80, NQKV, 4, generator=gen).to(torch.bfloat16).to(DEV)
    slots = torch.randperm(80, generator=gen)[:48].to(DEV)
    static_x = torch.zeros(48, K, dtype=torch.bfloat16, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    p0 = pool.clone()
    with torch.cuda.stream(side):
        run_fused(static_x, ws, cw, cb, pool, slots)  # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    pool.copy_(p0)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = run_fused(static_x, ws, cw, cb, pool, slots)
    pool.copy_(p0)
    for step in range(3):
        x = torch.randn(48, K, generator=gen).to(torch.bfloat16).to(DEV)
        before = pool.clone()
        eager = run_fused(x, ws, cw, cb, pool, slots)
        after = pool.clone()
        pool.copy_(before)
        torch.cuda.synchronize()
        static_x.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        for got, ref in zip(outs, eager):
            assert torch.equal(got, ref), step
        assert torch.equal(pool, after), step


def _count_calls(monkeypatch):
    from engine.kernels import gdn_layer
    calls, out_calls = [], []
    real = gdn_layer.gdn_in_proj_decode
    monkeypatch.setattr(gdn_layer, "gdn_in_proj_decode", lambda *a, **k: calls.append(1) or real(*a, **k))
    real_out = gdn_layer.gdn_out_proj_decode
    monkeypatch.setattr(gdn_layer, "gdn_out_proj_decode", lambda *a, **k: out_calls.append(1) or real_out(*a, **k))
    return calls, out_calls


def _layer_on_pools(name, slots, n_pre, n_dec, num_slots, state_heads, monkeypatch):
    """Sequences prefilled one at a time into their slots, then batched decode
    steps that take the fused input side, against HF's module run per
    sequence with its own cache (fixture, tests/golden/make_golden.py)."""
    from engine.kernels import gated_delta_net_forward
    from engine.runtime import GDNSlotPools
    golden = lc.load_golden()
    cfg, layer = lc.gpu_layer(name, golden)
    calls, out_calls = _count_calls(monkeypatch)
    hv = cfg.linear_num_value_heads
    conv_dim = 2 * cfg.linear_num_key_heads * 128 + hv * 128
    pools = GDNSlotPools.allocate([0], num_slots, conv_dim=conv_dim, num_v_heads=hv, device=torch.device(DEV))
    cache = types.SimpleNamespace(gdn_slot_pools=pools)
    for i in range(n_pre):
        print(f"{name}: prefill {i} into slot {slots[i]}", flush=True)
        pools.bind(torch.tensor([slots[i]]), is_prefill=True)
        with torch.no_grad():
            y = gated_delta_net_forward(layer, torch.from_numpy(golden[f"{name}.pre{i}.x"]).to(DEV, torch.bfloat16),
                                        cache_params=cache)
        assert lc.layer_close(y, golden[f"{name}.pre{i}.y"]), i
    assert not calls
    for step in range(n_dec):
        pools.bind(torch.tensor(slots), is_prefill=False)
        with torch.no_grad():
            y = gated_delta_net_forward(layer, torch.from_numpy(golden[f"{name}.dec{step}.x"]).to(DEV, torch.bfloat16),
                                        cache_params=cache)
        assert lc.layer_close(y, golden[f"{name}.dec{step}.y"]), step
    assert len(calls) == n_dec and len(out_calls) == n_dec
    conv_pool, rec_pool = pools.layer(0)
    for i, s in enumerate(slots):
        assert lc.state_close(rec_pool[s], golden[f"{name}.seq{i}.state"], state_heads), i
        assert lc.conv_close(conv_pool[s], golden[f"{name}.seq{i}.conv"]), i


def test_layer_decode_takes_the_fused_kernel_and_matches_hf(monkeypatch):
    """A 1024-wide GDN layer (the fused kernel's smallest K): three sequences
    prefilled through the slot pools, then decode steps."""
    _layer_on_pools("w1024", [4, 1, 2], 3, 3, 6, [0, 3], monkeypatch)


def test_layer_decode_at_model_shapes_takes_the_fused_kernel(monkeypatch):
    """The Qwen3.5-MoE GDN layer (hidden 2048, 16 k-heads, 32 v-heads): two
    sequences prefilled into slots, then batched decode steps."""
    _layer_on_pools("model", [2, 0], 2, 2, 4, lc.MODEL_STATE_HEADS, monkeypatch)


def run_out(x, w):
    from engine.kernels.in_proj import gdn_out_proj_decode
    return gdn_out_proj_decode(x, w)


@pytest.mark.parametrize("m,k,n", [(64, 4096, 2048), (1, 4096, 2048), (5, 4096, 2048), (100, 4096, 2048),
                                   (256, 4096, 2048), (3, 2048, 1024), (40, 1024, 192), (7, 512, 64),
                                   (9, 1536, 128), (6, 3072, 256), (70, 8192, 128),
                                   (1, 2048, 1024), (1, 512, 64), (1, 1536, 128)])
def test_out_proj_matches_oracle(m, k, n):
    """Against the exact sum: one bf16 ulp plus the fp32 summation error (one
    row with K / 512 in {1, 2, 4, 8} takes the GEMV kernel, the rest the
    split-K pair)."""
    print(f"out_proj_decode oracle case M={m} K={k} N={n}", flush=True)
    gen = torch.Generator().manual_seed(90 + m + n)
    x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(DEV)
    w = (0.02 * torch.randn(n, k, generator=gen)).to(torch.bfloat16).to(DEV)
    y = run_out(x, w)
    assert y.shape == (m, n) and y.dtype == torch.bfloat16
    ref = proj.out_proj(np64(x), np64(w))
    assert bf16_close(y, ref)
    assert tap_close(np64(y), ref, x, w)


def test_out_proj_matches_hipblaslt_and_is_deterministic():
    """torch F.linear (hipBLASLt) to the bf16 bound; repeated calls, also
    after calls of other shapes on the same workspace, give the same bits;
    a strided x view gives the same bits as its contiguous copy."""
    import torch.nn.functional as F
    gen = torch.Generator().manual_seed(91)
    x = torch.randn(64, 4096, generator=gen).to(torch.bfloat16).to(DEV)
    w = (0.02 * torch.randn(2048, 4096, generator=gen)).to(torch.bfloat16).to(DEV)
    y = run_out(x, w)
    assert bf16_close(y, np64(F.linear(x, w)))
    run_out(x[:5], w)
    run_out(torch.randn(300, 4096, generator=gen).to(torch.bfloat16).to(DEV), w)
    assert torch.equal(run_out(x, w), y)
    wide = torch.zeros(64, 4160, dtype=torch.bfloat16, device=DEV)
    wide[:, :4096] = x
    assert torch.equal(run_out(wide[:, :4096], w), y)
    assert torch.equal(run_out(x[:, None], w)[:, 0], y)


def test_out_proj_graph_replays_match_eager():
    gen = torch.Generator().manual_seed(92)
    w = (0.02 * torch.randn(2048, 4096, generator=gen)).to(torch.bfloat16).to(DEV)
    static_x = torch.zeros(48, 4096, dtype=torch.bfloat16, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run_out(static_x, w)  # warm-up (and the workspace) outside the capture
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = run_out(static_x, w)
    for step in range(3):
        x = torch.randn(48, 4096, generator=gen).to(torch.bfloat16).to(DEV)
        eager = run_out(x, w)
        torch.cuda.synchronize()
        static_x.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), step
