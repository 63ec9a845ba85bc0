"""Benchmark of the Gated DeltaNet hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-prefill]

Headline (``value``): decode throughput of one GDN layer at batch 64
(configuration 1), tokens/s: one step = one ``fused_recurrent_gated_delta_rule``
launch over 64 sequences that updates the fp32 slot pool in place.  Inputs
are resident in HBM before timing.  Steps rotate over 4 disjoint 256 MiB
state pools (1 GiB), so no step's state can be served by the 256 MB
Infinity Cache from an earlier step.  ``value`` is the rate of plain
(eager) launches on the stream, host launch path included; the rate of the
same steps replayed from a HIP graph (one step on each pool) is reported
beside it.

The JSON line also carries
  roofline      decode kernel: algorithmic bytes per launch / mean kernel time
                (K back-to-back launches between two HIP events on the launch
                stream) against the 8 TB/s HBM peak;
  prefill       chunk-64 prefill at T=4096 (configuration 2): tok/s and the
                dense-equivalent flop rate against the 2.5 PFLOP/s bf16 peak
                (q/k at 16 heads; prefill_qk_repeated: q/k repeated to 32 heads
                as HF passes them); prefill_b16_t1038 (and _qk_repeated): the
                reference's own profiled shape, 16 sequences of 1038 tokens;
  layer_glue    the GDN layer glue around the prefill core at configuration 2's
                shape: HF's torch glue (gates, q/k repeat, RMSNormGated) vs
                the fused kernels, and the gated-norm kernel's HBM rate;
  decode_in_proj a decode step's input side at B=64 (row f-4): the four GDN
                input projections and the conv window update as one kernel
                (gdn_in_proj_decode) vs hipBLASLt projections + the conv
                update kernel, both replayed from HIP graphs over 6 weight
                sets (304 MB, past the Infinity Cache), with the fused
                kernel's HBM rate;
  layer_decode  one whole GDN layer decode step at B=64 (rows f-2, f-4 and the
                core together): ``gated_delta_net_forward`` on engine slot
                pools, four layers with their own weights and 256 MiB state
                pools replayed from one HIP graph; the same with the unfused
                input side; and the reference cache's per-step gather + scatter
                of the same slots, which the pools remove;
  cpu_baseline  the CPU oracle (numpy fp32, sequences split over the host's
                cores) on a bounded sample of the same decode workload.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "paris-hackathon-2026-inference_amd"))

HBM_PEAK = 8.0e12           # B/s, MI355X HBM3E (vendor figure)
MFMA_BF16_PEAK = 2.5e15     # dense flop/s
# bytes per decode launch at B=64: state read + write 268,435,456; q, k (16 heads) 524,288;
# v 524,288; o 524,288; g, beta 16,384; slot ids 256
DECODE_BYTES = 270_024_960
# HBM bytes per decode launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE, each scaled by
# the same counter on a plain 128 MiB copy (profiles/gdn_decode_b64_hbm_traffic_pmc.md)
DECODE_TRAFFIC_MEASURED = 274_600_550
# dense-equivalent flops per (chunk, head): 2C^2(3K+2V) + 6CKV + (2/3)C^3, C=64, K=V=128
PREFILL_FLOP_PER_CHUNK_HEAD = 11_709_099


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill measurements")
    ap.add_argument("--no-prefill-repeated", action="store_true",
                    help="skip the prefill timing with q/k repeated to 32 heads")
    ap.add_argument("--no-layer-glue", action="store_true",
                    help="skip the fused vs torch layer-glue timing (gates, q/k repeat, gated norm)")
    ap.add_argument("--no-conv", action="store_true", help="skip the prefill conv measurement")
    ap.add_argument("--no-in-proj", action="store_true", help="skip the decode projection measurements")
    ap.add_argument("--no-layer-decode", action="store_true", help="skip the whole-layer decode measurement")
    ap.add_argument("--pools", type=int, default=4, help="rotating decode state pools")
    ap.add_argument("--prefill-only", action="store_true",
                    help="time only the configuration 2 prefill and the B=16 x T=1038 batch (for counter "
                         "profiles; prints no headline value)")
    ap.add_argument("--layer-only", action="store_true",
                    help="time only the decode projections and the whole-layer decode steps (for counter "
                         "profiles; prints no headline value)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run the HBM ceiling probes: a plain 128 MiB device copy (also the "
                         "rocprofv3 FETCH_SIZE/WRITE_SIZE calibration), the same bytes in place, and a "
                         "1 GiB read-only stream")
    return ap.parse_args()


def copy_probe(torch, reps=20):
    """The box's HBM streaming ceilings for the decode kernel's traffic.

    * copy: a plain device-to-device copy of 128 MiB each way (torch ``copy_``, run by ROCm
      as ``__amd_rocclr_copyBuffer``), the 268 MB one B=64 decode step moves; its traffic
      counters also calibrate the decode kernel's FETCH_SIZE / WRITE_SIZE;
    * in place: the same 128 MiB read and written back in place (torch ``mul_``), the
      decode kernel's own pattern (it updates the slot pool in place);
    * read-only: a row-wise sum over 1 GiB of fp32 (rows of 4,096).
    Each rotates over 4 buffers, so that no call reads what the previous one left in the
    Infinity Cache; times are per call, from events around all calls (the rocprofv3 kernel
    trace of the same run gives the kernels alone)."""
    n = (128 << 20) // 4
    src = [torch.randn(n, device="cuda") for _ in range(4)]
    dst = [torch.empty(n, device="cuda") for _ in range(4)]
    big = [torch.randn((1 << 30) // 4, device="cuda") for _ in range(2)]
    rows = torch.empty((1 << 30) // 4 // 4096, device="cuda")

    def timed(fn, count):
        fn(0)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(count):
            fn(i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / count

    t_copy = timed(lambda i: dst[i % 4].copy_(src[(i + 1) % 4]), reps)
    t_inpl = timed(lambda i: src[i % 4].mul_(1.0000001), reps)
    t_read = timed(lambda i: torch.sum(big[i % 2].view(-1, 4096), dim=1, out=rows), max(4, reps // 2))
    mb = 2 * (128 << 20)
    print(json.dumps({"copy_probe_bytes_each_way": 128 << 20, "reps": reps,
                      "copy_us": t_copy * 1e6, "copy_tb_per_s": mb / t_copy / 1e12,
                      "inplace_us": t_inpl * 1e6, "inplace_tb_per_s": mb / t_inpl / 1e12,
                      "read_stream_bytes": 1 << 30, "read_us": t_read * 1e6,
                      "read_tb_per_s": (1 << 30) / t_read / 1e12}), flush=True)


def bench_decode(torch, steps, warmup, n_pools):
    from engine import configs
    from engine.kernels import fused_recurrent_gated_delta_rule

    c = configs.config1()
    dev = torch.device("cuda", 0)
    q, k, v, g, beta = (c[x].to(dev) for x in ("q", "k", "v", "g", "beta"))
    slots = c["slots"].to(dev)
    pools = [c["pool"].to(dev)]
    for _ in range(1, n_pools):
        pools.append(torch.randn_like(pools[0]).mul_(0.1))
    b = q.shape[0]

    def step(i):
        return fused_recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=pools[i % n_pools],
                                                ssm_state_indices=slots, inplace_final_state=True,
                                                use_qk_l2norm_in_kernel=True)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()

    # kernel time: K back-to-back eager launches between two events on the launch stream
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    kernel_s = e0.elapsed_time(e1) * 1e-3 / steps

    # eager whole-job rate (host launch path included)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    torch.cuda.synchronize()
    eager_wall = time.perf_counter() - t0

    # graph replay: one graph holding one step on each pool, replayed steps / n_pools times
    try:
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            for i in range(n_pools):
                step(i)
        stream.wait_stream(side)
        torch.cuda.synchronize()
        gph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gph):
            for i in range(n_pools):
                step(i)
        for _ in range(max(1, warmup // n_pools)):
            gph.replay()
        torch.cuda.synchronize()
        reps = max(1, steps // n_pools)
        t0 = time.perf_counter()
        for _ in range(reps):
            gph.replay()
        torch.cuda.synchronize()
        graph_wall = (time.perf_counter() - t0) * steps / (reps * n_pools)
    except RuntimeError as e:  # capture unavailable: fall back to the eager figure
        print(f"bench.py: graph capture failed ({e}); reporting eager launches", file=sys.stderr)
        graph_wall = None
    return dict(tokens=b, steps=steps, kernel_s=kernel_s, eager_wall=eager_wall, graph_wall=graph_wall)


def bench_decode_batches(torch, batches=(1, 4, 16, 64), reps=100):
    """The decode step of configuration 1 at smaller batches (the first B
    rows of its inputs and slots; pool of 128 slots, 4 pools rotating so that
    the touched states come from HBM): time per step from a HIP graph of 20
    steps (below B = 64 an eager step is bound by the host's launch path,
    about 20 us, not by the GPU), also eager, and the HBM fraction of the
    state bytes (2 x B x 2 MiB read + written)."""
    from engine import configs
    from engine.kernels import fused_recurrent_gated_delta_rule

    c = configs.config1()
    dev = torch.device("cuda", 0)
    q, k, v, g, beta = (c[x].to(dev) for x in ("q", "k", "v", "g", "beta"))
    slots = c["slots"].to(dev)
    pools = [c["pool"].to(dev)] + [torch.randn_like(c["pool"]).to(dev).mul_(0.1) for _ in range(3)]
    out = {}
    for b in batches:
        i = [0]

        def step():
            i[0] += 1
            return fused_recurrent_gated_delta_rule(q[:b], k[:b], v[:b], g[:b], beta[:b],
                                                    initial_state=pools[i[0] % 4], ssm_state_indices=slots[:b],
                                                    inplace_final_state=True, use_qk_l2norm_in_kernel=True)

        t_eager = _time(torch, step, reps)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        gph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gph):
            for _ in range(20):
                step()
        t = _time(torch, gph.replay, reps) / 20
        byts = 2 * b * 32 * 128 * 128 * 4
        out[f"B{b}"] = {"us": t * 1e6, "tok_per_s": b / t, "frac": byts / t / HBM_PEAK, "eager_us": t_eager * 1e6}
    return out


def bench_prefill(torch, reps=120, warmup=3, repeat_qk=False, n_sets=3):
    """Configuration 2.  With repeat_qk, q and k arrive repeated to the 32 v-heads
    (HF's repeat_interleave before the call), the layout the reference's boundary
    actually receives; otherwise they keep their 16 heads (native GQA).  Calls
    rotate over ``n_sets`` input sets (about 100 MB each), so that the inputs of
    a call were last touched ``n_sets`` calls earlier and the 256 MB Infinity
    Cache does not serve them from the previous call."""
    from engine import configs
    from engine.kernels import chunk_gated_delta_rule

    dev = torch.device("cuda", 0)
    sets = []
    for i in range(n_sets):  # configuration 2's generator with one seed per set
        c = configs.config2(seed=2 + 1000 * i)
        q, k, v, g, beta = (c[x].to(dev) for x in ("q", "k", "v", "g", "beta"))
        if repeat_qk:
            rep = v.shape[2] // q.shape[2]
            q, k = q.repeat_interleave(rep, dim=2), k.repeat_interleave(rep, dim=2)
        sets.append((q, k, v, g, beta))
    t = sets[0][0].shape[1]

    def run(i):
        return chunk_gated_delta_rule(*sets[i % n_sets], output_final_state=True, use_qk_l2norm_in_kernel=True)

    i = [0]

    def call():
        run(i[0])
        i[0] += 1

    per = _time(torch, call, reps, warmup)
    flop = PREFILL_FLOP_PER_CHUNK_HEAD * ((t + 63) // 64) * 32
    set_mb = sum(x.numel() * x.element_size() for x in sets[0]) / 1e6
    return {"config": f"prefill B=1 T=4096 Hk={sets[0][0].shape[2]} Hv=32 d=128 bf16, chunk 64, zero h0, "
                      f"final state out; {n_sets} input sets of {set_mb:.0f} MB rotated call by call",
            "tok_per_s": t / per, "ms": per * 1e3, "reps": reps, "timing": "median of per-call events",
            "mfma": {"achieved": flop / per / 1e12, "peak": MFMA_BF16_PEAK / 1e12, "unit": "TFLOP/s",
                     "frac": flop / per / MFMA_BF16_PEAK, "flop_per_call": flop}}


def bench_prefill_non_bf16(torch, dtype, reps=5):
    """Configuration 2 (B=1, T=4096) with q/k/v given in fp32 or fp16 instead
    of bf16: the chunk entry then runs the token recurrence in fp32 on the
    inputs as given (the MFMA chunk path takes bf16 operands only).  Few
    reps: one call is milliseconds."""
    from engine import configs
    from engine.kernels import chunk_gated_delta_rule

    dev = torch.device("cuda", 0)
    c = configs.config2(seed=2)
    q, k, v = (c[x].to(dev, dtype) for x in ("q", "k", "v"))
    g, beta = c["g"].to(dev), c["beta"].to(dev)
    t = q.shape[1]

    def run():
        return chunk_gated_delta_rule(q, k, v, g, beta, output_final_state=True, use_qk_l2norm_in_kernel=True)

    per = _time(torch, run, reps, warmup=1)
    return {"config": f"prefill B=1 T={t} Hk=16 Hv=32 d=128, q/k/v {str(dtype).replace('torch.', '')}, "
                      "zero h0, final state out (token recurrence)",
            "ms": per * 1e3, "tok_per_s": t / per, "reps": reps}


def bench_prefill_b16(torch, reps=100, repeat_qk=False):
    """The reference's own profiled prefill shape (its profile of fla's chunk
    kernel: 1.659 ms per layer on H200): a dense batch of 16 sequences of 1038
    tokens (17 chunks each), q/k at 16 heads (with repeat_qk: repeated to the
    32 v-heads, as HF passes them), v at 32, zero h0, final states out; the
    batch is scanned by the persistent scan."""
    from engine import configs
    from engine.kernels import chunk_gated_delta_rule

    dev = torch.device("cuda", 0)
    b, t = 16, 1038
    c = configs.config2(seed=47, t=b * t)
    q, k, v, g, beta = (c[x].to(dev).reshape(b, t, *c[x].shape[2:]) for x in ("q", "k", "v", "g", "beta"))
    if repeat_qk:
        q, k = q.repeat_interleave(2, dim=2), k.repeat_interleave(2, dim=2)

    def run():
        return chunk_gated_delta_rule(q, k, v, g, beta, output_final_state=True, use_qk_l2norm_in_kernel=True)

    per = _time(torch, run, reps)
    flop = PREFILL_FLOP_PER_CHUNK_HEAD * b * ((t + 63) // 64) * 32
    return {"config": f"B=16 x T=1038 (17 chunks each), Hk={q.shape[2]} Hv=32 d=128 bf16, zero h0, final states out",
            "us": per * 1e6, "tok_per_s": b * t / per,
            "mfma": {"achieved": flop / per / 1e12, "peak": MFMA_BF16_PEAK / 1e12, "unit": "TFLOP/s",
                     "frac": flop / per / MFMA_BF16_PEAK, "flop": flop},
            "reference_h200_us": 1659.0}


def bench_varlen(torch, reps=100):
    """Configuration 3: 16 packed sequences (lengths U{128..2048}, seeded) as
    HF's layer runs them after the input projections: the causal conv + SiLU
    over the packed [sum L, 8192] projection with cu_seqlens (windows from
    zero), q|k|v as strided views of its output, then the chunk prefill with
    cu_seqlens, per-sequence initial states [16, 32, 128, 128] and final
    states out.  Algorithmic units as configurations 2 and the conv."""
    from engine import configs
    from engine.kernels import causal_conv1d_fn, chunk_gated_delta_rule

    c = configs.config3()
    dev = torch.device("cuda", 0)
    cu = c["cu_seqlens"].to(dev)
    x, w, g, beta, h0 = (c[k].to(dev) for k in ("x", "conv_w", "g", "beta", "h0"))
    lens = (c["cu_seqlens"][1:] - c["cu_seqlens"][:-1]).tolist()
    total = int(sum(lens))
    conv_out = [None]

    def conv():
        conv_out[0] = causal_conv1d_fn(x, w, None, activation="silu", cu_seqlens=cu)
        return conv_out[0]

    def gdn():
        q, k, v = configs.split_qkv(conv_out[0])
        return chunk_gated_delta_rule(q, k, v, g, beta, initial_state=h0, output_final_state=True,
                                      use_qk_l2norm_in_kernel=True, cu_seqlens=cu)

    conv()
    t_conv = _time(torch, conv, reps)
    t_gdn = _time(torch, gdn, reps)
    t_all = _time(torch, lambda: (conv(), gdn()), reps)
    flop = PREFILL_FLOP_PER_CHUNK_HEAD * 32 * sum((n + 63) // 64 for n in lens)
    conv_bytes = total * 8192 * 2 * 2
    gdn_bytes = total * (16 * 128 * 2 * 2 + 32 * 128 * 2 * 2 + 32 * 4 * 2) + 2 * 16 * 2 * 2 ** 20
    return {"config": f"configuration 3: 16 sequences, sum L = {total}, conv (8192 channels, SiLU) + chunk "
                      "prefill with cu_seqlens, h0 in, final states out",
            "tok_per_s": total / t_all, "us": t_all * 1e6, "conv_us": t_conv * 1e6, "gdn_us": t_gdn * 1e6,
            "gdn_mfma": {"achieved": flop / t_gdn / 1e12, "peak": MFMA_BF16_PEAK / 1e12, "unit": "TFLOP/s",
                         "frac": flop / t_gdn / MFMA_BF16_PEAK, "flop": flop},
            "conv_hbm": {"achieved": conv_bytes / t_conv / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                         "frac": conv_bytes / t_conv / HBM_PEAK, "bytes": conv_bytes},
            "gdn_bytes": gdn_bytes}


def bench_spec_verify(torch, reps=100):
    """Configuration 4: a speculative verify step of B=32 sequences x T=4
    tokens on a 64-slot fp32 pool (the recurrence reading each slot's state
    and writing all four per-token states as snapshots, the pool untouched),
    then the commit of each sequence's accepted snapshot into its slot.
    Algorithmic bytes: states read 64 MiB + snapshots written 256 MiB +
    commit 64 MiB read + 64 MiB written = 469,762,048 B (+ q, k, v, o)."""
    from engine import configs
    from engine.kernels import fused_recurrent_gated_delta_rule, gdn_state_commit

    c = configs.config4()
    dev = torch.device("cuda", 0)
    q, k, v, g, beta = (c[x].to(dev) for x in ("q", "k", "v", "g", "beta"))
    pool, slots, acc = c["pool"].to(dev), c["slots"].to(dev), c["accepted"].to(dev)
    b, t = q.shape[:2]
    snaps = torch.empty(b, t, 32, 128, 128, device=dev)

    def verify():
        return fused_recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=pool, ssm_state_indices=slots,
                                                snapshots=snaps, use_qk_l2norm_in_kernel=True)

    def commit():
        return gdn_state_commit(pool, slots, snaps, acc)

    verify()
    t_v, t_c = _time(torch, verify, reps), _time(torch, commit, reps)
    state = 32 * 128 * 128 * 4
    v_bytes, c_bytes = b * state + b * t * state, 2 * b * state
    return {"config": "configuration 4: B=32, T=4 verify on a 64-slot fp32 pool, snapshots [32, 4, 32, 128, 128], "
                      "accepted lengths U{1..4}, commit",
            "verify_us": t_v * 1e6, "commit_us": t_c * 1e6, "tok_per_s": b * t / (t_v + t_c),
            "verify_hbm": {"achieved": v_bytes / t_v / 1e9, "frac": v_bytes / t_v / HBM_PEAK, "bytes": v_bytes},
            "commit_hbm": {"achieved": c_bytes / t_c / 1e9, "frac": c_bytes / t_c / HBM_PEAK, "bytes": c_bytes},
            "total_bytes": v_bytes + c_bytes, "peak_GBps": HBM_PEAK / 1e9}


def _time(torch, fn, reps, warmup=3):
    """Median, over ``reps`` calls, of the time between two events recorded
    on the current stream just before and just after each call (seconds).
    A call that the host launches more slowly than the GPU runs it (a small
    eager step) is timed with its launch gap, as the caller would see it."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for e0, e1 in ev:
        e0.record(stream)
        fn()
        e1.record(stream)
    torch.cuda.synchronize()
    return statistics.median(e0.elapsed_time(e1) for e0, e1 in ev) * 1e-3


def bench_conv_prefill(torch, reps=100):
    """Row a-6's prefill conv (``causal_conv1d_fn`` + SiLU, width 4) over the
    qkv projection rows as the layer feeds it (token-major [T, 8192] bf16,
    transformers modeling_qwen3_5_moe.py:443-444, 468-474), for one 4096-token and one 16384-token
    sequence.  Algorithmic bytes: x read once and y written once, 2 x 2 B per
    (token, channel); the 3-token halo each 64-token tile re-reads adds ~2%."""
    from engine import configs
    from engine.kernels import causal_conv1d_fn

    dev = torch.device("cuda", 0)
    gen = torch.Generator().manual_seed(43)
    c = configs.CONV_DIM
    w = torch.randn(c, 4, generator=gen).to(dev, torch.bfloat16)
    out = {"config": f"C={c}, width 4, SiLU, bf16, token-major input (one sequence)"}
    for t in (4096, 16384):
        xs = [torch.randn(1, t, c, generator=gen).to(dev, torch.bfloat16) for _ in range(2)]
        i = [0]

        def run():
            i[0] ^= 1
            return causal_conv1d_fn(xs[i[0]].transpose(1, 2), w, None, activation="silu")

        us = _time(torch, run, reps) * 1e6
        byts = 2 * t * c * 2
        out[f"T{t}"] = {"us": us, "achieved_GBps": byts / us / 1e3, "peak_GBps": HBM_PEAK / 1e9,
                        "frac": byts / us / 1e3 / (HBM_PEAK / 1e9), "bytes": byts}
        del xs
    return out


def bench_layer_glue(torch, reps=100):
    """Configuration 2's shape through the GDN layer glue (row f-1): the glue as
    HF's layer forward runs it in torch around the core (gates,
    modeling_qwen3_5_moe.py:495-497; q/k repeat_interleave, :498-500;
    RMSNormGated, :169-185 / :535-538) versus the fused path (gates in the
    chunk kernel's prologue, native 16-head q/k, one-pass norm kernel)."""
    import torch.nn.functional as F
    from engine import configs
    from engine.kernels import chunk_gated_delta_rule, chunk_gated_delta_rule_from_projections, rms_norm_gated

    c = configs.config2()
    dev = torch.device("cuda", 0)
    q, k, v = (c[x].to(dev) for x in ("q", "k", "v"))
    t, hv = v.shape[1], v.shape[2]
    gen = torch.Generator().manual_seed(41)
    a = torch.randn(1, t, hv, generator=gen).to(dev, torch.bfloat16)
    b = torch.randn(1, t, hv, generator=gen).to(dev, torch.bfloat16)
    A_log = torch.log(torch.empty(hv).uniform_(1, 16, generator=gen)).to(dev)
    dt_bias = torch.randn(hv, generator=gen).to(dev)
    z = torch.randn(1, t, hv, 128, generator=gen).to(dev, torch.bfloat16)
    w = (1 + 0.2 * torch.randn(128, generator=gen)).to(dev, torch.bfloat16)

    def torch_norm(x, gate):  # the module's steps (fp32 variance, weight in the input dtype, silu gate)
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
        return (w * xf.to(x.dtype) * F.silu(gate.float())).to(x.dtype)

    def glue_torch():
        beta = b.sigmoid()
        g = -A_log.float().exp() * F.softplus(a.float() + dt_bias)
        rep = hv // q.shape[2]
        o, s = chunk_gated_delta_rule(q.repeat_interleave(rep, dim=2), k.repeat_interleave(rep, dim=2), v, g, beta,
                                      output_final_state=True, use_qk_l2norm_in_kernel=True)
        return torch_norm(o.reshape(-1, 128), z.reshape(-1, 128)), s

    def glue_fused():
        o, s = chunk_gated_delta_rule_from_projections(q, k, v, a, b, A_log, dt_bias, output_final_state=True)
        return rms_norm_gated(o, z, w), s

    o_ref = glue_torch()[0].reshape(1, t, hv, 128).float()
    y = glue_fused()[0].float()
    dev_err = ((y - o_ref).abs().max() / o_ref.abs().max()).item()
    t_torch, t_fused = _time(torch, glue_torch, reps), _time(torch, glue_fused, reps)
    x0 = torch.randn(1, t, hv, 128, generator=gen).to(dev, torch.bfloat16)
    t_norm = _time(torch, lambda: rms_norm_gated(x0, z, w), 100)
    t_norm_torch = _time(torch, lambda: torch_norm(x0.reshape(-1, 128), z.reshape(-1, 128)), 100)
    norm_bytes = 3 * x0.numel() * 2  # x, z in, y out (bf16)
    return {"config": "configuration 2 shape (T=4096, Hk=16, Hv=32, d=128), bf16; a, b [T, 32] bf16, z [T, 32, 128]",
            "torch_glue_us": t_torch * 1e6, "fused_us": t_fused * 1e6, "speedup": t_torch / t_fused,
            "max_diff_vs_torch_glue_rel_to_max": dev_err,
            "rmsnorm_gated": {"us": t_norm * 1e6, "torch_us": t_norm_torch * 1e6,
                              "achieved_GBps": norm_bytes / t_norm / 1e9, "peak_GBps": HBM_PEAK / 1e9,
                              "frac": norm_bytes / t_norm / HBM_PEAK, "bytes": norm_bytes}}


def _median_time(fn, min_reps=5, budget_s=3.0):
    """Median wall time of fn() over >= min_reps runs (and about budget_s), after one warmup run."""
    fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < min_reps or time.perf_counter() - t_start < budget_s:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(budget_s=6.0):
    """CPU oracle (numpy fp32) on bounded samples of configurations 0-4, each
    split over the host cores this run may use, plus configuration 1 on one
    thread.  Threads: the cores in this process's affinity mask, capped at
    OMP_NUM_THREADS (the GPU box gives one GPU's job a 16-core share of its
    host and sets OMP_NUM_THREADS=16 accordingly).  Each figure is the median
    of timed runs after one warmup (time.perf_counter)."""
    import numpy as np
    from engine import configs
    from oracle import conv, gdn

    affinity = len(os.sched_getaffinity(0))
    n = max(1, min(affinity, int(os.environ.get("OMP_NUM_THREADS", affinity) or affinity)))
    ex = cf.ThreadPoolExecutor(n)
    out = {"cores": n, "affinity_cores": affinity, "cpu_model": _cpu_model(), "kind": "port",
           "unit": "tok/s"}

    def split(total, parts):
        parts = max(1, min(parts, total))
        return [slice(i * total // parts, (i + 1) * total // parts) for i in range(parts)]

    # configuration 1 (the headline): one decode step over 64 gathered slot states
    c = configs.config1()
    args = [c[x].float().numpy() for x in ("q", "k", "v", "g", "beta")]
    h0 = c["pool"].numpy()[c["slots"].numpy()]

    def run_part(sl):
        return gdn.recurrent_gated_delta_rule(*(a[sl] for a in args), initial_state=h0[sl], dtype=np.float32)

    per, reps = _median_time(lambda: list(ex.map(run_part, split(64, n))), budget_s=budget_s)
    per1, reps1 = _median_time(lambda: run_part(slice(0, 64)), budget_s=3.0)
    out.update({"value": 64 / per, "gb_per_s": DECODE_BYTES / per / 1e9,
                "sample": f"configuration 1 decode steps (B=64, one layer, 64 gathered slot states) with the numpy "
                          f"fp32 oracle, sequences split over {n} threads; median of {reps} steps after one warmup, "
                          f"{per * 1e3:.1f} ms/step",
                "one_thread": {"value": 64 / per1, "unit": "tok/s", "cores": 1,
                               "sample": f"the same step on one thread, median of {reps1}: {per1 * 1e3:.1f} ms/step"}})

    def by_heads(q, k, v, g, beta, fn, **kw):
        """Run fn over groups of whole k-heads (and their v-heads) in parallel."""
        hk, hv = q.shape[2], v.shape[2]
        grp = hv // hk

        def run(ks):
            vs = slice(ks.start * grp, ks.stop * grp)
            return fn(q[:, :, ks], k[:, :, ks], v[:, :, vs], g[:, :, vs], beta[:, :, vs], dtype=np.float32, **kw)
        return lambda: list(ex.map(run, split(hk, n)))

    # configuration 0: fp32 recurrence, B=1, T=256
    c0 = configs.config0()
    a0 = [c0[x].numpy() for x in ("q", "k", "v", "g", "beta")]
    per0, reps0 = _median_time(by_heads(*a0, gdn.recurrent_gated_delta_rule), min_reps=3, budget_s=3.0)
    t0 = a0[0].shape[1]
    out["config0"] = {"value": t0 / per0, "unit": "tok/s",
                      "sample": f"configuration 0 (fp32 recurrence, T={t0}, 32 v-heads), k-head groups over {n} "
                                f"threads; median of {reps0}, {per0 * 1e3:.1f} ms per run"}

    # configuration 2: chunk prefill, T=4096
    c2 = configs.config2()
    a2 = [c2[x].float().numpy() for x in ("q", "k", "v", "g", "beta")]
    per2, reps2 = _median_time(by_heads(*a2, gdn.chunk_gated_delta_rule), min_reps=3, budget_s=3.0)
    t2 = a2[0].shape[1]
    flop2 = PREFILL_FLOP_PER_CHUNK_HEAD * ((t2 + 63) // 64) * 32
    out["prefill"] = {"value": t2 / per2, "unit": "tok/s", "gflop_per_s": flop2 / per2 / 1e9,
                      "sample": f"configuration 2 (T={t2}, all 32 v-heads) through the numpy fp32 chunk oracle, "
                                f"k-head groups over {n} threads; median of {reps2} runs after one warmup, "
                                f"{per2:.2f} s per run"}

    # configuration 3 (bounded): the first 4 of its 16 sequences -- conv over the 8192-wide
    # projection, then the chunk rule with cu_seqlens and initial states
    c3 = configs.config3()
    cu = c3["cu_seqlens"].numpy()[:5]
    n3 = int(cu[-1])
    x3 = c3["x"][:n3].float().numpy()
    w3 = c3["conv_w"].float().numpy()
    g3, b3 = c3["g"][:, :n3].numpy(), c3["beta"][:, :n3].numpy()
    h03 = c3["h0"][:4].numpy()

    def run3():
        cparts = split(x3.shape[1], n)
        ys = list(ex.map(lambda sl: conv.causal_conv1d_varlen(x3[:, sl], w3[sl], cu, activation="silu",
                                                              dtype=np.float32)[0], cparts))
        y = np.concatenate(ys, axis=1)
        q = y[:, :2048].reshape(1, n3, 16, 128)
        k = y[:, 2048:4096].reshape(1, n3, 16, 128)
        v = y[:, 4096:].reshape(1, n3, 32, 128)

        def heads(ks):
            vs = slice(ks.start * 2, ks.stop * 2)
            return gdn.chunk_gated_delta_rule_varlen(q[:, :, ks], k[:, :, ks], v[:, :, vs], g3[:, :, vs],
                                                     b3[:, :, vs], cu, h03[:, vs], dtype=np.float32)
        return list(ex.map(heads, split(16, n)))

    per3, reps3 = _median_time(run3, min_reps=3, budget_s=4.0)
    out["config3"] = {"value": n3 / per3, "unit": "tok/s",
                      "sample": f"configuration 3's first 4 sequences ({n3} tokens): numpy fp32 conv (channel groups) "
                                f"then the chunk oracle with cu_seqlens and h0 (k-head groups), {n} threads; median "
                                f"of {reps3}, {per3:.2f} s per run"}

    # configuration 4: speculative verify, B=32, T=4, snapshots and commit
    c4 = configs.config4()
    a4 = [c4[x].float().numpy() for x in ("q", "k", "v", "g", "beta")]
    pool4, slots4, acc4 = c4["pool"].numpy(), c4["slots"].numpy(), c4["accepted"].numpy()

    def run4_part(sl):  # each part gets the pool rows of its own slots
        return gdn.spec_verify(pool4[slots4[sl]], np.arange(sl.stop - sl.start), *(a[sl] for a in a4), acc4[sl],
                               dtype=np.float32)

    per4, reps4 = _median_time(lambda: list(ex.map(run4_part, split(len(slots4), n))), min_reps=3, budget_s=3.0)
    b4, tt4 = a4[0].shape[0], a4[0].shape[1]
    out["config4"] = {"value": b4 * tt4 / per4, "unit": "verified tok/s",
                      "sample": f"configuration 4 (B={b4}, T={tt4}: snapshots and commit) with the numpy fp32 oracle, "
                                f"sequences over {n} threads; median of {reps4}, {per4 * 1e3:.1f} ms per step"}
    ex.shutdown()
    return out


def bench_in_proj(torch, sets=6, reps=100):
    """Row f-4 at the decode batch (64 rows, hidden 2048, Qwen3.5-MoE GDN
    shapes): the fused input-projection kernel against the unfused path HF's
    layer takes (four nn.Linear on hipBLASLt, then causal_conv1d_update on
    the slot pool).  Each path is captured once per weight set into one
    HIP graph; the graph is replayed ``reps`` times, each replay between two
    events, and the median replay is reported."""
    import torch.nn.functional as F
    from engine.kernels import causal_conv1d_update, gdn_in_proj_decode

    dev = torch.device("cuda", 0)
    m, k, n = 64, 2048, (8192, 4096, 32, 32)
    gen = torch.Generator().manual_seed(51)
    wsets = [[(0.02 * torch.randn(c, k, generator=gen)).to(dev, torch.bfloat16) for c in n] for _ in range(sets)]
    cw = (0.5 * torch.randn(n[0], 4, generator=gen)).to(dev, torch.bfloat16)
    pool = torch.randn(128, n[0], 4, generator=gen).to(dev, torch.bfloat16)
    slots = torch.randperm(128, generator=gen)[:m].to(dev)
    x = torch.randn(m, k, generator=gen).to(dev, torch.bfloat16)

    def fused(ws):
        return gdn_in_proj_decode(x, *ws, cw, None, pool, slots)

    def unfused(ws):
        qkv, z, b, a = (F.linear(x, w) for w in ws)
        return causal_conv1d_update(qkv[:, :, None], pool, cw, None, "silu", conv_state_indices=slots), z, b, a

    def graph_us(fn):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for ws in wsets:
                fn(ws)
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for ws in wsets:
                fn(ws)
        return _time(torch, g.replay, reps, warmup=2) / sets * 1e6

    t_fused, t_unfused = graph_us(fused), graph_us(unfused)
    t_eager = _time(torch, lambda: fused(wsets[0]), reps) * 1e6
    wbytes = sum(c for c in n) * k * 2
    byts = wbytes + m * k * 2 + m * sum(n) * 2 + 2 * m * n[0] * 8  # weights, x, outputs, windows read + written
    return {"config": "B=64 rows, hidden 2048 -> qkv 8192 (conv width 4, 128-slot bf16 pool) / z 4096 / b 32 / a 32, bf16",
            "fused_us": t_fused, "unfused_hipblaslt_us": t_unfused, "speedup": t_unfused / t_fused,
            "fused_eager_us": t_eager,
            "roofline": {"bound": "hbm", "achieved": byts / t_fused / 1e3, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                         "frac": byts / (t_fused * 1e-6) / HBM_PEAK, "bytes_per_launch": byts,
                         "kernel": "gdn::in_proj_xs_kernel<16, 4>"}}


def bench_out_proj(torch, sets=16, reps=100):
    """Row f-4's output side at the decode batch: ``out_proj`` (4096 -> 2048,
    bf16) for 64 rows, the split-K kernel pair against hipBLASLt (torch
    F.linear), each captured once per weight set into one HIP graph (16 sets:
    268 MB of weights, past the 256 MB Infinity Cache)."""
    import torch.nn.functional as F
    from engine.kernels import gdn_out_proj_decode

    dev = torch.device("cuda", 0)
    m, k, n = 64, 4096, 2048
    gen = torch.Generator().manual_seed(53)
    wsets = [(0.02 * torch.randn(n, k, generator=gen)).to(dev, torch.bfloat16) for _ in range(sets)]
    x = torch.randn(m, k, generator=gen).to(dev, torch.bfloat16)

    def graph_us(fn):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for w in wsets:
                fn(w)
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for w in wsets:
                fn(w)
        return _time(torch, g.replay, reps, warmup=2) / sets * 1e6

    t_ours = graph_us(lambda w: gdn_out_proj_decode(x, w))
    t_lt = graph_us(lambda w: F.linear(x, w))
    byts = n * k * 2 + m * k * 2 + m * n * 2  # weights, x, y
    return {"config": "B=64 rows, out_proj 4096 -> 2048, bf16",
            "us": t_ours, "hipblaslt_us": t_lt, "speedup": t_lt / t_ours,
            "roofline": {"bound": "hbm", "achieved": byts / t_ours / 1e3, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                         "frac": byts / (t_ours * 1e-6) / HBM_PEAK, "bytes_per_call": byts,
                         "kernels": "gdn::out_proj_partial_kernel (4 splits of 1024) + gdn::out_proj_sum_kernel<4> "
                                    "(2 MiB of fp32 partials written and read besides)"}}


def bench_layer_decode(torch, layers=4, reps=100, batch=64):
    """One GDN layer decode step at B=64 with Qwen3.5-MoE layer shapes (hidden
    2048, 16 k-heads, 32 v-heads of 128, conv width 4; random bf16 weights):
    HF's ``Qwen3_5MoeGatedDeltaNet`` with ``gated_delta_net_forward`` on
    engine slot pools (128 slots, 64 bound).  ``layers`` such layers, each
    with its own weights and pools (256 MiB recurrent pool each, so neither
    the weights nor the states stay in the 256 MB Infinity Cache), one step
    of each captured into one HIP graph; the graph is replayed ``reps``
    times.  Also: the same steps with the unfused input side (hipBLASLt
    projections + conv update kernel), with out_proj on hipBLASLt, and the
    gather + scatter the reference cache runs around every step for the same
    slots (``index_select`` of both pools before, ``index_copy_`` after,
    engine/runtime/kv_cache.py:189-208)."""
    import types
    from unittest import mock
    from transformers.models.qwen3_5_moe import modeling_qwen3_5_moe as hf
    from transformers.models.qwen3_5_moe.configuration_qwen3_5_moe import Qwen3_5MoeTextConfig
    from engine.kernels import gated_delta_net_forward, gdn_layer
    from engine.runtime import GDNSlotPools

    dev = torch.device("cuda", 0)
    cfg = Qwen3_5MoeTextConfig(hidden_size=2048, num_hidden_layers=layers, layer_types=["linear_attention"] * layers,
                               linear_num_key_heads=16, linear_num_value_heads=32, linear_key_head_dim=128,
                               linear_value_head_dim=128, linear_conv_kernel_dim=4, rms_norm_eps=1e-6)
    torch.manual_seed(61)
    mods = [hf.Qwen3_5MoeGatedDeltaNet(cfg, layer_idx=i).eval().to(dev, torch.bfloat16) for i in range(layers)]
    pools = GDNSlotPools.allocate(range(layers), 128, conv_dim=8192, num_v_heads=32, device=dev, max_batch=64)
    gen = torch.Generator().manual_seed(62)
    torch.cuda.manual_seed(62)
    for i in range(layers):
        conv, rec = pools.layer(i)
        rec.normal_(0.0, 0.1)
        conv.normal_(0.0, 1.0)
    slots = torch.randperm(128, generator=gen)[:batch]
    x = torch.randn(batch, 1, 2048, generator=gen).to(dev, torch.bfloat16)
    cache = types.SimpleNamespace(gdn_slot_pools=pools)
    pools.bind(slots, is_prefill=False)
    dslots = slots.to(dev)

    def steps():
        with torch.no_grad():
            for m in mods:
                gated_delta_net_forward(m, x, cache_params=cache)

    def gather_scatter():
        for i in range(layers):
            conv, rec = pools.layer(i)
            c, r = conv.index_select(0, dslots), rec.index_select(0, dslots)
            conv.index_copy_(0, dslots, c)
            rec.index_copy_(0, dslots, r)

    def graph_us(fn):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        return _time(torch, g.replay, reps, warmup=2) / layers * 1e6

    t_fused = graph_us(steps)
    with mock.patch.object(gdn_layer, "_fused_decode_fits", lambda *a, **k: False):
        t_unfused = graph_us(steps)
    with mock.patch.object(gdn_layer, "_out_proj_fits", lambda *a, **k: False):
        t_lt_out = graph_us(steps)
    t_gs = graph_us(gather_scatter)
    return {"config": f"one GDN layer decode step, B={batch} of 128 slots, hidden 2048, Hk=16 Hv=32 d=128, conv 4, "
                      "bf16 weights (random), fp32 state pools; 4 layers per graph, own weights and pools",
            "step_us": t_fused, "tok_per_s": batch / (t_fused * 1e-6),
            "step_unfused_input_us": t_unfused,
            "step_hipblaslt_out_proj_us": t_lt_out,
            "reference_cache_gather_scatter_us": t_gs,
            "note": "step = fused input side + recurrence on the pool + gated norm + split-K out_proj; "
                    "the reference runs its gather + scatter in addition to the layer step"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); the GDN path "
              "shards over sequences and heads with no exchange inside the path", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.copy_probe:
        copy_probe(torch)
        return
    if args.prefill_only:  # the prefill kernels alone (for counter profiles); no headline value
        print(json.dumps({"prefill": bench_prefill(torch), "prefill_b16_t1038": bench_prefill_b16(torch)}),
              flush=True)
        return
    if args.layer_only:  # the decode projections and layer steps alone (for counter profiles)
        print(json.dumps({"decode_in_proj": bench_in_proj(torch), "decode_out_proj": bench_out_proj(torch),
                          "layer_decode": bench_layer_decode(torch)}), flush=True)
        return
    d = bench_decode(torch, args.steps, args.warmup, args.pools)
    wall = d["eager_wall"]
    value = d["tokens"] * d["steps"] / wall
    achieved = DECODE_BYTES / d["kernel_s"]
    out = {
        "metric": "GDN decode tok/s @B=64 (HBM GB/s); prefill tok/s @T=4096 (MFMA %)",
        "value": value,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": d["steps"],
        "warmup": args.warmup,
        "ms_per_step": wall / d["steps"] * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic, seeded (configuration 1: bf16 q/k/v, fp32 gates and state pool ~N(0,0.1))",
        "config": {"workload": "GDN decode, one layer, B=64, Hk=16 Hv=32 d=128, fp32 slot pool [128,32,128,128] "
                               "updated in place, 4 rotating pools",
                   "global_batch": 64, "seq_len": 1, "parallelism": "none (1 GPU)", "launch": "eager"},
        "graph_tok_per_s": (d["tokens"] * d["steps"] / d["graph_wall"]) if d["graph_wall"] else None,
        "roofline": {"bound": "hbm", "achieved": achieved / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK, "traffic": DECODE_TRAFFIC_MEASURED,
                     "kernel": "gdn::recurrent_kernel<32, 64>", "kernel_us": d["kernel_s"] * 1e6,
                     "bytes_per_launch": DECODE_BYTES},
    }
    out["decode_batches"] = bench_decode_batches(torch)
    if not args.no_prefill:
        out["prefill"] = bench_prefill(torch)
        if not args.no_prefill_repeated:
            out["prefill_qk_repeated"] = bench_prefill(torch, repeat_qk=True)
        for dt, key in ((torch.float32, "prefill_f32_qkv"), (torch.float16, "prefill_f16_qkv")):
            out[key] = bench_prefill_non_bf16(torch, dt)
            out[key]["x_bf16_call"] = out[key]["ms"] / out["prefill"]["ms"]
        if not args.no_layer_glue:
            out["layer_glue"] = bench_layer_glue(torch)
        out["varlen"] = bench_varlen(torch)
        out["prefill_b16_t1038"] = bench_prefill_b16(torch)
        if not args.no_prefill_repeated:
            out["prefill_b16_t1038_qk_repeated"] = bench_prefill_b16(torch, repeat_qk=True)
    out["spec_verify"] = bench_spec_verify(torch)
    if not args.no_conv:
        out["conv_prefill"] = bench_conv_prefill(torch)
    if not args.no_in_proj:
        out["decode_in_proj"] = bench_in_proj(torch)
        out["decode_out_proj"] = bench_out_proj(torch)
    if not args.no_layer_decode:
        out["layer_decode"] = bench_layer_decode(torch)
        out["layer_decode_b1"] = bench_layer_decode(torch, batch=1)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
