"""The HIP kernels are capturable into HIP graphs (the reference's decode
graph path, engine/runtime/cuda_graphs.py:259-359, had to swap its kernels
for torch code because the Triton/Helion ones were not): no host sync, no
allocation inside the library, every launch on the caller's stream.

Each graph is replayed several times with eager work and synchronisations
in between, and every replay is checked against the eager result."""
import pytest
import torch

from engine import configs
from engine.kernels import chunk_gated_delta_rule, fused_recurrent_gated_delta_rule

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

DEV = "cuda"


def capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()  # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def test_decode_step_graph_replays_match_eager():
    c = configs.config1(batch=16, num_slots=32)
    q, k, v, g, beta = (c[x].to(DEV) for x in ("q", "k", "v", "g", "beta"))
    slots = c["slots"].to(DEV)
    pool0 = c["pool"].to(DEV)
    pool = pool0.clone()

    def step():
        return fused_recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=pool, ssm_state_indices=slots,
                                                inplace_final_state=True, use_qk_l2norm_in_kernel=True)[0]

    o_eager = step().clone()
    pool_eager = pool.clone()
    graph, o_graph = capture(step)
    for _ in range(3):
        pool.copy_(pool0)                      # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(o_graph, o_eager)
        assert torch.equal(pool, pool_eager)


@pytest.mark.parametrize("t", [300, 4200])  # one segment; two (64 chunks each)
def test_chunk_prefill_graph_replays_match_eager(t):
    c = configs.config2(seed=12, t=t)
    q, k, v, g, beta = (c[x].to(DEV) for x in ("q", "k", "v", "g", "beta"))
    h0 = torch.randn(1, 32, 128, 128, generator=torch.Generator().manual_seed(4)).mul(0.1).to(DEV)

    def run():
        return chunk_gated_delta_rule(q, k, v, g, beta, initial_state=h0, output_final_state=True,
                                      use_qk_l2norm_in_kernel=True)

    o_eager, s_eager = (t.clone() for t in run())
    graph, (o_graph, s_graph) = capture(run)
    for _ in range(3):
        torch.cuda.synchronize()
        scratch = torch.randn(1 << 20, device=DEV)  # unrelated eager work
        del scratch
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(o_graph, o_eager)
        assert torch.equal(s_graph, s_eager)


@pytest.mark.parametrize("lens", [[1402, 1130, 590, 319, 404, 422, 421, 1909, 1501, 245, 2033, 1583, 810, 335, 401, 289],
                                  [700, 0, 1300]])
def test_varlen_prefill_graph_replays_match_eager(lens):
    """Packed sequences from a graph: configuration 3's lengths (512 pairs:
    the per-pair kernel, its workgroups ranking the lengths in the kernel) and
    three sequences with an empty one (the persistent scan, with the chunk
    table built on the device)."""
    import numpy as np
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=DEV)
    c = configs.config2(seed=13, t=int(sum(lens)))
    q, k, v, g, beta = (c[x].to(DEV) for x in ("q", "k", "v", "g", "beta"))
    h0 = torch.randn(len(lens), 32, 128, 128, generator=torch.Generator().manual_seed(5)).mul(0.1).to(DEV)

    def run():
        return chunk_gated_delta_rule(q, k, v, g, beta, initial_state=h0, output_final_state=True,
                                      use_qk_l2norm_in_kernel=True, cu_seqlens=cu)

    o_eager, s_eager = (t.clone() for t in run())
    graph, (o_graph, s_graph) = capture(run)
    for _ in range(3):
        torch.cuda.synchronize()
        scratch = torch.randn(1 << 20, device=DEV)  # unrelated eager work
        del scratch
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(o_graph, o_eager)
        assert torch.equal(s_graph, s_eager)
