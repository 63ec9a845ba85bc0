"""The allocation-free decode out_proj entry point (gdn_out_proj_decode_noalloc).

Called through the C ABI on two calls in a row -- the second with fewer
rows, so stale partial sums of the first call would show -- and compared
bit for bit with gdn_out_proj_decode, which runs the same kernels on a
caller workspace.  The entry point has no counterpart in the reference; it
serves callers that cannot allocate (graph capture, serving loops).
"""
import pytest
import torch

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

DEV = "cuda"


@pytest.mark.parametrize("k", [3072, 4096])
def test_noalloc_out_proj_matches_the_workspace_entry_point(k):
    """K = 3072 and 4096 (3 and 4 splits of 1024): the partial sums in the
    built-in scratch."""
    from engine.kernels import _lib
    from engine.kernels.in_proj import gdn_out_proj_decode
    lib = _lib.load()
    gen = torch.Generator().manual_seed(101)
    n = 2048
    assert lib.gdn_out_proj_workspace_bytes(64, k, n) == (k // 1024) * 64 * n * 4
    w = (0.02 * torch.randn(n, k, generator=gen)).to(torch.bfloat16).to(DEV)
    for m in (64, 5, 1, 33):  # each call after a larger one: no stale partials may leak in
        print(f"noalloc out_proj M={m} K={k} N={n}", flush=True)
        x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(DEV)
        y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
        st = lib.gdn_out_proj_decode_noalloc(x.data_ptr(), k, w.data_ptr(), m, k, n, y.data_ptr(), n,
                                             torch.cuda.current_stream().cuda_stream)
        _lib.check(st, "gdn_out_proj_decode_noalloc")
        ref = gdn_out_proj_decode(x, w)
        torch.cuda.synchronize()
        assert torch.equal(y, ref), m


def test_noalloc_out_proj_python_wrapper_and_graph_replay():
    """The wrapper writes into the caller's tensor; a captured call replays
    to the eager result (nothing is allocated inside the capture)."""
    from engine.kernels.in_proj import gdn_out_proj_decode, gdn_out_proj_decode_noalloc
    gen = torch.Generator().manual_seed(102)
    k, n, m = 4096, 2048, 48
    w = (0.02 * torch.randn(n, k, generator=gen)).to(torch.bfloat16).to(DEV)
    static_x = torch.zeros(m, k, dtype=torch.bfloat16, device=DEV)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    assert gdn_out_proj_decode_noalloc(static_x, w, out) is out
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gdn_out_proj_decode_noalloc(static_x, w, out)
    for step in range(3):
        x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(DEV)
        ref = gdn_out_proj_decode(x, w)
        torch.cuda.synchronize()
        static_x.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), step
