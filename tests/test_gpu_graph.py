"""HIP graph capture of the linear paths (serving loops capture their decode GEMVs): each path is captured once, after
an eager warm-up (path tuning, workspaces), then replayed four times with new activations written between replays and
eager work and synchronizations in between; every replay must equal the eager result bit for bit. No path records a
memset (its split partials are rewritten by every call), so replays after the first stay correct."""
import pytest
import torch

pytestmark = pytest.mark.gpu

# (m, path, K, N); small at N = 13824 runs the row-balanced kernel, at N = 1536 the split form
CASES = [(1, "lines", 5120, 1536), (2, "lines", 5120, 1536), (3, "lines", 5120, 1536), (4, "lines", 13824, 1536),
         (4, "lines", 1028, 1536), (8, "small", 5120, 1536), (16, "small", 13824, 1536), (32, "small", 5120, 13824),
         (40, "block", 5120, 1536), (40, "exact", 5120, 1536), (300, "row", 1536, 1536)]


@pytest.mark.parametrize("m,mode,k,n", CASES)
def test_graph_replay(wq, m, mode, k, n):
    print(f"graph replay m={m} mode={mode} k={k} n={n}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(m * 7 + k)
    xs = [torch.randn(m, k, device="cuda", generator=g).bfloat16() for _ in range(5)]
    w = torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda", generator=g)
    s = (torch.rand(n, device="cuda", generator=g) + 0.5) / 127
    b = (0.02 * torch.randn(n, device="cuda", generator=g)).bfloat16()
    x = xs[0].clone()
    out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    # warm-up on a side stream, as torch's capture recipe does
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            wq.linear(x, w, s, b, mode=mode, out=out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        wq.linear(x, w, s, b, mode=mode, out=out)
    for r in range(1, 5):
        x.copy_(xs[r])
        ref = wq.linear(xs[r], w, s, b, mode=mode)  # eager, on the same stream, between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {r} differs from the eager call"
