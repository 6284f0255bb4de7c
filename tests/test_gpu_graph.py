"""The layer forward under HIP graph capture: g5moe_forward (router, dispatch, the
grouped GEMMs, combine) allocates nothing,
synchronises nothing and records no memset nodes, so a serving loop can capture
it once and replay it.  Each replay, with the program's own eager work and a
synchronisation between replays, must give the eager result bit for bit; the
input is changed in place between replays and the replay must follow it."""
import pytest
import torch

from genet5_amd import ops, synth
from test_gpu_parity import layer_tensors

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [20000, 4550])
def test_forward_graph_replays_equal_eager(cuda_device, n):
    d, F, E, k = 768, 3072, 16, 2
    print(f"graph capture n={n}", flush=True)
    inp = synth.make_layer(n, d_model=d, d_ff=F, n_experts=E, top_k=k, seed=3, dtype="bf16")
    x, wr, wgu, wd, _ = layer_tensors(inp, cuda_device)
    x2 = (x.float() * 0.5).to(torch.bfloat16)
    buf = ops.ForwardBuffers(n, d, F, E, k, x.dtype, cuda_device)
    xin = x.clone()
    # eager references for both inputs
    y_a = ops.moe_forward(x, wr, wgu, wd, k, buffers=buf).clone()
    y_b = ops.moe_forward(x2, wr, wgu, wd, k, buffers=buf).clone()
    torch.cuda.synchronize()
    s = torch.cuda.Stream(cuda_device)
    s.wait_stream(torch.cuda.current_stream(cuda_device))
    with torch.cuda.stream(s):  # warm the capture stream (library caches)
        ops.moe_forward(xin, wr, wgu, wd, k, buffers=buf)
    torch.cuda.current_stream(cuda_device).wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = ops.moe_forward(xin, wr, wgu, wd, k, buffers=buf)
    for rep in range(6):
        src = x if rep % 2 == 0 else x2
        xin.copy_(src)
        g.replay()
        junk = torch.randn(1 << 20, device=cuda_device).sum()  # eager work between replays
        torch.cuda.synchronize()
        want = y_a if rep % 2 == 0 else y_b
        assert torch.equal(y, want), f"replay {rep}"
        del junk


def test_module_forward_graph_replays_equal_eager(cuda_device):
    """The drop-in module itself under capture (inference: no grad, eval mode), as a
    serving loop or torch.cuda.graphs-based runtime would use it: outputs and
    workspace come from the caching allocator's graph pool, and the weight caches
    are built before capture.  Replays follow in-place input changes."""
    from genet5_amd.moe import MoEFeedForward
    d, F, E, k, n = 768, 3072, 16, 2, 4550
    print(f"module graph capture n={n}", flush=True)
    torch.manual_seed(0)
    m = MoEFeedForward(d, F, 0.1, num_experts=E, top_k=k).to(cuda_device).to(torch.bfloat16)
    m.eval()
    g = torch.Generator(device=cuda_device).manual_seed(4)
    x1 = torch.randn(2, n // 2, d, device=cuda_device, generator=g).to(torch.bfloat16)
    x2 = torch.randn(2, n // 2, d, device=cuda_device, generator=g).to(torch.bfloat16)
    with torch.no_grad():
        y1, y2 = m(x1).clone(), m(x2).clone()
        xin = x1.clone()
        s = torch.cuda.Stream(cuda_device)
        s.wait_stream(torch.cuda.current_stream(cuda_device))
        with torch.cuda.stream(s):
            m(xin)
        torch.cuda.current_stream(cuda_device).wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            y = m(xin)
        for rep in range(4):
            xin.copy_(x1 if rep % 2 == 0 else x2)
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, y1 if rep % 2 == 0 else y2), f"replay {rep}"
