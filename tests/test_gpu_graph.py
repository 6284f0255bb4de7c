"""The layer forward under HIP graph capture: g5moe_forward (router, dispatch, the
grouped GEMMs with the gate|up launch's claimed tail, combine) allocates nothing,
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
    with torch.cuda.stream(s):  # warm the capture stream (library caches, claim slots)
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
