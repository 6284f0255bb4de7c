"""Concurrent layer forwards on two HIP streams, each with its own workspace and
outputs (the ABI's contract for overlapping calls): both results must equal the
same forwards run one after the other, bit for bit.  The two layers differ in
shape (so one stream's launches are not a replay of the other's) and each stream
runs several forwards back to back, so the gate|up launches of the two streams
are in flight together.  The same holds for a forward captured in a HIP graph and replayed on
one stream while eager forwards with another workspace run on a second."""
import pytest
import torch

from genet5_amd import ops, synth
from test_gpu_parity import layer_tensors

pytestmark = pytest.mark.gpu


def test_two_streams_equal_serial(cuda_device):
    print("two-stream forwards", flush=True)
    a = synth.make_layer(20000, d_model=768, d_ff=3072, n_experts=16, top_k=2, seed=5,
                         dtype="bf16")
    b = synth.make_layer(9000, d_model=768, d_ff=3072, n_experts=8, top_k=2, seed=6,
                         dtype="bf16")
    ta, tb = layer_tensors(a, cuda_device), layer_tensors(b, cuda_device)
    bufa = ops.ForwardBuffers(20000, 768, 3072, 16, 2, torch.bfloat16, cuda_device)
    bufb = ops.ForwardBuffers(9000, 768, 3072, 8, 2, torch.bfloat16, cuda_device)

    def fwd(t, buf):
        x, wr, wgu, wd, bias = t
        return ops.moe_forward(x, wr, wgu, wd, 2, bias=bias, buffers=buf)

    ya = fwd(ta, bufa).clone()
    yb = fwd(tb, bufb).clone()
    torch.cuda.synchronize()

    sa, sb = torch.cuda.Stream(cuda_device), torch.cuda.Stream(cuda_device)
    sa.wait_stream(torch.cuda.current_stream(cuda_device))
    sb.wait_stream(torch.cuda.current_stream(cuda_device))
    outs_a, outs_b = [], []
    for _ in range(4):
        with torch.cuda.stream(sa):
            outs_a.append(fwd(ta, bufa).clone())
        with torch.cuda.stream(sb):
            outs_b.append(fwd(tb, bufb).clone())
    torch.cuda.synchronize()
    for i, (oa, ob) in enumerate(zip(outs_a, outs_b)):
        assert torch.equal(oa, ya), f"stream A forward {i}"
        assert torch.equal(ob, yb), f"stream B forward {i}"


def test_graph_replay_beside_eager_stream(cuda_device):
    """A captured forward (its workspace the capture's own) replayed on stream A while
    eager forwards with their own workspace run on stream B: every output equals the
    serial result."""
    print("graph replay beside an eager stream", flush=True)
    a = synth.make_layer(20000, d_model=768, d_ff=3072, n_experts=16, top_k=2, seed=7,
                         dtype="bf16")
    b = synth.make_layer(16000, d_model=768, d_ff=3072, n_experts=16, top_k=2, seed=8,
                         dtype="bf16")
    ta, tb = layer_tensors(a, cuda_device), layer_tensors(b, cuda_device)
    bufa = ops.ForwardBuffers(20000, 768, 3072, 16, 2, torch.bfloat16, cuda_device)
    bufb = ops.ForwardBuffers(16000, 768, 3072, 16, 2, torch.bfloat16, cuda_device)

    def fwd(t, buf):
        x, wr, wgu, wd, bias = t
        return ops.moe_forward(x, wr, wgu, wd, 2, bias=bias, buffers=buf)

    ya = fwd(ta, bufa).clone()
    yb = fwd(tb, bufb).clone()
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(cuda_device), torch.cuda.Stream(cuda_device)
    sa.wait_stream(torch.cuda.current_stream(cuda_device))
    with torch.cuda.stream(sa):
        fwd(ta, bufa)
    torch.cuda.current_stream(cuda_device).wait_stream(sa)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=sa):
        y = fwd(ta, bufa)
    torch.cuda.synchronize()
    outs_a, outs_b = [], []
    for _ in range(4):
        with torch.cuda.stream(sa):
            g.replay()
            outs_a.append(y.clone())
        with torch.cuda.stream(sb):
            outs_b.append(fwd(tb, bufb).clone())
    torch.cuda.synchronize()
    for i, (oa, ob) in enumerate(zip(outs_a, outs_b)):
        assert torch.equal(oa, ya), f"graph replay {i}"
        assert torch.equal(ob, yb), f"eager forward {i}"
