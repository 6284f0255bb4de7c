"""The training step of the drop-in module captured in HIP graphs.

torch.cuda.make_graphed_callables captures `y = m(x)` and `y.backward(dy)` of
MoEFeedForward (dropout 0, d 768, F 3072, 16 experts, top-2) as a forward and a
backward graph.  Capture fails on any synchronisation (a host read, an event
wait, a blocking copy), so this is the test that the training path has none:
the backward sizes its padded operands from N k + 384 E, a bound the host knows,
and the kernels find each expert's rows from offsets on the device.  Every
replay, with a new input copied in, must equal the eager step bit for bit: the
output, the input gradient and the four parameter gradients."""
import pytest
import torch

from genet5_amd.moe import MoEFeedForward

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [4550, 3000])
def test_training_step_graph_replays_equal_eager(cuda_device, n):
    dev = cuda_device
    print(f"graphed training step n={n}", flush=True)
    torch.manual_seed(0)
    m = MoEFeedForward(768, 3072, 0.0, num_experts=16, top_k=2).to(dev).to(torch.bfloat16)
    m.train()
    g = torch.Generator(device=dev).manual_seed(2)
    xs = [torch.randn(n, 768, device=dev, generator=g).to(torch.bfloat16) for _ in range(3)]
    dys = [torch.randn(n, 768, device=dev, generator=g).to(torch.bfloat16) for _ in range(3)]
    params = (m.router.weight, m.w_gate, m.w_up, m.w_down)

    def eager(x, dy):
        m.zero_grad(set_to_none=True)
        xr = x.clone().requires_grad_(True)
        y = m(xr)
        y.backward(dy)
        return y.detach().clone(), xr.grad.clone(), [p.grad.clone() for p in params]

    refs = [eager(x, dy) for x, dy in zip(xs, dys)]
    torch.cuda.synchronize()
    sample = xs[0].clone().requires_grad_(True)
    m.zero_grad(set_to_none=True)
    # make_graphed_callables warms the callable up on a side stream and captures the
    # backward (torch.autograd.grad over the parameters) on its capture stream, so
    # the parameters' AccumulateGrad nodes belong to another stream than the
    # replays' backward on the current one; torch flags that (input_buffer.cpp) as a
    # possible extra synchronisation.  The replays are checked bit for bit against
    # the eager steps, so the notice is switched off for the capture and replays.
    torch.autograd.graph.set_warn_on_accumulate_grad_stream_mismatch(False)
    try:
        gm = torch.cuda.make_graphed_callables(m, (sample,))
        torch.cuda.synchronize()
        for rep in range(6):
            i = rep % 3
            m.zero_grad(set_to_none=True)
            xr = xs[i].clone().requires_grad_(True)
            y = gm(xr)
            y.backward(dys[i])
            torch.cuda.synchronize()
            y_ref, dx_ref, g_ref = refs[i]
            assert torch.equal(y, y_ref), f"replay {rep}: y"
            assert torch.equal(xr.grad, dx_ref), f"replay {rep}: dx"
            for p, gr in zip(params, g_ref):
                assert torch.equal(p.grad, gr), f"replay {rep}: parameter gradient"
    finally:
        torch.autograd.graph.set_warn_on_accumulate_grad_stream_mismatch(True)
