"""Edge cases of the token count through the C ABI: an empty batch (N = 0), a batch
whose every assignment names no expert (all experts empty with N > 0), and a
single token.

Several kernels run grids past their data (padded gate gradient, the padded GEMM
rows, the router's persistent batches, pad_rows, the input gradient's pipeline);
their loads are guarded, not only their stores.  These tests drive each
token-dependent entry point at the boundaries:

  * N = 0: every entry point succeeds, writes nothing where there are no rows,
    and writes zeros where its output has rows that do not depend on the tokens
    (the padded backward operands, the weight gradients);
  * every top-k index out of range (N = 64): the dispatch places nothing, every
    expert GEMM has zero rows, the combine gives zeros, the gate gradient gives
    dw = 0 and zero padded dY rows, and the weight gradients are zero;
  * N = 1: the module's forward and backward against the float64 oracle."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from oracle import moe_oracle as mo
from genet5_amd import _lib, ops, synth
from genet5_amd.moe import MoEFeedForward
from test_gpu_parity import host

pytestmark = pytest.mark.gpu

d, F, E, k = 256, 512, 4, 2


def bf(*shape, dev, fill=None):
    if fill is None:
        return torch.empty(*shape, dtype=torch.bfloat16, device=dev)
    return torch.full(shape, fill, dtype=torch.bfloat16, device=dev)


def test_empty_batch_every_entry_point(cuda_device):
    dev = cuda_device
    print("N = 0 through every token-dependent entry point", flush=True)
    s = _lib.make_shape(0, d, F, E, k, _lib.DTYPE_BF16)
    S = ops._stream(dev)
    P = ops._ptr
    i32 = dict(dtype=torch.int32, device=dev)
    f32 = dict(dtype=torch.float32, device=dev)
    x, wr = bf(0, d, dev=dev), (torch.randn(E, d, device=dev) * 0.05).to(torch.bfloat16)
    wg = (torch.randn(E, F, d, device=dev) * 0.05).to(torch.bfloat16)
    wu = (torch.randn(E, F, d, device=dev) * 0.05).to(torch.bfloat16)
    wd = (torch.randn(E, d, F, device=dev) * 0.05).to(torch.bfloat16)
    wgu, wgu_t = ops.pack_gate_up_transposed(wg, wu)
    wd_t = ops.transpose_experts(wd)
    idx, w = torch.empty(0, k, **i32), torch.empty(0, k, **f32)
    counts = torch.full((E,), 7, **i32)
    offsets = torch.full((E + 1,), 7, **i32)
    perm, inv = torch.empty(0, **i32), torch.empty(0, **i32)
    ws = ops.workspace(s, dev)
    _lib.call("g5moe_router_topk", P(x), P(wr), None, P(idx), P(w), None, ctypes.byref(s), S)
    _lib.call("g5moe_dispatch", P(idx), P(counts), P(offsets), P(perm), P(inv), P(ws),
              ctypes.byref(s), S)
    torch.cuda.synchronize()
    assert host(counts).tolist() == [0] * E and host(offsets).tolist() == [0] * (E + 1)
    c2, o2 = torch.full((E,), 7, **i32), torch.full((E + 1,), 7, **i32)
    _lib.call("g5moe_dispatch_noalloc", P(idx), P(c2), P(o2), P(perm), P(inv), ctypes.byref(s),
              S)
    torch.cuda.synchronize()
    assert host(c2).tolist() == [0] * E and host(o2).tolist() == [0] * (E + 1)
    yp = bf(0, d, dev=dev)
    gu = bf(0, 2 * F, dev=dev)
    _lib.call("g5moe_expert_gate_up", P(x), P(perm), P(offsets), P(wgu), P(ws), ctypes.byref(s), S)
    _lib.call("g5moe_expert_down", P(offsets), P(wd), P(yp), P(ws), ctypes.byref(s), S)
    _lib.call("g5moe_expert_swiglu", P(x), P(perm), P(offsets), P(wgu), P(wd), P(yp), P(ws),
              ctypes.byref(s), S)
    _lib.call("g5moe_expert_gate_up_raw", P(x), P(perm), P(offsets), P(wgu), P(gu), P(ws),
              ctypes.byref(s), S)
    for fn in ("g5moe_expert_gate_up_train", "g5moe_expert_gate_up_train_factors"):
        ws.fill_(0x55)
        _lib.call(fn, P(x), P(perm), P(offsets), P(wgu), P(gu), P(ws), None, ctypes.byref(s), S)
        h = ws[ops._h_offset(s): ops._h_offset(s) + ops.H_SLACK * F * 2]
        torch.cuda.synchronize()
        assert not h.any(), fn  # the slack rows the weight gradient reads are zeroed
    y = bf(0, d, dev=dev)
    _lib.call("g5moe_combine", P(yp), P(inv), P(w), P(y), ctypes.byref(s), S)
    _lib.call("g5moe_combine_residual", P(yp), P(inv), P(w), P(x), ctypes.c_float(1.0), P(y),
              ctypes.byref(s), S)
    nw = torch.ones(d, **f32)
    _lib.call("g5moe_add_rmsnorm_router", P(x), P(x), P(nw), ctypes.c_float(1e-6), P(wr), None,
              P(y), P(y), P(idx), P(w), None, ctypes.byref(s), S)
    _lib.call("g5moe_rmsnorm", P(x), P(x), P(nw), ctypes.c_float(1e-6), None, P(y), 0, d,
              _lib.DTYPE_BF16, S)
    _lib.call("g5moe_forward", P(x), P(wr), None, P(wgu), P(wd), P(y), P(idx), P(w), P(counts),
              P(offsets), P(perm), P(inv), P(ws), ctypes.byref(s), S)
    # backward stages
    dw = torch.empty(0, k, **f32)
    dlg = torch.empty(0, E, **f32)
    _lib.call("g5moe_gate_grad", P(x), P(yp), P(inv), P(w), P(dw), P(yp), ctypes.byref(s), S)
    _lib.call("g5moe_router_grad", P(dw), P(w), P(idx), None, P(dlg), ctypes.byref(s), S)
    for kmax in (0, 384):
        rows = E * 384   # both layouts: 384 rows per empty expert
        dy_pad = bf(rows + ops.ROW_PAD, d, dev=dev, fill=3.0)
        _lib.call("g5moe_gate_grad_padded", None, None, None, None, P(offsets), None, P(dy_pad),
                  kmax, ctypes.byref(s), S)
        dgu = bf(rows + ops.ROW_PAD, 2 * F, dev=dev, fill=3.0)
        _lib.call("g5moe_dh_swiglu_backward", P(dy_pad), kmax, P(offsets), P(wd_t), None, P(dgu),
                  ctypes.byref(s), S)
        dgu2 = bf(rows + ops.ROW_PAD, 2 * F, dev=dev, fill=3.0)
        hp = bf(rows, F, dev=dev, fill=3.0)
        _lib.call("g5moe_swiglu_backward", None, None, None, P(offsets), None, P(hp), P(dgu2),
                  kmax, None, ctypes.byref(s), S)
        xp = bf(rows, d, dev=dev, fill=3.0)
        _lib.call("g5moe_pad_rows", None, None, P(offsets), P(xp), d, kmax, ctypes.byref(s), S)
        grads = [torch.full((E, d, F), 3.0, dtype=torch.bfloat16, device=dev),
                 torch.full((E, F, d), 3.0, dtype=torch.bfloat16, device=dev),
                 torch.full((E, F, d), 3.0, dtype=torch.bfloat16, device=dev)]
        h = bf(ops.H_SLACK, F, dev=dev, fill=0.0)
        _lib.call("g5moe_weight_grad_sorted_h", P(dy_pad), P(h), P(grads[0]), P(dgu), P(xp),
                  P(grads[1]), P(grads[2]), P(offsets), kmax, ctypes.byref(s), S)
        torch.cuda.synchronize()
        for name, t in (("dy_pad", dy_pad[:rows]), ("dgu", dgu[:rows]), ("dgu2", dgu2[:rows]),
                        ("h_pad", hp), ("x_pad", xp)):
            assert not t.any(), (kmax, name)
        for t in grads:
            assert not t.any(), kmax
    xT = bf(E, d, 64, dev=dev, fill=3.0)
    _lib.call("g5moe_pad_transpose", None, None, P(offsets), P(xT), d, 64, ctypes.byref(s), S)
    c = bf(0, F, dev=dev)
    _lib.call("g5moe_grouped_gemm", P(dy_pad), P(offsets), P(wd_t), P(c), 0, d, F, E, S)
    _lib.call("g5moe_grouped_gemm_padded", P(dy_pad), 0, P(offsets), P(wd_t), P(c), 0, d, F, E,
              S)
    _lib.call("g5moe_input_grad", P(yp), P(inv), P(dlg), P(wr), P(y), ctypes.byref(s), S)
    d_wr = ops.router_weight_grad(dlg, x, s)
    torch.cuda.synchronize()
    assert not xT.any()
    assert d_wr.shape == (E, d) and not d_wr.any()


def test_every_assignment_out_of_range(cuda_device):
    """Top-k indices that name no expert (E itself): nothing is placed, and every
    later stage sees empty experts."""
    dev = cuda_device
    n = 64
    print(f"every assignment out of range, N = {n}", flush=True)
    s = _lib.make_shape(n, d, F, E, k, _lib.DTYPE_BF16)
    g = torch.Generator(device=dev).manual_seed(4)
    x = torch.randn(n, d, device=dev, generator=g).to(torch.bfloat16)
    wg = (torch.randn(E, F, d, device=dev, generator=g) * 0.05).to(torch.bfloat16)
    wu = (torch.randn(E, F, d, device=dev, generator=g) * 0.05).to(torch.bfloat16)
    wd = (torch.randn(E, d, F, device=dev, generator=g) * 0.05).to(torch.bfloat16)
    wgu, wgu_t = ops.pack_gate_up_transposed(wg, wu)
    wd_t = ops.transpose_experts(wd)
    idx = torch.full((n, k), E, dtype=torch.int32, device=dev)
    w = torch.full((n, k), 0.5, dtype=torch.float32, device=dev)
    counts, offsets, perm, inv = ops.dispatch(idx, E, d)
    torch.cuda.synchronize()
    assert host(counts).tolist() == [0] * E and host(offsets).tolist() == [0] * (E + 1)
    assert (host(inv) == -1).all()
    y_perm = ops.expert_swiglu(x, perm, offsets, wgu, wd, k)
    y = ops.combine(y_perm, inv, w, torch.bfloat16)
    torch.cuda.synchronize()
    assert not y.any()
    dy = torch.randn(n, d, device=dev, generator=g).to(torch.bfloat16)
    P = ops.packed_rows(n * k, E)
    dy_pad = bf(P + ops.ROW_PAD, d, dev=dev, fill=3.0)
    dw = torch.full((n, k), 5.0, dtype=torch.float32, device=dev)
    _lib.call("g5moe_gate_grad_padded", ops._ptr(dy), ops._ptr(y_perm), ops._ptr(inv),
              ops._ptr(w), ops._ptr(offsets), ops._ptr(dw), ops._ptr(dy_pad), 0,
              ctypes.byref(s), ops._stream(dev))
    x_pad = ops.pad_rows(x, perm, offsets, E, 0, k, n_assignments=n * k)
    torch.cuda.synchronize()
    assert not dw.any()
    assert not dy_pad[:E * 384].any() and not x_pad[:E * 384].any()


def test_single_token_module_vs_oracle(cuda_device):
    dev = cuda_device
    print("N = 1 through the module, forward and backward", flush=True)
    torch.manual_seed(3)
    m = MoEFeedForward(d, F, 0.0, num_experts=E, top_k=k).to(dev).to(torch.bfloat16)
    with torch.no_grad():
        for p in (m.w_gate, m.w_up, m.w_down):
            p.normal_(0, 0.05)
    x = torch.randn(1, d, device=dev).to(torch.bfloat16).requires_grad_(True)
    R = torch.randn(1, d, device=dev)
    y = m(x)
    (y.float() * R).sum().backward()
    bits = lambda t: t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)
    xb, wrb = bits(x), bits(m.router.weight)
    fwd = oracle.moe_forward(xb, wrb, bits(m.w_gate), bits(m.w_up), bits(m.w_down), k,
                             storage="bf16")
    got = host(y).astype(np.float64)
    err = np.abs(got - fwd["y"]).max() / np.abs(fwd["y"]).max()
    assert err <= 2e-2, err
    ref = oracle.moe_backward(xb, wrb, bits(m.w_gate), bits(m.w_up), bits(m.w_down),
                              fwd["topk_idx"], synth.f32_to_bf16_bits(R.cpu().numpy()))
    for got_t, key in ((x.grad, "dx"), (m.router.weight.grad, "d_w_router"),
                       (m.w_gate.grad, "d_w_gate"), (m.w_up.grad, "d_w_up"),
                       (m.w_down.grad, "d_w_down")):
        a = host(got_t).astype(np.float64)
        r = ref[key]
        e = np.abs(a - r).max() / max(np.abs(r).max(), 1e-30)
        print(f"  {key}: max_rel={e:.3e}", flush=True)
        assert e <= 1.5e-2, (key, e)
