"""GPU backward of the MoE layer (through the C ABI and the module's autograd)
against the float64 oracle backward (oracle.moe_backward, pinned by finite
differences and float64 torch autograd).

Exact where the contract fixes the arithmetic: dy_perm = bf16(w * dy) bit for bit,
and the gate gradient dw (bf16 x bf16 products are exact in fp32, so the lane
chain and tree order reproduce in numpy).  Everything downstream passes through
bf16 buffers (dY, dh, dGU, h, dX_perm, bf16 weight gradients), so the gradients are
checked normwise against float64: max|err| / max|ref| <= 1.5e-2 and
mean|err| / mean|ref| <= 6e-3, about twice the measured error (max 7e-3, mean
4e-3 at d = 768, F = 3072, E = 16, N = 2048; printed by each test)."""
import numpy as np
import pytest
import torch

import oracle
from oracle import moe_oracle as mo
from genet5_amd import ops, synth
from genet5_amd.moe import MoEFeedForward
from test_gpu_parity import dev_t, host, layer_tensors

pytestmark = pytest.mark.gpu

MAX_REL = 1.5e-2
MEAN_REL = 6e-3


def normwise(got, ref):
    err = np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64))
    r = np.abs(np.asarray(ref, np.float64))
    return err.max() / max(r.max(), 1e-30), err.mean() / max(r.mean(), 1e-30)


def check(name, got, ref):
    mx, mean = normwise(got, ref)
    print(f"  {name}: max_rel={mx:.3e} mean_rel={mean:.3e}", flush=True)
    assert mx <= MAX_REL and mean <= MEAN_REL, (name, mx, mean)


@pytest.mark.parametrize("n,d,F,E,k", [
    (2048, 768, 3072, 16, 2),
    (700, 256, 512, 8, 2),
    (333, 512, 384, 4, 3),
])
def test_backward_stages_vs_oracle(cuda_device, n, d, F, E, k):
    print(f"backward n={n} d={d} F={F} E={E} k={k}", flush=True)
    inp = synth.make_layer(n, d_model=d, d_ff=F, n_experts=E, top_k=k, seed=21, dtype="bf16")
    x, wr, wgu, wd, _ = layer_tensors(inp, cuda_device)
    rng = np.random.default_rng(5)
    dy_np = synth.f32_to_bf16_bits(rng.standard_normal((n, d)).astype(np.float32))
    dy = dev_t(dy_np, cuda_device, True)
    y, logits, idx, w, offsets, perm, inv_pos, y_perm, gu = ops.moe_forward_train(x, wr, wgu,
                                                                                 wd, k)
    torch.cuda.synchronize()
    ref_i, _ = oracle.topk_gates_c(oracle.router_logits(inp.x, inp.w_router), k)
    np.testing.assert_array_equal(idx.cpu().numpy(), ref_i)
    # the training forward (gate|up GEMM storing h and the raw products) gives the
    # inference forward's output bit for bit, and its kept products equal the
    # backward's recompute (g5moe_expert_gate_up_raw) bit for bit
    assert torch.equal(y, ops.moe_forward(x, wr, wgu, wd, k))
    from genet5_amd import _lib
    import ctypes
    shape = _lib.make_shape(n, d, F, E, k, _lib.DTYPE_BF16)
    gu_re = torch.empty_like(gu)
    _lib.call("g5moe_expert_gate_up_raw", ops._ptr(x), ops._ptr(perm), ops._ptr(offsets),
              ops._ptr(wgu), ops._ptr(gu_re), ops._ptr(ops.workspace(shape, cuda_device)),
              ctypes.byref(shape), ops._stream(cuda_device))
    torch.cuda.synchronize()
    assert torch.equal(gu, gu_re)

    # gate gradient: dy_perm exact, dw in the contract's order (exact products)
    dw = torch.empty((n, k), dtype=torch.float32, device=cuda_device)
    dyp = torch.empty((n * k + ops.ROW_PAD, d), dtype=torch.bfloat16, device=cuda_device)
    _lib.call("g5moe_gate_grad", ops._ptr(dy), ops._ptr(y_perm), ops._ptr(inv_pos),
              ops._ptr(w), ops._ptr(dw), ops._ptr(dyp), ctypes.byref(shape),
              ops._stream(cuda_device))
    torch.cuda.synchronize()
    ip = inv_pos.cpu().numpy().reshape(n, k)
    wn = w.cpu().numpy()
    dyf = mo.bf16_to_f32(dy_np)
    exp_dyp = mo.round_bf16(wn[:, :, None] * dyf[:, None, :])
    got_dyp = host(dyp[: n * k])
    np.testing.assert_array_equal(got_dyp[ip.reshape(-1)], exp_dyp.reshape(n * k, d))
    yp = host(y_perm)[ip.reshape(-1)].reshape(n, k, d)
    L = d // 64
    prod = (dyf[:, None, :] * yp).reshape(n, k, 64, L)   # exact in fp32
    acc = np.zeros((n, k, 64), np.float32)
    for i in range(L):
        acc = acc + prod[..., i]
    m = 32
    while m >= 1:
        acc = acc[..., :m] + acc[..., m:2 * m]
        m //= 2
    np.testing.assert_array_equal(dw.cpu().numpy().view(np.uint32), acc[..., 0].view(np.uint32))

    dx, d_wr, d_wgu, d_wd = ops.moe_backward(dy, x, wr, wgu, wd, k, idx, w, offsets, perm,
                                             inv_pos, y_perm, gu=gu)
    recomputed = ops.moe_backward(dy, x, wr, wgu, wd, k, idx, w, offsets, perm, inv_pos, y_perm)
    # the forward's non-blocking host copy of the offsets, handed to the backward
    offs_host = torch.full((E + 1,), -1, dtype=torch.int32, pin_memory=True)
    ready = torch.cuda.Event()
    fw2 = ops.moe_forward_train(x, wr, wgu, wd, k, offsets_host=offs_host, offsets_ready=ready)
    ready.synchronize()
    assert offs_host.tolist() == offsets.tolist()
    via_host = ops.moe_backward(dy, x, wr, wgu, wd, k, idx, w, offsets, perm, inv_pos, y_perm,
                                gu=fw2[8], offsets_host=offs_host)
    torch.cuda.synchronize()
    for a, b, c in zip((dx, d_wr, d_wgu, d_wd), recomputed, via_host):
        assert torch.equal(a, b) and torch.equal(a, c)
    ref = oracle.moe_backward(inp.x, inp.w_router, inp.w_gate, inp.w_up, inp.w_down, ref_i, dy_np)
    d_wg, d_wu = ops.unpack_gate_up(d_wgu)
    check("dx", host(dx), ref["dx"])
    check("d_w_router", host(d_wr), ref["d_w_router"])
    check("d_w_gate", host(d_wg), ref["d_w_gate"])
    check("d_w_up", host(d_wu), ref["d_w_up"])
    check("d_w_down", host(d_wd), ref["d_w_down"])


@pytest.mark.parametrize("aux,data_loss", [(0.0, True), (0.01, True), (1.0, False)])
def test_module_autograd_vs_oracle(cuda_device, aux, data_loss):
    """loss = sum(y * R) (+ the load-balancing loss).  With data_loss False the loss
    is the load-balancing term alone, so the router and input gradients come only
    through the logits and the expert weights get none."""
    torch.manual_seed(7)
    d, F, E, k, n = 256, 512, 8, 2, 900
    m = MoEFeedForward(d, F, 0.0, num_experts=E, top_k=k).to(cuda_device).to(torch.bfloat16)
    with torch.no_grad():
        for p in (m.w_gate, m.w_up, m.w_down):
            p.normal_(0, 0.05)
        m.router.weight.normal_(0, 0.05)
    m.aux_loss_coef = aux
    x = torch.randn(n, d, device=cuda_device).to(torch.bfloat16).requires_grad_(True)
    R = torch.randn(n, d, device=cuda_device) if data_loss else torch.zeros(n, d, device=cuda_device)
    y = m(x)
    loss = (y.float() * R).sum()
    if aux > 0:
        assert m.aux_loss is not None and m.aux_loss.requires_grad
        loss = loss + m.aux_loss
    loss.backward()
    bits = lambda t: t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)
    xb, wrb = bits(x), bits(m.router.weight)
    logits = mo.bf16_to_f32(xb).astype(np.float64) @ mo.bf16_to_f32(wrb).astype(np.float64).T
    idx, _ = oracle.topk_gates_c(oracle.router_logits(xb, wrb), k)
    grad_logits = None
    if aux > 0:
        # d/dlogits of aux * E * sum_e f_e * mean_t softmax(logits_t)_e, f fixed
        f = np.bincount(idx.reshape(-1), minlength=E) / idx.size
        p = np.exp(logits - logits.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        gp = aux * E * f / n
        grad_logits = p * (gp[None, :] - (p * gp[None, :]).sum(axis=1, keepdims=True))
    dy = synth.f32_to_bf16_bits(R.cpu().numpy())  # dL/dy = R, in the bf16 the backward takes
    ref = oracle.moe_backward(xb, wrb, bits(m.w_gate), bits(m.w_up), bits(m.w_down), idx, dy,
                              grad_logits=grad_logits)
    print(f"module aux={aux} data_loss={data_loss}", flush=True)
    check("x.grad", host(x.grad), ref["dx"])
    check("router.grad", host(m.router.weight.grad), ref["d_w_router"])
    for name, p, key in (("w_gate.grad", m.w_gate, "d_w_gate"), ("w_up.grad", m.w_up, "d_w_up"),
                         ("w_down.grad", m.w_down, "d_w_down")):
        if data_loss:
            check(name, host(p.grad), ref[key])
        else:
            assert not np.any(ref[key]) and not torch.any(p.grad), name


def test_padded_weight_gradient_operands(cuda_device):
    """g5moe_pad_transpose (plain rows and gathered x rows) and the padded outputs
    of g5moe_swiglu_backward against numpy, with empty experts and ragged counts:
    the rows land per expert at kmax spacing and every padding entry is zero."""
    import ctypes
    from genet5_amd import _lib
    rng = np.random.default_rng(9)
    E, k, d, F = 6, 2, 128, 128
    counts = np.array([0, 70, 5, 0, 130, 35], np.int32)
    nk = int(counts.sum())
    n = nk // k
    offsets = np.zeros(E + 1, np.int32)
    offsets[1:] = np.cumsum(counts)
    perm = rng.permutation(nk).astype(np.int32)
    kmax = 192
    shape = _lib.make_shape(n, d, F, E, k, _lib.DTYPE_BF16)
    S = ops._stream(cuda_device)
    rows = synth.f32_to_bf16_bits(rng.standard_normal((nk, d)).astype(np.float32))
    x = synth.f32_to_bf16_bits(rng.standard_normal((n, d)).astype(np.float32))
    t_off = dev_t(offsets, cuda_device)
    t_perm = dev_t(perm, cuda_device)
    out = torch.full((E, d, kmax), 7, dtype=torch.int16, device=cuda_device).view(torch.bfloat16)
    outx = torch.full((E, d, kmax), 7, dtype=torch.int16, device=cuda_device).view(torch.bfloat16)
    _lib.call("g5moe_pad_transpose", ops._ptr(dev_t(rows, cuda_device, True)), None,
              ops._ptr(t_off), ops._ptr(out), d, kmax, ctypes.byref(shape), S)
    _lib.call("g5moe_pad_transpose", ops._ptr(dev_t(x, cuda_device, True)), ops._ptr(t_perm),
              ops._ptr(t_off), ops._ptr(outx), d, kmax, ctypes.byref(shape), S)
    # swiglu backward on random dh / gu
    dh = synth.f32_to_bf16_bits(rng.standard_normal((nk, F)).astype(np.float32))
    gu = synth.f32_to_bf16_bits(rng.standard_normal((nk, 2 * F)).astype(np.float32))
    dgu = torch.empty((nk + ops.ROW_PAD, 2 * F), dtype=torch.bfloat16, device=cuda_device)
    h_pad = torch.full((E, kmax, F), 7, dtype=torch.int16, device=cuda_device).view(torch.bfloat16)
    dgu_pad = torch.full((E, kmax, 2 * F), 7, dtype=torch.int16,
                         device=cuda_device).view(torch.bfloat16)
    _lib.call("g5moe_swiglu_backward", ops._ptr(dev_t(dh, cuda_device, True)),
              ops._ptr(dev_t(gu, cuda_device, True)), None, ops._ptr(t_off), ops._ptr(dgu),
              ops._ptr(h_pad), ops._ptr(dgu_pad), kmax, None, ctypes.byref(shape), S)
    torch.cuda.synchronize()
    bits = lambda t: t.cpu().view(torch.int16).numpy().view(np.uint16)
    exp = np.zeros((E, d, kmax), np.uint16)
    expx = np.zeros((E, d, kmax), np.uint16)
    exp_h = np.zeros((E, kmax, F), np.uint16)
    exp_g = np.zeros((E, kmax, 2 * F), np.uint16)
    g_sorted = bits(dgu)[:nk]
    # h = silu(g) * u from the packed layout, in float64, compared after rounding below
    gf = mo.bf16_to_f32(gu).reshape(nk, F // 32, 2, 32)
    g, u = gf[:, :, 0].reshape(nk, F).astype(np.float64), gf[:, :, 1].reshape(nk, F).astype(np.float64)
    h_ref = g / (1 + np.exp(-g)) * u
    for e in range(E):
        o0, o1 = offsets[e], offsets[e + 1]
        exp[e, :, : o1 - o0] = rows[o0:o1].T
        expx[e, :, : o1 - o0] = x[perm[o0:o1] // k].T
        exp_g[e, : o1 - o0] = g_sorted[o0:o1]
    np.testing.assert_array_equal(bits(out), exp)
    np.testing.assert_array_equal(bits(outx), expx)
    np.testing.assert_array_equal(bits(dgu_pad), exp_g)
    hp = bits(h_pad)
    for e in range(E):
        o0, o1 = offsets[e], offsets[e + 1]
        assert not hp[e, o1 - o0:].any()
        got = mo.bf16_to_f32(hp[e, : o1 - o0]).astype(np.float64)
        np.testing.assert_allclose(got, h_ref[o0:o1], rtol=8e-3, atol=1e-6)


@pytest.mark.parametrize("d,k,garbage", [(768, 2, 7.0), (256, 2, float("nan")),
                                         (512, 1, float("nan")), (128, 4, 7.0)])
def test_gate_grad_padded_equals_sorted(cuda_device, d, k, garbage):
    """g5moe_gate_grad_padded writes the same dw as g5moe_gate_grad bit for bit,
    and dY scaled by the gates at row e*kmax + j for sorted position
    offsets[e] + j (equal to g5moe_pad_rows over the sorted copy), zero rows past
    each expert's count (the buffer starts as garbage), with empty experts, an
    assignment outside [0, E) (inv_pos -1, dw 0) and ragged counts; the dh
    product over it equals the sorted product bit for bit."""
    import ctypes
    from genet5_amd import _lib
    print(f"gate_grad_padded d={d} k={k}", flush=True)
    rng = np.random.default_rng(31)
    E, F = 6, 256
    counts = np.array([300, 0, 41, 0, 513, 3], np.int32)
    counts[-1] += (-(int(counts.sum()) + 1)) % k   # N k assignments in all
    nk_valid = int(counts.sum())
    nk = nk_valid + 1                    # one assignment is not placed
    assert nk % k == 0
    n = nk // k
    offsets = np.zeros(E + 1, np.int32)
    offsets[1:] = np.cumsum(counts)
    dropped = 7
    inv = np.full(nk, -1, np.int32)
    inv[np.arange(nk) != dropped] = rng.permutation(nk_valid).astype(np.int32)
    kmax = ops.wgrad_kmax(int(counts.max()))
    shape = _lib.make_shape(n, d, F, E, k, _lib.DTYPE_BF16)
    S = ops._stream(cuda_device)
    t_off = dev_t(offsets, cuda_device)
    t_inv = dev_t(inv, cuda_device)
    w = torch.tensor(rng.random((n, k)).astype(np.float32), device=cuda_device)
    dy = dev_t(synth.f32_to_bf16_bits(rng.standard_normal((n, d)).astype(np.float32)),
               cuda_device, True)
    y_perm = dev_t(synth.f32_to_bf16_bits(rng.standard_normal((nk_valid, d))
                                          .astype(np.float32)), cuda_device, True)
    dw1 = torch.full((n, k), 5.0, dtype=torch.float32, device=cuda_device)
    dw2 = torch.full_like(dw1, 5.0)
    dyp = torch.zeros((nk_valid + ops.ROW_PAD, d), dtype=torch.bfloat16, device=cuda_device)
    buf = torch.full((E * kmax + ops.ROW_PAD, d), garbage, dtype=torch.bfloat16,
                     device=cuda_device)
    _lib.call("g5moe_gate_grad", ops._ptr(dy), ops._ptr(y_perm), ops._ptr(t_inv), ops._ptr(w),
              ops._ptr(dw1), ops._ptr(dyp), ctypes.byref(shape), S)
    _lib.call("g5moe_gate_grad_padded", ops._ptr(dy), ops._ptr(y_perm), ops._ptr(t_inv),
              ops._ptr(w), ops._ptr(t_off), ops._ptr(dw2), ops._ptr(buf), kmax,
              ctypes.byref(shape), S)
    ref_pad = ops.pad_rows(dyp, None, t_off, E, kmax, k)
    torch.cuda.synchronize()
    assert torch.equal(dw1.view(torch.int32), dw2.view(torch.int32))
    assert float(dw2.view(-1)[dropped]) == 0.0
    got = buf[:E * kmax].view(E, kmax, d)
    assert torch.equal(got.view(torch.int16), ref_pad.view(torch.int16))
    for e in range(E):
        m = int(counts[e])
        assert torch.equal(got[e, :m], dyp[offsets[e]:offsets[e + 1]])
        assert not torch.any(got[e, m:].view(torch.int16))      # +0.0 bits
    # the dh product over the padded dY equals the sorted one: the trailing
    # buffer rows (never written, NaN here in one case) reach only discarded
    # output rows
    wt = (torch.randn(E, F, d, device=cuda_device) * 0.05).to(torch.bfloat16)
    dh_ref = ops.grouped_gemm(dyp, nk_valid, t_off, wt)
    dh = ops.grouped_gemm_padded(buf, kmax, nk_valid, t_off, wt)
    torch.cuda.synchronize()
    assert torch.equal(dh, dh_ref)


def test_padded_dx_product_equals_sorted(cuda_device):
    """g5moe_grouped_gemm_padded over the SwiGLU backward's per-expert padded dGU
    equals g5moe_grouped_gemm over the sorted dGU bit for bit (same rows, same
    kernel), with empty experts, ragged counts and a partial last tile; the SwiGLU
    backward writes the same padded outputs whether or not it also writes the
    sorted copy."""
    import ctypes
    from genet5_amd import _lib
    rng = np.random.default_rng(12)
    E, k, d, F = 5, 2, 256, 256
    counts = np.array([300, 0, 41, 513, 2], np.int32)
    nk = int(counts.sum())
    n = nk // k
    offsets = np.zeros(E + 1, np.int32)
    offsets[1:] = np.cumsum(counts)
    kmax = 576
    shape = _lib.make_shape(n, d, F, E, k, _lib.DTYPE_BF16)
    S = ops._stream(cuda_device)
    t_off = dev_t(offsets, cuda_device)
    dh = dev_t(synth.f32_to_bf16_bits(rng.standard_normal((nk, F)).astype(np.float32)),
               cuda_device, True)
    gu = dev_t(synth.f32_to_bf16_bits(rng.standard_normal((nk, 2 * F)).astype(np.float32)),
               cuda_device, True)
    dgu = torch.empty((nk + ops.ROW_PAD, 2 * F), dtype=torch.bfloat16, device=cuda_device)
    h1 = torch.empty((E, kmax, F), dtype=torch.bfloat16, device=cuda_device)
    p1 = torch.empty((E * kmax + ops.ROW_PAD, 2 * F), dtype=torch.bfloat16, device=cuda_device)
    h2 = torch.empty_like(h1)
    p2 = torch.empty_like(p1)
    _lib.call("g5moe_swiglu_backward", ops._ptr(dh), ops._ptr(gu), None, ops._ptr(t_off),
              ops._ptr(dgu), ops._ptr(h1), ops._ptr(p1), kmax, None, ctypes.byref(shape), S)
    _lib.call("g5moe_swiglu_backward", ops._ptr(dh), ops._ptr(gu), None, ops._ptr(t_off), None,
              ops._ptr(h2), ops._ptr(p2), kmax, None, ctypes.byref(shape), S)
    wt = (torch.randn(E, d, 2 * F, device=cuda_device) * 0.05).to(torch.bfloat16)
    ref = ops.grouped_gemm(dgu, nk, t_off, wt)
    got = ops.grouped_gemm_padded(p1, kmax, nk, t_off, wt)
    torch.cuda.synchronize()
    assert torch.equal(h1, h2) and torch.equal(p1[:E * kmax], p2[:E * kmax])
    assert torch.equal(got, ref)
    # and against an fp32 product of the same bf16 rows
    dg = dgu[:nk].float()
    for e in range(E):
        o0, o1 = offsets[e], offsets[e + 1]
        if o1 > o0:
            exp = dg[o0:o1] @ wt[e].float().T
            torch.testing.assert_close(got[o0:o1].float(), exp, rtol=2e-2, atol=2e-2)


def test_weight_grad_kernel_vs_fp32(cuda_device):
    """g5moe_weight_grad (both products in one launch) against float32 torch
    products per expert, over token-major padded operands from g5moe_pad_rows,
    with an empty expert, a one-row expert, counts on and just past the 192-row
    k-step groups, and large experts.  Also: g5moe_pad_rows copies rows exactly
    (zero past each count), an empty expert's gradients are exactly zero, and
    each product alone gives the same bits as the two in one launch (an output
    element's reduction order does not depend on the launch's other tiles)."""
    import ctypes
    from genet5_amd import _lib
    dev = cuda_device
    g = torch.Generator(device=dev).manual_seed(5)
    E, d, F, k = 7, 256, 512, 2
    counts = [0, 1, 192, 384, 385, 2000, 4100]
    offsets = np.zeros(E + 1, np.int32)
    offsets[1:] = np.cumsum(counts)
    T = int(offsets[-1])
    n_tok = (T + k - 1) // k
    t_off = torch.tensor(offsets, dtype=torch.int32, device=dev)
    dy = torch.randn(T + ops.ROW_PAD, d, device=dev, generator=g).to(torch.bfloat16)
    x = torch.randn(n_tok, d, device=dev, generator=g).to(torch.bfloat16)
    perm = torch.randperm(n_tok * k, device=dev, generator=g)[:T].to(torch.int32)
    kmax = ops.wgrad_kmax(max(counts))
    print(f"  E={E} d={d} F={F} counts={counts} kmax={kmax}", flush=True)
    dy_pad = ops.pad_rows(dy, None, t_off, E, kmax, k)
    x_pad = ops.pad_rows(x, perm, t_off, E, kmax, k)
    h_pad = torch.zeros(E, kmax, F, dtype=torch.bfloat16, device=dev)
    dgu_pad = torch.zeros(E, kmax, 2 * F, dtype=torch.bfloat16, device=dev)
    for e, c in enumerate(counts):
        h_pad[e, :c] = torch.randn(c, F, device=dev, generator=g).to(torch.bfloat16)
        dgu_pad[e, :c] = torch.randn(c, 2 * F, device=dev, generator=g).to(torch.bfloat16)
    d_wd, d_wgu = ops.weight_grad(dy_pad, h_pad, dgu_pad, x_pad, t_off, kmax, top_k=k)
    # each product alone
    shape = _lib.make_shape(n_tok, d, F, E, k, _lib.DTYPE_BF16)
    wd1 = torch.empty_like(d_wd)
    wgu1 = torch.empty_like(d_wgu)
    S = ops._stream(dev)
    _lib.call("g5moe_weight_grad", ops._ptr(dy_pad), ops._ptr(h_pad), ops._ptr(wd1), None, None,
              None, ops._ptr(t_off), kmax, ctypes.byref(shape), S)
    _lib.call("g5moe_weight_grad", None, None, None, ops._ptr(dgu_pad), ops._ptr(x_pad),
              ops._ptr(wgu1), ops._ptr(t_off), kmax, ctypes.byref(shape), S)
    torch.cuda.synchronize()
    assert torch.equal(wd1, d_wd) and torch.equal(wgu1, d_wgu)
    for e, c in enumerate(counts):
        o0, o1 = int(offsets[e]), int(offsets[e + 1])
        assert torch.equal(dy_pad[e, :c], dy[o0:o1])
        assert torch.equal(x_pad[e, :c], x[(perm[o0:o1] // k).long()])
        assert not dy_pad[e, c:].any() and not x_pad[e, c:].any()
        if c == 0:
            assert not d_wd[e].any() and not d_wgu[e].any()
            continue
        ref_wd = dy[o0:o1].float().t() @ h_pad[e, :c].float()
        ref_wgu = dgu_pad[e, :c].float().t() @ x_pad[e, :c].float()
        for got, ref, name in ((d_wd[e], ref_wd, "dWd"), (d_wgu[e], ref_wgu, "dWgu")):
            err = (got.float() - ref).abs().max().item() / max(ref.abs().max().item(), 1e-30)
            print(f"  expert {e} ({c} rows) {name}: max_rel={err:.2e}", flush=True)
            assert err <= 8e-3, (e, name, err)


@pytest.mark.parametrize("counts", [[0, 1, 192, 384, 385, 2000, 4100], [700, 3, 0, 0]])
def test_weight_grad_sorted_h_equals_padded(cuda_device, counts):
    """g5moe_weight_grad_sorted_h (h in sorted order with H_SLACK zero rows after
    the last expert's, gate and up gradients written unpacked) against
    g5moe_weight_grad on the padded copy of the same h: bit for bit, since the
    rows past an expert's count meet dY's zero rows.  Empty experts first and last
    (the last ones read only the zero slack rows)."""
    import ctypes
    from genet5_amd import _lib
    dev = cuda_device
    g = torch.Generator(device=dev).manual_seed(11)
    E, d, F, k = len(counts), 256, 512, 2
    offsets = np.zeros(E + 1, np.int32)
    offsets[1:] = np.cumsum(counts)
    T = int(offsets[-1])
    n_tok = (T + k - 1) // k
    t_off = torch.tensor(offsets, dtype=torch.int32, device=dev)
    dy = torch.randn(T + ops.ROW_PAD, d, device=dev, generator=g).to(torch.bfloat16)
    x = torch.randn(n_tok, d, device=dev, generator=g).to(torch.bfloat16)
    perm = torch.randperm(n_tok * k, device=dev, generator=g)[:T].to(torch.int32)
    h = torch.zeros(T + ops.H_SLACK, F, dtype=torch.bfloat16, device=dev)
    h[:T] = torch.randn(T, F, device=dev, generator=g).to(torch.bfloat16)
    dgu = torch.randn(T + ops.ROW_PAD, 2 * F, device=dev, generator=g).to(torch.bfloat16)
    kmax = ops.wgrad_kmax(max(counts))
    print(f"  E={E} counts={counts} kmax={kmax}", flush=True)
    dy_pad = ops.pad_rows(dy, None, t_off, E, kmax, k)
    x_pad = ops.pad_rows(x, perm, t_off, E, kmax, k)
    h_pad = ops.pad_rows(h, None, t_off, E, kmax, k)
    dgu_pad = ops.pad_rows(dgu, None, t_off, E, kmax, k)
    d_wd, d_wgu = ops.weight_grad(dy_pad, h_pad, dgu_pad, x_pad, t_off, kmax, top_k=k)
    wd2 = torch.empty_like(d_wd)
    wg2 = torch.empty(E, F, d, dtype=torch.bfloat16, device=dev)
    wu2 = torch.empty_like(wg2)
    shape = _lib.make_shape(n_tok, d, F, E, k, _lib.DTYPE_BF16)
    _lib.call("g5moe_weight_grad_sorted_h", ops._ptr(dy_pad), ops._ptr(h), ops._ptr(wd2),
              ops._ptr(dgu_pad), ops._ptr(x_pad), ops._ptr(wg2), ops._ptr(wu2), ops._ptr(t_off),
              kmax, ctypes.byref(shape), ops._stream(dev))
    torch.cuda.synchronize()
    wg, wu = ops.unpack_gate_up(d_wgu)
    assert torch.equal(wd2, d_wd)
    assert torch.equal(wg2, wg) and torch.equal(wu2, wu)
    assert d_wd.abs().sum() > 0 and wg.abs().sum() > 0


@pytest.mark.parametrize("n,E,d", [(0, 16, 768), (1, 16, 768), (129, 9, 256), (4096, 4, 512),
                                   (36400, 16, 768)])
def test_router_weight_grad_vs_float64(cuda_device, n, E, d):
    """g5moe_router_weight_grad against the float64 product dlogits^T x: within one
    bf16 ulp of the result plus the fp32 accumulation bound 2e-5 * (|dlogits|^T |x|),
    and the same bits on a second call (fixed reduction order)."""
    from genet5_amd import _lib
    dev = cuda_device
    g = torch.Generator(device=dev).manual_seed(n + E)
    x = torch.randn(n, d, device=dev, generator=g).to(torch.bfloat16)
    dl = torch.randn(n, E, device=dev, generator=g) * 1e-2
    shape = _lib.make_shape(n, d, 512, E, 2, _lib.DTYPE_BF16)
    got = ops.router_weight_grad(dl, x, shape)
    again = ops.router_weight_grad(dl, x, shape)
    torch.cuda.synchronize()
    assert torch.equal(got, again)
    xf = x.float().cpu().numpy().astype(np.float64)
    df = dl.cpu().numpy().astype(np.float64)
    ref = df.T @ xf
    bound = 2.0 ** -8 * np.abs(ref) + 2e-5 * (np.abs(df).T @ np.abs(xf))
    err = np.abs(host(got).astype(np.float64) - ref)
    print(f"  n={n} E={E} d={d}: max err/bound {float((err / np.maximum(bound, 1e-30)).max()):.3f}",
          flush=True)
    assert np.all(err <= bound)


def _split_packed(t, F):
    """[rows, 2F] packed gate|up order -> (gate [rows, F], up [rows, F])."""
    v = t.view(t.shape[0], F // 32, 2, 32)
    return v[:, :, 0].reshape(t.shape[0], F), v[:, :, 1].reshape(t.shape[0], F)


@pytest.mark.parametrize("p", [0.0, 0.2])
@pytest.mark.parametrize("n,d,F,E,k", [(2048, 768, 3072, 16, 2), (700, 256, 512, 8, 2)])
def test_gate_up_train_factors(cuda_device, n, d, F, E, k, p):
    """g5moe_expert_gate_up_train_factors: h bit for bit g5moe_expert_gate_up_train's
    (same dropout), and the factors A = m u s (1 + g (1 - s)), B = m g s against
    float64 from the raw products (which are bf16-rounded, the kernel's are not:
    normwise 1.5e-2 / 4e-3; measured 6e-3 / 2e-3), exactly zero where the mask drops."""
    from oracle import moe_oracle as mo2
    print(f"factors n={n} d={d} F={F} E={E} k={k} p={p}", flush=True)
    inp = synth.make_layer(n, d_model=d, d_ff=F, n_experts=E, top_k=k, seed=21, dtype="bf16")
    x, wr, wgu, wd, _ = layer_tensors(inp, cuda_device)
    drop = (p, 0x1234_5678_9ABC) if p > 0 else None
    raw = ops.moe_forward_train(x, wr, wgu, wd, k, dropout=drop, return_h=True)
    fac = ops.moe_forward_train(x, wr, wgu, wd, k, dropout=drop, return_h=True, factors=True)
    torch.cuda.synchronize()
    for i in range(8):  # y, logits, routing, y_perm: the same
        assert torch.equal(raw[i], fac[i]), i
    assert torch.equal(raw[9], fac[9])  # h, and its zero slack rows
    assert not raw[9][n * k:].any()
    g, u = (t.float().cpu().numpy().astype(np.float64) for t in _split_packed(raw[8], F))
    a, b = (host(t).astype(np.float64) for t in _split_packed(fac[8], F))
    perm = raw[5].cpu().numpy()
    if p > 0:
        m = mo2.dropout_keep(perm, F, p, drop[1]) * float(mo2.dropout_scale(p))
    else:
        m = np.ones_like(g)
    s = 1.0 / (1.0 + np.exp(-g))
    a_ref = m * u * s * (1.0 + g * (1.0 - s))
    b_ref = m * g * s
    for got, ref, name in ((a, a_ref, "A"), (b, b_ref, "B")):
        mx, mean = normwise(got, ref)
        print(f"  {name}: max_rel={mx:.3e} mean_rel={mean:.3e}", flush=True)
        assert mx <= 1.5e-2 and mean <= 4e-3, (name, mx, mean)
        assert np.all(got[m == 0] == 0), name


@pytest.mark.parametrize("counts", [[0, 1, 192, 255, 256, 385, 2000, 4100], [700, 3, 0, 0]])
def test_dh_swiglu_fused_equals_staged(cuda_device, counts):
    """g5moe_dh_swiglu_backward against the staged computation: dh from
    g5moe_grouped_gemm_padded (the same product, stored bf16), times the factors in
    fp32 with one bf16 rounding (torch) — bit for bit in every expert's rows, zeros
    in the rows up to the weight gradient's row count, rows past it untouched."""
    import ctypes
    from genet5_amd import _lib
    dev = cuda_device
    g = torch.Generator(device=dev).manual_seed(3)
    E, d, F, k = len(counts), 768, 512, 2
    offsets = np.zeros(E + 1, np.int32)
    offsets[1:] = np.cumsum(counts)
    T = int(offsets[-1])
    t_off = torch.tensor(offsets, dtype=torch.int32, device=dev)
    kmax = ops.wgrad_kmax(max(counts))
    dy = torch.randn(T + ops.ROW_PAD, d, device=dev, generator=g).to(torch.bfloat16)
    dy_buf = torch.zeros(E * kmax + ops.ROW_PAD, d, dtype=torch.bfloat16, device=dev)
    dy_buf[:E * kmax] = ops.pad_rows(dy, None, t_off, E, kmax, k).view(E * kmax, d)
    wd_t = (torch.randn(E, F, d, device=dev, generator=g) * 0.05).to(torch.bfloat16)
    fac = torch.randn(T, 2 * F, device=dev, generator=g).to(torch.bfloat16)
    sentinel = torch.full((E * kmax + ops.ROW_PAD, 2 * F), -7.0, dtype=torch.bfloat16,
                          device=dev)
    dgu = sentinel.clone()
    n_tok = (T + k - 1) // k
    shape = _lib.make_shape(n_tok, d, F, E, k, _lib.DTYPE_BF16)
    print(f"  counts={counts} kmax={kmax}", flush=True)
    _lib.call("g5moe_dh_swiglu_backward", ops._ptr(dy_buf), kmax, ops._ptr(t_off),
              ops._ptr(wd_t), ops._ptr(fac), ops._ptr(dgu), ctypes.byref(shape),
              ops._stream(dev))
    dh = ops.grouped_gemm_padded(dy_buf, kmax, T, t_off, wd_t)  # [T, F] bf16
    a, b = _split_packed(fac, F)
    dg = (dh.float() * a.float()).to(torch.bfloat16)
    du = (dh.float() * b.float()).to(torch.bfloat16)
    ref = torch.stack([dg.view(T, F // 32, 32), du.view(T, F // 32, 32)], 2).reshape(T, 2 * F)
    torch.cuda.synchronize()
    for e, c in enumerate(counts):
        o0 = int(offsets[e])
        kr = max(384, 192 * -(-c // 192))
        rows = dgu[e * kmax: e * kmax + kmax]
        assert torch.equal(rows[:c], ref[o0:o0 + c]), e
        assert not rows[c:kr].any(), e
        assert torch.equal(rows[kr:], sentinel[:kmax - kr]), e
    assert torch.equal(dgu[E * kmax:], sentinel[E * kmax:])


@pytest.mark.parametrize("n,d,E,k", [(36400, 768, 16, 2), (4097, 768, 16, 2), (1, 768, 16, 2),
                                     (777, 256, 16, 2), (300, 128, 16, 2), (500, 512, 8, 2),
                                     (333, 768, 16, 1)])
def test_input_grad_bit_exact(cuda_device, n, d, E, k):
    """g5moe_input_grad against the C restatement (oracle.input_grad_c, pinned by
    exact rationals) bit for bit: the persistent kernel (k = 2, E = 16, bf16:
    router weights held in registers, rows walked with prefetch, ragged last
    block) and the per-token kernel (other shapes), with skipped positions."""
    import ctypes
    from genet5_amd import _lib
    dev = cuda_device
    g = torch.Generator(device=dev).manual_seed(n + d)
    dxp = torch.randn(n * k, d, device=dev, generator=g).to(torch.bfloat16)
    inv = torch.randperm(n * k, device=dev, generator=g).to(torch.int32)
    inv[::7] = -1
    dl = torch.randn(n, E, device=dev, generator=g) * 0.1
    wr = torch.randn(E, d, device=dev, generator=g).to(torch.bfloat16)
    dx = torch.empty(n, d, dtype=torch.bfloat16, device=dev)
    shape = _lib.make_shape(n, d, 512, E, k, _lib.DTYPE_BF16)
    _lib.call("g5moe_input_grad", ops._ptr(dxp), ops._ptr(inv), ops._ptr(dl), ops._ptr(wr),
              ops._ptr(dx), ctypes.byref(shape), ops._stream(dev))
    torch.cuda.synchronize()
    bits = lambda t: t.cpu().view(torch.int16).numpy().view(np.uint16)
    ref = oracle.input_grad_c(bits(dxp), inv.cpu().numpy(), dl.cpu().numpy(), bits(wr))
    np.testing.assert_array_equal(bits(dx), ref)


@pytest.mark.parametrize("E,F,d", [(16, 3072, 768), (3, 128, 128), (2, 512, 256)])
def test_pack_gate_up_transposed(cuda_device, E, F, d):
    """g5moe_pack_gate_up_transposed: the packed weight bit for bit g5moe_pack_gate_up's,
    and the transpose bit for bit g5moe_transpose_experts of it; with a NULL packed
    output only the transpose is written."""
    import ctypes
    from genet5_amd import _lib
    g = torch.Generator(device=cuda_device).manual_seed(E * F)
    wg = torch.randn(E, F, d, device=cuda_device, generator=g).to(torch.bfloat16)
    wu = torch.randn(E, F, d, device=cuda_device, generator=g).to(torch.bfloat16)
    wgu, wgu_t = ops.pack_gate_up_transposed(wg, wu)
    ref = ops.pack_gate_up(wg, wu)
    ref_t = ops.transpose_experts(ref)
    only_t = torch.empty_like(wgu_t)
    shape = _lib.make_shape(0, d, F, E, 1, _lib.DTYPE_BF16)
    _lib.call("g5moe_pack_gate_up_transposed", ops._ptr(wg), ops._ptr(wu), None,
              ops._ptr(only_t), ctypes.byref(shape), ops._stream(cuda_device))
    torch.cuda.synchronize()
    assert torch.equal(wgu, ref)
    assert torch.equal(wgu_t, ref_t)
    assert torch.equal(only_t, ref_t)
    # against torch: 32-row blocks of gate then up rows per expert, and its transpose
    packed = torch.cat([wg.view(E, F // 32, 32, d), wu.view(E, F // 32, 32, d)], dim=2)
    packed = packed.view(E, 2 * F, d)
    assert torch.equal(wgu, packed)
    assert torch.equal(wgu_t, packed.transpose(1, 2).contiguous())
    # operands and outputs at an odd element offset (2-byte aligned): the same bits
    # through the kernel that makes 2-byte accesses
    n = E * F * d

    def odd(t):
        buf = torch.empty(t.numel() + 1, dtype=torch.bfloat16, device=cuda_device)
        v = buf[1:].view(t.shape)
        v.copy_(t)
        return v

    wg_o, wu_o = odd(wg), odd(wu)
    wgu_o, wgu_t_o = odd(torch.zeros_like(wgu)), odd(torch.zeros_like(wgu_t))
    assert wg_o.data_ptr() % 16 != 0 and wgu_t_o.data_ptr() % 16 != 0 and n > 0
    _lib.call("g5moe_pack_gate_up_transposed", ops._ptr(wg_o), ops._ptr(wu_o), ops._ptr(wgu_o),
              ops._ptr(wgu_t_o), ctypes.byref(shape), ops._stream(cuda_device))
    torch.cuda.synchronize()
    assert torch.equal(wgu_o, packed)
    assert torch.equal(wgu_t_o, wgu_t)


@pytest.mark.parametrize("E,R,C", [(16, 3072, 768), (16, 768, 3072), (3, 128, 192), (1, 64, 64)])
def test_transpose_experts_equals_torch(cuda_device, E, R, C):
    """g5moe_transpose_experts bit for bit torch's transpose(1, 2), with 16-byte
    aligned tensors (the kernel with 16-byte accesses) and with the source and the
    output at an odd element offset (the kernel with 2-byte accesses)."""
    from genet5_amd import _lib
    g = torch.Generator(device=cuda_device).manual_seed(R + C)
    w = torch.randn(E, R, C, device=cuda_device, generator=g).to(torch.bfloat16)
    ref = w.transpose(1, 2).contiguous()
    assert torch.equal(ops.transpose_experts(w), ref)
    wbuf = torch.empty(E * R * C + 1, dtype=torch.bfloat16, device=cuda_device)
    obuf = torch.zeros(E * R * C + 1, dtype=torch.bfloat16, device=cuda_device)
    w_o, out_o = wbuf[1:].view(E, R, C), obuf[1:].view(E, C, R)
    w_o.copy_(w)
    assert w_o.data_ptr() % 16 != 0 and out_o.data_ptr() % 16 != 0
    _lib.call("g5moe_transpose_experts", ops._ptr(w_o), ops._ptr(out_o), E, R, C,
              ops._stream(cuda_device))
    torch.cuda.synchronize()
    assert torch.equal(out_o, ref)
    assert obuf[0].item() == 0  # nothing written before the output


def test_module_autograd_skewed_routing_vs_oracle(cuda_device):
    """The module's training path (factor-storing forward, fused dh + SwiGLU backward,
    sorted-h weight gradient) under skewed routing — a direction shared by the
    tokens and one expert's router row, so that this expert takes about half of
    the assignments and others few — against the float64 oracle backward."""
    torch.manual_seed(17)
    d, F, E, k, n = 768, 3072, 16, 2, 3000
    m = MoEFeedForward(d, F, 0.0, num_experts=E, top_k=k).to(cuda_device).to(torch.bfloat16)
    with torch.no_grad():
        for p in (m.w_gate, m.w_up, m.w_down):
            p.normal_(0, 0.02)
        m.router.weight.normal_(0, 0.05)
        # a direction shared by the tokens and expert 3's router row
        sgn = torch.randint(0, 2, (d,), device=cuda_device).float() * 2 - 1
        m.router.weight[3] += (0.03 * sgn).to(torch.bfloat16)
    x = (torch.randn(n, d, device=cuda_device) + 0.3 * sgn).to(torch.bfloat16).requires_grad_(True)
    R = torch.randn(n, d, device=cuda_device)
    y = m(x)
    (y.float() * R).sum().backward()
    bits = lambda t: t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)
    xb, wrb = bits(x), bits(m.router.weight)
    idx, _ = oracle.topk_gates_c(oracle.router_logits(xb, wrb), k)
    counts = np.bincount(idx.reshape(-1), minlength=E)
    print(f"  counts {counts.tolist()}", flush=True)
    assert counts.max() > 0.4 * n * k
    ref = oracle.moe_backward(xb, wrb, bits(m.w_gate), bits(m.w_up), bits(m.w_down), idx,
                              synth.f32_to_bf16_bits(R.cpu().numpy()))
    check("x.grad", host(x.grad), ref["dx"])
    check("router.grad", host(m.router.weight.grad), ref["d_w_router"])
    check("w_gate.grad", host(m.w_gate.grad), ref["d_w_gate"])
    check("w_up.grad", host(m.w_up.grad), ref["d_w_up"])
    check("w_down.grad", host(m.w_down.grad), ref["d_w_down"])
