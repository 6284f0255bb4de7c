"""GPU parity of the pre-norm and residual-combine entry points, through the C ABI.

g5moe_add_rmsnorm_router: the sum rows, the normed rows and the router logits are
bit-exact against the C oracle (the reduction order, the correctly rounded division
and sqrt and every rounding are fixed by the contract); top-k indices equal; gates
within 2e-6 of the oracle's float64 softmax; and the routing equals what
g5moe_router_topk gives on the normed rows the kernel wrote.

g5moe_combine / g5moe_combine_residual: bit-exact against the C oracle (fma in slot
order, one rounding, then the residual composition's roundings).
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import moe_oracle as mo
from genet5_amd import ops, synth
from test_gpu_parity import dev_t

pytestmark = pytest.mark.gpu


def as_dev(a: np.ndarray, device) -> torch.Tensor:
    return dev_t(a, device, bf16=(a.dtype == np.uint16))


def bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy().view(np.uint32)


def act(rng, shape, dtype, scale=1.0):
    a = (rng.standard_normal(shape) * scale).astype(np.float32)
    return synth.f32_to_bf16_bits(a) if dtype == "bf16" else a


@pytest.mark.parametrize("n,d,E,k,dtype,add", [
    (36400, 768, 16, 2, "bf16", True),
    (2048, 768, 16, 2, "f32", True),
    (1000, 512, 8, 2, "bf16", False),
    (333, 256, 16, 4, "f32", False),
    (1, 128, 4, 1, "bf16", True),
    (65, 128, 5, 1, "bf16", False),
])
def test_add_rmsnorm_router_bit_exact(cuda_device, n, d, E, k, dtype, add):
    print(f"add_rmsnorm_router n={n} d={d} E={E} k={k} {dtype} add={add}", flush=True)
    rng = np.random.default_rng(n + d)
    res = act(rng, (n, d), dtype)
    xa = act(rng, (n, d), dtype, 0.5) if add else None
    nw = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    wr = act(rng, (E, d), dtype, 0.02)
    bias = synth.zipf_router_bias(E) if E == 16 else None
    eps = 1e-6
    dev = cuda_device
    normed, ssum, idx, w, logits = ops.add_rmsnorm_router(
        as_dev(res, dev), as_dev(nw, dev), eps, as_dev(wr, dev), k,
        x_add=None if xa is None else as_dev(xa, dev),
        bias=None if bias is None else as_dev(bias, dev), return_logits=True)
    torch.cuda.synchronize()
    n_ref, s_ref = oracle.add_rmsnorm(res, nw, eps, xa)
    np.testing.assert_array_equal(bits(normed), n_ref.view(bits(normed).dtype))
    if add:
        np.testing.assert_array_equal(bits(ssum), s_ref.view(bits(ssum).dtype))
    else:
        assert ssum is None
    l_ref = oracle.router_logits(n_ref, wr, bias)
    np.testing.assert_array_equal(bits(logits), l_ref.view(np.uint32))
    i_ref, g_ref = oracle.topk_gates_c(l_ref, k)
    np.testing.assert_array_equal(idx.cpu().numpy(), i_ref)
    np.testing.assert_allclose(w.cpu().numpy(), g_ref, rtol=0, atol=2e-6)
    # composition: the fused routing is the router applied to the rows it wrote
    idx2, w2 = ops.router_topk(normed, as_dev(wr, dev), k,
                               bias=None if bias is None else as_dev(bias, dev))
    assert torch.equal(idx2, idx) and torch.equal(w2, w)


@pytest.mark.parametrize("n,d,dtype,add", [
    (36400, 768, "bf16", False),
    (2049, 768, "bf16", True),
    (1000, 512, "f32", True),
    (17, 256, "f32", False),
    (1, 128, "bf16", True),
])
def test_rmsnorm_bit_exact(cuda_device, n, d, dtype, add):
    """g5moe_rmsnorm: normed and sum rows bit-exact against the C oracle's add_rmsnorm
    and equal to the fused norm+router kernel's normed rows."""
    print(f"rmsnorm n={n} d={d} {dtype} add={add}", flush=True)
    rng = np.random.default_rng(n * 7 + d)
    res = act(rng, (n, d), dtype)
    xa = act(rng, (n, d), dtype, 0.5) if add else None
    nw = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    dev = cuda_device
    r_t, nw_t = as_dev(res, dev), as_dev(nw, dev)
    xa_t = None if xa is None else as_dev(xa, dev)
    if add:
        normed, ssum = ops.rmsnorm(r_t, nw_t, 1e-6, x_add=xa_t, return_sum=True)
    else:
        normed, ssum = ops.rmsnorm(r_t, nw_t, 1e-6), None
    wr = as_dev(act(rng, (4, d), dtype, 0.02), dev)
    fused, fsum, _, _ = ops.add_rmsnorm_router(r_t, nw_t, 1e-6, wr, 1, x_add=xa_t)
    torch.cuda.synchronize()
    n_ref, s_ref = oracle.add_rmsnorm(res, nw, 1e-6, xa)
    np.testing.assert_array_equal(bits(normed), n_ref.view(bits(normed).dtype))
    assert torch.equal(normed, fused)
    if add:
        np.testing.assert_array_equal(bits(ssum), s_ref.view(bits(ssum).dtype))
        assert torch.equal(ssum, fsum)


def test_add_rmsnorm_router_rejects_sum_without_add(cuda_device):
    from genet5_amd import _lib
    import ctypes
    s = _lib.make_shape(4, 128, 128, 4, 1, _lib.DTYPE_BF16)
    t = torch.zeros(4, 128, dtype=torch.bfloat16, device=cuda_device)
    st = _lib.lib().g5moe_add_rmsnorm_router(
        None, ctypes.c_void_p(t.data_ptr()), ctypes.c_void_p(t.data_ptr()), ctypes.c_float(1e-6),
        ctypes.c_void_p(t.data_ptr()), None, ctypes.c_void_p(t.data_ptr()),
        ctypes.c_void_p(t.data_ptr()), ctypes.c_void_p(t.data_ptr()),
        ctypes.c_void_p(t.data_ptr()), None, ctypes.byref(s), None)
    assert st == 1 and b"sum_out" in _lib.lib().g5moe_last_error()


def combine_inputs(rng, n, d, k):
    y_perm = synth.f32_to_bf16_bits(rng.standard_normal((n * k, d)).astype(np.float32))
    inv = rng.permutation(n * k).astype(np.int32)
    if n * k > 4:
        inv[rng.choice(n * k, size=max(1, n * k // 50), replace=False)] = -1
    w = rng.random((n, k)).astype(np.float32)
    w /= w.sum(axis=1, keepdims=True)
    return y_perm, inv, w


@pytest.mark.parametrize("n,d,k,dtype,alpha", [
    (36400, 768, 2, "bf16", 1.0),
    (999, 768, 2, "f32", 1.0 / np.sqrt(3.0)),
    (100, 256, 4, "bf16", 1.0 / np.sqrt(2.0)),
    (1, 128, 1, "bf16", 1.0),
])
def test_combine_and_combine_residual_bit_exact(cuda_device, n, d, k, dtype, alpha):
    print(f"combine n={n} d={d} k={k} {dtype} alpha={alpha:.4f}", flush=True)
    rng = np.random.default_rng(n * k + d)
    y_perm, inv, w = combine_inputs(rng, n, d, k)
    res = act(rng, (n, d), dtype)
    dev = cuda_device
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    ty, ti, tw = as_dev(y_perm, dev), as_dev(inv, dev), as_dev(w, dev)
    y = ops.combine(ty, ti, tw, tdt)
    tr = as_dev(res, dev)
    out = ops.combine_residual(ty, ti, tw, tr, alpha)
    torch.cuda.synchronize()
    ref_y = oracle.combine_c(y_perm, inv, w, out_dtype=dtype)
    np.testing.assert_array_equal(bits(y), ref_y.view(bits(y).dtype))
    ref = oracle.combine_c(y_perm, inv, w, res, alpha, out_dtype=dtype)
    np.testing.assert_array_equal(bits(out), ref.view(bits(out).dtype))
    # in place: out aliases the residual
    ops.combine_residual(ty, ti, tw, tr, alpha, out=tr)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(tr), ref.view(bits(tr).dtype))
