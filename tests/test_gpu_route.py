"""g5moe_route — the router kernel with the dispatch's rank pass inside it, then
the placement from its per-chunk counts — against g5moe_router_topk followed by
g5moe_dispatch through the C ABI, bit for bit (topk_idx, topk_w, counts,
offsets, perm, inv_pos), and against the definition of the dispatch: perm is
the stable argsort of topk_idx.flatten(), inv_pos its inverse, counts the
per-expert histogram and offsets their exclusive scan.

The router cuts the tokens into chunks of 2 * tpp (one workgroup's tokens per
round), so the shapes cover its regimes: a single 2-token batch, partial last
chunks, one round with idle workgroups, several rounds (N above 768 workgroups
x 128 tokens), each d the router supports, E from 1 to 16, k from 1 to 4, bf16
and f32 activations, and routing pushed by the bias onto one or two experts or
skewed across them.  g5moe_add_rmsnorm_route is checked the same way against
g5moe_add_rmsnorm_router followed by g5moe_dispatch."""
import ctypes

import numpy as np
import pytest
import torch

from genet5_amd import _lib, ops
from test_gpu_parity import host

pytestmark = pytest.mark.gpu

# (N, d, E, k, x dtype, bias)
CASES = [
    (1, 768, 16, 2, "bf16", None),
    (3, 128, 4, 1, "bf16", None),
    (5, 256, 2, 2, "bf16", "one"),
    (37, 512, 16, 4, "f32", None),
    (100, 768, 8, 3, "bf16", "two"),
    (1000, 768, 16, 2, "bf16", None),
    (4550, 768, 16, 2, "bf16", "skew"),
    (36400, 768, 16, 2, "bf16", None),
    (36400, 768, 16, 2, "f32", None),
    (36401, 256, 16, 4, "bf16", None),
    (120000, 768, 16, 2, "bf16", None),
    (200000, 128, 1, 1, "bf16", None),
]


def _bias(kind, E, dev):
    if kind is None:
        return None
    b = torch.zeros(E, dtype=torch.float32, device=dev)
    if kind == "one":
        b[0] = 100.0
    elif kind == "two":
        b[:2] = 100.0
    else:
        b.copy_(torch.linspace(0.0, 2.0, E, device=dev))
    return b


@pytest.mark.parametrize("N,d,E,k,dt,bias_kind", CASES)
def test_route_equals_router_then_dispatch(cuda_device, N, d, E, k, dt, bias_kind):
    dev = cuda_device
    print(f"route N={N} d={d} E={E} k={k} {dt} bias={bias_kind}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(N * 131 + d + E * 7 + k)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    x = torch.randn(N, d, generator=g).to(tdt).to(dev)
    wr = (torch.randn(E, d, generator=g) * 0.05).to(tdt).to(dev)
    bias = _bias(bias_kind, E, dev)
    s = _lib.make_shape(N, d, 256, E, k, _lib.DTYPE_BF16 if dt == "bf16" else _lib.DTYPE_F32)
    S = ops._stream(dev)
    P = ops._ptr
    i32 = dict(dtype=torch.int32, device=dev)
    f32 = dict(dtype=torch.float32, device=dev)
    ws = ops.workspace(s, dev)
    out = []
    for fused in (True, False):
        idx, w = torch.full((N, k), -7, **i32), torch.full((N, k), -7.0, **f32)
        counts, offsets = torch.full((E,), -7, **i32), torch.full((E + 1,), -7, **i32)
        perm, inv = torch.full((N * k,), -7, **i32), torch.full((N * k,), -7, **i32)
        logits = torch.full((N, E), -7.0, **f32) if N % 2 else None   # optional output
        ws.fill_(0xA5)   # nothing the route reads may come from an earlier call
        if fused:
            _lib.call("g5moe_route", P(x), P(wr), P(bias), P(idx), P(w), P(logits), P(counts),
                      P(offsets), P(perm), P(inv), P(ws), ctypes.byref(s), S)
        else:
            _lib.call("g5moe_router_topk", P(x), P(wr), P(bias), P(idx), P(w), P(logits),
                      ctypes.byref(s), S)
            _lib.call("g5moe_dispatch", P(idx), P(counts), P(offsets), P(perm), P(inv), P(ws),
                      ctypes.byref(s), S)
        torch.cuda.synchronize()
        out.append([host(t) for t in (idx, w, counts, offsets, perm, inv)]
                   + ([host(logits)] if logits is not None else []))
    for name, a, b in zip(("topk_idx", "topk_w", "counts", "offsets", "perm", "inv_pos",
                           "logits"), out[0], out[1]):
        assert a.dtype == b.dtype and np.array_equal(a.view(np.uint32), b.view(np.uint32)), name
    idx, _, counts, offsets, perm, inv = out[0][:6]
    flat = idx.reshape(-1).astype(np.int64)
    ref_perm = np.argsort(flat, kind="stable")
    assert np.array_equal(perm, ref_perm)
    assert np.array_equal(inv[ref_perm], np.arange(N * k))
    ref_counts = np.bincount(flat, minlength=E)
    assert np.array_equal(counts, ref_counts)
    assert np.array_equal(offsets, np.concatenate([[0], np.cumsum(ref_counts)]))
    if bias_kind in ("one", "two"):
        assert set(np.unique(idx[:, : (1 if bias_kind == "one" else 2)])) <= {0, 1}


def test_route_empty_batch(cuda_device):
    dev = cuda_device
    print("route N = 0", flush=True)
    E, k = 4, 2
    s = _lib.make_shape(0, 256, 256, E, k, _lib.DTYPE_BF16)
    i32 = dict(dtype=torch.int32, device=dev)
    counts, offsets = torch.full((E,), 7, **i32), torch.full((E + 1,), 7, **i32)
    ws = ops.workspace(s, dev)
    P = ops._ptr
    _lib.call("g5moe_route", None, None, None, None, None, None, P(counts), P(offsets), None,
              None, P(ws), ctypes.byref(s), ops._stream(dev))
    torch.cuda.synchronize()
    assert host(counts).tolist() == [0] * E and host(offsets).tolist() == [0] * (E + 1)


def test_ops_route_equals_stage_calls(cuda_device):
    """ops.route (the Python mirror, with logits, own or caller workspace) against
    ops.router_topk + ops.dispatch."""
    dev = cuda_device
    print("ops.route N=4550 d=768 E=16 k=2", flush=True)
    g = torch.Generator(device="cpu").manual_seed(7)
    x = torch.randn(4550, 768, generator=g).to(torch.bfloat16).to(dev)
    wr = (torch.randn(16, 768, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    idx, w, logits = ops.router_topk(x, wr, 2, return_logits=True)
    ref = (idx, w) + ops.dispatch(idx, 16, 768) + (logits,)
    ws = ops.workspace(_lib.make_shape(4550, 768, 3072, 16, 2, _lib.DTYPE_BF16), dev)
    for kw in (dict(), dict(ws=ws, d_ff=3072)):
        got = ops.route(x, wr, 2, return_logits=True, **kw)
        torch.cuda.synchronize()
        for a, b in zip(got, ref):
            assert torch.equal(a.view(torch.int32), b.view(torch.int32))


# (N, d, E, k, x dtype, x_add given)
NORM_CASES = [
    (1, 768, 16, 2, "bf16", True),
    (3, 128, 4, 1, "bf16", False),
    (37, 512, 16, 4, "f32", True),
    (100, 768, 8, 3, "bf16", False),
    (4550, 768, 16, 2, "bf16", True),
    (45500, 768, 16, 2, "bf16", True),
    (45500, 768, 16, 2, "bf16", False),
    (36401, 256, 16, 4, "f32", False),
    (120000, 768, 16, 2, "bf16", True),
]


@pytest.mark.parametrize("N,d,E,k,dt,with_add", NORM_CASES)
def test_add_rmsnorm_route_equals_norm_router_then_dispatch(cuda_device, N, d, E, k, dt,
                                                            with_add):
    """g5moe_add_rmsnorm_route against g5moe_add_rmsnorm_router followed by
    g5moe_dispatch, bit for bit: normed rows, the sum, topk_idx, topk_w, logits,
    counts, offsets, perm, inv_pos.  Its router grid (two workgroups per CU)
    differs from the plain router's, so its chunks do too."""
    dev = cuda_device
    print(f"add_rmsnorm_route N={N} d={d} E={E} k={k} {dt} x_add={with_add}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(N * 17 + d + E * 5 + k)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    res = torch.randn(N, d, generator=g).to(tdt).to(dev)
    xa = torch.randn(N, d, generator=g).to(tdt).to(dev) if with_add else None
    nw = (1.0 + 0.1 * torch.randn(d, generator=g)).to(dev)
    wr = (torch.randn(E, d, generator=g) * 0.05).to(tdt).to(dev)
    bias = _bias("skew", E, dev) if N % 3 == 0 else None
    s = _lib.make_shape(N, d, 256, E, k, _lib.DTYPE_BF16 if dt == "bf16" else _lib.DTYPE_F32)
    S = ops._stream(dev)
    P = ops._ptr
    i32 = dict(dtype=torch.int32, device=dev)
    f32 = dict(dtype=torch.float32, device=dev)
    ws = ops.workspace(s, dev)
    eps = ctypes.c_float(1e-6)
    out = []
    for fused in (True, False):
        normed = torch.full((N, d), -7.0, dtype=tdt, device=dev)
        ssum = torch.full((N, d), -7.0, dtype=tdt, device=dev) if with_add else None
        idx, w = torch.full((N, k), -7, **i32), torch.full((N, k), -7.0, **f32)
        counts, offsets = torch.full((E,), -7, **i32), torch.full((E + 1,), -7, **i32)
        perm, inv = torch.full((N * k,), -7, **i32), torch.full((N * k,), -7, **i32)
        logits = torch.full((N, E), -7.0, **f32) if N % 2 else None
        ws.fill_(0xA5)
        if fused:
            _lib.call("g5moe_add_rmsnorm_route", P(xa), P(res), P(nw), eps, P(wr), P(bias),
                      P(ssum), P(normed), P(idx), P(w), P(logits), P(counts), P(offsets),
                      P(perm), P(inv), P(ws), ctypes.byref(s), S)
        else:
            _lib.call("g5moe_add_rmsnorm_router", P(xa), P(res), P(nw), eps, P(wr), P(bias),
                      P(ssum), P(normed), P(idx), P(w), P(logits), ctypes.byref(s), S)
            _lib.call("g5moe_dispatch", P(idx), P(counts), P(offsets), P(perm), P(inv), P(ws),
                      ctypes.byref(s), S)
        torch.cuda.synchronize()
        out.append([host(t.view(torch.int16) if t.dtype == torch.bfloat16 else t)
                    for t in (normed, idx, w, counts, offsets, perm, inv)]
                   + ([host(ssum.view(torch.int16) if tdt == torch.bfloat16 else ssum)]
                      if with_add else [])
                   + ([host(logits)] if logits is not None else []))
    for i, (a, b) in enumerate(zip(out[0], out[1])):
        assert a.dtype == b.dtype and np.array_equal(a, b), i
    idx, counts, perm = out[0][1], out[0][3], out[0][5]
    flat = idx.reshape(-1).astype(np.int64)
    assert np.array_equal(perm, np.argsort(flat, kind="stable"))
    assert np.array_equal(counts, np.bincount(flat, minlength=E))


def test_add_rmsnorm_route_empty_batch(cuda_device):
    dev = cuda_device
    print("add_rmsnorm_route N = 0", flush=True)
    E, k = 4, 2
    s = _lib.make_shape(0, 256, 256, E, k, _lib.DTYPE_BF16)
    i32 = dict(dtype=torch.int32, device=dev)
    counts, offsets = torch.full((E,), 7, **i32), torch.full((E + 1,), 7, **i32)
    ws = ops.workspace(s, dev)
    P = ops._ptr
    _lib.call("g5moe_add_rmsnorm_route", None, None, None, ctypes.c_float(1e-6), None, None,
              None, None, None, None, None, P(counts), P(offsets), None, None, P(ws),
              ctypes.byref(s), ops._stream(dev))
    torch.cuda.synchronize()
    assert host(counts).tolist() == [0] * E and host(offsets).tolist() == [0] * (E + 1)


def test_ops_add_rmsnorm_route_equals_stage_calls(cuda_device):
    """ops.add_rmsnorm_route (with logits, own or caller workspace) against
    ops.add_rmsnorm_router + ops.dispatch."""
    dev = cuda_device
    print("ops.add_rmsnorm_route N=4550 d=768 E=16 k=2", flush=True)
    g = torch.Generator(device="cpu").manual_seed(11)
    res = torch.randn(4550, 768, generator=g).to(torch.bfloat16).to(dev)
    xa = torch.randn(4550, 768, generator=g).to(torch.bfloat16).to(dev)
    nw = torch.ones(768, device=dev)
    wr = (torch.randn(16, 768, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    normed, ssum, idx, w, logits = ops.add_rmsnorm_router(res, nw, 1e-6, wr, 2, x_add=xa,
                                                          return_logits=True)
    ref = (normed, ssum, idx, w) + ops.dispatch(idx, 16, 768) + (logits,)
    ws = ops.workspace(_lib.make_shape(4550, 768, 3072, 16, 2, _lib.DTYPE_BF16), dev)
    for kw in (dict(), dict(ws=ws, d_ff=3072)):
        got = ops.add_rmsnorm_route(res, nw, 1e-6, wr, 2, x_add=xa, return_logits=True, **kw)
        torch.cuda.synchronize()
        for a, b in zip(got, ref):
            assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else
                               a.view(torch.int32),
                               b.view(torch.int16) if b.dtype == torch.bfloat16 else
                               b.view(torch.int32))
