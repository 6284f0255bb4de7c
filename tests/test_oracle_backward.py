"""Pins for the oracle's float64 backward (oracle.moe_backward): central finite
differences of a scalar loss in random directions, and torch.autograd (float64,
CPU) on an independent torch restatement of the same forward.  A wrong SwiGLU
derivative, a dropped gate factor, a missing renormalisation term or a transposed
weight gradient fails both."""
import numpy as np
import pytest
import torch

import oracle


def problem(seed, N=6, d=64, F=64, E=4, k=2):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((N, d))
    wr = rng.standard_normal((E, d)) * 0.5
    wg = rng.standard_normal((E, F, d)) * 0.2
    wu = rng.standard_normal((E, F, d)) * 0.2
    wd = rng.standard_normal((E, d, F)) * 0.2
    logits = x @ wr.T
    idx = np.argsort(-logits, axis=1, kind="stable")[:, :k].astype(np.int32)
    # the perturbations below must not change the top-k choice
    srt = np.sort(logits, axis=1)[:, ::-1]
    assert np.min(srt[:, k - 1] - srt[:, k]) > 1e-3
    R = rng.standard_normal((N, d))
    G = rng.standard_normal((N, E))
    return x, wr, wg, wu, wd, idx, R, G


def loss(x, wr, wg, wu, wd, idx, R, G):
    """L = sum(y * R) + sum(logits * G) with the oracle forward for fixed routing."""
    out = oracle.moe_backward(x, wr, wg, wu, wd, idx, np.zeros_like(x))
    return float((out["y"] * R).sum() + ((x @ wr.T) * G).sum())


@pytest.mark.parametrize("seed", [0, 1])
def test_backward_matches_central_differences(seed):
    x, wr, wg, wu, wd, idx, R, G = problem(seed)
    g = oracle.moe_backward(x, wr, wg, wu, wd, idx, R, grad_logits=G)
    rng = np.random.default_rng(100 + seed)
    eps = 1e-6
    args = dict(x=x, wr=wr, wg=wg, wu=wu, wd=wd)
    names = dict(x="dx", wr="d_w_router", wg="d_w_gate", wu="d_w_up", wd="d_w_down")
    for name, arr in args.items():
        v = rng.standard_normal(arr.shape)
        plus = dict(args, **{name: arr + eps * v})
        minus = dict(args, **{name: arr - eps * v})
        fd = (loss(idx=idx, R=R, G=G, **plus) - loss(idx=idx, R=R, G=G, **minus)) / (2 * eps)
        an = float((g[names[name]] * v).sum())
        assert abs(fd - an) <= 1e-6 * max(1.0, abs(an)), (name, fd, an)


def test_backward_matches_torch_autograd_float64():
    x, wr, wg, wu, wd, idx, R, G = problem(3, N=20, d=128, F=64, E=5, k=3)
    T = lambda a: torch.tensor(a, dtype=torch.float64, requires_grad=True)
    tx, twr, twg, twu, twd = T(x), T(wr), T(wg), T(wu), T(wd)
    ti = torch.from_numpy(idx).long()
    logits = tx @ twr.T
    w = torch.softmax(torch.gather(logits, 1, ti), dim=1)
    y = torch.zeros_like(tx)
    for s in range(ti.shape[1]):
        e = ti[:, s]
        g = torch.einsum("nd,nfd->nf", tx, twg[e])
        u = torch.einsum("nd,nfd->nf", tx, twu[e])
        h = torch.nn.functional.silu(g) * u
        y = y + w[:, s:s + 1] * torch.einsum("nf,ndf->nd", h, twd[e])
    L = (y * torch.from_numpy(R)).sum() + (logits * torch.from_numpy(G)).sum()
    L.backward()
    o = oracle.moe_backward(x, wr, wg, wu, wd, idx, R, grad_logits=G)
    for name, t in (("dx", tx), ("d_w_router", twr), ("d_w_gate", twg), ("d_w_up", twu),
                    ("d_w_down", twd)):
        np.testing.assert_allclose(o[name], t.grad.numpy(), rtol=1e-10, atol=1e-12,
                                   err_msg=name)
    np.testing.assert_allclose(o["y"], y.detach().numpy(), rtol=1e-12, atol=1e-12)
