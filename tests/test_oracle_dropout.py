"""Pins for the dropout mask (g5moe_dropout, oracle.moe_oracle.dropout_keep) and the
oracle's dropout forward/backward.  The mask is this build's own definition (the
reference's nn.Dropout draws from torch's Philox stream, which is not reproduced),
so it is pinned by an independent restatement plus the statistical properties a
dropout mask must have; the backward with a fixed mask is pinned by finite
differences and torch autograd in float64, as the mask-free backward is."""
import numpy as np
import pytest
import torch

from oracle import moe_oracle as mo


def test_numpy_mask_equals_pure_python():
    rng = np.random.default_rng(0)
    for seed in (0, 1, 2 ** 32 - 1, 2 ** 32, 0x0123456789ABCDEF, 2 ** 64 - 1):
        for p in (0.1, 0.37, 0.5, 0.9):
            a = np.concatenate([rng.integers(0, 2 ** 31, 40), [0, 1, 2 ** 31 - 1]])
            keep = mo.dropout_keep(a, 70, p, seed)
            for i, ai in enumerate(a):
                for f in (0, 1, 2, 3, 31, 32, 68, 69):
                    assert keep[i, f] == mo.dropout_keep_py(int(ai), f, p, seed), (seed, p, ai, f)


def test_fmix32_bijective_with_avalanche():
    x = np.arange(1 << 20, dtype=np.uint32) * np.uint32(2654435761)
    y = mo._fmix32_np(x)
    assert np.unique(y).size == x.size
    # each input bit flips about half of the 32 output bits
    base = mo._fmix32_np(np.arange(4096, dtype=np.uint32))
    for bit in range(32):
        flipped = mo._fmix32_np(np.arange(4096, dtype=np.uint32) ^ np.uint32(1 << bit))
        d = np.unpackbits((base ^ flipped).view(np.uint8)).reshape(4096, 32).sum(1).mean()
        assert 15.0 < d < 17.0, (bit, d)
    assert mo._fmix32_py(0) == 0 and int(mo._fmix32_np(np.array([12345], np.uint32))[0]) == \
        mo._fmix32_py(12345)


@pytest.mark.parametrize("p", [0.1, 0.3, 0.5])
def test_kept_fraction_within_binomial_bound(p):
    keep = mo.dropout_keep(np.arange(4096), 256, p, 99)
    n = keep.size
    q = (65536 - mo.dropout_threshold(p)) / 65536
    assert abs(keep.mean() - q) <= 6 * np.sqrt(q * (1 - q) / n)
    # per row and per column the counts are binomial too (no stuck rows/columns)
    rows = keep.mean(axis=1)
    assert np.abs(rows - q).max() <= 6 * np.sqrt(q * (1 - q) / 256)


def test_neighbours_uncorrelated():
    p, n_rows, n_cols = 0.5, 4096, 256
    k = mo.dropout_keep(np.arange(n_rows), n_cols, p, 7).astype(np.float64)
    lim = lambda n: 6 / np.sqrt(n)
    corr = lambda a, b: np.corrcoef(a.ravel(), b.ravel())[0, 1]
    assert abs(corr(k[:, 0::2], k[:, 1::2])) < lim(k[:, 0::2].size)      # the two halves of a hash
    assert abs(corr(k[:, 1:-1:2], k[:, 2::2])) < lim(k[:, 2::2].size)    # adjacent hashes
    assert abs(corr(k[:-1], k[1:])) < lim(k[1:].size)                    # adjacent rows
    k2 = mo.dropout_keep(np.arange(n_rows), n_cols, p, 8).astype(np.float64)
    assert abs(corr(k, k2)) < lim(k.size)                                # adjacent seeds
    k3 = mo.dropout_keep(np.arange(n_rows), n_cols, p, 7 + (1 << 32)).astype(np.float64)
    assert abs(corr(k, k3)) < lim(k.size)                                # high seed word


def test_threshold_scale_and_extremes():
    assert mo.dropout_threshold(0.0) == 0 and mo.dropout_scale(0.0) == np.float32(1.0)
    assert mo.dropout_keep(np.arange(64), 64, 0.0, 5).all()
    assert mo.dropout_threshold(1.0) == 65536 and mo.dropout_scale(1.0) == 0.0
    assert not mo.dropout_keep(np.arange(64), 64, 1.0, 5).any()
    assert mo.dropout_threshold(0.1) == 6554
    assert mo.dropout_scale(0.1) == np.float32(65536 / (65536 - 6554))
    assert mo.dropout_threshold(0.5) == 32768 and mo.dropout_scale(0.5) == np.float32(2.0)


def problem(seed, N=6, d=64, F=64, E=4, k=2):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((N, d))
    wr = rng.standard_normal((E, d)) * 0.5
    wg = rng.standard_normal((E, F, d)) * 0.2
    wu = rng.standard_normal((E, F, d)) * 0.2
    wd = rng.standard_normal((E, d, F)) * 0.2
    logits = x @ wr.T
    idx = np.argsort(-logits, axis=1, kind="stable")[:, :k].astype(np.int32)
    srt = np.sort(logits, axis=1)[:, ::-1]
    assert np.min(srt[:, k - 1] - srt[:, k]) > 1e-3
    return x, wr, wg, wu, wd, idx, rng.standard_normal((N, d)), rng.standard_normal((N, E))


def test_dropout_backward_matches_central_differences():
    x, wr, wg, wu, wd, idx, R, G = problem(4)
    keep = mo.dropout_keep(np.arange(idx.size), wg.shape[1], 0.3, 11)
    sc = float(mo.dropout_scale(0.3))
    g = mo.moe_backward(x, wr, wg, wu, wd, idx, R, grad_logits=G, keep=keep, scale=sc)
    def loss(**a):
        o = mo.moe_backward(a["x"], a["wr"], a["wg"], a["wu"], a["wd"], idx, np.zeros_like(x),
                            keep=keep, scale=sc)
        return float((o["y"] * R).sum() + ((a["x"] @ a["wr"].T) * G).sum())
    args = dict(x=x, wr=wr, wg=wg, wu=wu, wd=wd)
    names = dict(x="dx", wr="d_w_router", wg="d_w_gate", wu="d_w_up", wd="d_w_down")
    rng = np.random.default_rng(5)
    eps = 1e-6
    for name, arr in args.items():
        v = rng.standard_normal(arr.shape)
        fd = (loss(**dict(args, **{name: arr + eps * v}))
              - loss(**dict(args, **{name: arr - eps * v}))) / (2 * eps)
        an = float((g[names[name]] * v).sum())
        assert abs(fd - an) <= 1e-6 * max(1.0, abs(an)), (name, fd, an)
    # the mask matters: without it the gradients differ
    g0 = mo.moe_backward(x, wr, wg, wu, wd, idx, R, grad_logits=G)
    assert not np.allclose(g0["d_w_down"], g["d_w_down"])


def test_dropout_backward_matches_torch_autograd_float64():
    x, wr, wg, wu, wd, idx, R, G = problem(6, N=20, d=128, F=64, E=5, k=3)
    keep = mo.dropout_keep(np.arange(idx.size), wg.shape[1], 0.25, 3)
    sc = float(mo.dropout_scale(0.25))
    T = lambda a: torch.tensor(a, dtype=torch.float64, requires_grad=True)
    tx, twr, twg, twu, twd = T(x), T(wr), T(wg), T(wu), T(wd)
    ti = torch.from_numpy(idx).long()
    tk = torch.from_numpy(keep.reshape(x.shape[0], idx.shape[1], -1)).double() * sc
    logits = tx @ twr.T
    w = torch.softmax(torch.gather(logits, 1, ti), dim=1)
    y = torch.zeros_like(tx)
    for s in range(ti.shape[1]):
        e = ti[:, s]
        g = (tx[:, None, :] * twg[e]).sum(-1)
        u = (tx[:, None, :] * twu[e]).sum(-1)
        h = torch.nn.functional.silu(g) * u * tk[:, s]
        y = y + w[:, s:s + 1] * (h[:, None, :] * twd[e]).sum(-1)
    L = (y * torch.from_numpy(R)).sum() + (logits * torch.from_numpy(G)).sum()
    L.backward()
    o = mo.moe_backward(x, wr, wg, wu, wd, idx, R, grad_logits=G, keep=keep, scale=sc)
    for name, t in (("dx", tx), ("d_w_router", twr), ("d_w_gate", twg), ("d_w_up", twu),
                    ("d_w_down", twd)):
        np.testing.assert_allclose(o[name], t.grad.numpy(), rtol=1e-10, atol=1e-12,
                                   err_msg=name)


def test_forward_with_dropout_is_masked_composition():
    """moe_forward(dropout=(p, seed)) equals the float64 backward's y with the mask
    of dropout_keep by assignment (two code paths, one definition)."""
    x, wr, wg, wu, wd, idx, _, _ = problem(8, N=30, d=64, F=64, E=4, k=2)
    f32 = lambda a: a.astype(np.float32)
    out = mo.moe_forward(f32(x), f32(wr), f32(wg), f32(wu), f32(wd), 2, dtype=np.float64,
                         dropout=(0.4, 77))
    keep = mo.dropout_keep(np.arange(out["perm"].size), 64, 0.4, 77)
    ref = mo.moe_backward(f32(x), f32(wr), f32(wg), f32(wu), f32(wd), out["topk_idx"],
                          np.zeros_like(x), keep=keep, scale=float(mo.dropout_scale(0.4)))
    np.testing.assert_allclose(out["y"], ref["y"], rtol=1e-5, atol=1e-6)
    plain = mo.moe_forward(f32(x), f32(wr), f32(wg), f32(wu), f32(wd), 2, dtype=np.float64)
    assert not np.allclose(plain["y"], out["y"])
