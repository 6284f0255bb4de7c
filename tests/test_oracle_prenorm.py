"""Pins for the oracle's pre-norm (residual add + RMSNorm) and combine restatements
(oracle.add_rmsnorm, oracle.add_rmsnorm_np, oracle.combine_c): each checked against
an independent restatement, a library routine (torch's own bf16 ops), a closed form
or float64, chosen so that a plausible mistake (sequential instead of tree order,
rsqrt instead of the correctly rounded sqrt and division, a dropped rounding, a
fused product in the residual sum) fails one of them."""
from fractions import Fraction

import numpy as np
import pytest
import torch

import oracle
from oracle import moe_oracle as mo
from genet5_amd import synth
from test_oracle import add_exact, fma_exact, round_f32


def bf16_bits(a: np.ndarray) -> np.ndarray:
    return synth.f32_to_bf16_bits(np.asarray(a, np.float32))


def rows(n, d, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    return mo.round_bf16((rng.standard_normal((n, d)) * scale).astype(np.float32))


# ---- add + RMSNorm ---------------------------------------------------------------

@pytest.mark.parametrize("n,d,add,eps", [(300, 768, True, 1e-6), (64, 128, False, 1e-6),
                                         (33, 512, True, 1e-5), (5, 256, False, 0.0)])
def test_add_rmsnorm_c_equals_numpy_restatement_bf16(n, d, add, eps):
    r = rows(n, d, 1)
    xa = rows(n, d, 2, 0.5) if add else None
    w = np.random.default_rng(3).standard_normal(d).astype(np.float32)
    nc, sc = oracle.add_rmsnorm(bf16_bits(r), w, eps, None if xa is None else bf16_bits(xa))
    nn, sn = oracle.add_rmsnorm_np(r, w, eps, xa)
    np.testing.assert_array_equal(mo.bf16_to_f32(nc).view(np.uint32), nn.view(np.uint32))
    if add:
        np.testing.assert_array_equal(mo.bf16_to_f32(sc).view(np.uint32), sn.view(np.uint32))
    else:
        assert sc is None and sn is None


def rmsnorm_pure(r: np.ndarray, w: np.ndarray, eps: float, xa=None) -> np.ndarray:
    """Exact-rational restatement for fp32 rows (fma, division and sqrt rounded once)."""
    N, d = r.shape
    L = d // 64
    out = np.zeros((N, d), np.float32)
    for t in range(N):
        s = [r[t, j] if xa is None else add_exact(xa[t, j], r[t, j]) for j in range(d)]
        lanes = []
        for c in range(64):
            acc = np.float32(0.0)
            for i in range(L):
                acc = fma_exact(s[c * L + i], s[c * L + i], acc)
            lanes.append(acc)
        for bit in (32, 16, 8, 4, 2, 1):
            lanes = [add_exact(lanes[l], lanes[l + bit]) for l in range(bit)]
        mean = round_f32(Fraction(float(lanes[0])) / d)
        v = add_exact(mean, np.float32(eps))
        root = np.float32(np.sqrt(np.float64(v)))  # f64 sqrt of an f32, rounded to f32: exact rounding
        rstd = round_f32(Fraction(1) / Fraction(float(root)))
        for j in range(d):
            a = round_f32(Fraction(float(s[j])) * Fraction(float(rstd)))
            out[t, j] = round_f32(Fraction(float(a)) * Fraction(float(w[j])))
    return out


def test_add_rmsnorm_c_matches_exact_rational_fp32():
    """fp32 rows, where s*s is inexact and the fused multiply-add is visible."""
    rng = np.random.default_rng(7)
    r = rng.standard_normal((2, 128)).astype(np.float32)
    xa = rng.standard_normal((2, 128)).astype(np.float32)
    w = rng.standard_normal(128).astype(np.float32)
    got, _ = oracle.add_rmsnorm(r, w, 1e-6, xa)
    ref = rmsnorm_pure(r, w, 1e-6, xa)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_add_rmsnorm_power_of_two_rows_known_answer():
    """Rows of +-2^p with eps = 0: ss = d * 4^p exactly, rstd = 2^-p exactly, so the
    output is T(sign * w) bit for bit."""
    d = 768
    w = mo.round_bf16(np.random.default_rng(0).standard_normal(d).astype(np.float32))
    sign = np.where(np.random.default_rng(1).random(d) < 0.5, -1.0, 1.0).astype(np.float32)
    r = np.stack([sign * np.float32(2.0 ** p) for p in (-6, 0, 5)])
    got, _ = oracle.add_rmsnorm(bf16_bits(r), w, 0.0)
    np.testing.assert_array_equal(mo.bf16_to_f32(got), np.broadcast_to(sign * w, r.shape))


def test_rmsnorm_sum_order_is_the_lane_tree():
    """A row whose sum of squares rounds differently in sequential order: the
    oracle follows the contract's lane/tree order."""
    d = 128  # L = 2: lane c holds columns 2c, 2c + 1
    s = np.zeros((1, d), np.float32)
    s[0, 0] = 4096.0          # square 2^24 in lane 0
    s[0, 2::2] = 1.0          # squares of 1 in lanes 1..63
    w = np.ones(d, np.float32)
    seq = np.float32(0)
    for v in s[0]:
        seq = np.float32(seq + np.float32(v * v))
    # the contract's tree over the 64 lane partials (each lane: 2 squares)
    lanes = (s.reshape(64, 2) ** 2).sum(axis=1).astype(np.float32)
    m = 32
    while m >= 1:
        lanes = lanes[:m] + lanes[m:2 * m]
        m //= 2
    assert lanes[0] != seq  # the two orders round differently on this row
    nc, _ = oracle.add_rmsnorm(bf16_bits(s), w, 0.0)
    rstd_tree = np.float32(1) / np.sqrt(lanes[0] / np.float32(d))
    rstd_seq = np.float32(1) / np.sqrt(seq / np.float32(d))
    assert rstd_tree != rstd_seq
    expect = mo.round_bf16(s * rstd_tree)
    np.testing.assert_array_equal(mo.bf16_to_f32(nc), expect)


def test_add_rmsnorm_close_to_float64():
    r = rows(200, 768, 11, 3.0)
    xa = rows(200, 768, 12, 0.1)
    w = np.random.default_rng(13).standard_normal(768).astype(np.float32)
    got, s = oracle.add_rmsnorm(r, w, 1e-6, xa)  # fp32 rows: no output rounding
    s64 = r.astype(np.float64) + xa.astype(np.float64)
    ref = s64 / np.sqrt((s64 ** 2).mean(axis=1, keepdims=True) + 1e-6) * w.astype(np.float64)
    assert np.max(np.abs(got - ref)) <= 8 * np.finfo(np.float32).eps * np.max(np.abs(ref))


def test_residual_add_equals_torch_bf16_add():
    r = rows(64, 256, 21)
    xa = rows(64, 256, 22, 0.3)
    _, s = oracle.add_rmsnorm(bf16_bits(r), np.ones(256, np.float32), 1e-6, bf16_bits(xa))
    ref = (torch.from_numpy(xa).to(torch.bfloat16) + torch.from_numpy(r).to(torch.bfloat16))
    np.testing.assert_array_equal(s, ref.view(torch.int16).numpy().view(np.uint16))


# ---- combine ---------------------------------------------------------------------

def combine_case(n, d, k, seed):
    rng = np.random.default_rng(seed)
    y_perm = bf16_bits(rng.standard_normal((n * k, d)).astype(np.float32))
    inv = rng.permutation(n * k).astype(np.int32)
    w = rng.random((n, k)).astype(np.float32)
    w /= w.sum(axis=1, keepdims=True)
    return y_perm, inv, w


def test_combine_c_k1_unit_gate_is_identity():
    y_perm, inv, _ = combine_case(50, 256, 1, 0)
    w = np.ones((50, 1), np.float32)
    out = oracle.combine_c(y_perm, inv, w)
    np.testing.assert_array_equal(out, y_perm[inv])
    out32 = oracle.combine_c(y_perm, inv, w, out_dtype="f32")
    np.testing.assert_array_equal(out32, mo.bf16_to_f32(y_perm[inv]))


def test_combine_c_matches_exact_rational():
    y_perm, inv, w = combine_case(3, 64, 2, 1)
    inv[1] = -1  # a skipped slot
    got = oracle.combine_c(y_perm, inv, w, out_dtype="f32")
    yp = mo.bf16_to_f32(y_perm)
    for t in range(3):
        for j in range(64):
            acc = np.float32(0)
            for s in range(2):
                p = inv[t * 2 + s]
                if p >= 0:
                    acc = fma_exact(w[t, s], yp[p, j], acc)
            assert got[t, j].view(np.uint32) == np.float32(acc).view(np.uint32)


@pytest.mark.parametrize("alpha", [1.0, 1.0 / np.sqrt(3.0)])
def test_combine_residual_equals_torch_composition(alpha):
    """out = residual + y * alpha with torch's own bf16 (and fp32) elementwise ops."""
    y_perm, inv, w = combine_case(40, 128, 2, 2)
    res = rows(40, 128, 3)
    y = oracle.combine_c(y_perm, inv, w)  # the MoE output, bf16
    out = oracle.combine_c(y_perm, inv, w, bf16_bits(res), alpha)
    tr = torch.from_numpy(res).to(torch.bfloat16)
    ty = torch.from_numpy(y.view(np.int16)).view(torch.bfloat16)
    ref = tr + ty * alpha
    np.testing.assert_array_equal(out, ref.view(torch.int16).numpy().view(np.uint16))
    y32 = oracle.combine_c(y_perm, inv, w, out_dtype="f32")
    out32 = oracle.combine_c(y_perm, inv, w, res, alpha, out_dtype="f32")
    ref32 = torch.from_numpy(res) + torch.from_numpy(y32) * np.float32(alpha)
    np.testing.assert_array_equal(out32.view(np.uint32), ref32.numpy().view(np.uint32))


def test_input_grad_c_matches_exact_rational():
    """oracle.input_grad_c: each slot addition and each fma rounded once to fp32, in
    slot then expert order (a skipped position included); fp32 and bf16 outputs."""
    rng = np.random.default_rng(4)
    n, d, k, E = 3, 64, 2, 5
    dxp = bf16_bits(rng.standard_normal((n * k, d)).astype(np.float32))
    inv = rng.permutation(n * k).astype(np.int32)
    inv[3] = -1
    dl = (rng.standard_normal((n, E)) * 0.1).astype(np.float32)
    wr = rng.standard_normal((E, d)).astype(np.float32)
    got = oracle.input_grad_c(dxp, inv, dl, wr, out_dtype="f32")
    xp = mo.bf16_to_f32(dxp)
    for t in range(n):
        for j in range(d):
            acc = np.float32(0)
            for s in range(k):
                p = inv[t * k + s]
                if p >= 0:
                    acc = add_exact(acc, xp[p, j])
            for e in range(E):
                acc = fma_exact(dl[t, e], wr[e, j], acc)
            assert got[t, j].view(np.uint32) == np.float32(acc).view(np.uint32), (t, j)
    wb = bf16_bits(wr)
    gb = oracle.input_grad_c(dxp, inv, dl, wb, out_dtype="bf16")
    g32 = oracle.input_grad_c(dxp, inv, dl, mo.bf16_to_f32(wb), out_dtype="f32")
    np.testing.assert_array_equal(gb, bf16_bits(g32))


def test_input_grad_c_without_logits_is_slot_sum():
    rng = np.random.default_rng(5)
    dxp = bf16_bits(rng.standard_normal((40, 128)).astype(np.float32))
    inv = rng.permutation(40).astype(np.int32)
    out = oracle.input_grad_c(dxp, inv, np.zeros((20, 16), np.float32),
                              np.ones((16, 128), np.float32), out_dtype="f32")
    xp = mo.bf16_to_f32(dxp)[inv].reshape(20, 2, 128)
    np.testing.assert_array_equal(out, xp[:, 0] + xp[:, 1])
