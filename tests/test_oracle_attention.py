"""Pins for the oracle's varlen ALiBi attention (oracle.attention_varlen): a library
routine (torch's scaled_dot_product_attention in float64 with the bias as an explicit
mask), closed forms and structural invariants, chosen so that a plausible mistake
(a wrong bias sign, global instead of sequence-local positions, a transposed score
matrix, a missing scale, the wrong key/value head for a query head, attending across
sequences) fails one of them.  Also the C ABI's argument checks for the attention
entry point, which run before any GPU work."""
import ctypes
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from genet5_amd import _lib
from genet5_amd.attention import alibi_slopes


def rand_qkv(T, H, Hkv, D, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((T, H, D)) * scale
    k = rng.standard_normal((T, Hkv, D)) * scale
    v = rng.standard_normal((T, Hkv, D))
    return q, k, v


def sdpa_reference(q, k, v, cu, scale, slopes):
    """torch SDPA (float64, CPU) per sequence with the ALiBi bias as attn_mask."""
    T, H, D = q.shape
    g = H // k.shape[1]
    out = np.zeros((T, H, D))
    for a, b in zip(cu[:-1], cu[1:]):
        if b <= a:
            continue
        L = b - a
        qs = torch.tensor(q[a:b]).permute(1, 0, 2)                       # [H, L, D]
        ks = torch.tensor(k[a:b]).repeat_interleave(g, dim=1).permute(1, 0, 2)
        vs = torch.tensor(v[a:b]).repeat_interleave(g, dim=1).permute(1, 0, 2)
        pos = torch.arange(L, dtype=torch.float64)
        dist = (pos[:, None] - pos[None, :]).abs()
        bias = -torch.tensor(slopes, dtype=torch.float64)[:, None, None] * dist[None]
        o = F.scaled_dot_product_attention(qs, ks, vs, attn_mask=bias, scale=scale)
        out[a:b] = o.permute(1, 0, 2).numpy()
    return out


@pytest.mark.parametrize("cu,H,Hkv,D", [([0, 5, 22, 23, 63], 4, 2, 16),
                                        ([0, 70, 140], 6, 6, 64),
                                        ([0, 3, 3, 40], 3, 1, 8)])
def test_equals_torch_sdpa_with_explicit_bias(cu, H, Hkv, D):
    q, k, v = rand_qkv(cu[-1], H, Hkv, D, seed=1, scale=1.5)
    slopes = np.array(alibi_slopes(H)) * 4.0
    scale = 1.0 / math.sqrt(D)
    got = oracle.attention_varlen(q, k, v, cu, scale, slopes)
    ref = sdpa_reference(q, k, v, cu, scale, slopes)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_zero_queries_no_bias_give_sequence_mean():
    cu = [0, 7, 20]
    q, k, v = rand_qkv(20, 2, 2, 8, seed=2)
    got = oracle.attention_varlen(np.zeros_like(q), k, v, cu, 0.125, None)
    for a, b in zip(cu[:-1], cu[1:]):
        np.testing.assert_allclose(got[a:b], np.broadcast_to(v[a:b].mean(0), got[a:b].shape),
                                   rtol=1e-13, atol=1e-13)


def test_zero_queries_with_slope_give_geometric_weights():
    # second sequence starts at token 9: positions must be sequence-local
    cu = [0, 9, 30]
    s = 0.37
    q, k, v = rand_qkv(30, 1, 1, 4, seed=3)
    got = oracle.attention_varlen(np.zeros_like(q), k, v, cu, 0.5, [s])
    for a, b in zip(cu[:-1], cu[1:]):
        L = b - a
        for i in range(L):
            w = np.array([math.exp(-s * abs(i - j)) for j in range(L)])
            expect = (w[:, None] * v[a:b, 0]).sum(0) / w.sum()
            np.testing.assert_allclose(got[a + i, 0], expect, rtol=1e-12, atol=1e-13)


def test_dominant_key_returns_its_value():
    T, D = 12, 16
    q = np.zeros((T, 1, D))
    k = np.zeros((T, 1, D))
    v = np.random.default_rng(4).standard_normal((T, 1, D))
    q[:, 0, 0] = 30.0
    k[5, 0, 0] = 30.0
    got = oracle.attention_varlen(q, k, v, [0, T], 1.0 / 4.0, None)
    np.testing.assert_allclose(got[:, 0], np.broadcast_to(v[5, 0], (T, D)), atol=1e-12)


def test_packing_equals_separate_sequences():
    cu = [0, 11, 12, 40]
    q, k, v = rand_qkv(40, 4, 2, 8, seed=5)
    sl = alibi_slopes(4)
    packed = oracle.attention_varlen(q, k, v, cu, 0.3, sl)
    for a, b in zip(cu[:-1], cu[1:]):
        alone = oracle.attention_varlen(q[a:b], k[a:b], v[a:b], [0, b - a], 0.3, sl)
        np.testing.assert_array_equal(packed[a:b], alone)


def test_gqa_equals_repeated_heads():
    cu = [0, 15, 33]
    q, k, v = rand_qkv(33, 6, 2, 8, seed=6)
    sl = alibi_slopes(6)
    got = oracle.attention_varlen(q, k, v, cu, 0.4, sl)
    rep = oracle.attention_varlen(q, np.repeat(k, 3, axis=1), np.repeat(v, 3, axis=1), cu, 0.4,
                                  sl)
    np.testing.assert_array_equal(got, rep)


def test_lse_closed_form_and_row_subset():
    cu = [0, 6, 19]
    q, k, v = rand_qkv(19, 2, 2, 4, seed=7)
    _, lse = oracle.attention_varlen(np.zeros_like(q), k, v, cu, 1.0, None, return_lse=True)
    for a, b in zip(cu[:-1], cu[1:]):
        np.testing.assert_allclose(lse[:, a:b], math.log(b - a), rtol=1e-14)
    full, lf = oracle.attention_varlen(q, k, v, cu, 0.5, [0.3, 0.1], return_lse=True)
    rows = np.array([0, 5, 6, 18])
    sub, ls = oracle.attention_varlen(q, k, v, cu, 0.5, [0.3, 0.1], rows=rows, return_lse=True)
    np.testing.assert_array_equal(sub[rows], full[rows])
    np.testing.assert_array_equal(ls[:, rows], lf[:, rows])
    assert np.isnan(sub[1]).all()


def test_alibi_slopes_closed_form():
    assert alibi_slopes(8) == [2.0 ** -(i + 1) for i in range(8)]
    s12 = alibi_slopes(12)
    assert s12[:8] == [2.0 ** -(i + 1) for i in range(8)]
    np.testing.assert_allclose(s12[8:], [2.0 ** -0.5, 2.0 ** -1.5, 2.0 ** -2.5, 2.0 ** -3.5],
                               rtol=1e-15)


# ---- C ABI argument checks (no GPU work) ---------------------------------------

def attn_shape(**kw):
    base = dict(n_seqs=2, max_seqlen=100, total_tokens=200, n_heads=12, n_kv_heads=12,
                head_dim=64, reserved=0, q_token_stride=768, q_head_stride=64,
                k_token_stride=768, k_head_stride=64, v_token_stride=768, v_head_stride=64,
                o_token_stride=768, o_head_stride=64)
    base.update(kw)
    return _lib.AttnShape(**base)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(head_dim=128), 2, "head_dim"),
    (dict(n_kv_heads=5), 1, "divide"),
    (dict(n_kv_heads=0), 1, "divide"),
    (dict(reserved=3), 1, "reserved"),
    (dict(n_seqs=-1), 1, ">= 0"),
    (dict(q_token_stride=770), 2, "multiple of 8"),
    (dict(v_head_stride=-64), 2, "multiple of 8"),
    (dict(n_heads=70000, n_kv_heads=70000), 2, "65535"),
    (dict(total_tokens=2 ** 31), 2, "int32"),
])
def test_attn_invalid_shapes_rejected(g5lib, kw, code, msg):
    s = attn_shape(**kw)
    st = g5lib.g5moe_attn_varlen_fwd(None, None, None, None, None, None, ctypes.c_float(0.125),
                                     None, None, ctypes.byref(s), None)
    err = g5lib.g5moe_last_error().decode()
    assert st == code and msg in err, (st, err)
    n = ctypes.c_size_t(0)
    assert g5lib.g5moe_attn_workspace_size(ctypes.byref(s), ctypes.byref(n)) == code


def test_attn_null_and_misaligned_pointers_rejected(g5lib):
    s = attn_shape()
    st = g5lib.g5moe_attn_varlen_fwd(None, None, None, None, None, None, ctypes.c_float(0.125),
                                     None, None, ctypes.byref(s), None)
    assert st == 1 and "NULL" in g5lib.g5moe_last_error().decode()
    n = ctypes.c_size_t(0)
    assert g5lib.g5moe_attn_workspace_size(ctypes.byref(s), ctypes.byref(n)) == 0
    assert n.value == 256  # 12 heads x ceil(200 / 64) blocks x 4 bytes, 256-byte aligned
    s_big = attn_shape(total_tokens=36400)
    assert g5lib.g5moe_attn_workspace_size(ctypes.byref(s_big), ctypes.byref(n)) == 0
    assert n.value == (12 * 569 * 4 + 255) // 256 * 256
    p = ctypes.c_void_p(0x1000)
    bad = ctypes.c_void_p(0x1008)
    st = g5lib.g5moe_attn_varlen_fwd(p, p, bad, p, p, None, ctypes.c_float(0.125), None, None,
                                     ctypes.byref(s), None)
    assert st == 2 and "aligned" in g5lib.g5moe_last_error().decode()
    st = g5lib.g5moe_attn_varlen_fwd(p, p, p, p, p, None, ctypes.c_float(float("nan")), None,
                                     None, ctypes.byref(s), None)
    assert st == 1 and "finite" in g5lib.g5moe_last_error().decode()
    # nothing to do: no pointer is touched
    s0 = attn_shape(n_seqs=0)
    assert g5lib.g5moe_attn_varlen_fwd(None, None, None, None, None, None, ctypes.c_float(1.0),
                                       None, None, ctypes.byref(s0), None) == 0


def test_attn_wrappers_refuse_cpu_and_unsupported_modes():
    from genet5_amd import attention
    q = torch.zeros(4, 12, 64, dtype=torch.bfloat16)
    cu = torch.tensor([0, 4], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="GPU only"):
        attention.attn_varlen_fwd(q, q, q, cu, 4, 0.125)
    with pytest.raises(NotImplementedError, match="dropout"):
        attention.flash_attn_varlen_func(q, q, q, cu, cu, 4, 4, dropout_p=0.1)
    with pytest.raises(NotImplementedError, match="causal"):
        attention.flash_attn_varlen_func(q, q, q, cu, cu, 4, 4, causal=True)
    with pytest.raises(NotImplementedError, match="head_dim"):
        attention.FlashAttention(attention.FlashAttentionConfig(embed_dim=768, num_heads=6))
