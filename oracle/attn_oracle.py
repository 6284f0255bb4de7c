"""CPU restatement of varlen bidirectional ALiBi attention — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, as the checker.

attention_varlen(q, k, v, cu_seqlens, softmax_scale, alibi_slopes, rows, return_lse)
    For every sequence s of the packed batch (tokens cu_seqlens[s] ..
    cu_seqlens[s+1]) and query head h:
        out[t, h] = sum_j softmax_j(q[t, h] . k[j, h'] * scale - slope_h * |i - j|) v[j, h']
    over the keys j of the same sequence, i and j sequence-local positions,
    h' = h // (H // Hkv), in float64.  This is flash_attn_varlen_func as
    GeneT5's FlashAttention.forward calls it (lib/blocks/_flash_att.py:76-88:
    cu_seqlens_q = cu_seqlens_k, causal=False, softmax_scale =
    1/sqrt(head_dim) at :52), with flash-attn's alibi_slopes bias, which for
    non-causal self-attention is -slope * |i + seqlen_k - seqlen_q - j| =
    -slope * |i - j|.  `rows` restricts the computation to some query tokens
    (global indices), for large inputs.  lse = log sum_j exp(score) per (h, t).
    Pins (tests/test_oracle_attention.py): torch's scaled_dot_product_attention
    in float64 with the explicit bias as attn_mask, per sequence (a library
    routine); zero queries and zero slopes give the mean of v over the
    sequence (closed form); zero queries with a slope give the closed-form
    weights e^{-s|i-j|} / sum_j e^{-s|i-j|}; a dominant key returns its value
    row; packing sequences equals running them one by one; GQA equals repeating
    the key/value heads; lse equals the closed form log sum exp on a case with
    known scores.
"""
from __future__ import annotations

from typing import Optional, Sequence

import numpy as np


def attention_varlen(q: np.ndarray, k: np.ndarray, v: np.ndarray, cu_seqlens: Sequence[int],
                     softmax_scale: float, alibi_slopes: Optional[Sequence[float]] = None,
                     rows: Optional[np.ndarray] = None, return_lse: bool = False):
    """q [T, H, D], k/v [T, Hkv, D] (any float dtype) -> out [T, H, D] float64
    (rows not in `rows` are NaN), and lse [H, T] float64 when return_lse."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    T, H, D = q.shape
    Hkv = k.shape[1]
    if H % Hkv:
        raise ValueError("Hkv must divide H")
    g = H // Hkv
    cu = [int(c) for c in cu_seqlens]
    slopes = np.zeros(H) if alibi_slopes is None else np.asarray(alibi_slopes, np.float64)
    want = np.ones(T, bool) if rows is None else np.isin(np.arange(T), np.asarray(rows))
    out = np.full((T, H, D), np.nan)
    lse = np.full((H, T), np.nan)
    for s in range(len(cu) - 1):
        a, b = cu[s], cu[s + 1]
        if b <= a:
            continue
        qi = np.nonzero(want[a:b])[0]  # sequence-local query positions
        if qi.size == 0:
            continue
        kj = np.arange(b - a)
        dist = np.abs(qi[:, None] - kj[None, :]).astype(np.float64)
        for h in range(H):
            hk = h // g
            sc = (q[a + qi, h] @ k[a:b, hk].T) * softmax_scale - slopes[h] * dist
            mx = sc.max(axis=1, keepdims=True)
            e = np.exp(sc - mx)
            den = e.sum(axis=1, keepdims=True)
            out[a + qi, h] = (e @ v[a:b, hk]) / den
            lse[h, a + qi] = (mx + np.log(den))[:, 0]
    return (out, lse) if return_lse else out
